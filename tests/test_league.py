"""League workload (BASELINE C5): device-side grouping of the opponents' rows, the grouped
policy launch with device row ranges and per-network normalisation, the opponent redraw and the
fuel-exhaustion termination inside the post-physics step, and the LeagueRollout wiring.

Exact checks: the grouping is numpy's stable argsort; grouped launches equal per-network
launches bit for bit; redrawn opponents follow Philox + the weights' CDF; fuel-exhaustion flags
are the oracle's flags OR'd with the fuel rule; GAE of the buffers is the float32 checker's."""
import importlib.util
import os

import numpy as np
import pytest
import torch

import oracle_lib
from conftest import ROOT, import_pkg
from test_policy import oracle_sample, philox
from test_rollout import _check_against_reference

_spec = importlib.util.spec_from_file_location("gae_oracle", os.path.join(ROOT, "oracle", "gae_oracle.py"))
GO = importlib.util.module_from_spec(_spec)
_spec.loader.exec_module(GO)


def test_zipf_weights():
    w = import_pkg("ppo").zipf_weights(8, 1.1)
    assert abs(sum(w) - 1.0) < 1e-12
    for k in range(1, 8):
        assert abs(w[k] / w[0] - (k + 1) ** -1.1) < 1e-12


@pytest.mark.gpu
@pytest.mark.parametrize("n,ng", [(65536, 8), (70001, 5), (1000, 3), (5, 16), (0, 2),
                                  (1000003, 16)])
def test_group_rows_is_stable_sort(gpu, n, ng):
    L = import_pkg("_lib")
    rng = np.random.default_rng(n + ng)
    a = rng.integers(0, ng, n).astype(np.int32)
    if n > 10:
        a[::97] = ng + 3                                   # ids out of range are dropped
    rows = torch.full((max(n, 1),), -1, dtype=torch.int32, device=gpu)
    offs = torch.full((ng + 1,), -1, dtype=torch.int32, device=gpu)
    at = torch.as_tensor(a, device=gpu)
    work = torch.empty(max(8, L.lib().f16_group_workspace_bytes(n)), dtype=torch.uint8,
                       device=gpu)
    rc = L.lib().f16_group_rows(L.ptr(at) if n else None, n, ng, 2, 1, L.ptr(rows), L.ptr(offs),
                                L.ptr(work), L.stream_handle(gpu))
    L.check(rc, "f16_group_rows")
    valid = a < ng
    order = np.argsort(np.where(valid, a, ng), kind="stable")[:int(valid.sum())]
    ref_rows = 2 * order + 1
    ref_offs = np.concatenate([[0], np.cumsum(np.bincount(a[valid], minlength=ng))])
    np.testing.assert_array_equal(offs.cpu().numpy(), ref_offs)
    np.testing.assert_array_equal(rows.cpu().numpy()[:len(ref_rows)], ref_rows)


def _nets(P, k, dim, gpu, seed):
    return [P.MLPActorCritic(dim, init="normal", generator=torch.Generator().manual_seed(seed + i)).to(gpu)
            for i in range(k)]


@pytest.mark.gpu
@pytest.mark.parametrize("packed,empty", [(True, False), (False, False), (True, True)])
def test_grouped_launch_with_device_offsets(gpu, orc, packed, empty):
    """One launch over rows grouped on the device equals one launch per network, each with its
    own normalisation statistics: with the groups' tiles packed into one grid dimension and with
    one grid row per group, and with a group that gets no rows (empty=True: ids avoid group 2)."""
    P = import_pkg("policy")
    L = import_pkg("_lib")
    nenv, ng, D = 3000, 5, 214
    nets = _nets(P, ng, D, gpu, 40)
    norms = []
    rng = np.random.default_rng(41)
    for _ in range(ng):
        nm = P.RunningNorm(D, gpu)
        nm.mean.copy_(torch.as_tensor(rng.normal(0, 0.3, D).astype(np.float32)))
        nm.var.copy_(torch.as_tensor(rng.uniform(0.5, 2.0, D).astype(np.float32)))
        norms.append(nm)
    obs = torch.as_tensor(rng.normal(0, 1, (2 * nenv, D)).astype(np.float32), device=gpu)
    ids = rng.integers(0, ng, nenv).astype(np.int32)
    if empty:
        ids[ids == 2] = 3
    assign = torch.as_tensor(ids, device=gpu)
    rows = torch.empty(nenv, dtype=torch.int32, device=gpu)
    offs = torch.empty(ng + 1, dtype=torch.int32, device=gpu)
    work = torch.empty(max(8, L.lib().f16_group_workspace_bytes(nenv)), dtype=torch.uint8,
                       device=gpu)
    L.check(L.lib().f16_group_rows(L.ptr(assign), nenv, ng, 2, 1, L.ptr(rows), L.ptr(offs),
                                   L.ptr(work), L.stream_handle(gpu)), "f16_group_rows")
    step = P.PolicyStep(D, device=gpu, seed=9)
    acts = torch.zeros(2 * nenv, 4, dtype=torch.float64, device=gpu)
    lg = torch.empty(nenv, 84, dtype=torch.float32, device=gpu)
    step(obs, [(n, None, None, nm) for n, nm in zip(nets, norms)], rows=rows,
         group_offsets=offs, max_group_rows=nenv, nphys=2 * nenv, step=3, salt=1,
         env_actions=acts, logits_out=lg, packed=packed)
    o = offs.cpu().numpy()
    assert (o[3] - o[2] == 0) == empty
    r = rows.cpu().numpy()
    for g in range(ng):
        if o[g + 1] == o[g]:
            continue
        sub = obs[rows[o[g]:o[g + 1]].long()].contiguous()
        lg2 = torch.empty(o[g + 1] - o[g], 84, dtype=torch.float32, device=gpu)
        step(sub, [(nets[g], 0, o[g + 1] - o[g])], norm=norms[g], logits_out=lg2)
        torch.testing.assert_close(lg[o[g]:o[g + 1]], lg2, rtol=0, atol=0)
    idx, _ = oracle_sample(orc, lg.cpu().numpy(), r.astype(np.int64), seed=9, step=3, salt=1)
    ref = np.zeros((2 * nenv, 4))
    ref[r] = P.action_to_env(torch.as_tensor(idx), 21).double().numpy()
    np.testing.assert_array_equal(acts.cpu().numpy(), ref)


def _sim_states(gpu, nenv, seed, fuel=None):
    icm = import_pkg("ic")
    rng = np.random.default_rng(seed)
    rows = icm.contest_rows(rng, nenv)
    if fuel is not None:
        rows[:, 9] = fuel
    sim = import_pkg().GpuDogfight(nenv, fcs_rate=60)
    sim.seed_rows(torch.as_tensor(rows, device=gpu))
    return sim


@pytest.mark.gpu
def test_post_step_opponent_redraw_and_fuel_exhaustion(gpu, orc):
    nenv, P_ = 256, 32
    fuel = np.full(2 * nenv, 2000.0)
    fuel[2 * np.arange(0, nenv, 5) + 1] = 0.0          # every 5th engagement's target is empty
    sim = _sim_states(gpu, nenv, 51, fuel)
    pool = _sim_states(gpu, P_, 52).states.reshape(P_, 2, 101).contiguous()
    R = import_pkg("obs_reward")
    L = import_pkg("_lib")
    obr = R.BatchObsReward(nenv)
    obr.t_sec[nenv // 2:].fill_(199.95)                 # the second half also times out
    st0 = sim.states.cpu().numpy()
    ob = oracle_lib.ObrOracle(orc, nenv)
    s9 = ob.state9(st0)
    _, te_o, tr_o = ob.step(s9, np.zeros((2 * nenv, 4)))
    t_sec = np.zeros(nenv); t_sec[nenv // 2:] = 199.95
    fuel_out = (fuel.reshape(nenv, 2) <= 0).any(1)
    te_ref = te_o | fuel_out
    tr_ref = (~te_ref) & (t_sec + 0.1 >= 200.0 - 1e-8)
    cdf = torch.tensor([0.5, 0.8, 1.0], dtype=torch.float32, device=gpu)
    assign = torch.full((nenv,), 7, dtype=torch.int32, device=gpu)
    te, tr, dn = (torch.empty(nenv, dtype=torch.uint8, device=gpu) for _ in range(3))
    obs = torch.zeros(2 * nenv, 184, dtype=torch.float32, device=gpu)
    c = R.reward_cfg_struct(R.MY_REWARD_CONFIG, 304.8, 200.0, 0, 5.0, fuel_exhaustion=True)
    rec = obr._recon()
    seed, step = 77, 5
    io = L.F16EnvStepIO(states=sim._state_soa.data_ptr(), ld=sim.nac,
                        actions=sim.actions.data_ptr(), ic_pool=pool.data_ptr(), pool_size=P_,
                        pick=None, seed=seed, step=step, obs_dim=184, obs=obs.data_ptr(),
                        term=te.data_ptr(), trunc=tr.data_ptr(), done=dn.data_ptr(),
                        opp_assign=assign.data_ptr(), opp_cdf=cdf.data_ptr(), n_opp=3)
    L.check(L.lib().f16_env_post_step(L.ctypes.byref(io), L.ctypes.byref(rec), L.ctypes.byref(c),
                                      L.stream_handle(gpu)), "f16_env_post_step")
    np.testing.assert_array_equal(te.cpu().numpy().astype(bool), te_ref)
    np.testing.assert_array_equal(tr.cpu().numpy().astype(bool), tr_ref)
    done = te_ref | tr_ref
    assert fuel_out.any() and done.any() and (~done).any()
    got = assign.cpu().numpy()
    cdf_np = cdf.cpu().numpy()
    for e in range(nenv):
        if not done[e]:
            assert got[e] == 7
            continue
        x0 = philox(orc, [e, step, 1, 0x0FF0A55E], [seed, 0])[0]
        u = np.float32((x0 >> 8) * 2.0 ** -24)
        assert got[e] == int(np.argmax(cdf_np > u)), e


@pytest.mark.gpu
def test_league_rollout_buffers(gpu, orc):
    P = import_pkg("policy")
    R = import_pkg("ppo")
    E = import_pkg("rl_env").GpuDogfightVecEnv
    nenv, T = 1024, 8
    env = E(nenv, seed=5, obs_dim=214, ic_pool_size=64, fuel_exhaustion=True,
            fuel_lbs_range=(0.0, 3.0))
    net = P.MLPActorCritic(214, init="normal", generator=torch.Generator().manual_seed(1)).to(gpu)
    opps = _nets(P, 8, 214, gpu, 60)                 # BASELINE C5's eight opponent networks
    ro = R.LeagueRollout(env, net, opps, T=T, seed=0)
    ro.reset(stagger=False)
    a0 = env.opp_assign.clone()
    g0 = ro.global_step
    adv, ret, stats = ro.collect()
    torch.cuda.synchronize()
    assert bool(stats["trajectory_finite"])
    step = P.PolicyStep(214, device=gpu, seed=0)
    rows = (2 * np.arange(nenv)).astype(np.int64)
    for t in range(T):
        lg = torch.empty(nenv, 84, dtype=torch.float32, device=gpu)
        v = torch.empty(nenv, dtype=torch.float32, device=gpu)
        step(ro.b_obs[t], [(net, 0, nenv)], norm=None, logits_out=lg, value=v)
        assert torch.equal(v, ro.b_val[t]), t
        _check_against_reference(net, ro.b_obs[t], lg, ro.b_val[t])
        idx, lp = oracle_sample(orc, lg.cpu().numpy(), rows, seed=0, step=g0 + t)
        np.testing.assert_array_equal(ro.b_act[t].cpu().numpy(), idx)
    ref_adv, ref_ret = GO.gae_f32(ro.b_rew.cpu().numpy(), ro.b_val.cpu().numpy(),
                                  ro.b_done.cpu().numpy(), ro.last_val.cpu().numpy(),
                                  ro.next_done.cpu().numpy(), 0.99, 0.95)
    np.testing.assert_array_equal(adv.cpu().numpy(), ref_adv)
    np.testing.assert_array_equal(ret.cpu().numpy(), ref_ret)
    # the low-fuel workload finishes engagements, and their opponents get redrawn
    done_any = ro.b_done[1:].sum().item() + ro.next_done.sum().item()
    assert done_any > 0
    assert not torch.equal(a0, env.opp_assign)
    assert len(np.unique(env.opp_assign.cpu().numpy())) == 8   # every opponent network has rows
    acts = env.sim.actions.cpu().numpy()
    grid = P.make_action_grid(21).double().numpy()
    assert np.isin(acts[1::2, :3], grid).all()           # opponents' controls are grid values


@pytest.mark.gpu
def test_full_c5_league_rollout(gpu, orc):
    """BASELINE C5 at its stated size: 65,536 engagements x 128 steps, 214-D, eight opponent
    networks drawn from Zipf(1.1) weights, fuel exhaustion (the bench's fuel range) so
    engagements end and their opponents are redrawn inside the window.  GAE of the whole buffer
    bit-exact against the float32 checker; on a 1,024-engagement sample of every 16th step, the
    learner's stored values and the logits of its stored observations against the float64
    reference evaluation and its stored draws against the draw checker; every opponent network
    has engagements."""
    P = import_pkg("policy")
    R = import_pkg("ppo")
    E = import_pkg("rl_env").GpuDogfightVecEnv
    nenv, T = 65536, 128
    env = E(nenv, seed=0, obs_dim=214, fuel_exhaustion=True, fuel_lbs_range=(100.0, 3000.0))
    mk = lambda s: P.MLPActorCritic(214, init="normal", init_std=0.02,
                                    generator=torch.Generator().manual_seed(s)).to(gpu)
    net, opps = mk(0), [mk(100 + k) for k in range(8)]
    ro = R.LeagueRollout(env, net, opps, T=T, seed=0)
    ro.reset(stagger=False)
    g0 = ro.global_step
    adv, ret, stats = ro.collect()
    torch.cuda.synchronize()
    assert bool(stats["trajectory_finite"])
    assert float(ro.b_done[1:].sum()) + float(ro.next_done.sum()) > 0
    assert len(np.unique(env.opp_assign.cpu().numpy())) == 8
    ref_adv, ref_ret = GO.gae_f32(ro.b_rew.cpu().numpy(), ro.b_val.cpu().numpy(),
                                  ro.b_done.cpu().numpy(), ro.last_val.cpu().numpy(),
                                  ro.next_done.cpu().numpy(), 0.99, 0.95)
    np.testing.assert_array_equal(adv.cpu().numpy(), ref_adv)
    np.testing.assert_array_equal(ret.cpu().numpy(), ref_ret)
    step = P.PolicyStep(214, device=gpu, seed=0)
    sample = np.sort(np.random.default_rng(8).choice(nenv, 1024, replace=False))
    st = torch.as_tensor(sample, device=gpu)
    for t in range(0, T, 16):
        lg = torch.empty(nenv, 84, dtype=torch.float32, device=gpu)
        v = torch.empty(nenv, dtype=torch.float32, device=gpu)
        step(ro.b_obs[t], [(net, 0, nenv)], norm=None, logits_out=lg, value=v)
        assert torch.equal(v[st], ro.b_val[t][st]), t
        _check_against_reference(net, ro.b_obs[t], lg, ro.b_val[t], st)
        idx, _ = oracle_sample(orc, lg[st].cpu().numpy(), 2 * sample, seed=0, step=g0 + t)
        np.testing.assert_array_equal(ro.b_act[t][st].cpu().numpy(), idx)
