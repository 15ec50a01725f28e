"""GPU: the self-play rollout collector (BASELINE C4 sequence) end to end.

The pieces are each checked against the reference elsewhere (physics, observation/reward, policy
step, GAE); here the wiring: every buffer row is what the step that wrote it consumed.
  * b_act / b_logp are the draws of the policy evaluated on b_obs[t] at counter step t
    (re-evaluated from the stored normalised observations, draws checked by the CPU checker);
  * the controls sent to the physics are action_to_env of the last draws;
  * b_done[t] is the done flag entering step t; adv/ret are GAE of the buffers (float32 checker);
  * two collectors from the same seeds produce identical buffers.
"""
import importlib.util
import os

import numpy as np
import pytest
import torch

from conftest import ROOT, import_pkg
from test_policy import _ref_forward, oracle_sample

_spec = importlib.util.spec_from_file_location("gae_oracle", os.path.join(ROOT, "oracle", "gae_oracle.py"))
GO = importlib.util.module_from_spec(_spec)
_spec.loader.exec_module(GO)

pytestmark = pytest.mark.gpu


def _collector(gpu, nenv=256, T=12, seed=3, env_kw=None, **kw):
    E = import_pkg("rl_env").GpuDogfightVecEnv
    P = import_pkg("policy")
    R = import_pkg("ppo")
    env = E(nenv, seed=seed, ic_pool_size=64, **(env_kw or {}))
    net = P.MLPActorCritic(184, init="normal", generator=torch.Generator().manual_seed(seed)).to(gpu)
    ro = R.SelfPlayRollout(env, net, T=T, gamma=0.99, lam=0.95, seed=0, **kw)
    ro.reset(stagger=True, max_stagger_steps=8)
    return ro


def _check_against_reference(net, nobs, logits, value, rows=None):
    """Logits and values of stored rows against the float64 evaluation of the same network with
    the kernel's bf16 roundings (the policy test's tolerance: 5e-3 x max(1, std), 99 % within
    1e-4 x that scale)."""
    x = nobs.cpu().numpy() if rows is None else nobs[rows].cpu().numpy()
    ref_l, ref_v = _ref_forward(net, x)
    for got, ref in ((logits, ref_l), (value, ref_v)):
        got = got.cpu().numpy() if rows is None else got[rows].cpu().numpy()
        scale = max(1.0, float(np.std(ref)))
        err = np.abs(got - ref)
        assert err.max() < 5e-3 * scale
        assert np.quantile(err, 0.99) < 1e-4 * scale


def test_rollout_buffers_consistent(gpu, orc):
    ro = _collector(gpu)
    T, nac, nenv = ro.T, ro.nac, ro.nenv
    g0 = ro.global_step
    adv, ret, stats = ro.collect()
    torch.cuda.synchronize()
    assert bool(stats["trajectory_finite"])
    P = import_pkg("policy")
    step = P.PolicyStep(184, device=gpu, seed=0)
    for t in range(T):
        lg = torch.empty(nac, 84, dtype=torch.float32, device=gpu)
        v = torch.empty(nac, dtype=torch.float32, device=gpu)
        step(ro.b_obs[t], [(ro.net, 0, nac)], norm=None, logits_out=lg, value=v)
        assert torch.equal(v, ro.b_val[t]), t
        _check_against_reference(ro.net, ro.b_obs[t], lg, ro.b_val[t])
        idx, lp = oracle_sample(orc, lg.cpu().numpy(), np.arange(nac), seed=0, step=g0 + t)
        np.testing.assert_array_equal(ro.b_act[t].cpu().numpy(), idx)
        assert np.abs(ro.b_logp[t].cpu().numpy() - lp).max() < 1e-5
    last = P.action_to_env(ro.b_act[T - 1].cpu(), 21).double()
    np.testing.assert_array_equal(ro.env.sim.actions.cpu().numpy(), last.numpy())
    # normalised observations are clipped to +-10
    assert float(ro.b_obs.abs().max()) <= 10.0
    # GAE of the buffers, (T, nac) columns with the done flag shared by the 2 planes
    ref_adv, ref_ret = GO.gae_f32(ro.b_rew.cpu().numpy(), ro.b_val.cpu().numpy(),
                                  ro.b_done.cpu().numpy(), ro.last_val.cpu().numpy(),
                                  ro.next_done.cpu().numpy(), 0.99, 0.95, nagents=2)
    np.testing.assert_array_equal(adv.reshape(T, nac).cpu().numpy(), ref_adv)
    np.testing.assert_array_equal(ret.reshape(T, nac).cpu().numpy(), ref_ret)


def test_rollout_deterministic(gpu):
    a, b = _collector(gpu, nenv=128, T=6), _collector(gpu, nenv=128, T=6)
    ra, rb = a.collect(), b.collect()
    for name in ("b_obs", "b_act", "b_logp", "b_rew", "b_val", "b_done"):
        assert torch.equal(getattr(a, name), getattr(b, name)), name
    assert torch.equal(ra[0], rb[0]) and torch.equal(ra[1], rb[1])


BUFFERS = ("b_obs", "b_act", "b_logp", "b_rew", "b_val", "b_done", "last_val", "next_done",
           "finite_acc")


def _same_rollouts(a, b, n=4, refresh_at=2, outside_at=None):
    """n rollouts of the eager collector `a` and the graph collector `b`, with host work and
    synchronisation between replays; every buffer, the GAE outputs and the env state agree bit
    for bit after each one.  Before rollout `refresh_at` both networks' weights change and are
    re-packed (the graph picks up the refreshed blobs).  Before rollout `outside_at` both envs
    take three steps outside the collectors (an evaluation on the same env), which advance the
    envs' draw counters on the host only; the next replay must continue from them."""
    for r in range(n):
        if r == outside_at:
            act = torch.zeros(a.env.nac, 4, dtype=torch.float64, device=a.device)
            act[:, 3] = 0.7
            for ro in (a, b):
                for _ in range(3):
                    ro.env.step(act)
        if r == refresh_at:
            for ro in (a, b):
                with torch.no_grad():
                    for prm in ro.net.parameters():
                        prm.mul_(0.9)
                ro.net.pack()
        ra, rb = a.collect(), b.collect()
        torch.cuda.synchronize()
        x = torch.arange(1000, device=a.device).sum().item()      # eager work between replays
        assert x == 499500
        for name in BUFFERS:
            assert torch.equal(getattr(a, name), getattr(b, name)), (r, name)
        assert torch.equal(ra[0], rb[0]) and torch.equal(ra[1], rb[1]), r
        assert bool(ra[2]["trajectory_finite"]) == bool(rb[2]["trajectory_finite"])
        assert torch.equal(a.env.sim._state_soa, b.env.sim._state_soa), r
        assert a.global_step == b.global_step and a.env._post_steps == b.env._post_steps


def test_graph_rollout_equals_eager(gpu):
    """SelfPlayRollout(graph=True) records the rollout once as a HIP graph and replays it; its
    draws' counters advance on the device.  Four rollouts match the eager collector's."""
    a = _collector(gpu, nenv=512, T=8, stats=False)
    b = _collector(gpu, nenv=512, T=8, stats=False, graph=True)
    _same_rollouts(a, b)


def test_graph_rollout_after_outside_env_steps(gpu):
    """Env steps taken between two replays (outside the graph) move the replay's draw counters
    on as they move the eager collector's: the device counters are refilled from the host's
    before every replay."""
    a = _collector(gpu, nenv=256, T=6, stats=False)
    b = _collector(gpu, nenv=256, T=6, stats=False, graph=True)
    _same_rollouts(a, b, n=4, refresh_at=None, outside_at=3)


def test_graph_league_rollout_equals_eager(gpu):
    E = import_pkg("rl_env").GpuDogfightVecEnv
    P = import_pkg("policy")
    R = import_pkg("ppo")

    def make(graph):
        env = E(256, seed=5, obs_dim=214, ic_pool_size=64, fuel_exhaustion=True,
                fuel_lbs_range=(0.0, 3.0))
        mk = lambda s: P.MLPActorCritic(214, init="normal",
                                        generator=torch.Generator().manual_seed(s)).to(gpu)
        ro = R.LeagueRollout(env, mk(1), [mk(60 + k) for k in range(3)], T=6, seed=0, graph=graph)
        ro.reset(stagger=False)
        return ro
    a, b = make(False), make(True)
    _same_rollouts(a, b)
    assert a.b_done.sum().item() > 0          # autoresets and opponent redraws happened


@pytest.mark.parametrize("nenv,graph", [(200, False), (512, True)])
def test_fused_norm_partials_equal_separate_update(gpu, nenv, graph):
    """The post-physics launch forming the RunningNorm partial sums of the rows the next step
    normalises (then only the merge runs) gives the same statistics and buffers, bit for bit, as
    a separate f16_norm_update per step: over three rollouts with autoresets, a ragged last
    128-row block (nenv 200) and the fused collector recorded as a HIP graph."""
    short = {"max_engage_time_s": 1.5}          # every engagement ends within 15 decisions
    a = _collector(gpu, nenv=nenv, T=8, stats=False, fuse_norm=False, env_kw=short)
    b = _collector(gpu, nenv=nenv, T=8, stats=False, graph=graph, fuse_norm=True, env_kw=short)
    assert not a.fuse_norm and b.fuse_norm
    done = 0.0
    for r in range(3):
        ra, rb = a.collect(), b.collect()
        torch.cuda.synchronize()
        for name in BUFFERS:
            assert torch.equal(getattr(a, name), getattr(b, name)), (r, name)
        assert torch.equal(ra[0], rb[0]) and torch.equal(ra[1], rb[1]), r
        for name in ("mean", "var", "count"):
            assert torch.equal(getattr(a.norm, name), getattr(b.norm, name)), (r, name)
        done += a.b_done.sum().item()
    assert done > 0                            # rows rebuilt from the pool were in the sums


def test_full_c4_rollout(gpu, orc):
    """BASELINE C4 at its stated size: 16,384 engagements x 64 steps, the episode clocks
    staggered over the 200 s limit so engagements end inside the window.  GAE of the whole
    buffer bit-exact against the float32 checker; on a 1,024-row sample of every 8th step, the
    stored values and the logits of the stored observations against the float64 reference
    evaluation and the stored draws against the draw checker."""
    ro = _collector(gpu, nenv=16384, T=64, seed=11)
    ro.reset(stagger=True, max_stagger_steps=2000)
    T, nac = ro.T, ro.nac
    g0 = ro.global_step
    adv, ret, stats = ro.collect()
    torch.cuda.synchronize()
    assert bool(stats["trajectory_finite"])
    assert float(ro.b_done[1:].sum()) + float(ro.next_done.sum()) > 0     # autoresets happened
    ref_adv, ref_ret = GO.gae_f32(ro.b_rew.cpu().numpy(), ro.b_val.cpu().numpy(),
                                  ro.b_done.cpu().numpy(), ro.last_val.cpu().numpy(),
                                  ro.next_done.cpu().numpy(), 0.99, 0.95, nagents=2)
    np.testing.assert_array_equal(adv.reshape(T, nac).cpu().numpy(), ref_adv)
    np.testing.assert_array_equal(ret.reshape(T, nac).cpu().numpy(), ref_ret)
    P = import_pkg("policy")
    step = P.PolicyStep(184, device=gpu, seed=0)
    rows = np.sort(np.random.default_rng(7).choice(nac, 1024, replace=False))
    rows_t = torch.as_tensor(rows, device=gpu)
    for t in range(0, T, 8):
        lg = torch.empty(nac, 84, dtype=torch.float32, device=gpu)
        v = torch.empty(nac, dtype=torch.float32, device=gpu)
        step(ro.b_obs[t], [(ro.net, 0, nac)], norm=None, logits_out=lg, value=v)
        assert torch.equal(v[rows_t], ro.b_val[t][rows_t]), t
        _check_against_reference(ro.net, ro.b_obs[t], lg, ro.b_val[t], rows_t)
        idx, lp = oracle_sample(orc, lg[rows_t].cpu().numpy(), rows, seed=0, step=g0 + t)
        np.testing.assert_array_equal(ro.b_act[t][rows_t].cpu().numpy(), idx)
        assert np.abs(ro.b_logp[t][rows_t].cpu().numpy() - lp).max() < 1e-5
    assert float(ro.b_obs.abs().max()) <= 10.0
