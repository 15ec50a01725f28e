"""GPU: GpuDogfightVecEnv.step chained over many decisions at BASELINE C3/C4 size, each decision
replayed on the CPU restatement from the GPU's own state (the reference's step sequence,
research/competition_36500/runtime/cuda_fdm/rl_env.py:499-580: FDM decision -> advance ->
termination -> terminal observation -> pool autoreset -> reset_envs -> init_reward -> masked
build_obs).

Per decision: the physics of live engagements within 1e-10 relative per state variable, the
autoreset rows equal to their pool rows bit for bit, observations (live and terminal) within
1e-5, rewards and reconstructor doubles within 1e-8, termination / truncation / done flags
exact.  A short engagement time limit (the staggered reset spreads episode clocks over
0-12.8 s, the limit is 12 s) makes truncations and autoresets happen inside the window, on top
of the damage, HP and hard-deck terminations random manoeuvring produces.
"""
import numpy as np
import pytest
import torch

import oracle_lib
from conftest import import_pkg
from test_obs_gpu import OBS_TOL, VAL_TOL, _cmp_recon, _to_oracle

pytestmark = pytest.mark.gpu


def _bin_actions(rng, n):
    """Uniform 21-bin draws per channel through action_to_env (R/cuda_fdm/ppo_gpu.py:361-370)."""
    grid = np.linspace(-1.0, 1.0, 21)
    z = grid[rng.integers(0, 21, size=(n, 4))]
    z[:, 3] = 0.5 * z[:, 3] + 0.5
    return z


@pytest.mark.parametrize("obs_dim,nenv,ndec", [(184, 16384, 24), (214, 4096, 20)])
def test_env_step_chain_matches_oracle(gpu, orc, obs_dim, nenv, ndec, worst):
    E = import_pkg("rl_env").GpuDogfightVecEnv
    env = E(nenv, seed=5, ic_pool_size=256, obs_dim=obs_dim, max_engage_time_s=12.0)
    env.reset(stagger=True, max_stagger_steps=128)
    ext = obs_dim == 214
    rng = np.random.default_rng(17)
    pool = env.ic_pool.cpu().numpy()
    n = 2 * nenv
    seen = dict(done=0, trunc=0, term=0)
    for d in range(ndec):
        st0 = np.ascontiguousarray(env.sim.states.cpu().numpy())
        ob = _to_oracle(env.obr, orc, ext)
        act = _bin_actions(rng, n)
        pick = rng.integers(0, pool.shape[0], nenv)
        obs, rew, done, info = env.step(torch.as_tensor(act, device=gpu),
                                        reset_indices=torch.as_tensor(pick, device=gpu))
        # the reference's sequence on the oracle, from the GPU's pre-step state
        st1 = st0.copy()
        orc.step(st1, act, env.substeps, 60, want_obs=False)
        s9 = ob.state9(st1)
        r_o, te_o, tr_o = ob.step(s9, act, max_time=env.max_engage_time_s)
        tobs_o = ob.build_obs(s9, obs_dim)
        done_o = te_o | tr_o
        st2 = st1.copy()
        for e in np.nonzero(done_o)[0]:
            st2[2 * e:2 * e + 2] = pool[pick[e]]
        ob.reset_envs(done_o)
        s9r = ob.state9(st2)
        ob.init_reward(s9r, done_o)
        rows = np.repeat(done_o, 2)
        obs_o = tobs_o.copy()
        obs_o[rows] = ob.build_obs(s9r, obs_dim)[rows]
        # flags exact
        np.testing.assert_array_equal(info["terminated"].cpu().numpy(), te_o, err_msg=str(d))
        np.testing.assert_array_equal(info["truncated"].cpu().numpy(), tr_o, err_msg=str(d))
        np.testing.assert_array_equal(done.cpu().numpy(), done_o, err_msg=str(d))
        # physics: live rows per step, autoreset rows exactly the pool's
        got = env.sim.states.cpu().numpy()
        live = ~rows
        e_obs = np.abs(obs.reshape(n, obs_dim).cpu().numpy() - obs_o).max()
        worst(f"env chain {obs_dim}, state rel_err", oracle_lib.rel_err(got[live], st1[live]).max(),
              1e-10)
        worst(f"env chain {obs_dim}, reward |err|", np.abs(rew.reshape(n).cpu().numpy() - r_o).max(),
              VAL_TOL)
        worst(f"env chain {obs_dim}, observation |err|", e_obs, OBS_TOL)
        assert oracle_lib.rel_err(got[live], st1[live]).max() <= 1e-10, d
        np.testing.assert_array_equal(got[rows], st2[rows], err_msg=str(d))
        # observation, terminal observation, reward, reconstructor
        assert np.abs(rew.reshape(n).cpu().numpy() - r_o).max() <= VAL_TOL, d
        assert np.abs(info["terminal_obs"].reshape(n, obs_dim).cpu().numpy()
                      - tobs_o).max() <= OBS_TOL, d
        assert np.abs(obs.reshape(n, obs_dim).cpu().numpy() - obs_o).max() <= OBS_TOL, d
        _cmp_recon(env.obr, ob, ext)
        seen["done"] += int(done_o.sum())
        seen["trunc"] += int(tr_o.sum())
        seen["term"] += int(te_o.sum())
    # the window must have exercised autoresets of both kinds
    assert seen["trunc"] > 0 and seen["term"] > 0, seen


def test_env_step_chain_c5_league(gpu, orc, worst):
    """BASELINE C5's env path chained against the oracle: 65,536 engagements, 214-D (two launches:
    the physics, then the post-physics step with the vector-block tile), fuel exhaustion on
    (low-fuel initial conditions, so some engagements run dry inside the window; a 4.5 s limit on
    clocks staggered over 0-4 s truncates others), 8 opponents assigned
    from Zipf(1.1) weights and redrawn at autoreset, over 10 decisions each stepped from the
    GPU's own state.  Live states <= 1e-10 per variable, autoreset rows the pool's bit for bit,
    observations <= 1e-5, rewards and reconstructor <= 1e-8, termination / truncation / done
    exact, every redrawn opponent the Philox draw through the weights' CDF (the CPU reference's
    Philox4x32-10), every other assignment unchanged.  Fuel exhaustion is not in the reference
    model's reward path: a dry engagement terminates with no terminal reward, so where the
    oracle (without it) truncates such an engagement its timeout reward is taken off."""
    from test_policy import philox
    E, R = import_pkg("rl_env").GpuDogfightVecEnv, import_pkg("ppo")
    nenv, ndec, obs_dim = 65536, 10, 214
    env = E(nenv, seed=8, ic_pool_size=512, obs_dim=obs_dim, max_engage_time_s=4.5,
            fuel_exhaustion=True, fuel_lbs_range=(1.0, 400.0))
    env.reset(stagger=True, max_stagger_steps=40)
    w = R.zipf_weights(8)
    cdf = np.cumsum(w) / np.sum(w)
    cdf[-1] = 1.0
    env.opp_cdf = torch.tensor(cdf, dtype=torch.float32, device=gpu)
    env.opp_assign = torch.as_tensor(np.random.default_rng(3).integers(0, 8, nenv),
                                     dtype=torch.int32, device=gpu)
    assert not env.norm_fusable()                      # beyond the full-row tile: two launches
    cdf32 = env.opp_cdf.cpu().numpy()
    rng = np.random.default_rng(18)
    pool = env.ic_pool.cpu().numpy()
    n = 2 * nenv
    seen = dict(done=0, trunc=0, term=0, dry=0)
    for d in range(ndec):
        st0 = np.ascontiguousarray(env.sim.states.cpu().numpy())
        ob = _to_oracle(env.obr, orc, True)
        assign0 = env.opp_assign.cpu().numpy()
        step_id = env._post_steps & 0xffffffff
        act = _bin_actions(rng, n)
        pick = rng.integers(0, pool.shape[0], nenv)
        obs, rew, done, info = env.step(torch.as_tensor(act, device=gpu),
                                        reset_indices=torch.as_tensor(pick, device=gpu))
        st1 = st0.copy()
        orc.step(st1, act, env.substeps, 60, want_obs=False, nthreads=0)
        s9 = ob.state9(st1)
        r_o, te_o, tr_o = ob.step(s9, act, max_time=env.max_engage_time_s)
        dry = (st1[:, 14].reshape(nenv, 2) <= 0.0).any(1)
        te_ref = te_o | dry
        tr_ref = tr_o & ~dry
        done_o = te_ref | tr_ref
        # a dry engagement the oracle truncates loses the oracle's timeout reward
        fix = np.repeat(dry & tr_o & ~te_o, 2)
        hp = ob.hp.reshape(nenv, 2)
        hp_t = hp[:, ::-1].reshape(-1)
        timeout = np.where(ob.hp > hp_t, 5.0, np.where(ob.hp < hp_t, -5.0, -4.0))
        r_ref = np.where(fix, r_o - timeout, r_o)
        tobs_o = ob.build_obs(s9, obs_dim)
        st2 = st1.copy()
        for e in np.nonzero(done_o)[0]:
            st2[2 * e:2 * e + 2] = pool[pick[e]]
        ob.reset_envs(done_o)
        s9r = ob.state9(st2)
        ob.init_reward(s9r, done_o)
        rows = np.repeat(done_o, 2)
        obs_o = tobs_o.copy()
        obs_o[rows] = ob.build_obs(s9r, obs_dim)[rows]
        np.testing.assert_array_equal(info["terminated"].cpu().numpy(), te_ref, err_msg=str(d))
        np.testing.assert_array_equal(info["truncated"].cpu().numpy(), tr_ref, err_msg=str(d))
        np.testing.assert_array_equal(done.cpu().numpy(), done_o, err_msg=str(d))
        got = env.sim.states.cpu().numpy()
        live = ~rows
        e_state = oracle_lib.rel_err(got[live], st1[live]).max()
        e_rew = np.abs(rew.reshape(n).cpu().numpy() - r_ref).max()
        e_obs = np.abs(obs.reshape(n, obs_dim).cpu().numpy() - obs_o).max()
        worst("env chain C5 214, state rel_err", e_state, 1e-10)
        worst("env chain C5 214, reward |err|", e_rew, VAL_TOL)
        worst("env chain C5 214, observation |err|", e_obs, OBS_TOL)
        assert e_state <= 1e-10, d
        np.testing.assert_array_equal(got[rows], st2[rows], err_msg=str(d))
        assert e_rew <= VAL_TOL, d
        assert np.abs(info["terminal_obs"].reshape(n, obs_dim).cpu().numpy()
                      - tobs_o).max() <= OBS_TOL, d
        assert e_obs <= OBS_TOL, d
        _cmp_recon(env.obr, ob, True)
        # opponents: redrawn exactly where the engagement ended
        assign1 = env.opp_assign.cpu().numpy()
        np.testing.assert_array_equal(assign1[~done_o], assign0[~done_o], err_msg=str(d))
        for e in np.nonzero(done_o)[0]:
            x0 = philox(orc, [int(e), step_id, 1, 0x0FF0A55E], [env.seed, 0])[0]
            u = np.float32((x0 >> 8) * 2.0 ** -24)
            assert assign1[e] == int(np.argmax(cdf32 > u)), (d, e)
        seen["done"] += int(done_o.sum())
        seen["trunc"] += int(tr_ref.sum())
        seen["term"] += int(te_ref.sum())
        seen["dry"] += int((dry & ~te_o).sum())
    assert seen["trunc"] > 0 and seen["term"] > 0 and seen["dry"] > 0, seen
