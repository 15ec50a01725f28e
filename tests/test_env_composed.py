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
