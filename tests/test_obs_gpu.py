"""GPU parity of the observation / reward / termination kernels and of the fused post-physics
environment step (include/f16_obs.h, through the C ABI) against the CPU restatement of the
reference (oracle/obs_oracle.c, itself pinned to the reference's torch path by
tests/golden/obs_golden.npz) and against those golden vectors directly.

Tolerances (observations and rewards within 1e-5, termination flags
bit-exact): observations <= 1e-5 absolute (float32 outputs of unit-scale features); rewards
and reconstructor doubles <= 1e-8 absolute (the GPU and host transcendentals differ by an ulp,
which the geometry score's smoothsteps amplify by at most ~1e3); flags, action history, time,
autoreset state rows: exact.
"""
import numpy as np
import pytest
import torch

import oracle_lib
from conftest import import_pkg

pytestmark = pytest.mark.gpu
OBS_TOL = 1e-5
VAL_TOL = 1e-8
FT2M = 0.3048


def _obr(nenv, ext=False):
    obr = import_pkg("obs_reward").BatchObsReward(nenv)
    if ext:
        obr.enable_external_observations()
    return obr


def _to_oracle(obr, orc, ext=False):
    """An oracle reconstructor holding a copy of the GPU reconstructor's state."""
    ob = oracle_lib.ObrOracle(orc, obr.nenv, accel=ext)
    c = lambda t: t.detach().cpu().numpy()
    ob.hp[:] = c(obr.hp); ob.fuel[:] = c(obr.fuel); ob.t_sec[:] = c(obr.t_sec)
    ob.prev_att[:] = c(obr.prev_att); ob.prev_valid[:] = c(obr.prev_valid)
    ob.pqr[:] = c(obr.pqr); ob.dealt[:] = c(obr.last_dmg_dealt)
    ob.taken[:] = c(obr.last_dmg_taken); ob.hp_loss[:] = c(obr.hp_loss)
    ob.act_hist[:] = c(obr.act_hist); ob.prev_x[:] = c(obr.prev_x)
    ob.prev_x_valid[:] = c(obr.prev_x_valid); ob.prev_alt_log[:] = c(obr.prev_alt_log)
    if ext:
        ob.prev_vel_ned[:] = c(obr.external_previous_velocity)
        ob.accel[:] = c(obr.external_accel)
    return ob


def _cmp_recon(obr, ob, ext=False):
    c = lambda t: t.detach().cpu().numpy().astype(np.float64)
    pairs = [("hp", obr.hp, ob.hp), ("fuel", obr.fuel, ob.fuel), ("pqr", obr.pqr, ob.pqr),
             ("dealt", obr.last_dmg_dealt, ob.dealt), ("taken", obr.last_dmg_taken, ob.taken),
             ("hp_loss", obr.hp_loss, ob.hp_loss), ("prev_x", obr.prev_x, ob.prev_x),
             ("prev_alt_log", obr.prev_alt_log, ob.prev_alt_log),
             ("prev_att", obr.prev_att, ob.prev_att)]
    if ext:
        pairs += [("accel", obr.external_accel, ob.accel),
                  ("prev_vel", obr.external_previous_velocity, ob.prev_vel_ned)]
    for name, g, o in pairs:
        err = np.abs(c(g) - o).max() if o.size else 0.0
        assert err <= VAL_TOL * max(1.0, np.abs(o).max()), (name, err)
    np.testing.assert_array_equal(c(obr.t_sec), ob.t_sec)
    np.testing.assert_array_equal(c(obr.act_hist), ob.act_hist)
    np.testing.assert_array_equal(c(obr.prev_valid), ob.prev_valid)
    np.testing.assert_array_equal(c(obr.prev_x_valid), ob.prev_x_valid)


def _soa(gpu, states_aos):
    """A (nac, 101) transposed view of a structure-of-arrays device buffer."""
    st = torch.as_tensor(np.ascontiguousarray(states_aos).T.copy(), device=gpu)
    return st.t()


# ------------------------------------------------------------------------ golden replay
@pytest.mark.parametrize("mode", [0, 1, 2, 3])
def test_golden_replay_matches_reference(gpu, mode, worst):
    """The scripted reference sequence (damage, hard deck, HP death, timeout, masked resets)
    through the GPU kernels against the reference's own outputs."""
    g = oracle_lib.golden("obs_golden.npz")
    nenv = g["in_reset"].shape[1]
    obr = _obr(nenv)
    obr.hp.copy_(torch.as_tensor(g["in_hp0"], device=gpu))
    obr.t_sec.copy_(torch.as_tensor(g["in_t0"], device=gpu))
    obr.kernel_init_reward_state(_soa(gpu, g["in_states"][0]))
    key = lambda n: g[f"m{mode}_{n}"] if f"m{mode}_{n}" in g else g[f"m0_{n}"]
    for k in range(g["in_actions"].shape[0]):
        st = _soa(gpu, g["in_states"][k])
        act = torch.as_tensor(g["in_actions"][k], device=gpu)
        r, te, tr = obr.kernel_advance(st, act, reward_mode=mode)
        obs = obr.kernel_build_obs(st).cpu().numpy()
        worst("golden replay 184, reward |err|", np.abs(r.cpu().numpy() - key("reward")[k]).max(),
              VAL_TOL)
        worst("golden replay 184, observation |err|", np.abs(obs - g["m0_obs"][k]).max(), OBS_TOL)
        assert np.abs(r.cpu().numpy() - key("reward")[k]).max() <= VAL_TOL, (k, "reward")
        np.testing.assert_array_equal(te.cpu().numpy().astype(bool), g["m0_term"][k].astype(bool))
        np.testing.assert_array_equal(tr.cpu().numpy().astype(bool), g["m0_trunc"][k].astype(bool))
        assert np.abs(obs - g["m0_obs"][k]).max() <= OBS_TOL, (k, "obs")
        assert np.abs(obr.hp.cpu().numpy() - g["m0_hp"][k]).max() <= VAL_TOL
        assert np.abs(obr.prev_x.cpu().numpy() - key("prev_x")[k]).max() <= VAL_TOL
        np.testing.assert_array_equal(obr.t_sec.cpu().numpy(), g["m0_t_sec"][k])
        mask = torch.as_tensor(g["in_reset"][k], device=gpu)
        str_ = _soa(gpu, g["in_states_reset"][k])
        if g["in_reset"][k].any():
            obr.reset_envs(mask)
            obr.kernel_init_reward_state(str_, mask)
            obs = obr.kernel_build_obs(str_, mask).cpu().numpy()
        assert np.abs(obs - g["m0_obs_reset"][k]).max() <= OBS_TOL, (k, "obs_reset")


# ------------------------------------------------------------------------ random engagements
def _random_states(gpu, nenv, seed, rate=60):
    """Seeded valid aircraft states: positions within +-20 km of the contest centre, altitude
    150 m - 12 km (some below the hard deck), 100-350 m/s, any attitude; a third of the
    engagements put the partner 150-1300 m in front of the nose so damage cones engage."""
    icm = import_pkg("ic")
    rng = np.random.default_rng(seed)
    n = 2 * nenv
    north = 3500.0 + rng.uniform(-20000, 20000, n)
    east = rng.uniform(-20000, 20000, n)
    alt = rng.uniform(150.0, 12000.0, n)
    spd = rng.uniform(100.0, 350.0, n)
    phi = rng.uniform(-180, 180, n)
    theta = rng.uniform(-80, 80, n)
    psi = rng.uniform(0, 360, n)
    alpha = rng.uniform(-5, 15, n)
    beta = rng.uniform(-5, 5, n)
    close = rng.random(nenv) < 0.35
    for e in np.nonzero(close)[0]:
        a, b = 2 * e, 2 * e + 1
        th, ps = np.radians(theta[a]), np.radians(psi[a])
        r = rng.uniform(150.0, 1300.0)
        fwd = np.array([np.cos(th) * np.cos(ps), np.cos(th) * np.sin(ps), -np.sin(th)])
        off = rng.normal(0.0, 0.004 * r, 3)
        north[b], east[b] = north[a] + r * fwd[0] + off[0], east[a] + r * fwd[1] + off[1]
        alt[b] = alt[a] - r * fwd[2] - off[2]
        alt[a] = max(alt[a], 2000.0)
        alt[b] = max(alt[b], 1500.0)
        alpha[a] = beta[a] = 0.0
    la, lo, h = icm.ned_to_geodetic(north, east, -alt)
    rows = np.array([icm.ic_row(la[i], lo[i], h[i], spd[i] / FT2M, psi[i], 3000.0, phi[i],
                                theta[i], alpha[i], beta[i]) for i in range(n)])
    sim = import_pkg().GpuDogfight(nenv, fcs_rate=rate)
    sim.seed_rows(torch.as_tensor(rows, device=gpu))
    return sim


def _random_recon(gpu, obr, seed, s9=None):
    """Reconstructor mid-episode: random HP (some nearly dead), times (some at the limit),
    previous attitudes, histories, anchors and validity flags.  With s9, the previous attitude
    is the current one perturbed by 8 deg (sd) per axis, as one 0.1 s decision of fast
    manoeuvring; log_SO3 is ill-conditioned for rotations near pi, which no decision makes."""
    rng = np.random.default_rng(seed)
    n, ne = obr.nac, obr.nenv
    t = lambda x, dt=torch.float64: torch.as_tensor(x, dtype=dt, device=gpu)
    hp = rng.uniform(0.05, 1.0, n)
    hp[rng.random(n) < 0.1] = 1e-3
    obr.hp.copy_(t(hp))
    obr.fuel.copy_(t(rng.uniform(0.0, 1.0, n)))
    ts = rng.uniform(0.0, 199.0, ne)
    ts[rng.random(ne) < 0.1] = 199.95
    ts[rng.random(ne) < 0.2] = rng.choice([99.95, 120.0, 149.95, 160.0])
    obr.t_sec.copy_(t(ts))
    if s9 is None:
        att = np.stack([rng.uniform(-180, 180, n), rng.uniform(-80, 80, n),
                        rng.uniform(0, 360, n)], 1)
    else:
        att = s9[:, 3:6] + rng.normal(0.0, 8.0, (n, 3))
    obr.prev_att.copy_(t(att))
    obr.prev_valid.copy_(t(rng.random(n) < 0.8, torch.bool))
    obr.pqr.copy_(t(rng.normal(0, 0.3, (n, 3))))
    obr.last_dmg_dealt.copy_(t(rng.uniform(0, 1, n)))
    obr.last_dmg_taken.copy_(t(rng.uniform(0, 1, n)))
    obr.hp_loss.copy_(t(rng.uniform(0, 0.01, n)))
    obr.act_hist.copy_(t(rng.uniform(-1, 1, (n, 5, 4))))
    obr.prev_x.copy_(t(rng.uniform(-1, 1, n)))
    obr.prev_x_valid.copy_(t(rng.random(n) < 0.8, torch.bool))
    obr.prev_alt_log.copy_(t(rng.normal(2.0, 1.0, n)))
    if obr._acc_soa is not None:
        obr.external_previous_velocity.copy_(t(rng.normal(0, 200, (n, 3))))
        obr.external_accel.copy_(t(rng.normal(0, 20, (n, 3))))


@pytest.mark.parametrize("mode", [0, 1, 2, 3])
def test_random_engagements_match_oracle(gpu, orc, mode):
    nenv = 1024
    sim = _random_states(gpu, nenv, 10 + mode)
    obr = _obr(nenv)
    s9 = oracle_lib.ObrOracle(orc, nenv).state9(sim.states.cpu().numpy())
    _random_recon(gpu, obr, 20 + mode, s9)
    ob = _to_oracle(obr, orc)
    act = np.random.default_rng(30 + mode).uniform(-1, 1, (2 * nenv, 4))
    r, te, tr = obr.kernel_advance(sim.states, torch.as_tensor(act, device=gpu), reward_mode=mode)
    r_o, te_o, tr_o = ob.step(s9, act, mode=mode)
    np.testing.assert_array_equal(te.cpu().numpy().astype(bool), te_o)
    np.testing.assert_array_equal(tr.cpu().numpy().astype(bool), tr_o)
    assert np.abs(r.cpu().numpy() - r_o).max() <= VAL_TOL
    _cmp_recon(obr, ob)
    obs = obr.kernel_build_obs(sim.states).cpu().numpy()
    assert np.abs(obs - ob.build_obs(s9)).max() <= OBS_TOL
    # the workload must exercise what it claims to
    assert te_o.any() and (~te_o).any() and tr_o.any()
    assert (ob.dealt > 0).any() and (ob.hp <= 0).any()


def test_init_reward_masked(gpu, orc):
    nenv = 512
    sim = _random_states(gpu, nenv, 41)
    obr = _obr(nenv)
    _random_recon(gpu, obr, 42)
    ob = _to_oracle(obr, orc)
    mask = np.random.default_rng(43).random(nenv) < 0.5
    obr.kernel_init_reward_state(sim.states, torch.as_tensor(mask, device=gpu))
    ob.init_reward(ob.state9(sim.states.cpu().numpy()), mask)
    _cmp_recon(obr, ob)


@pytest.mark.parametrize("nenv", [512, 17000, 26000])
def test_external_214_matches_oracle(gpu, orc, nenv):
    """214-D variant: acceleration vectors spliced in before the action history.  17,000
    engagements build the 214-D rows through the vector-block tile and the 184-D rows through
    the full-row tile; 26,000 build both through the vector-block tile."""
    sim = _random_states(gpu, nenv, 51)
    obr = _obr(nenv, ext=True)
    s9 = oracle_lib.ObrOracle(orc, nenv).state9(sim.states.cpu().numpy())
    _random_recon(gpu, obr, 52, s9)
    ob = _to_oracle(obr, orc, ext=True)
    act = np.random.default_rng(53).uniform(-1, 1, (2 * nenv, 4))
    obr.kernel_advance(sim.states, torch.as_tensor(act, device=gpu))
    ob.step(s9, act)
    _cmp_recon(obr, ob, ext=True)
    obs = obr.build_external_obs(sim.states).cpu().numpy()
    ref = ob.build_obs(s9, obs_dim=214)
    assert obs.shape == (2 * nenv, 214)
    assert np.abs(obs - ref).max() <= OBS_TOL
    # the 184-D layout is the 214-D one without the acceleration block
    obs184 = obr.kernel_build_obs(sim.states).cpu().numpy()
    np.testing.assert_array_equal(obs184[:, :164], obs[:, :164])
    np.testing.assert_array_equal(obs184[:, 164:], obs[:, 194:])


def test_golden_replay_214_matches_root_reference(gpu, worst):
    """The scripted sequence through the GPU's 214-D path against the root lineage's own torch
    path (cuda_fdm/obs_reward.py advance :544-582, build_obs :585-721; golden written by
    tests/golden/make_obs_golden.py --root214): observation, acceleration and the previous NED
    velocity after every decision and after the masked resets."""
    g = oracle_lib.golden("obs_golden.npz")
    a = oracle_lib.golden("obs214_golden.npz")
    nenv = g["in_reset"].shape[1]
    obr = _obr(nenv, ext=True)
    obr.hp.copy_(torch.as_tensor(g["in_hp0"], device=gpu))
    obr.t_sec.copy_(torch.as_tensor(g["in_t0"], device=gpu))
    obr.kernel_init_reward_state(_soa(gpu, g["in_states"][0]))
    c = lambda t: t.detach().cpu().numpy().astype(np.float64)
    for k in range(g["in_actions"].shape[0]):
        st = _soa(gpu, g["in_states"][k])
        act = torch.as_tensor(g["in_actions"][k], device=gpu)
        r, te, tr = obr.kernel_advance(st, act)
        obs = obr.build_external_obs(st).cpu().numpy()
        worst("golden replay 214, observation |err|", np.abs(obs - a["a214_obs"][k]).max(), OBS_TOL)
        worst("golden replay 214, acceleration |err| m/s2",
              np.abs(c(obr.external_accel) - a["a214_accel"][k]).max(), VAL_TOL * 100)
        assert np.abs(obs - a["a214_obs"][k]).max() <= OBS_TOL, (k, "obs")
        assert np.abs(c(obr.external_accel) - a["a214_accel"][k]).max() <= VAL_TOL * 100, k
        assert np.abs(c(obr.external_previous_velocity)
                      - a["a214_prev_vel_ned"][k]).max() <= VAL_TOL * 300, k
        assert np.abs(c(r) - a["a214_reward"][k]).max() <= VAL_TOL, (k, "reward")
        np.testing.assert_array_equal(te.cpu().numpy().astype(bool), a["a214_term"][k])
        np.testing.assert_array_equal(tr.cpu().numpy().astype(bool), a["a214_trunc"][k])
        if g["in_reset"][k].any():
            mask = torch.as_tensor(g["in_reset"][k], device=gpu)
            str_ = _soa(gpu, g["in_states_reset"][k])
            obr.reset_envs(mask)
            obr.kernel_init_reward_state(str_, mask)
            obs = obr.build_external_obs(str_).cpu().numpy()
            assert np.abs(obs - a["a214_obs_reset"][k]).max() <= OBS_TOL, (k, "obs_reset")
            acc = c(obr.external_accel)
            assert np.abs(acc - a["a214_accel_reset"][k]).max() <= VAL_TOL * 100, k
            assert np.all(acc[np.repeat(g["in_reset"][k], 2)] == 0.0), k


def test_state9_kernel(gpu, orc):
    nenv = 256
    sim = _random_states(gpu, nenv, 61)
    out = torch.empty(2 * nenv, 9, dtype=torch.float64, device=gpu)
    L = import_pkg("_lib")
    rc = L.lib().f16_state9(L.ptr(sim._state_soa), sim.nac, sim.nac, L.ptr(out),
                            L.stream_handle(gpu))
    L.check(rc, "f16_state9")
    ref = oracle_lib.ObrOracle(orc, nenv).state9(sim.states.cpu().numpy())
    got = out.cpu().numpy()
    assert np.abs(got[:, :3] - ref[:, :3]).max() <= 1e-6          # metres
    assert np.abs(got[:, 3:6] - ref[:, 3:6]).max() <= 1e-9        # degrees
    assert np.abs(got[:, 6:] - ref[:, 6:]).max() <= 1e-10         # m/s


# ------------------------------------------------------------------------ fused env step
@pytest.mark.parametrize("obs_dim,nenv", [(184, 1024), (214, 1024), (184, 26000), (214, 17000)])
def test_env_post_step_matches_reference_sequence(gpu, orc, obs_dim, nenv):
    """f16_env_post_step against the reference's sequence (rl_env.py:540-580) replayed on the
    oracle: advance -> terminal obs -> pool autoreset -> reset_envs -> init_reward -> masked
    build_obs.  The large sizes exceed what the full-row staging tile keeps resident on an
    MI355X (768 / 512 wavefronts), so they run the vector-block tile with direct row stores."""
    ext = obs_dim == 214
    sim = _random_states(gpu, nenv, 71)
    pool_sim = _random_states(gpu, 64, 72)
    pool = pool_sim.states.reshape(64, 2, 101).contiguous()
    obr = _obr(nenv, ext)
    st0 = sim.states.cpu().numpy()
    _random_recon(gpu, obr, 73, oracle_lib.ObrOracle(orc, nenv).state9(st0))
    ob = _to_oracle(obr, orc, ext)
    act = np.random.default_rng(74).uniform(-1, 1, (2 * nenv, 4))
    pick = torch.as_tensor(np.random.default_rng(75).integers(0, 64, nenv), device=gpu)
    sim.actions.copy_(torch.as_tensor(act, device=gpu))
    L = import_pkg("_lib")
    R = import_pkg("obs_reward")
    n = 2 * nenv
    obs = torch.full((n, obs_dim), -7.0, dtype=torch.float32, device=gpu)
    tobs = torch.empty_like(obs)
    rew = torch.empty(n, dtype=torch.float64, device=gpu)
    rew32 = torch.empty(n, dtype=torch.float32, device=gpu)
    te, tr, dn, fin = (torch.empty(nenv, dtype=torch.uint8, device=gpu) for _ in range(4))
    dn32 = torch.empty(nenv, dtype=torch.float32, device=gpu)
    facc = torch.ones(nenv, dtype=torch.uint8, device=gpu)
    thp = torch.empty(n, dtype=torch.float64, device=gpu)
    talt = torch.empty(n, dtype=torch.float64, device=gpu)
    c = R.reward_cfg_struct(R.MY_REWARD_CONFIG, 304.8, 200.0, 0, 5.0)
    rec = obr._recon()
    io = L.F16EnvStepIO(states=sim._state_soa.data_ptr(), ld=sim.nac,
                        actions=sim.actions.data_ptr(), ic_pool=pool.data_ptr(), pool_size=64,
                        pick=pick.data_ptr(), obs_dim=obs_dim, obs=obs.data_ptr(),
                        terminal_obs=tobs.data_ptr(), reward=rew.data_ptr(),
                        reward_f32=rew32.data_ptr(), term=te.data_ptr(), trunc=tr.data_ptr(),
                        done=dn.data_ptr(), done_f32=dn32.data_ptr(),
                        terminal_hp=thp.data_ptr(), terminal_alt_m=talt.data_ptr(),
                        terminal_finite=fin.data_ptr(), finite_acc=facc.data_ptr())
    rc = L.lib().f16_env_post_step(L.ctypes.byref(io), L.ctypes.byref(rec), L.ctypes.byref(c),
                                   L.stream_handle(gpu))
    L.check(rc, "f16_env_post_step")
    # oracle replay of the reference sequence
    s9 = ob.state9(st0)
    r_o, te_o, tr_o = ob.step(s9, act)
    tobs_o = ob.build_obs(s9, obs_dim)
    thp_o = ob.hp.copy()
    done_o = te_o | tr_o
    st1 = st0.copy()
    pk = pick.cpu().numpy()
    pool_np = pool.cpu().numpy()
    for e in np.nonzero(done_o)[0]:
        st1[2 * e:2 * e + 2] = pool_np[pk[e]]
    ob.reset_envs(done_o)
    s9r = ob.state9(st1)
    ob.init_reward(s9r, done_o)
    obs_o = tobs_o.copy()
    obs_o[np.repeat(done_o, 2)] = ob.build_obs(s9r, obs_dim)[np.repeat(done_o, 2)]
    # compare
    np.testing.assert_array_equal(te.cpu().numpy().astype(bool), te_o)
    np.testing.assert_array_equal(tr.cpu().numpy().astype(bool), tr_o)
    np.testing.assert_array_equal(dn.cpu().numpy().astype(bool), done_o)
    np.testing.assert_array_equal(fin.cpu().numpy().astype(bool),
                                  np.isfinite(st0).all(1).reshape(nenv, 2).all(1))
    assert np.abs(rew.cpu().numpy() - r_o).max() <= VAL_TOL
    np.testing.assert_array_equal(rew32.cpu().numpy(), rew.cpu().numpy().astype(np.float32))
    np.testing.assert_array_equal(dn32.cpu().numpy(), done_o.astype(np.float32))
    np.testing.assert_array_equal(facc.cpu().numpy().astype(bool), fin.cpu().numpy().astype(bool))
    assert np.abs(thp.cpu().numpy() - thp_o).max() <= VAL_TOL
    alt_o = (np.linalg.norm(st0[:, 0:3], axis=1) - 20925646.32546) * FT2M
    assert np.abs(talt.cpu().numpy() - alt_o).max() <= 1e-6
    assert np.abs(tobs.cpu().numpy() - tobs_o).max() <= OBS_TOL
    assert np.abs(obs.cpu().numpy() - obs_o).max() <= OBS_TOL
    np.testing.assert_array_equal(sim.states.cpu().numpy(), st1)
    _cmp_recon(obr, ob, ext)
    assert done_o.any() and (~done_o).any()


@pytest.mark.parametrize("obs_dim,nenv,terminal", [
    (184, 1024, True), (184, 1024, False), (214, 1024, True), (214, 1024, False),
    (184, 300, True), (214, 33, False),
    (184, 26000, True), (184, 26000, False), (214, 17000, True)])
def test_env_post_step_two_wave_equals_one_wave(gpu, obs_dim, nenv, terminal):
    """f16_env_post_step against f16_env_post_step_onewave on identical inputs: every output,
    state row, reconstructor value and aux feature bit for bit, with finished engagements
    (autoreset rows), with and without terminal observations, with the full-row tile (1024
    engagements, and 300 and 33 whose last workgroup is partly filled: four wavefronts per 64
    aircraft) and the vector-block tile (26000 / 17000
    engagements exceed what the full-row tile keeps resident: an advance wave and a vector-block
    wave per 64 aircraft)."""
    ext = obs_dim == 214
    sim = _random_states(gpu, nenv, 171)
    pool = _random_states(gpu, 64, 172).states.reshape(64, 2, 101).contiguous()
    obr = _obr(nenv, ext)
    obr.enable_aux_capture()
    _random_recon(gpu, obr, 173)
    act = np.random.default_rng(174).uniform(-1, 1, (2 * nenv, 4))
    sim.actions.copy_(torch.as_tensor(act, device=gpu))
    pick = torch.as_tensor(np.random.default_rng(175).integers(0, 64, nenv), device=gpu)
    L = import_pkg("_lib")
    R = import_pkg("obs_reward")
    c = R.reward_cfg_struct(R.MY_REWARD_CONFIG, 304.8, 200.0, 0, 5.0)
    st0, rec0 = sim._state_soa.clone(), obr.clone_state()
    n = 2 * nenv
    results = []
    for fn in ("f16_env_post_step_onewave", "f16_env_post_step"):
        sim._state_soa.copy_(st0)
        obr.restore(rec0)
        out = {"obs": torch.full((n, obs_dim), -7.0, dtype=torch.float32, device=gpu),
               "tobs": torch.full((n, obs_dim), -9.0, dtype=torch.float32, device=gpu),
               "rew": torch.zeros(n, dtype=torch.float64, device=gpu),
               "rew32": torch.zeros(n, dtype=torch.float32, device=gpu),
               "thp": torch.zeros(n, dtype=torch.float64, device=gpu),
               "talt": torch.zeros(n, dtype=torch.float64, device=gpu),
               "dn32": torch.zeros(nenv, dtype=torch.float32, device=gpu),
               "facc": torch.ones(nenv, dtype=torch.uint8, device=gpu)}
        for k in ("te", "tr", "dn", "fin"):
            out[k] = torch.zeros(nenv, dtype=torch.uint8, device=gpu)
        rec = obr._recon()
        io = L.F16EnvStepIO(states=sim._state_soa.data_ptr(), ld=sim.nac,
                            actions=sim.actions.data_ptr(), ic_pool=pool.data_ptr(),
                            pool_size=64, pick=pick.data_ptr(), obs_dim=obs_dim,
                            obs=out["obs"].data_ptr(),
                            terminal_obs=out["tobs"].data_ptr() if terminal else None,
                            reward=out["rew"].data_ptr(), reward_f32=out["rew32"].data_ptr(),
                            term=out["te"].data_ptr(), trunc=out["tr"].data_ptr(),
                            done=out["dn"].data_ptr(), done_f32=out["dn32"].data_ptr(),
                            terminal_hp=out["thp"].data_ptr(),
                            terminal_alt_m=out["talt"].data_ptr(),
                            terminal_finite=out["fin"].data_ptr(), finite_acc=out["facc"].data_ptr())
        L.check(getattr(L.lib(), fn)(L.ctypes.byref(io), L.ctypes.byref(rec), L.ctypes.byref(c),
                                     L.stream_handle(gpu)), fn)
        torch.cuda.synchronize()
        snap = {k: v.cpu().numpy() for k, v in out.items()}
        snap["states"] = sim._state_soa.cpu().numpy()
        snap.update({"recon_" + k: v.cpu().numpy() for k, v in obr.clone_state().items()})
        results.append(snap)
    one, two = results
    assert one.keys() == two.keys()
    for k in one:
        np.testing.assert_array_equal(two[k], one[k], err_msg=k)
    done = one["dn"].astype(bool)
    assert done.any() and (~done).any()


@pytest.mark.parametrize("obs_dim", [184, 214])
def test_env_step_fused_finite_equals_state_scan(gpu, obs_dim):
    """GpuDogfightVecEnv.step with the physics launch's finite flags (F16EnvStepIO.state_finite)
    against the post-physics launch testing the 101 state values itself: every output, the
    reconstructor and the states agree bit for bit over several steps, with NaN and infinity
    planted in some engagements' states (terminal_state_finite false, autoreset)."""
    E = import_pkg("rl_env").GpuDogfightVecEnv
    envs = [E(300, seed=4, ic_pool_size=64, obs_dim=obs_dim) for _ in range(2)]
    envs[1].fused_finite = False
    for env in envs:
        env.reset(stagger=False)
    rng = np.random.default_rng(5)
    for k in range(4):
        act = torch.as_tensor(rng.uniform(-1, 1, (600, 4)), device=gpu)
        pick = torch.as_tensor(rng.integers(0, 64, 300), device=gpu)
        outs = []
        for env in envs:
            if k == 1:
                env.sim.states[17, 5] = float("nan")
                env.sim.states[40, 88] = float("inf")
                env.sim.states[301, 100] = float("nan")
            outs.append(env.step(act, reset_indices=pick))
        (oa, ra, da, ia), (ob, rb, db, ib) = outs
        bits = lambda t: t.contiguous().view(torch.int32 if t.element_size() == 4 else
                                             torch.int64 if t.element_size() == 8 else torch.uint8)
        same = lambda x, y: torch.equal(bits(x), bits(y))       # NaN-safe, bit for bit
        assert same(oa, ob) and same(ra, rb) and same(da, db), k
        for key in ia:
            assert same(ia[key], ib[key]), (k, key)
        assert same(envs[0].sim._state_soa, envs[1].sim._state_soa), k
        assert same(envs[0].obr.hp, envs[1].obr.hp)
        if k == 1:
            bad = (~ia["terminal_state_finite"]).nonzero().flatten().tolist()
            assert bad == [8, 20, 150], bad
            # termination tests the state9 row (rl_env.py:467-484): a NaN velocity terminates;
            # an infinite actuator state or PID integrator is clamped before it reaches state9
            assert bool(da[8])


@pytest.mark.parametrize("obs_dim,nenv", [(184, 300), (214, 300), (184, 20000)])
def test_env_step_pool_tables_equal_rebuild(gpu, obs_dim, nenv):
    """Autoresets that copy each pool row's observation, reward anchors and aux features from
    the env's pool tables (F16EnvStepIO.pool_obs) against autoresets that rebuild them: every
    output, the reconstructor, the aux features and the states agree bit for bit over steps
    with many autoresets (a 1.2 s engagement limit on staggered clocks), including a pick
    outside the pool (its NaN row is still built).  20,000 engagements exercise the
    vector-block tile layout."""
    E = import_pkg("rl_env").GpuDogfightVecEnv
    envs = [E(nenv, seed=9, ic_pool_size=64, obs_dim=obs_dim, max_engage_time_s=1.2)
            for _ in range(2)]
    envs[1].pool_tables = False
    for env in envs:
        env.enable_aux_capture()
        env.reset(stagger=True, max_stagger_steps=12)
    bits = lambda t: t.contiguous().view(torch.int32 if t.element_size() == 4 else
                                         torch.int64 if t.element_size() == 8 else torch.uint8)
    same = lambda x, y: torch.equal(bits(x), bits(y))       # NaN-safe, bit for bit
    rng = np.random.default_rng(6)
    resets = 0
    for k in range(8):
        act = torch.as_tensor(rng.uniform(-1, 1, (2 * nenv, 4)), device=gpu)
        pick = rng.integers(0, 64, nenv)
        if k == 3:
            pick[5] = 64                                    # outside the pool: NaN row
        pick = torch.as_tensor(pick, device=gpu)
        outs = [env.step(act, reset_indices=pick) for env in envs]
        (oa, ra, da, ia), (ob, rb, db, ib) = outs
        assert same(oa, ob) and same(ra, rb) and same(da, db), k
        for key in ia:
            assert same(ia[key], ib[key]), (k, key)
        assert same(envs[0].sim._state_soa, envs[1].sim._state_soa), k
        for name in ("hp", "fuel", "prev_x", "prev_x_valid", "prev_alt_log", "t_sec",
                     "aux_features", "_hist_soa", "_att_soa", "_pqr_soa"):
            assert same(getattr(envs[0].obr, name), getattr(envs[1].obr, name)), (k, name)
        resets += int(da.sum())
    assert resets > nenv // 4, resets
    assert envs[0]._pool_key is not None and envs[1]._pool_key is None


@pytest.mark.parametrize("obs_dim", [184, 214])
def test_env_step_pool_tables_follow_pool_replacement(gpu, obs_dim):
    """The pool tables follow the pool tensor itself, not its address: after
    `env.ic_pool = None` (the reference's evaluation reset, search_eval.py:78, redraws the pool
    on the next step) and after a restored pool of the same shape is assigned
    (ppo_gpu.py:2909), autoresets with tables equal autoresets that rebuild their rows, bit for
    bit, even when the caching allocator hands the new pool the freed pool's address."""
    E = import_pkg("rl_env").GpuDogfightVecEnv
    nenv = 200
    envs = [E(nenv, seed=21, ic_pool_size=64, obs_dim=obs_dim, max_engage_time_s=1.2)
            for _ in range(2)]
    envs[1].pool_tables = False
    for env in envs:
        env.enable_aux_capture()
        env.reset(stagger=True, max_stagger_steps=12)
    bits = lambda t: t.contiguous().view(torch.int32 if t.element_size() == 4 else
                                         torch.int64 if t.element_size() == 8 else torch.uint8)
    same = lambda x, y: torch.equal(bits(x), bits(y))
    donor = E(32, seed=77, ic_pool_size=64, obs_dim=obs_dim)
    donor._ensure_ic_pool()
    rng = np.random.default_rng(22)
    resets = 0
    for k in range(9):
        if k == 3:
            for env in envs:
                env.ic_pool = None                  # redrawn (same draws in both) on this step
        if k == 6:
            for env in envs:
                env.ic_pool = None
            torch.cuda.synchronize()
            for env in envs:                        # a restored pool of the same shape
                env.ic_pool = donor.ic_pool.clone()
        act = torch.as_tensor(rng.uniform(-1, 1, (2 * nenv, 4)), device=gpu)
        pick = torch.as_tensor(rng.integers(0, 64, nenv), device=gpu)
        (oa, ra, da, ia), (ob, rb, db, ib) = [env.step(act, reset_indices=pick) for env in envs]
        assert same(oa, ob) and same(ra, rb) and same(da, db), k
        for key in ia:
            assert same(ia[key], ib[key]), (k, key)
        assert same(envs[0].sim._state_soa, envs[1].sim._state_soa), k
        for name in ("prev_x", "prev_alt_log", "aux_features"):
            assert same(getattr(envs[0].obr, name), getattr(envs[1].obr, name)), (k, name)
        assert envs[0]._pool_src is envs[0].ic_pool
        resets += int(da.sum())
    assert resets > nenv // 4, resets


@pytest.mark.parametrize("obs_dim,nenv,fcs,roles", [
    (184, 300, 60, 2), (214, 300, 120, 2), (184, 16384, 60, 2), (214, 16384, 120, 2),
    (184, 20000, 60, 2), (184, 300, 60, 4), (214, 300, 120, 4), (184, 16384, 60, 4),
    (214, 16384, 120, 4), (184, 20, 60, 4), (214, 33, 120, 4), (184, 20000, 60, 4),
    (214, 17000, 120, 4)])
def test_env_step_one_launch_equals_two(gpu, obs_dim, nenv, fcs, roles):
    """f16_env_step (physics and post-physics step in one launch wherever the full-row tile is
    resident: 300 engagements, whose last workgroup is partly filled, and 16,384; at 17,000 and
    20,000 the entry issues the two launches itself), and roles=4: four wavefronts per 64
    aircraft in both phases, against sim.step + f16_env_post_step: every output,
    the states, the kept actions, the reconstructor and the aux features bit for bit over steps
    with autoresets (staggered 1.2 s engagements), terminal observations on and off, a separate
    action tensor (the launch copies it into sim.actions) and a non-contiguous one (copied
    before the launch), NaN planted in a state and a pick outside the pool; then rollout steps
    (step_rollout) with a device step counter and, where fusable, the RunningNorm partial sums
    merged into the statistics, and plane 0's float32 rewards written alone (reward0_f32)."""
    E = import_pkg("rl_env").GpuDogfightVecEnv
    P = import_pkg("policy")
    envs = [E(nenv, seed=11, ic_pool_size=64, obs_dim=obs_dim, max_engage_time_s=1.2,
              fcs_rate=fcs) for _ in range(2)]
    envs[1].fused_step = False
    envs[0].step_roles = roles
    for env in envs:
        env.enable_aux_capture()
        env.reset(stagger=True, max_stagger_steps=12)
    bits = lambda t: t.contiguous().view(torch.int32 if t.element_size() == 4 else
                                         torch.int64 if t.element_size() == 8 else torch.uint8)
    same = lambda x, y: torch.equal(bits(x), bits(y))       # NaN-safe, bit for bit
    names = ("hp", "fuel", "prev_x", "prev_x_valid", "prev_alt_log", "t_sec", "aux_features",
             "_hist_soa", "_att_soa", "_pqr_soa")
    rng = np.random.default_rng(12)
    resets = 0
    for k in range(6):
        act = rng.uniform(-1, 1, (2 * nenv, 4))
        act_t = (torch.as_tensor(act.T.copy(), device=gpu).t() if k == 2 else
                 torch.as_tensor(act, device=gpu))
        pick = rng.integers(0, 64, nenv)
        if k == 3:
            pick[5] = 64                                    # outside the pool: NaN row
        pick = torch.as_tensor(pick, device=gpu)
        outs = []
        for env in envs:
            if k == 1:
                env.sim.states[17, 5] = float("nan")
            outs.append(env.step(act_t, reset_indices=pick if k % 2 == 1 else None,
                                 capture_terminal_obs=k != 4))
        (oa, ra, da, ia), (ob, rb, db, ib) = outs
        assert same(oa, ob) and same(ra, rb) and same(da, db), k
        for key in ia:
            assert (ia[key] is None) == (ib[key] is None), (k, key)
            assert ia[key] is None or same(ia[key], ib[key]), (k, key)
        assert same(envs[0].sim._state_soa, envs[1].sim._state_soa), k
        assert same(envs[0].sim.actions, envs[1].sim.actions), k
        assert same(envs[0].sim.actions, torch.as_tensor(act, device=gpu)), k
        for name in names:
            assert same(getattr(envs[0].obr, name), getattr(envs[1].obr, name)), (k, name)
        if k == 1:
            assert not bool(ia["terminal_state_finite"][8])
        resets += int(da.sum())
    assert resets > nenv // 4 or nenv < 100, resets
    nac = 2 * nenv
    norms = [P.RunningNorm(obs_dim, gpu) for _ in envs]
    bases = [torch.full((), 40, dtype=torch.int32, device=gpu) for _ in envs]
    bufs = [{"rew": torch.zeros(nac, dtype=torch.float32, device=gpu),
             "dn": torch.zeros(nenv, dtype=torch.float32, device=gpu),
             "facc": torch.ones(nenv, dtype=torch.uint8, device=gpu)} for _ in envs]
    rew0 = torch.full((nenv,), -5.0, dtype=torch.float32, device=gpu)
    fusable = envs[0].norm_fusable()
    assert fusable == (nenv <= 16384)
    for t in range(3):
        act = torch.as_tensor(rng.uniform(-1, 1, (nac, 4)), device=gpu)
        obs = []
        for env, norm, base, b in zip(envs, norms, bases, bufs):
            env.sim.actions.copy_(act)
            obs.append(env.step_rollout(b["rew"], b["dn"], b["facc"], step_base=base, step=t,
                                        norm=norm if fusable else None,
                                        reward0_f32=rew0 if env is envs[0] else None))
            if fusable:
                norm.merge(nac)
        assert same(obs[0], obs[1]), t
        assert same(rew0, bufs[1]["rew"][0::2]), t         # plane 0's rewards alone
        for key in bufs[0]:
            assert same(bufs[0][key], bufs[1][key]), (t, key)
        assert same(envs[0].sim._state_soa, envs[1].sim._state_soa), t
        for name in names:
            assert same(getattr(envs[0].obr, name), getattr(envs[1].obr, name)), (t, name)
        if fusable:
            for f in ("mean", "var", "count"):
                assert same(getattr(norms[0], f), getattr(norms[1], f)), (t, f)
    if fusable:
        assert float(norms[0].count) > 1.0


def test_step_training_and_capture_switch(gpu):
    """The root lineage's surface (cuda_fdm/rl_env.py:518-529): step_training and
    step(capture_terminal_obs=False) return the same observation, reward, done and info as a
    capturing step, with info["terminal_obs"] None; the instance default survives a failing
    step_training."""
    E = import_pkg("rl_env").GpuDogfightVecEnv
    envs = [E(200, seed=3, ic_pool_size=32, max_engage_time_s=0.5) for _ in range(3)]
    for env in envs:
        env.reset(stagger=True, max_stagger_steps=5)
    rng = np.random.default_rng(2)
    for k in range(6):
        act = torch.as_tensor(rng.uniform(-1, 1, (400, 4)), device=gpu)
        pick = torch.as_tensor(rng.integers(0, 32, 200), device=gpu)
        torch.manual_seed(k)
        a = envs[0].step(act, reset_indices=pick)
        b = envs[1].step(act, reset_indices=pick, capture_terminal_obs=False)
        c = envs[2].step(act, reset_indices=pick, terminal_obs=False)
        assert a[3]["terminal_obs"] is not None
        assert b[3]["terminal_obs"] is None and c[3]["terminal_obs"] is None
        for x, y in ((a, b), (a, c)):
            for i in range(3):
                assert torch.equal(x[i], y[i]), (k, i)
            for key in x[3]:
                if key != "terminal_obs":
                    assert torch.equal(x[3][key], y[3][key]), (k, key)
    # step_training draws its own pool picks (inside the post-physics launch)
    env = envs[2]
    out = env.step_training(torch.zeros(400, 4, dtype=torch.float64, device=gpu))
    assert out[3]["terminal_obs"] is None and env._capture_terminal_obs
    with pytest.raises((ValueError, RuntimeError)):
        env.step_training(torch.zeros(3, 4, dtype=torch.float64, device=gpu))
    assert env._capture_terminal_obs is True
    assert env.step(torch.zeros(400, 4, dtype=torch.float64, device=gpu))[3]["terminal_obs"] is not None


def test_env_post_step_bad_pick_poisons_state(gpu):
    """A pool index out of range never reads out of bounds: the engagement becomes NaN."""
    nenv = 4
    sim = _random_states(gpu, nenv, 81)
    obr = _obr(nenv)
    obr.t_sec.fill_(199.95)          # every engagement truncates -> autoreset for all
    pool = sim.states.reshape(nenv, 2, 101).contiguous()
    pick = torch.tensor([0, 4, -1, 1], dtype=torch.int64, device=gpu)
    L = import_pkg("_lib")
    R = import_pkg("obs_reward")
    n = 2 * nenv
    obs = torch.zeros(n, 184, dtype=torch.float32, device=gpu)
    dn = torch.empty(nenv, dtype=torch.uint8, device=gpu)
    c = R.reward_cfg_struct(R.MY_REWARD_CONFIG, 0.0, 200.0, 0, 5.0)
    rec = obr._recon()
    io = L.F16EnvStepIO(states=sim._state_soa.data_ptr(), ld=sim.nac,
                        actions=sim.actions.data_ptr(), ic_pool=pool.data_ptr(), pool_size=nenv,
                        pick=pick.data_ptr(), obs_dim=184, obs=obs.data_ptr(), done=dn.data_ptr())
    rc = L.lib().f16_env_post_step(L.ctypes.byref(io), L.ctypes.byref(rec), L.ctypes.byref(c),
                                   L.stream_handle(gpu))
    L.check(rc, "f16_env_post_step")
    st = sim.states.cpu().numpy().reshape(nenv, 2, 101)
    assert dn.cpu().numpy().all()
    assert np.isfinite(st[[0, 3]]).all()
    assert np.isnan(st[[1, 2]]).all()


def test_env_post_step_kernel_picks(gpu, orc):
    """pick = NULL: finished engagements take pool row floor(P x0 / 2^32) of Philox4x32-10
    (key = seed, counter = (e, step, 0, 0x5EED5EED))."""
    from test_policy import philox
    nenv, P = 64, 48
    sim = _random_states(gpu, nenv, 91)
    pool = _random_states(gpu, P, 92).states.reshape(P, 2, 101).contiguous()
    obr = _obr(nenv)
    obr.t_sec.fill_(199.95)                              # all truncate
    L = import_pkg("_lib")
    R = import_pkg("obs_reward")
    obs = torch.zeros(2 * nenv, 184, dtype=torch.float32, device=gpu)
    c = R.reward_cfg_struct(R.MY_REWARD_CONFIG, 0.0, 200.0, 0, 5.0)
    rec = obr._recon()
    seed, step = 0x1234_5678_9ABC, 17
    io = L.F16EnvStepIO(states=sim._state_soa.data_ptr(), ld=sim.nac,
                        actions=sim.actions.data_ptr(), ic_pool=pool.data_ptr(), pool_size=P,
                        pick=None, seed=seed, step=step, obs_dim=184, obs=obs.data_ptr())
    L.check(L.lib().f16_env_post_step(L.ctypes.byref(io), L.ctypes.byref(rec), L.ctypes.byref(c),
                                      L.stream_handle(gpu)), "f16_env_post_step")
    st = sim.states.cpu().numpy().reshape(nenv, 2, 101)
    pn = pool.cpu().numpy()
    for e in range(nenv):
        x0 = philox(orc, [e, step, 0, 0x5EED5EED], [seed & 0xffffffff, seed >> 32])[0]
        np.testing.assert_array_equal(st[e], pn[(x0 * P) >> 32])


# ------------------------------------------------------------------------ the env object
def test_vec_env_contract(gpu):
    """GpuDogfightVecEnv reset()/step() shapes, dtypes, info keys, autoreset bookkeeping."""
    E = import_pkg("rl_env").GpuDogfightVecEnv
    env = E(64, seed=3, ic_pool_size=32)
    obs = env.reset(stagger=True, max_stagger_steps=6)
    assert obs.shape == (64, 2, 184) and obs.dtype == torch.float32
    assert torch.isfinite(obs).all()
    rng = torch.Generator(device=gpu).manual_seed(0)
    for k in range(40):
        a = torch.rand(64, 2, 4, generator=rng, device=gpu, dtype=torch.float64) * 2 - 1
        a[..., 3] = (a[..., 3] + 1) / 2
        obs, rew, done, info = env.step(a)
        assert obs.shape == (64, 2, 184) and rew.shape == (64, 2) and done.shape == (64,)
        assert rew.dtype == torch.float64 and done.dtype == torch.bool
        assert set(info) == {"terminated", "truncated", "terminal_obs", "terminal_hp",
                             "terminal_alt_m", "done", "terminal_state_finite"}
        assert torch.equal(done, info["terminated"] | info["truncated"])
        if done.any():
            # autoreset engagements restart the clock and full HP
            assert (env.obr.t_sec[done] == 0).all()
            assert (env.obr.hp.view(64, 2)[done] == 1).all()
        live = ~done
        assert torch.equal(obs[live], info["terminal_obs"][live])
    s9 = env.state9()
    assert s9.shape == (64, 2, 9)
    ev = env.reset_evaluation(paired=True, seed_block=1)
    assert ev.shape == (64, 2, 184)
    np.testing.assert_array_equal(env.sim.states[:64].cpu().numpy(),
                                  env.sim.states[64:].cpu().numpy())


def test_staggered_warmup_is_device_resident(gpu):
    """The staggered warm-up (rl_env.py:386-434) runs without one host synchronisation (torch's
    sync debug mode would raise), captures every engagement at a whole number of decisions below
    the bound (the engagement clock restarts with each re-seed), and leaves every aircraft finite
    and above the 100 m departure floor."""
    E = import_pkg("rl_env").GpuDogfightVecEnv
    env = E(512, seed=11, ic_pool_size=64)
    env.reset(stagger=False)
    env._ensure_ic_pool()                  # built once per environment, before any warm-up
    torch.cuda.synchronize()
    steps = 24
    torch.cuda.set_sync_debug_mode("error")
    try:
        finite = env._staggered_warmup(steps, None)
    finally:
        torch.cuda.set_sync_debug_mode(0)
    assert bool(finite)
    t = env.obr.t_sec.cpu().numpy()
    k = np.round(t / env.obr.dt)
    np.testing.assert_allclose(t, k * env.obr.dt, atol=1e-9)
    assert k.min() >= 0 and k.max() < steps and len(np.unique(k)) > steps // 2
    s9 = env.state9().cpu().numpy()
    assert np.isfinite(s9).all() and (-s9[:, :, 2] > 100.0).all()
    obs = env._build_obs_all()
    assert torch.isfinite(obs).all()


def test_env_step_argument_errors_launch_nothing(gpu):
    """f16_env_step rejects a bad call before launching anything: no substeps, an FCS rate other
    than 60/120, no finite-flag buffer, controls overlapping io.actions, RunningNorm partials past
    the resident full-row tile (the two-launch case) -- the states and observations stay as they
    were."""
    E = import_pkg("rl_env").GpuDogfightVecEnv
    L = import_pkg("_lib")
    env = E(20000, seed=2, ic_pool_size=16)
    env.reset(stagger=False)
    env._ensure_ic_pool()
    lib = L.lib()
    st0, obs0 = env.sim._state_soa.clone(), env._obs.clone()
    fin = torch.zeros(env.nac, dtype=torch.uint8, device=gpu)
    act = torch.zeros(env.nac, 4, dtype=torch.float64, device=gpu)
    work = torch.zeros(1 << 20, dtype=torch.float64, device=gpu)
    cnt = torch.zeros(2, dtype=torch.float32, device=gpu)
    c = env._cfg_struct()

    def call(actions_ptr, substeps, rate, fin_ptr, norm=False):
        io = env._io(None)
        if norm:
            io.norm_partial, io.norm_count = work.data_ptr(), cnt.data_ptr()
            io.norm_count_snap = cnt.data_ptr() + 4
        return lib.f16_env_step(L.ctypes.byref(io), L.ctypes.byref(env._rec), L.ctypes.byref(c),
                                actions_ptr, substeps, rate, fin_ptr, L.stream_handle(gpu))

    EINVAL, ERATE = -1, -2
    assert call(act.data_ptr(), 0, 60, fin.data_ptr()) == EINVAL
    assert call(act.data_ptr(), 6, 90, fin.data_ptr()) == ERATE
    assert call(act.data_ptr(), 6, 60, None) == EINVAL
    overlap = env.sim.actions.data_ptr() + 8 * 4 * 3           # 3 rows into io.actions
    assert call(overlap, 6, 60, fin.data_ptr()) == EINVAL
    assert not env.norm_fusable()
    assert call(act.data_ptr(), 6, 60, fin.data_ptr(), norm=True) == EINVAL
    torch.cuda.synchronize()
    assert torch.equal(env.sim._state_soa, st0) and torch.equal(env._obs, obs0)
    assert call(act.data_ptr(), 6, 60, fin.data_ptr()) == 0    # the same call, valid
    torch.cuda.synchronize()
    assert not torch.equal(env.sim._state_soa, st0)
    assert torch.equal(env.sim.actions, act)                  # the controls were kept


def test_obs_argument_errors(gpu):
    obr = _obr(8)
    st = torch.zeros(16, 101, dtype=torch.float64, device=gpu)
    with pytest.raises(TypeError):
        obr.kernel_build_obs(st.float())
    with pytest.raises(ValueError):
        obr.kernel_build_obs(st[:8])
    with pytest.raises(ValueError):
        obr.kernel_advance(st, torch.zeros(16, 4, dtype=torch.float64, device=gpu), reward_mode=7)
    with pytest.raises(TypeError):
        obr.kernel_advance(st, torch.zeros(16, 4, dtype=torch.float32, device=gpu))
    with pytest.raises(ValueError):
        obr._build(st, None, 200, obr.obs_buf)
