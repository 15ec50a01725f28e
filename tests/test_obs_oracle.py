"""CPU: the observation / reward / termination restatement (oracle/obs_oracle.c) against the
golden vectors written from the reference's own torch path (tests/golden/make_obs_golden.py:
research/competition_36500/runtime/cuda_fdm/obs_reward.py BatchObsReward with
enable_kernel=False, and cuda_fdm/rl_env.py's state9 bridge and termination rule).

The scenario drives every branch the reference has: tier-1 tail-chase damage, mutual head-on
damage, hard-deck exits of either plane, an HP death, a timeout truncation, and masked resets
followed by the re-anchoring of the reward state.  All four reward modes are checked.
"""
import numpy as np
import pytest

import oracle_lib

# torch's batched 3x3 products accumulate in another order than the oracle's plain sums, and the
# state9 bridge's Bowring latitude carries ~1e-9 m of that into N/E; everything downstream
# inherits it, scaled by the observation's normalisations (all <= 1/300 per metre).
TOL = {"s9": 1e-7, "reward": 1e-10, "obs": 1e-6, "hp": 1e-11, "pqr": 1e-12, "prev_x": 1e-11,
       "fuel": 1e-14, "obs_reset": 1e-6}


@pytest.fixture(scope="module")
def gold():
    return oracle_lib.golden("obs_golden.npz")


def _replay(orc, g, mode):
    """Run the oracle through the golden's scripted sequence, collecting what it produced."""
    nenv = g["in_reset"].shape[1]
    ob = oracle_lib.ObrOracle(orc, nenv)
    ob.hp[:] = g["in_hp0"]
    ob.t_sec[:] = g["in_t0"]
    ob.init_reward(ob.state9(g["in_states"][0]))
    rec = {k: [] for k in ("s9", "reward", "term", "trunc", "obs", "hp", "pqr", "prev_x", "fuel",
                           "obs_reset", "t_sec", "act_hist")}
    for k in range(g["in_actions"].shape[0]):
        s9 = ob.state9(g["in_states"][k])
        r, te, tr = ob.step(s9, g["in_actions"][k], mode=mode)
        rec["s9"].append(s9); rec["reward"].append(r); rec["term"].append(te)
        rec["trunc"].append(tr); rec["obs"].append(ob.build_obs(s9))
        rec["hp"].append(ob.hp.copy()); rec["pqr"].append(ob.pqr.copy())
        rec["prev_x"].append(ob.prev_x.copy()); rec["fuel"].append(ob.fuel.copy())
        rec["t_sec"].append(ob.t_sec.copy()); rec["act_hist"].append(ob.act_hist.copy())
        m = g["in_reset"][k]
        s9r = ob.state9(g["in_states_reset"][k])
        if m.any():
            ob.reset_envs(m)
            ob.init_reward(s9r, m)
        rec["obs_reset"].append(ob.build_obs(s9r))
    return {k: np.array(v) for k, v in rec.items()}


def _gold_key(g, mode, name):
    key = f"m{mode}_{name}"
    return g[key] if key in g else g[f"m0_{name}"]


@pytest.mark.parametrize("mode", [0, 1, 2, 3])
def test_obs_reward_oracle_matches_reference(orc, gold, mode):
    out = _replay(orc, gold, mode)
    for name, tol in TOL.items():
        ref = _gold_key(gold, mode, name)
        err = np.abs(out[name].astype(np.float64) - ref.astype(np.float64)).max()
        assert err <= tol, (mode, name, err)
    assert np.array_equal(out["term"], gold["m0_term"].astype(bool))
    assert np.array_equal(out["trunc"], gold["m0_trunc"].astype(bool))
    np.testing.assert_array_equal(out["t_sec"], gold["m0_t_sec"])
    np.testing.assert_array_equal(out["act_hist"].reshape(gold["m0_act_hist"].shape),
                                  gold["m0_act_hist"])


def test_golden_covers_every_branch(gold):
    """The fixture must actually exercise what the parity test claims to pin."""
    term, trunc = gold["m0_term"].astype(bool), gold["m0_trunc"].astype(bool)
    assert term.any() and trunc.any()
    hp = gold["m0_hp"]
    assert (hp <= 0.0).any(), "an HP death"
    assert ((hp < 1.0) & (hp > 0.0)).any(), "partial damage"
    alt = -gold["m0_s9"][..., 2]
    assert (alt < 304.8).any(), "a hard-deck exit"
    assert gold["in_reset"].any(), "masked resets"
    # shaping differs between modes (mode 1 is altitude hunting), damage terms differ in 2/3
    r = [gold[f"m{m}_reward"] for m in range(4)]
    assert not np.allclose(r[0], r[1]) and not np.allclose(r[0], r[2]) and not np.allclose(r[0], r[3])


def test_state9_closed_forms(orc):
    """state9 at the official origin: N = E = 0, D = -altitude, level attitude, body velocity
    (IC rows carry feet and feet per second)."""
    import importlib
    icm = importlib.import_module("2026_ai_pilot_challenge-1st_solution_amd.ic")
    lat, lon = 37.240778, 131.869556
    rows = np.array([icm.ic_row(lat, lon, 3000.0, 800.0, 0.0, 6000.0),
                     icm.ic_row(lat, lon, 5000.0, 700.0, 90.0, 6000.0)])
    st = orc.seed(rows, 60)
    ob = oracle_lib.ObrOracle(orc, 1)
    s9 = ob.state9(st)
    # the bridge's latitude is Bowring's one-step formula: sub-millimetre at these altitudes
    np.testing.assert_allclose(s9[:, :2], 0.0, atol=1e-3)
    np.testing.assert_allclose(-s9[:, 2], [3000.0 * 0.3048, 5000.0 * 0.3048], rtol=0, atol=1e-6)
    np.testing.assert_allclose(s9[:, 5], [0.0, 90.0], atol=1e-9)
    np.testing.assert_allclose(s9[:, 3], 0.0, atol=1e-9)
    np.testing.assert_allclose(s9[:, 6], [800.0 * 0.3048, 700.0 * 0.3048], rtol=1e-9)


def test_damage_rate_tiers(orc):
    """Observation scalar 20-23 and the HP integral at known cone geometry (closed form)."""
    ob = oracle_lib.ObrOracle(orc, 1)
    # plane 0 at the origin heading north, plane 1 dead ahead at 700 m, both level
    s9 = np.zeros((2, 9))
    s9[1, 0] = 700.0
    s9[:, 2] = -5000.0
    s9[:, 6] = 200.0
    ob.init_reward(s9)
    ob.step(s9, np.zeros((2, 4)))
    r_ft = 700.0 * 3.28084
    rate = (3000.0 - r_ft) / 2500.0          # tier 1, exact alignment
    assert abs(ob.hp[1] - (1.0 - rate * 0.1)) < 1e-15
    assert ob.hp[0] == 1.0                     # plane 1 looks away (ATA 180)
    assert abs(ob.dealt[0] - rate) < 1e-15 and abs(ob.taken[1] - rate) < 1e-15


# ------------------------------------------------------------------ 214-D acceleration block
ACC0 = 164          # 214-D: own accel x 5 frames at [164:179], target accel x 5 at [179:194]


@pytest.fixture(scope="module")
def gold214():
    return oracle_lib.golden("obs214_golden.npz")


def test_obs214_oracle_matches_root_reference(orc, gold, gold214):
    """The oracle's 214-D path against the root lineage's own CPU torch path
    (cuda_fdm/obs_reward.py BatchObsReward(device="cpu", enable_kernel=False): advance's NED
    velocity difference at :569-575 and build_obs's accel columns at :702-712), driven by
    tests/golden/make_obs_golden.py --root214 on the 184-D golden's scripted states."""
    g, a = gold, gold214
    nenv = g["in_reset"].shape[1]
    ob = oracle_lib.ObrOracle(orc, nenv, accel=True)
    ob.hp[:] = g["in_hp0"]
    ob.t_sec[:] = g["in_t0"]
    ob.init_reward(ob.state9(g["in_states"][0]))
    for k in range(g["in_actions"].shape[0]):
        s9 = ob.state9(g["in_states"][k])
        r, te, tr = ob.step(s9, g["in_actions"][k])
        obs = ob.build_obs(s9, obs_dim=214)
        assert np.abs(obs.astype(np.float64) - a["a214_obs"][k]).max() <= 1e-6, k
        assert np.abs(ob.accel - a["a214_accel"][k]).max() <= 1e-9, k
        assert np.abs(ob.prev_vel_ned - a["a214_prev_vel_ned"][k]).max() <= 1e-9, k
        assert np.abs(r - a["a214_reward"][k]).max() <= 1e-10, k
        np.testing.assert_array_equal(te, a["a214_term"][k])
        np.testing.assert_array_equal(tr, a["a214_trunc"][k])
        m = g["in_reset"][k]
        s9r = ob.state9(g["in_states_reset"][k])
        if m.any():
            ob.reset_envs(m)
            ob.init_reward(s9r, m)
        obs = ob.build_obs(s9r, obs_dim=214)
        assert np.abs(obs.astype(np.float64) - a["a214_obs_reset"][k]).max() <= 1e-6, k
        assert np.abs(ob.accel - a["a214_accel_reset"][k]).max() <= 1e-9, k
        assert np.abs(ob.prev_vel_ned - a["a214_prev_vel_ned_reset"][k]).max() <= 1e-9, k


def test_obs214_golden_is_the_184_layout_plus_accel(gold, gold214):
    """The root lineage's 214-D row is the 184-D row with the acceleration block spliced in
    before the action history (claude_code/my_observation.py VECTOR_SPECS: own_accel and
    tgt_accel appended after tgt_omega), and its reward under the default configuration equals
    the 184-D lineage's; the golden must also hold non-zero accelerations to pin anything."""
    a, g = gold214, gold
    np.testing.assert_array_equal(a["a214_obs"][..., :ACC0], g["m0_obs"][..., :ACC0])
    np.testing.assert_array_equal(a["a214_obs"][..., ACC0 + 30:], g["m0_obs"][..., ACC0:])
    np.testing.assert_array_equal(a["a214_reward"], g["m0_reward"])
    assert np.all(a["a214_accel"][0] == 0.0)               # first decision: no previous velocity
    assert np.abs(a["a214_accel"][1:]).max() > 5.0
    reset_rows = np.repeat(g["in_reset"], 2, axis=1)       # masked resets zero the block
    assert np.all(a["a214_accel_reset"][reset_rows] == 0.0)


def _level_s9(north, east, alt, roll, pitch, yaw, u, v=0.0, w=0.0):
    return np.array([north, east, -alt, roll, pitch, yaw, u, v, w], np.float64)


def test_accel_closed_forms(orc):
    """Closed forms of the acceleration features, independent of the restatement's formula:
    (1) constant NED velocity -> zero acceleration in every frame; (2) a body velocity change
    dv with a known attitude gives R_b2n dv / dt, with R_b2n from scipy's intrinsic Z-Y-X
    (yaw, pitch, roll) rotation, the aerospace convention; (3) every frame is orthonormal, so
    each of the 5 frame projections keeps the vector's norm; (4) the target block of one plane
    is the own block of its partner; (5) the first decision after a reset is zero."""
    from scipy.spatial.transform import Rotation
    dt = 0.1
    rng = np.random.default_rng(3)
    ob = oracle_lib.ObrOracle(orc, 1, accel=True)
    att = [(25.0, 10.0, 70.0), (-40.0, -15.0, 200.0)]
    vb0 = [np.array([220.0, 4.0, 9.0]), np.array([180.0, -6.0, 3.0])]

    def s9_of(vb, att_, pos_shift):
        rows = []
        for i in range(2):
            r, p, y = att_[i]
            rows.append(_level_s9(3500.0 + 900.0 * i + pos_shift, 200.0 * i, 5000.0 + 50 * i,
                                  r, p, y, *vb[i]))
        return np.array(rows)

    s9a = s9_of(vb0, att, 0.0)
    ob.init_reward(s9a)
    ob.step(s9a, np.zeros((2, 4)))
    assert np.all(ob.accel == 0.0)                         # (5): prev_valid was 0
    obs = ob.build_obs(s9a, obs_dim=214)
    assert np.all(obs[:, ACC0:ACC0 + 30] == 0.0)
    # (1) same attitude and body velocity, aircraft moved: velocity in NED unchanged
    s9b = s9_of(vb0, att, 25.0)
    ob.step(s9b, np.zeros((2, 4)))
    np.testing.assert_allclose(ob.accel, 0.0, atol=1e-10)
    # (2) a body velocity change and a new attitude
    att2 = [(26.0, 10.5, 71.0), (-39.0, -14.5, 201.0)]
    vb1 = [vb0[0] + rng.normal(0, 2.0, 3), vb0[1] + rng.normal(0, 2.0, 3)]
    s9c = s9_of(vb1, att2, 50.0)
    ob.step(s9c, np.zeros((2, 4)))
    for i in range(2):
        Rn0 = Rotation.from_euler("ZYX", att[i][::-1], degrees=True).as_matrix()
        Rn1 = Rotation.from_euler("ZYX", att2[i][::-1], degrees=True).as_matrix()
        want = (Rn1 @ vb1[i] - Rn0 @ vb0[i]) / dt
        np.testing.assert_allclose(ob.accel[i], want, rtol=1e-9, atol=1e-9)
        assert np.linalg.norm(want) < 150.0                # no clamp below
    obs = ob.build_obs(s9c, obs_dim=214).astype(np.float64)
    for i in range(2):
        own = obs[i, ACC0:ACC0 + 15].reshape(5, 3) * 150.0     # normalize(x, -150, 150) = x/150
        np.testing.assert_allclose(own[0], ob.accel[i], rtol=0, atol=150.0 * 2e-7)  # world
        np.testing.assert_allclose(np.linalg.norm(own, axis=1), np.linalg.norm(ob.accel[i]),
                                   rtol=1e-5)                                     # (3)
        # body frame = R_n2b a
        Rn1 = Rotation.from_euler("ZYX", att2[i][::-1], degrees=True).as_matrix()
        np.testing.assert_allclose(own[1], Rn1.T @ ob.accel[i], rtol=0, atol=150.0 * 2e-7)
        # (4) the partner's target block: world, mybody(own body), oppbody, myvel, los of the
        # partner hold this plane's acceleration
        tgt = obs[i ^ 1, ACC0 + 15:ACC0 + 30].reshape(5, 3) * 150.0
        np.testing.assert_allclose(tgt[0], ob.accel[i], rtol=0, atol=150.0 * 2e-7)
        np.testing.assert_allclose(tgt[2], Rn1.T @ ob.accel[i], rtol=0, atol=150.0 * 2e-7)
        np.testing.assert_allclose(np.linalg.norm(tgt, axis=1), np.linalg.norm(ob.accel[i]),
                                   rtol=1e-5)
    # (5) a masked reset zeroes the block and its history
    ob.reset_envs(np.array([True]))
    ob.step(s9c, np.zeros((2, 4)))
    assert np.all(ob.accel == 0.0)
