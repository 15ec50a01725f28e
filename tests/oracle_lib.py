"""ctypes view of the CPU checkers under oracle/ (test infrastructure only).

liborc.so is the C restatement of the reference's Python model; oracle/_ref/libf16ref_*.so
is the reference's own host-compilable C model built from its sources (present only where the
reference checkout was available at build time)."""
import ctypes
import os
import subprocess

import numpy as np

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
ORACLE = os.path.join(ROOT, "oracle")
D = ctypes.POINTER(ctypes.c_double)
_c, _i, _l = ctypes.c_double, ctypes.c_int, ctypes.c_long


def _p(a):
    return None if a is None else a.ctypes.data_as(D)


class Oracle:
    def __init__(self, L):
        self.L = L
        sig = {
            "orc_table1d": (_c, [D, D, _i, _c]),
            "orc_table2d": (_c, [D, _i, D, _i, D, _c, _c]),
            "orc_model_image": (D, []),
            "orc_mass": (None, [_c, D]),
            "orc_atmos": (None, [_c, D]),
            "orc_fdm_step1": (None, [D, D, _i, _i, D]),
            "orc_fdm_step_batch": (None, [D, D, _l, _i, _i, D, _i]),
            "orc_fdm_rollout": (None, [D, D, _l, _i, _i, _i, _i]),
            "orc_build_seed": (None, [D, _i, D]),
            "orc_euler_to_quat": (None, [_c, _c, _c, D]),
            "orc_quat_to_T": (None, [D, D]),
            "orc_mat_to_quat": (None, [D, D]),
            "orc_mat_to_euler": (None, [D, D]),
            "orc_gravity_j2": (None, [D, _c, D]),
            "orc_vcal_from_mach": (_c, [_c, _c]),
            "orc_idleff": (_c, []),
            "orc_geodetic_to_ecef": (None, [_c, _c, _c, D]),
            "orc_num_threads": (_i, []),
        }
        for name, (res, args) in sig.items():
            f = getattr(L, name)
            f.restype = res
            f.argtypes = args

    def table1d(self, x, y, key):
        x = np.ascontiguousarray(x, dtype=np.float64); y = np.ascontiguousarray(y, dtype=np.float64)
        return self.L.orc_table1d(_p(x), _p(y), len(x), key)

    def table2d(self, rx, cx, d, r, c):
        rx, cx, d = (np.ascontiguousarray(a, dtype=np.float64) for a in (rx, cx, d))
        return self.L.orc_table2d(_p(rx), len(rx), _p(cx), len(cx), _p(d), r, c)

    def mass(self, fuel):
        o = np.zeros(25)
        self.L.orc_mass(fuel, _p(o))
        return dict(cg=o[0:3], mass=o[3], J=o[4:13].reshape(3, 3), Jinv=o[13:22].reshape(3, 3), rp=o[22:25])

    def atmos(self, alt_ft):
        o = np.zeros(6)
        self.L.orc_atmos(alt_ft, _p(o))
        return dict(zip(("T", "P", "rho", "a", "sigma", "densalt"), o))

    def seed(self, ic_rows, fcs_rate=120):
        ic_rows = np.ascontiguousarray(ic_rows, dtype=np.float64).reshape(-1, 10)
        out = np.zeros((len(ic_rows), 101))
        for i, r in enumerate(ic_rows):
            r = np.ascontiguousarray(r)
            self.L.orc_build_seed(_p(r), fcs_rate, _p(out[i]))
        return out

    def step(self, states, actions, substeps, fcs_rate=120, want_obs=True, nthreads=0):
        """In place on a C-contiguous (nac, 101) array; returns the (nac, 17) output."""
        assert states.flags.c_contiguous and states.dtype == np.float64
        actions = np.ascontiguousarray(actions, dtype=np.float64)
        obs = np.zeros((states.shape[0], 17)) if want_obs else None
        self.L.orc_fdm_step_batch(_p(states), _p(actions), states.shape[0], substeps, fcs_rate,
                                  _p(obs), nthreads)
        return obs

    def rollout(self, states, actions, substeps, fcs_rate=120, nthreads=0):
        actions = np.ascontiguousarray(actions, dtype=np.float64)
        self.L.orc_fdm_rollout(_p(states), _p(actions), states.shape[0], actions.shape[0],
                               substeps, fcs_rate, nthreads)


class RefModel:
    """The reference's own fdm.cuh compiled for the host (oracle/_ref)."""

    def __init__(self, path):
        self.L = ctypes.CDLL(path)
        self.L.ref_fdm_step_batch.argtypes = [D, D, _l, _i, D, _i]
        self.L.ref_fdm_rollout.argtypes = [D, D, _l, _i, _i, _i]
        self.L.ref_fcs_rate.restype = _i

    def step(self, states, actions, substeps, nthreads=0):
        actions = np.ascontiguousarray(actions, dtype=np.float64)
        obs = np.zeros((states.shape[0], 17))
        self.L.ref_fdm_step_batch(_p(states), _p(actions), states.shape[0], substeps, _p(obs), nthreads)
        return obs


def build():
    subprocess.run(["make", "-s", "-C", ORACLE], check=True)


def load():
    """The C restatement; F16_ORACLE_LIB names another build of it (the sanitizer build of
    `make -C oracle sanitize`, run with its runtime preloaded)."""
    path = os.environ.get("F16_ORACLE_LIB") or os.path.join(ORACLE, "liborc.so")
    if not os.path.exists(path):
        build()
    return Oracle(ctypes.CDLL(path))


def load_ref(fcs_rate=120):
    path = os.path.join(ORACLE, "_ref", f"libf16ref_{fcs_rate}.so")
    return RefModel(path) if os.path.exists(path) else None


def golden(name):
    return np.load(os.path.join(ROOT, "tests", "golden", name))


# Column groups whose members share one physical scale: the components of one vector or
# quaternion of the 101-double state (cuda_fdm/ic.py:92-114) and of the 17-value output.
def _spans(*bounds):
    return [list(range(a, b)) for a, b in zip(bounds, bounds[1:])]


STATE_GROUPS = (_spans(0, 3, 6, 10, 13, 14, 15, 18, 21, 25, 29, 33, 37, 40, 43, 46, 49, 52,
                       55, 58, 61, 64, 67, 70, 73, 74, 75, 76, 77, 79, 82)
                + [[k] for k in range(82, 101)])
OBS_GROUPS = _spans(0, 3, 6, 9, 12, 14, 15, 16, 17)


def rel_err(got, want, floor_frac=1e-3):
    """Per-state-variable relative error |got - want| / max(|want|, floor), where the floor is
    floor_frac times the largest magnitude of the variable's group (the vector it belongs to)
    over the batch.  Components that are zero by symmetry (e.g. the roll acceleration of a
    wings-level aircraft, pure rounding noise) are judged on their vector's scale."""
    got = np.asarray(got, dtype=np.float64); want = np.asarray(want, dtype=np.float64)
    groups = {101: STATE_GROUPS, 17: OBS_GROUPS}.get(want.shape[-1])
    if groups is None:
        groups = [[k] for k in range(want.shape[-1])]
    scale = np.zeros(want.shape[-1])
    for g in groups:
        scale[g] = np.max(np.abs(want[..., g])) if want.size else 0.0
    den = np.maximum(np.abs(want), np.maximum(floor_frac * scale, 1e-300))
    return np.abs(got - want) / den



def scaled_abs_err(got, want):
    """|got - want| / (largest |want| of the variable's group over the batch): the absolute
    difference in units of its vector's magnitude (rel_err with floor_frac = 1 and no per-entry
    denominator).  A component passing through zero -- an acceleration in level flight, a body
    rate between manoeuvres -- is judged by the scale at which its vector is computed."""
    return np.abs(np.asarray(got, dtype=np.float64) - np.asarray(want, dtype=np.float64)) / \
        _group_scale(want)


def _group_scale(want):
    want = np.asarray(want, dtype=np.float64)
    groups = {101: STATE_GROUPS, 17: OBS_GROUPS}.get(want.shape[-1])
    if groups is None:
        groups = [[k] for k in range(want.shape[-1])]
    scale = np.zeros(want.shape[-1])
    for g in groups:
        scale[g] = np.max(np.abs(want[..., g])) if want.size else 0.0
    return np.maximum(scale, 1e-300)


def raw_rel_err(got, want):
    """|got - want| / |want| with no floor (entries whose reference value is exactly zero report
    the absolute difference): the per-variable figure before rel_err's scale floor."""
    got = np.asarray(got, dtype=np.float64); want = np.asarray(want, dtype=np.float64)
    d = np.abs(got - want)
    return np.where(want != 0, d / np.where(want != 0, np.abs(want), 1.0), d)

# ------------------------------------------------------------------ observation / reward oracle
class _OrcObrStruct(ctypes.Structure):
    _fields_ = [("nenv", ctypes.c_long)] + [
        (n, ctypes.c_void_p) for n in ("hp", "fuel", "t_sec", "prev_att", "prev_valid", "pqr",
                                      "dealt", "taken", "hp_loss", "act_hist", "prev_x",
                                      "prev_x_valid", "prev_alt_log", "prev_vel_ned", "accel")]


REWARD_CFG = np.array([1.0, 10.0, 0.0001, 5.0, -5.0, 5.0, -5.0, -4.0])  # MY_REWARD_CONFIG
REWARD_CFG_KEYS = ("own_damage_weight", "damage_scale", "shaping_reward_scale", "win_reward",
                   "loss_reward", "timeout_win_reward", "timeout_loss_reward",
                   "timeout_draw_reward")


class ObrOracle:
    """Numpy-backed reconstructor state + the C restatement of BatchObsReward."""

    def __init__(self, orc, nenv, accel=False):
        self.L = orc.L
        n = 2 * nenv
        self.nenv = nenv
        self.hp = np.ones(n); self.fuel = np.ones(n); self.t_sec = np.zeros(nenv)
        self.prev_att = np.zeros((n, 3)); self.prev_valid = np.zeros(n, np.uint8)
        self.pqr = np.zeros((n, 3)); self.dealt = np.zeros(n); self.taken = np.zeros(n)
        self.hp_loss = np.zeros(n); self.act_hist = np.zeros((n, 5, 4)); self.prev_x = np.zeros(n)
        self.prev_x_valid = np.zeros(n, np.uint8); self.prev_alt_log = np.zeros(n)
        self.prev_vel_ned = np.zeros((n, 3)) if accel else None
        self.accel = np.zeros((n, 3)) if accel else None
        L = self.L
        L.orc_state9.argtypes = [D, D]
        L.orc_state9_batch.argtypes = [D, _l, D]
        L.orc_obr_reset_envs.argtypes = [ctypes.c_void_p, ctypes.c_void_p]
        L.orc_obr_init_reward.argtypes = [ctypes.c_void_p, D, ctypes.c_void_p]
        L.orc_obr_step.argtypes = [ctypes.c_void_p, D, D, D, ctypes.c_int, ctypes.c_double,
                                   ctypes.c_double, ctypes.c_double, D, ctypes.c_void_p,
                                   ctypes.c_void_p]
        L.orc_obr_build_obs.argtypes = [ctypes.c_void_p, D, ctypes.c_int, ctypes.c_void_p,
                                        ctypes.c_void_p]

    def _struct(self):
        s = _OrcObrStruct()
        s.nenv = self.nenv
        for name, _ in _OrcObrStruct._fields_[1:]:
            arr = getattr(self, name)
            setattr(s, name, None if arr is None else arr.ctypes.data)
        return s

    def state9(self, states):
        states = np.ascontiguousarray(states, dtype=np.float64).reshape(-1, 101)
        out = np.zeros((states.shape[0], 9))
        self.L.orc_state9_batch(_p(states), states.shape[0], _p(out))
        return out

    def reset_envs(self, mask=None):
        s = self._struct()
        m = None if mask is None else np.ascontiguousarray(mask, np.uint8)
        self.L.orc_obr_reset_envs(ctypes.byref(s), None if m is None else m.ctypes.data)

    def init_reward(self, s9, mask=None):
        s = self._struct()
        s9 = np.ascontiguousarray(s9, np.float64)
        m = None if mask is None else np.ascontiguousarray(mask, np.uint8)
        self.L.orc_obr_init_reward(ctypes.byref(s), _p(s9), None if m is None else m.ctypes.data)

    def step(self, s9, actions, mode=0, coef=5.0, cfg=REWARD_CFG, min_alt=304.8, max_time=200.0):
        s = self._struct()
        s9 = np.ascontiguousarray(s9, np.float64)
        actions = np.ascontiguousarray(actions, np.float64)
        cfg = np.ascontiguousarray(cfg, np.float64)
        reward = np.zeros(2 * self.nenv)
        term = np.zeros(self.nenv, np.uint8); trunc = np.zeros(self.nenv, np.uint8)
        self.L.orc_obr_step(ctypes.byref(s), _p(s9), _p(actions), _p(cfg), mode, coef, min_alt,
                            max_time, _p(reward), term.ctypes.data, trunc.ctypes.data)
        return reward, term.astype(bool), trunc.astype(bool)

    def build_obs(self, s9, obs_dim=184, mask=None):
        s = self._struct()
        s9 = np.ascontiguousarray(s9, np.float64)
        obs = np.zeros((2 * self.nenv, obs_dim), np.float32)
        m = None if mask is None else np.ascontiguousarray(mask, np.uint8)
        self.L.orc_obr_build_obs(ctypes.byref(s), _p(s9), obs_dim,
                                 None if m is None else m.ctypes.data, obs.ctypes.data)
        return obs


# ------------------------------------------------------------------ drift envelope (BASELINE C1)
# 8 replicas of C1 (seeds 0-7): 64 head-on engagements each, 600 decisions of i.i.d. 21-bin
# actions, FCS at 120 Hz.  tests/golden/make_drift_envelope.py writes the reference pair's
# divergence curve on exactly these inputs.
DRIFT_REPLICAS, DRIFT_NENV, DRIFT_NDEC = 8, 64, 600
DRIFT_QUANTILES = (0.5, 0.75, 0.9, 1.0)
# the stated bound: every quantile of the divergence at decision d <= DRIFT_K x the reference
# pair's same quantile anywhere in decisions d .. d + DRIFT_LAG (floored at DRIFT_FLOOR_FT)
DRIFT_K, DRIFT_LAG, DRIFT_FLOOR_FT = 30.0, 50, 1e-6
EARTH_RADIUS_FT = 20925646.32546


def c1_replicas(icm):
    """IC rows (1024, 10) and actions (600, 1024, 4) of the 8 C1 replicas."""
    ic = np.concatenate([icm.sample_headon(DRIFT_NENV, seed=s) for s in range(DRIFT_REPLICAS)])
    acts = np.concatenate([icm.random_bin_actions(DRIFT_NDEC, 2 * DRIFT_NENV, seed=s)
                           for s in range(DRIFT_REPLICAS)], axis=1)
    return ic, acts


def altitude_m(states):
    return (np.linalg.norm(states[:, 0:3], axis=1) - EARTH_RADIUS_FT) * 0.3048


def drift_quantiles(a, b, alive):
    """DRIFT_QUANTILES of |ECI position a - b| (ft) over the aircraft in `alive`."""
    div = np.linalg.norm(a[:, 0:3] - b[:, 0:3], axis=1)[alive]
    return np.array([np.quantile(div, q) if div.size else 0.0 for q in DRIFT_QUANTILES])


def drift_envelope(env, d):
    """The bound at decision index d (0-based) for each quantile, from the fixture."""
    ref = env["pos_ft"]
    return DRIFT_K * np.maximum(DRIFT_FLOOR_FT, ref[d:min(d + DRIFT_LAG, len(ref) - 1) + 1].max(0))
