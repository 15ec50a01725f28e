"""Initial-condition sampling and the discrete action grid.

* ``ned_to_geodetic`` places an aircraft given in the contest's N/E/D frame about the official
  origin (37.240778 N, 131.869556 E, cuda_fdm/rl_env.py:33-37) at a geodetic latitude and
  longitude, with altitude MSL = -D (cuda_fdm/rl_env.py:165-173).  The reference uses pymap3d
  for the horizontal inverse; this is an independent WGS84 implementation (tangent-plane ->
  ECEF, then Bowring's iteration to convergence).  IC sampling is not on the parity path: the
  same IC rows feed the GPU and the CPU restatement.
* samplers for the BASELINE workloads (head-on and tail-chase engagements);
* ``action_grid`` / ``bins_to_controls``: 21 bins on [-1, 1], throttle = 0.5 z + 0.5
  (research/competition_36500/runtime/cuda_fdm/ppo_gpu.py:178-181, 361-370);
* ``build_seed_vector``: one IC's 101-value seed state under the reference's name and keywords,
  computed by the device seeding kernel (the reference's host helpers geodetic_to_ecef,
  ic_to_seedargs and _flatten_state are that kernel's steps, cuda_fdm/ic.py:18-114).
"""
import math

import numpy as np

ORIGIN_LAT_DEG = 37.240778
ORIGIN_LON_DEG = 131.869556
WGS84_A_M = 6378137.0
WGS84_E2 = 0.0066943799901411
FT2M = 0.3048
M2FT = 1.0 / FT2M


def _geodetic_to_ecef_m(lat, lon, h):
    s, c = np.sin(lat), np.cos(lat)
    n = WGS84_A_M / np.sqrt(1.0 - WGS84_E2 * s * s)
    return ((n + h) * c * np.cos(lon), (n + h) * c * np.sin(lon), (n * (1.0 - WGS84_E2) + h) * s)


def ned_to_geodetic(n, e, d, lat0=ORIGIN_LAT_DEG, lon0=ORIGIN_LON_DEG, h0=0.0):
    """N/E/D metres about (lat0, lon0, h0) -> (lat_deg, lon_deg, alt_ft) with alt = -D."""
    n, e, d = (np.asarray(v, dtype=np.float64) for v in (n, e, d))
    la0, lo0 = math.radians(lat0), math.radians(lon0)
    x0, y0, z0 = _geodetic_to_ecef_m(la0, lo0, h0)
    sl, cl, so, co = math.sin(la0), math.cos(la0), math.sin(lo0), math.cos(lo0)
    u = -d
    x = x0 - sl * co * n - so * e + cl * co * u
    y = y0 - sl * so * n + co * e + cl * so * u
    z = z0 + cl * n + sl * u
    lon = np.arctan2(y, x)
    p = np.hypot(x, y)
    lat = np.arctan2(z, p * (1.0 - WGS84_E2))
    for _ in range(8):
        s = np.sin(lat)
        nn = WGS84_A_M / np.sqrt(1.0 - WGS84_E2 * s * s)
        lat = np.arctan2(z + WGS84_E2 * nn * s, p)
    return np.degrees(lat), np.degrees(lon), -d * M2FT


def build_seed_vector(lat_deg, lon_deg, alt_ft, vt_fps, gamma_deg=0.0, phi_deg=0.0, psi_deg=0.0,
                      theta_deg=0.0, alpha_deg=0.0, beta_deg=0.0, lat_type="geodetic",
                      fuel_lbs=6000.0, throttle=0.8, fcs_rate=120, device="cuda"):
    """The 101-value seed state of one initial condition (cuda_fdm/ic.py:117-138: the same
    keywords in the same order), as a list of floats, computed on the device by f16_seed_batch
    (no host model).  As in the reference, gamma_deg and throttle do not enter the seed (the
    flight-path angle is not used by its ic_to_seedargs; the throwaway force path runs at 0.8
    throttle).  fcs_rate: 120 for the root lineage, 60 for the 184-D one.  Only geodetic
    latitude is supported (ValueError otherwise, before any device work)."""
    if lat_type != "geodetic":
        raise ValueError("only geodetic IC latitude is supported")
    import torch
    from .gpu_env import GpuDogfight
    sim = GpuDogfight(1, planes_per_env=1, fcs_rate=fcs_rate, device=device)
    row = [[lat_deg, lon_deg, alt_ft, vt_fps, phi_deg, theta_deg, psi_deg, alpha_deg, beta_deg,
            fuel_lbs]]
    sim.seed_rows(torch.tensor(row, dtype=torch.float64, device=sim.device))
    return sim.states[0].tolist()


def ic_row(lat_deg, lon_deg, alt_ft, vt_fps, psi_deg, fuel_lbs, phi_deg=0.0, theta_deg=0.0,
           alpha_deg=0.0, beta_deg=0.0):
    return [lat_deg, lon_deg, alt_ft, vt_fps, phi_deg, theta_deg, psi_deg, alpha_deg, beta_deg,
            fuel_lbs]


def sample_headon(nenv, seed=0, fuel_lbs=6972.0):
    """BASELINE C1: alt U[3,10] km, speed U[150,300] m/s, separation U[5,15] km, opposing
    headings on the north axis about N = 3500 m (rl_env.py:252-258 pattern).  Returns (2*nenv, 10)
    IC rows, plane 0 at N = c + d/2 heading 180 deg, plane 1 at N = c - d/2 heading 0 deg."""
    rng = np.random.default_rng(seed)
    alt = rng.uniform(3000.0, 10000.0, nenv)
    spd = rng.uniform(150.0, 300.0, nenv)
    sep = rng.uniform(5000.0, 15000.0, nenv)
    c = 3500.0
    rows = np.zeros((2 * nenv, 10))
    for plane, sign, psi in ((0, 1.0, 180.0), (1, -1.0, 0.0)):
        la, lo, h = ned_to_geodetic(c + sign * 0.5 * sep, np.zeros(nenv), -alt)
        for k in range(nenv):
            rows[2 * k + plane] = ic_row(la[k], lo[k], h[k], spd[k] * M2FT, psi, fuel_lbs)
    return rows


def sample_tailchase(nenv, seed=0, fuel_lbs=6972.0):
    """BASELINE C2: both aircraft share a random heading; the pursuer (plane 0) sits 1-3 km
    behind the target (plane 1); alt U[4,8] km, speed U[200,280] m/s.  Returns (2*nenv, 10)."""
    rng = np.random.default_rng(seed)
    alt = rng.uniform(4000.0, 8000.0, nenv)
    spd = rng.uniform(200.0, 280.0, nenv)
    gap = rng.uniform(1000.0, 3000.0, nenv)
    psi = rng.uniform(0.0, 360.0, nenv)
    cn, ce = 3500.0, 0.0
    hn, he = np.cos(np.radians(psi)), np.sin(np.radians(psi))
    rows = np.zeros((2 * nenv, 10))
    lt, ot, ht = ned_to_geodetic(cn + 0.5 * gap * hn, ce + 0.5 * gap * he, -alt)
    lp, op, hp = ned_to_geodetic(cn - 0.5 * gap * hn, ce - 0.5 * gap * he, -alt)
    for k in range(nenv):
        rows[2 * k] = ic_row(lp[k], op[k], hp[k], spd[k] * M2FT, psi[k], fuel_lbs)
        rows[2 * k + 1] = ic_row(lt[k], ot[k], ht[k], spd[k] * M2FT, psi[k], fuel_lbs)
    return rows


def sample_random_valid(nenv, seed=0, fuel_lbs=6972.0):
    """BASELINE C3: a random valid state per aircraft -- position within +-20 km of the contest
    centre (north and east; altitude 0.5-12 km, so every aircraft starts above the hard deck),
    airspeed U[100, 350] m/s, any attitude (roll U[-180, 180], pitch U[-89, 89], heading
    U[0, 360] deg: a uniformly random direction of the body axes' Euler parameterisation),
    alpha U[-10, 40] and beta U[-25, 25] deg (inside the aero tables' breakpoints, so the
    quaternion and velocity agree on them), fuel U[0.2, 1] of full.  Returns (2*nenv, 10) IC
    rows; the device seeding (f16_seed_batch) turns them into consistent 101-value states."""
    rng = np.random.default_rng(seed)
    n = 2 * nenv
    north = 3500.0 + rng.uniform(-20000.0, 20000.0, n)
    east = rng.uniform(-20000.0, 20000.0, n)
    alt = rng.uniform(500.0, 12000.0, n)
    spd = rng.uniform(100.0, 350.0, n)
    phi = rng.uniform(-180.0, 180.0, n)
    theta = rng.uniform(-89.0, 89.0, n)
    psi = rng.uniform(0.0, 360.0, n)
    alpha = rng.uniform(-10.0, 40.0, n)
    beta = rng.uniform(-25.0, 25.0, n)
    fuel = rng.uniform(0.2, 1.0, n) * fuel_lbs
    la, lo, h = ned_to_geodetic(north, east, -alt)
    rows = np.zeros((n, 10))
    rows[:, 0], rows[:, 1], rows[:, 2], rows[:, 3] = la, lo, h, spd * M2FT
    rows[:, 4], rows[:, 5], rows[:, 6] = phi, theta, psi
    rows[:, 7], rows[:, 8], rows[:, 9] = alpha, beta, fuel
    return rows


def action_grid(num_bins=21):
    """linspace(-1, 1, num_bins) (ppo_gpu.py:178-181)."""
    return np.linspace(-1.0, 1.0, num_bins)


def bins_to_controls(idx, num_bins=21):
    """(..., 4) integer bins -> (..., 4) controls; throttle = 0.5 z + 0.5 (ppo_gpu.py:361-370)."""
    g = action_grid(num_bins)
    u = g[np.asarray(idx)]
    u[..., 3] = 0.5 * u[..., 3] + 0.5
    return u


def random_bin_actions(ndec, nac, seed=0, num_bins=21):
    """(ndec, nac, 4) controls from i.i.d. uniform bins (BASELINE C1/C2 action model)."""
    rng = np.random.default_rng(seed)
    return bins_to_controls(rng.integers(0, num_bins, size=(ndec, nac, 4)), num_bins)


# contest distribution (research/competition_36500/runtime/cuda_fdm/rl_env.py:199-212)
CONTEST_CENTER_N = 3500.0
CONTEST_CENTER_E = 0.0
CONTEST_ALT_FT = (2000.0, 30000.0)
CONTEST_SPEED_MPS = (200.0, 300.0)
CONTEST_DIST_A_FT = (2000.0, 2500.0, 3000.0)
CONTEST_DIST_HEADON_FT = 5539.0 / FT2M
CONTEST_FUEL_LBS = 3000.0


def _contest_draw(rng, scenario_b_prob=0.0, alt_ft=None, speed=None, side_swap=None,
                  scenario_b=None, head_swap=None, dist_ft=None, fuel_range=None):
    """One engagement's draws, in the reference's order (rl_env.py:218-250): altitude, speed,
    side swap, scenario B, then heading swap and 3-9 distance (scenario A only), then the optional
    per-aircraft fuel.  Returns (own_n, tgt_n, d, speed_fps, own_hdg, tgt_hdg, fuel0, fuel1)."""
    alt_ft = float(rng.uniform(*CONTEST_ALT_FT) if alt_ft is None else alt_ft)
    speed = float(rng.uniform(*CONTEST_SPEED_MPS) if speed is None else speed)
    side_swap = bool(rng.integers(0, 2) if side_swap is None else side_swap)
    scenario_b = bool(rng.random() < scenario_b_prob if scenario_b is None else scenario_b)
    if scenario_b:
        half = 0.5 * CONTEST_DIST_HEADON_FT * FT2M
        own_hdg, tgt_hdg = (0.0, 180.0) if side_swap else (180.0, 0.0)
    else:
        head_swap = bool(rng.integers(0, 2) if head_swap is None else head_swap)
        # rng.integers(0, 3) consumes the Generator's stream exactly as rng.choice of a 3-element
        # array does (the reference's call), at a seventh of the cost
        dist_ft = float(CONTEST_DIST_A_FT[int(rng.integers(0, 3))] if dist_ft is None else dist_ft)
        half = 0.5 * dist_ft * FT2M
        own_hdg, tgt_hdg = (270.0, 90.0) if head_swap else (90.0, 270.0)
    own_n = CONTEST_CENTER_N + (-half if side_swap else half)
    tgt_n = CONTEST_CENTER_N + (half if side_swap else -half)
    # fuel_range (lb): per-aircraft fuel drawn after the reference's draws (league workload with
    # fuel exhaustion); None keeps the contest's 3000 lb
    f = (rng.uniform(*fuel_range, size=2) if fuel_range is not None
         else (CONTEST_FUEL_LBS, CONTEST_FUEL_LBS))
    return (own_n, tgt_n, -alt_ft * FT2M, speed * M2FT, own_hdg, tgt_hdg, float(f[0]),
            float(f[1]))


def _rows_from_draws(dr):
    """(P, 8) draws -> (2P, 10) IC rows; the geodetic conversion runs once over all aircraft."""
    dr = np.asarray(dr, dtype=np.float64).reshape(-1, 8)
    P = dr.shape[0]
    n = np.stack([dr[:, 0], dr[:, 1]], axis=1).reshape(-1)
    d = np.repeat(dr[:, 2], 2)
    la, lo, h = ned_to_geodetic(n, np.full(2 * P, CONTEST_CENTER_E), d)
    rows = np.zeros((2 * P, 10))
    rows[:, 0], rows[:, 1], rows[:, 2] = la, lo, h
    rows[:, 3] = np.repeat(dr[:, 3], 2)
    rows[:, 6] = dr[:, 4:6].reshape(-1)
    rows[:, 9] = dr[:, 6:8].reshape(-1)
    return rows


def contest_pair(rng, scenario_b_prob=0.0, **fixed):
    """One engagement's (own, target) IC rows from the contest distribution (rl_env.py:218-250).
    Scenario A puts the two aircraft abeam on the north axis with opposite east/west headings;
    B is head-on.  Keyword arguments fix individual draws (alt_ft, speed, side_swap, scenario_b,
    head_swap, dist_ft, fuel_range)."""
    return [list(r) for r in _rows_from_draws([_contest_draw(rng, scenario_b_prob, **fixed)])]


def contest_rows(rng, npairs, scenario_b_prob=0.0, fuel_range=None):
    """(2*npairs, 10) IC rows, plane 0 = ownship, plane 1 = target: the per-engagement draws in
    the reference's order, then one vectorised geodetic conversion."""
    if npairs == 0:
        return np.zeros((0, 10))
    return _rows_from_draws([_contest_draw(rng, scenario_b_prob, fuel_range=fuel_range)
                             for _ in range(npairs)])
