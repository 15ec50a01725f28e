"""Host-side IC sampling and the action grid (no GPU)."""
import math

import numpy as np

from conftest import import_pkg


def test_ned_to_geodetic_known_answers():
    icm = import_pkg("ic")
    la, lo, h = icm.ned_to_geodetic(0.0, 0.0, -1000.0)
    assert abs(la - icm.ORIGIN_LAT_DEG) < 1e-9 and abs(lo - icm.ORIGIN_LON_DEG) < 1e-9
    assert h == 1000.0 / 0.3048                       # MSL = -D (cuda_fdm/rl_env.py:165-173)
    # 1 km north / east move the point by the local meridian / prime-vertical radii
    a, e2 = 6378137.0, 0.0066943799901411
    s = math.sin(math.radians(icm.ORIGIN_LAT_DEG))
    M = a * (1 - e2) / (1 - e2 * s * s) ** 1.5
    N = a / math.sqrt(1 - e2 * s * s)
    la, lo, _ = icm.ned_to_geodetic(1000.0, 0.0, 0.0)
    assert abs(math.radians(la - icm.ORIGIN_LAT_DEG) * M - 1000.0) < 0.05
    la, lo, _ = icm.ned_to_geodetic(0.0, 1000.0, 0.0)
    assert abs(math.radians(lo - icm.ORIGIN_LON_DEG) * N * math.cos(math.radians(icm.ORIGIN_LAT_DEG)) - 1000.0) < 0.05


def test_action_grid_mapping():
    """Centre bin -> zero stick, throttle 0.5 (ppo_gpu_val.py (A) known answer)."""
    icm = import_pkg("ic")
    u = icm.bins_to_controls(np.array([[10, 10, 10, 10], [0, 20, 0, 20]]))
    assert np.array_equal(u[0], [0.0, 0.0, 0.0, 0.5])
    assert np.array_equal(u[1], [-1.0, 1.0, -1.0, 1.0])


def test_samplers_shapes_and_ranges():
    icm = import_pkg("ic")
    r = icm.sample_headon(8, seed=1)
    assert r.shape == (16, 10)
    assert (r[0::2, 6] == 180.0).all() and (r[1::2, 6] == 0.0).all()
    alt_m = r[:, 2] * 0.3048
    assert ((alt_m >= 3000 - 1e-6) & (alt_m <= 10000 + 1e-6)).all()
    t = icm.sample_tailchase(8, seed=1)
    assert (t[0::2, 6] == t[1::2, 6]).all()           # shared heading
    assert (t[:, 9] == 6972.0).all()
