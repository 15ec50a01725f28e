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


def _pairwise_contest(rng, npairs, scenario_b_prob, fuel_range):
    """The reference's per-engagement draws (rl_env.py:218-250, rng.choice for the 3-9 distance)
    converted one engagement at a time."""
    icm = import_pkg("ic")
    rows = []
    for _ in range(npairs):
        alt = rng.uniform(2000.0, 30000.0)
        spd = rng.uniform(200.0, 300.0)
        side = bool(rng.integers(0, 2))
        b = rng.random() < scenario_b_prob
        if b:
            half, hdg = 0.5 * 5539.0, ((0.0, 180.0) if side else (180.0, 0.0))
        else:
            head = bool(rng.integers(0, 2))
            half = 0.5 * float(rng.choice(np.asarray([2000.0, 2500.0, 3000.0]))) * 0.3048
            hdg = (270.0, 90.0) if head else (90.0, 270.0)
        fuel = rng.uniform(*fuel_range, size=2) if fuel_range else (3000.0, 3000.0)
        for k, sgn in ((0, -1.0 if side else 1.0), (1, 1.0 if side else -1.0)):
            la, lo, h = icm.ned_to_geodetic(3500.0 + sgn * half, 0.0, -alt * 0.3048)
            rows.append([la, lo, h, spd / 0.3048, 0, 0, hdg[k], 0, 0, fuel[k]])
    return np.asarray(rows, dtype=np.float64)


def test_contest_rows_match_pairwise_draws():
    """The batched sampler (per-engagement draws, one vectorised geodetic conversion) gives the
    rows of drawing and converting engagement by engagement with the reference's calls, from the
    same Generator state, and leaves the Generator where the pairwise draws leave it."""
    icm = import_pkg("ic")
    for kw in (dict(scenario_b_prob=0.0, fuel_range=None), dict(scenario_b_prob=0.35, fuel_range=None),
               dict(scenario_b_prob=0.0, fuel_range=(1500.0, 3000.0))):
        r1, r2 = np.random.default_rng(7), np.random.default_rng(7)
        a = icm.contest_rows(r1, 300, **kw)
        b = _pairwise_contest(r2, 300, **kw)
        np.testing.assert_allclose(a, b, rtol=0, atol=1e-9)
        assert r1.random() == r2.random()
    # scenario A: abeam on the north axis, east/west headings, 3-9 separations
    a = icm.contest_rows(np.random.default_rng(1), 200)
    assert set(np.unique(a[:, 6])) <= {90.0, 270.0} and (a[0::2, 6] != a[1::2, 6]).all()
    assert icm.contest_rows(np.random.default_rng(1), 0).shape == (0, 10)


def test_build_seed_vector_refuses_geocentric_before_device_work():
    """The reference's keyword interface (cuda_fdm/ic.py:117-138); geocentric latitude is not
    supported and is refused on the host, before any device call."""
    import pytest
    icm = import_pkg("ic")
    with pytest.raises(ValueError, match="geodetic"):
        icm.build_seed_vector(37.0, 131.0, 10000.0, 800.0, lat_type="geocentric")
