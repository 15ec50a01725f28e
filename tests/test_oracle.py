"""CPU checks that pin the C restatement of the reference model (oracle/f16_oracle.c).

Each check is chosen so that a plausible restatement mistake (wrong operand, sign, index or
order; a dropped term) fails it: closed forms and textbook formulas, invariants, brute force on
small tables, values printed in the reference's own generated header, golden vectors written
from the reference's Python, and the reference's own host-compiled C model (oracle/_ref)."""
import ast
import importlib
import importlib.util
import math
import os
import re

import numpy as np
import pytest

import oracle_lib
from conftest import ROOT

REF = "/root/reference"
IMG_HDR = os.path.join(ROOT, "2026_ai_pilot_challenge-1st_solution_amd", "csrc", "f16_model_gen.h")


def header_defines():
    out = {}
    for line in open(IMG_HDR):
        m = re.match(r"#define (F16M_\w+) \((.*)\)$", line.strip())
        if m:
            try:
                out[m.group(1)] = float(m.group(2))
            except ValueError:
                pass
        m = re.match(r"#define (F16M_\w+) (\d+)$", line.strip())
        if m:
            out[m.group(1)] = int(m.group(2))
    return out


def image(orc):
    n = header_defines()["F16M_IMAGE_LEN"]
    p = orc.L.orc_model_image()
    return np.ctypeslib.as_array(p, shape=(n,)).copy()


# ------------------------------------------------------------------ tables
def test_table1d_closed_forms(orc):
    x = [-0.175, -0.087, 0.0, 0.087, 0.175, 0.262]
    y = [0.003, 0.001, 0.0, 0.001, 0.002, 0.004]
    for xi, yi in zip(x, y):                      # exact at breakpoints
        assert orc.table1d(x, y, xi) == yi
    assert orc.table1d(x, y, -1.0) == y[0]        # clamped, no extrapolation
    assert orc.table1d(x, y, 5.0) == y[-1]
    for a, b, ya, yb in zip(x, x[1:], y, y[1:]):  # interior: the linear closed form
        for t in (0.25, 0.5, 0.9):
            k = a + t * (b - a)
            want = (k - a) / (b - a) * (yb - ya) + ya
            assert abs(orc.table1d(x, y, k) - want) <= 1e-16 * max(1.0, abs(want))
    ks = np.linspace(-0.3, 0.4, 301)              # brute force against numpy's interpolation
    got = np.array([orc.table1d(x, y, k) for k in ks])
    assert np.allclose(got, np.interp(ks, x, y), rtol=0, atol=1e-16)
    assert math.isnan(orc.table1d(x, y, float("nan")))


def test_table2d_closed_forms(orc):
    rx = np.array([-0.175, -0.087, 0.0, 0.087])
    cx = np.array([-0.436, -0.218, 0.0, 0.218, 0.436])
    rng = np.random.default_rng(3)
    d = rng.normal(size=(4, 5))
    for i in range(4):                              # corners exact
        for j in range(5):
            assert abs(orc.table2d(rx, cx, d, rx[i], cx[j]) - d[i, j]) <= 1e-15 * abs(d[i, j]) + 1e-16
    for _ in range(200):                            # bilinear closed form inside
        r, c = rng.uniform(rx[0], rx[-1]), rng.uniform(cx[0], cx[-1])
        i = np.searchsorted(rx, r) ; i = min(max(i, 1), 3)
        j = np.searchsorted(cx, c) ; j = min(max(j, 1), 4)
        tr = (r - rx[i - 1]) / (rx[i] - rx[i - 1]); tc = (c - cx[j - 1]) / (cx[j] - cx[j - 1])
        want = ((1 - tr) * (1 - tc) * d[i - 1, j - 1] + tr * (1 - tc) * d[i, j - 1]
                + (1 - tr) * tc * d[i - 1, j] + tr * tc * d[i, j])
        assert abs(orc.table2d(rx, cx, d, r, c) - want) < 1e-13
    # factors clamp to [0, 1] on both axes
    assert abs(orc.table2d(rx, cx, d, -9.0, -9.0) - d[0, 0]) < 1e-15
    assert abs(orc.table2d(rx, cx, d, 9.0, 9.0) - d[-1, -1]) < 1e-14


# ------------------------------------------------------------------ model data vs the reference
def _py_literal(path, name):
    tree = ast.parse(open(path, encoding="utf-8").read())
    for node in tree.body:
        if isinstance(node, ast.Assign) and any(getattr(t, "id", None) == name for t in node.targets):
            return ast.literal_eval(node.value)
    raise KeyError(name)


@pytest.mark.skipif(not os.path.isdir(REF), reason="reference checkout absent")
def test_model_image_matches_reference_data(orc):
    """Our XML parser's tables equal the numbers in the reference's extracted data (read as
    text: cuda_fdm/ref/f16_aero_data.py, jsb_propulsion.py)."""
    img = image(orc)
    hd = header_defines()
    axes = _py_literal(os.path.join(REF, "cuda_fdm/ref/f16_aero_data.py"), "AXES")
    for ax, fns in axes.items():
        for f in fns:
            t = f["table"]
            if t is None:
                continue
            short = f["name"].split("/")[-1]
            off = hd[f"F16M_T_AERO_{short}_OFF"]
            rg = hd[f"F16M_T_AERO_{short}_RG"]
            if t["type"] == "1d":
                xs = [r[0] for r in t["rows"]]; ys = [r[1] for r in t["rows"]]
                assert list(img[rg:rg + len(xs)]) == xs, short
                assert list(img[off:off + len(ys)]) == ys, short
            else:
                cg = hd[f"F16M_T_AERO_{short}_CG"]
                nr, nc = len(t["rowvals"]), len(t["colvals"])
                assert list(img[rg:rg + nr]) == t["rowvals"], short
                assert list(img[cg:cg + nc]) == t["colvals"], short
                assert list(img[off:off + nr * nc]) == [v for row in t["data"] for v in row], short
    prop = os.path.join(REF, "cuda_fdm/ref/jsb_propulsion.py")
    for tname, key in (("ENG_IDLE", "_IDLE"), ("ENG_MIL", "_MIL"), ("ENG_AUG", "_AUG")):
        data = _py_literal(prop, key)
        off = hd[f"F16M_T_{tname}_OFF"]
        flat = [v for row in data for v in row]
        assert list(img[off:off + len(flat)]) == flat, tname


@pytest.mark.skipif(not os.path.isdir(REF), reason="reference checkout absent")
def test_derived_constants_match_reference_header():
    """Start-up constants equal the values printed in cuda_fdm/gen/f16_gen.cuh:9-60."""
    txt = open(os.path.join(REF, "cuda_fdm/gen/f16_gen.cuh"), encoding="utf-8").read()

    def arr(name):
        m = re.search(name + r"\[\d+\] = \{([^}]*)\}", txt)
        return [float(v) for v in m.group(1).split(",")]

    def scal(name):
        return float(re.search(r"double " + name + r" = ([^;]+);", txt).group(1))

    hdr = open(IMG_HDR).read()

    def harr(name):
        m = re.search(r"#define " + name + r"_INIT \{([^}]*)\}", hdr)
        return [float(v) for v in m.group(1).split(",")]
    for ours, theirs in (("F16M_ATM_LAPSE", "ATM_LAPSE"), ("F16M_ATM_PBRK", "ATM_PBRK"),
                         ("F16M_ATM_DBRK", "ATM_DBRK")):
        assert harr(ours) == arr(theirs), ours
    hd = header_defines()
    for ours, theirs in (("F16M_IDLEFF", "IdleFF"), ("F16M_SLGRAVITY", "SLGRAVITY"),
                         ("F16M_STD_SL_SOUNDSPEED", "STD_SL_SOUNDSPEED"), ("F16M_RENG", "Reng"),
                         ("F16M_FPSTOKTS", "FPSTOKTS"), ("F16M_WGS_E2", "E2")):
        assert hd[ours] == scal(theirs), ours


# ------------------------------------------------------------------ atmosphere
def test_isa_sea_level_known_answers(orc):
    a = orc.atmos(0.0)
    assert a["T"] == 518.67 and a["P"] == 2116.228
    assert a["rho"] == 0.0023769117527742576          # f16_gen.cuh ATM_DBRK[0]
    assert a["a"] == 1116.4485575897318               # f16_gen.cuh STD_SL_SOUNDSPEED
    assert a["sigma"] == 1.0
    assert abs(a["densalt"]) < 1e-9


def test_isa_troposphere_textbook(orc):
    """T = T0 + L h_gp and P = P0 (T/T0)^(-g0 M / (R* L)), with h_gp = h R/(R + h)."""
    FTTOM, KG2SL = 0.3048, 0.06852168
    Rstar = 8.31432 * (KG2SL / (1.8 * FTTOM * FTTOM))
    Mair = 28.9645 * KG2SL / 1000.0
    g0 = 9.80665 / FTTOM
    ER = 6356766.0 / FTTOM
    L = (389.97 - 518.67) / 36089.2388
    for h in (1000.0, 10000.0, 25000.0, 35000.0):
        hg = h * ER / (ER + h)
        T = 518.67 + L * hg
        P = 2116.228 * (T / 518.67) ** (-g0 * Mair / (Rstar * L))
        a = orc.atmos(h)
        assert abs(a["T"] - T) < 1e-10
        assert abs(a["P"] / P - 1) < 1e-12
        assert abs(a["densalt"] - h) < 1e-6           # standard day: density altitude = altitude
    # isothermal layer above the tropopause
    hg = 50000.0
    h = hg * ER / (ER - hg)
    a = orc.atmos(h)
    assert abs(a["T"] - 389.97) < 1e-9
    Pb = 472.6805793706109                            # f16_gen.cuh ATM_PBRK[1]
    P = Pb * math.exp(-g0 * Mair * (hg - 36089.2388) / (Rstar * 389.97))
    assert abs(a["P"] / P - 1) < 1e-11
    assert abs(a["densalt"] - h) < 1e-5


def test_image_reciprocal_widths(orc):
    """Every breakpoint grid carries 1 / (x[i+1] - x[i]) per interval (the kernels' bracket
    factor multiplies by it instead of dividing)."""
    img = image(orc)
    hd = header_defines()
    grids = [k[:-4] for k in hd if re.match(r"F16M_G\d+_\w+_OFF$", k)]
    assert len(grids) == 20
    for g in grids:
        off, n, riv = hd[g + "_OFF"], hd[g + "_LEN"], hd[g + "_RIV"]
        x = img[off:off + n]
        assert np.all(np.diff(x) > 0), g
        assert list(img[riv:riv + n - 1]) == [1.0 / (b - a) for a, b in zip(x, x[1:])], g


def test_image_isa_layer_constants(orc):
    """The per-layer atmosphere constants, used the way the kernels use them (pressure as
    exp(e log(1 + k dH)) or exp(e dH); density altitude as base + c (exp(x log(rho / rb)) - 1)
    or base + c log(rho / rb)), reproduce the oracle's pressure and density altitude over the
    whole table, and the standard day's density altitude is the altitude itself."""
    img = image(orc)
    hd = header_defines()
    L0, K = hd["F16M_ATM_LAYER_OFF"], hd["F16M_ATM_LAYER_STRIDE"]
    lay = img[L0:L0 + 8 * K].reshape(8, K)
    hdr = open(IMG_HDR).read()

    def harr(name):
        m = re.search(r"#define " + name + r"_INIT \{([^}]*)\}", hdr)
        return [float(v) for v in m.group(1).split(",")]
    alts, dbrk = harr("F16M_ATM_ALT"), harr("F16M_ATM_DBRK")
    ER = hd["F16M_EARTH_RADIUS_ISA"]
    for h in np.concatenate([np.linspace(-2000.0, 280000.0, 2001), [0.0, 36089.0, 65617.0]]):
        a = orc.atmos(h)
        gp = (h * ER) / (ER + h)
        b = sum(not (gp < alts[i]) for i in range(1, 8))
        base, pb, k, e = lay[b, :4]
        dH = gp - base
        P = pb * math.exp(e * (math.log(1.0 + k * dH) if k != 0.0 else dH))
        assert abs(P / a["P"] - 1) < 1e-13, h
        d = sum(not (a["rho"] >= dbrk[i]) for i in range(1, 8))
        dbase, irb, x, c = lay[d, 4:]
        lr = math.log(a["rho"] * irb)
        da = dbase + c * (math.exp(x * lr) - 1.0 if x != 0.0 else lr)
        da = (da * ER) / (ER - da)
        assert abs(da - a["densalt"]) < 1e-8 * max(1.0, abs(h)), h
        if 0.0 <= h <= 250000.0:
            assert abs(da - h) < 1e-6 * max(1.0, abs(h)), h


# ------------------------------------------------------------------ mass balance
def test_mass_closed_forms(orc):
    for fuel in (0.0, 3000.0, 6000.0, 6972.0):
        m = orc.mass(fuel)
        w = 17400.0 + fuel + 230.0
        assert abs(m["mass"] - w / 32.174049) < 1e-12
        cgx = (17400.0 * -193.0 + 230.0 * -336.2 + fuel * -174.4) / w
        cgz = (17400.0 * -5.1 + 0.0 + fuel * 5.0) / w
        assert abs(m["cg"][0] - cgx) < 1e-12 and abs(m["cg"][2] - cgz) < 1e-12
        assert m["cg"][1] == 0.0                    # symmetric tanks
        J, Ji = m["J"], m["Jinv"]
        assert np.array_equal(J, J.T)
        assert np.allclose(J @ Ji, np.eye(3), atol=1e-14)
        # parallel-axis: Ixx grows by the tanks' y offset (65 in) squared
        if fuel > 0:
            m0 = orc.mass(0.0)
            assert m["J"][0, 0] > m0["J"][0, 0]
        # moment reference point in body axes, ft
        assert abs(m["rp"][0] - (m["cg"][0] + 189.5) / 12.0) < 1e-12


# ------------------------------------------------------------------ frames
def test_frames_invariants(orc):
    import ctypes
    rng = np.random.default_rng(5)
    for _ in range(100):
        e = np.array([rng.uniform(-3, 3), rng.uniform(-1.5, 1.5), rng.uniform(0, 2 * np.pi)])
        q = np.zeros(4); T = np.zeros(9); q2 = np.zeros(4); e2 = np.zeros(3)
        orc.L.orc_euler_to_quat(e[0], e[1], e[2], oracle_lib._p(q))
        assert abs(np.linalg.norm(q) - 1) < 1e-15
        orc.L.orc_quat_to_T(oracle_lib._p(q), oracle_lib._p(T))
        M = T.reshape(3, 3)
        assert np.allclose(M @ M.T, np.eye(3), atol=1e-14)
        assert abs(np.linalg.det(M) - 1) < 1e-14
        orc.L.orc_mat_to_quat(oracle_lib._p(T), oracle_lib._p(q2))
        assert min(np.abs(q2 - q).max(), np.abs(q2 + q).max()) < 1e-14
        orc.L.orc_mat_to_euler(oracle_lib._p(T), oracle_lib._p(e2))
        assert abs(e2[1] - e[1]) < 1e-12
        d = np.angle(np.exp(1j * (e2[[0, 2]] - e[[0, 2]])))
        assert np.abs(d).max() < 1e-12
        assert 0.0 <= e2[2] < 2 * np.pi
    # heading 90 deg, level: body x points east
    q = np.zeros(4); T = np.zeros(9)
    orc.L.orc_euler_to_quat(0.0, 0.0, np.pi / 2, oracle_lib._p(q))
    orc.L.orc_quat_to_T(oracle_lib._p(q), oracle_lib._p(T))
    assert np.allclose(T.reshape(3, 3)[0], [0, 1, 0], atol=1e-15)


def test_gravity_j2_closed_form(orc):
    a, GM, J2 = 20925646.32546, 14.0764417572E15, 1.08262982E-03
    g = np.zeros(3)
    orc.L.orc_gravity_j2(oracle_lib._p(np.array([a, 0.0, 0.0])), 0.0, oracle_lib._p(g))
    assert abs(g[0] / (-GM / a ** 2 * (1 + 1.5 * J2)) - 1) < 1e-14 and g[1] == 0 and g[2] == 0
    orc.L.orc_gravity_j2(oracle_lib._p(np.array([0.0, 0.0, a])), math.pi / 2, oracle_lib._p(g))
    assert abs(g[2] / (-GM / a ** 2 * (1 - 3 * J2)) - 1) < 1e-14


def test_pitot_round_trip(orc):
    """At sea-level static pressure calibrated airspeed equals true airspeed: Vc = M a0."""
    for M in (0.1, 0.5, 0.9, 0.99):
        vc = orc.L.orc_vcal_from_mach(M, 2116.228)
        assert abs(vc / (M * 1116.4485575897318) - 1) < 1e-14
    # supersonic: the reference inverts the Rayleigh pitot formula with a fixed 10-pass
    # fixed-point iteration (jsb_auxiliary.py:33-35), which leaves a ~1e-8 residual
    for M in (1.2, 1.6, 2.0):
        vc = orc.L.orc_vcal_from_mach(M, 2116.228)
        assert abs(vc / (M * 1116.4485575897318) - 1) < 1e-6
    assert orc.L.orc_idleff() == 757.6485181409156     # f16_gen.cuh IdleFF


def test_geodetic_to_ecef_radius(orc):
    """|ecef| = a + alt on the geodetic normal (cuda_fdm/ic.py:18-45 contract)."""
    o = np.zeros(3)
    for lat in (0.0, 0.65, 1.2):
        for alt in (0.0, 10000.0, 30000.0):
            orc.L.orc_geodetic_to_ecef(lat, 2.3, alt, oracle_lib._p(o))
            assert abs(np.linalg.norm(o) - (20925646.32546 + alt)) < 1e-6


# ------------------------------------------------------------------ composed paths
@pytest.mark.parametrize("rate", [120, 60])
def test_seed_matches_reference_golden(orc, rate):
    """build_seed_vector golden vectors from the reference (tests/golden/make_fdm_golden.py):
    bit-for-bit, both lineages.  This also pins the force path the seed runs."""
    g = oracle_lib.golden("seed_golden.npz")
    got = orc.seed(g["ic"], rate)
    assert np.array_equal(got, g[f"seed_{rate}"])


@pytest.mark.parametrize("rate", [120, 60])
def test_step_matches_reference_c_model(orc, rate):
    """Per decision against the reference's own fdm.cuh built for the host (oracle/_ref)."""
    ref = oracle_lib.load_ref(rate)
    if ref is None:
        pytest.skip("oracle/_ref not built (reference checkout absent at build time)")
    assert ref.L.ref_fcs_rate() == rate
    g = oracle_lib.golden("seed_golden.npz")
    a_st = np.ascontiguousarray(g[f"seed_{rate}"]); b_st = a_st.copy()
    rng = np.random.default_rng(11)
    n = a_st.shape[0]
    for dec in range(10):
        act = np.stack([rng.uniform(-1, 1, n), rng.uniform(-1, 1, n), rng.uniform(-1, 1, n),
                        rng.uniform(0, 1, n)], 1)
        oa = orc.step(a_st, act, 6, rate)
        ob = ref.step(b_st, act, 6)
        assert oracle_lib.rel_err(a_st, b_st).max() < 1e-11, dec
        assert oracle_lib.rel_err(oa, ob).max() < 1e-11, dec


def test_substep_count_equivalence(orc):
    """S substeps in one call equal S single-substep calls (history bookkeeping)."""
    g = oracle_lib.golden("seed_golden.npz")
    a = np.ascontiguousarray(g["seed_120"][:8]); b = a.copy()
    act = np.tile([0.1, -0.2, 0.05, 0.7], (8, 1))
    orc.step(a, act, 6)
    for _ in range(6):
        orc.step(b, act, 1)
    assert np.array_equal(a, b)


# ------------------------------------------------------------------ drift envelope (C1)
def test_drift_envelope_fixture_shape():
    """The reference pair's curve (tests/golden/make_drift_envelope.py): quantiles ordered,
    the survivor count non-increasing, and the pair bit-identical over the first 50 decisions
    (fdm.cuh and the Python model round differently only in a few expressions)."""
    env = oracle_lib.golden("drift_envelope.npz")
    q = env["pos_ft"]
    assert q.shape == (oracle_lib.DRIFT_NDEC, len(oracle_lib.DRIFT_QUANTILES))
    assert (np.diff(q, axis=1) >= 0).all()
    assert (np.diff(env["alive"]) <= 0).all() and env["alive"][0] == 1024
    assert (q[:50] == 0).all() and q[-1, -1] > 0


def test_drift_envelope_rejects_planted_drift(orc):
    """The GPU drift bound has power: the CPU model against itself with the velocities of every
    aircraft perturbed by 1e-13 relative (normal, per decision) breaks the envelope well inside
    the 600 decisions, while the unperturbed pair never does."""
    icm = importlib.import_module("2026_ai_pilot_challenge-1st_solution_amd.ic")
    ic, acts = oracle_lib.c1_replicas(icm)
    env = oracle_lib.golden("drift_envelope.npz")
    a = orc.seed(ic, 120)
    b, c = a.copy(), a.copy()
    alive = np.ones(len(a), bool)
    rng = np.random.default_rng(0)
    broke = None
    for d in range(200):
        for x in (a, b, c):
            orc.step(x, acts[d], 6, want_obs=False)
        b[:, 3:6] *= 1.0 + 1e-13 * rng.standard_normal((len(b), 3))
        alive &= oracle_lib.altitude_m(a) > 304.8
        if d % 10 == 9:
            bound = oracle_lib.drift_envelope(env, d)
            assert (oracle_lib.drift_quantiles(a, c, alive) <= bound).all()
            if broke is None and (oracle_lib.drift_quantiles(a, b, alive) > bound).any():
                broke = d + 1
    assert broke is not None and broke <= 150, broke


# ------------------------------------------------------------------ FLOP-count fixture
def test_flop_fixture_reproduces():
    """tests/golden/fdm_flops.json (bench.py's algorithmic FLOPs per aircraft-substep) is what the
    counting build of the restatement (oracle/opcount.hpp) tallies on its samples; that build
    steps the aircraft bit for bit like the plain restatement, so it counts the restatement's
    own operations; and the counts sit within 2 % of the reference model's static count
    (1,550: 114 divisions, ~11 square roots, ~18 libm calls)."""
    import json
    spec = importlib.util.spec_from_file_location(
        "make_flops_golden", os.path.join(ROOT, "tests", "golden", "make_flops_golden.py"))
    M = importlib.util.module_from_spec(spec)
    spec.loader.exec_module(M)
    icm = importlib.import_module("2026_ai_pilot_challenge-1st_solution_amd.ic")
    orc, lib = M.load_counter()
    fix = json.load(open(os.path.join(ROOT, "tests", "golden", "fdm_flops.json")))
    for name, (ic, act, rate) in M.samples(icm).items():
        per, st = M.count(orc, lib, ic, act, rate)
        want = fix["per_aircraft_substep"][name]
        for k in M.KEYS + ("flop",):
            assert abs(per[k] - want[k]) <= 1e-6 * max(1.0, want[k]), (name, k)
        assert per["aircraft_substeps"] == want["aircraft_substeps"]
        plain = orc.seed(ic, rate)
        orc.rollout(plain, np.ascontiguousarray(act), 6, rate)
        assert np.array_equal(st, plain, equal_nan=True), name    # crashed rows: NaN signs vary
        assert abs(per["flop"] / 1550.0 - 1.0) < 0.02, (name, per["flop"])
