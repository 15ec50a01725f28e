#!/usr/bin/env python3
"""Generate the F-16 model data header from the JSBSim aircraft and engine XML.

Reads
  * ``aircraft/f16/f16.xml``  -- <metrics>, <mass_balance>, fuel tanks, the three FCS
    ``scheduled_gain`` tables and the whole <aerodynamics> block (kCLge + 40 axis functions);
  * ``engine/F100-PW-229.xml`` -- turbine constants and the Idle/Mil/Aug thrust tables,

and writes ``f16_model_gen.h``: one flat image of doubles holding every breakpoint grid
(identical breakpoint vectors are stored once) followed by every table body, ``#define``
offsets into that image, the model constants, and a descriptor list of the 40 aero
coefficient functions (factor properties in XML order, optional scalar value, optional
1-D/2-D table).  The header is plain C so the CPU oracle and the HIP kernels read the same
numbers; the kernel side additionally gets ``f16_aero_gen.inc``, straight-line device code
that evaluates the 40 functions with one bracket search per shared grid.

Semantics mirrored (reference files, for parity review):
  * function = product of its property factors, then its <value>, then its table
    (cuda_fdm/ref/jsb_aero.py:62-73);
  * 1-D table: clamp to end values, linear inside (cuda_fdm/ref/jsb_tables.py:22-40);
  * 2-D table: bracket per axis, factors clamped to [0,1] (cuda_fdm/ref/jsb_tables.py:56-80).

Usage:  python gen_f16_model.py [--assets DIR] [--out-dir DIR]
The default asset directory is the reference checkout's competition runtime assets; the
generated headers are committed, so building the library never needs the XML.
"""
import argparse
import os
import xml.etree.ElementTree as ET

DEFAULT_ASSETS = "/root/reference/third_party/competition_runtime/assets"

# property name -> (enum name, device expression used by the generated aero code)
AERO_VARS = [
    ("aero/qbar-psf", "QBAR", "qbar"),
    ("metrics/Sw-sqft", "SW", None),
    ("metrics/bw-ft", "BW", None),
    ("metrics/cbarw-ft", "CBAR", None),
    ("aero/alpha-rad", "ALPHA", "alpha"),
    ("aero/beta-rad", "BETA", "beta"),
    ("aero/bi2vel", "BI2VEL", "bi2vel"),
    ("aero/ci2vel", "CI2VEL", "ci2vel"),
    ("velocities/mach", "MACH", "mach"),
    ("aero/function/kCLge", "KCLGE", "kclge"),
    ("velocities/p-aero-rad_sec", "P", "p"),
    ("velocities/q-aero-rad_sec", "Q", "q"),
    ("velocities/r-aero-rad_sec", "R", "r"),
    ("fcs/aileron-pos-rad", "AIL", "ail"),
    ("fcs/elevator-pos-rad", "ELEV", "elev"),
    ("fcs/rudder-pos-rad", "RUD", "rud"),
    ("fcs/lef-pos-rad", "LEF", "lef"),
    ("fcs/flaperon-mix-rad", "FLAP", "flap"),
    ("fcs/speedbrake-pos-rad", "SB", "sb"),
    ("gear/gear-pos-norm", "GEAR", "gear"),
]
VAR_INDEX = {p: i for i, (p, _, _) in enumerate(AERO_VARS)}
AXES = ["DRAG", "SIDE", "LIFT", "ROLL", "PITCH", "YAW"]


def fnum(x):
    """Round-trip exact C literal for a double."""
    r = repr(float(x))
    if "e" not in r and "." not in r and "inf" not in r and "nan" not in r:
        r += ".0"
    return r


def _floats(text):
    return [float(t) for t in text.split()]


def parse_table(tel):
    ivs = tel.findall("independentVar")
    lines = [ln.split() for ln in tel.find("tableData").text.strip().splitlines() if ln.split()]
    if len(ivs) <= 1:
        return {"kind": 1, "row_var": ivs[0].text.strip() if ivs else None,
                "x": [float(l[0]) for l in lines], "y": [float(l[1]) for l in lines]}
    row_var = col_var = None
    for iv in ivs:
        if iv.get("lookup") == "row":
            row_var = iv.text.strip()
        elif iv.get("lookup") == "column":
            col_var = iv.text.strip()
    cols = [float(v) for v in lines[0]]
    rows, data = [], []
    for l in lines[1:]:
        rows.append(float(l[0]))
        vals = [float(v) for v in l[1:]]
        assert len(vals) == len(cols), "ragged 2-D table"
        data.append(vals)
    return {"kind": 2, "row_var": row_var, "col_var": col_var, "x": rows, "c": cols, "d": data}


def parse_function(fel):
    prod = fel.find("product")
    box = prod if prod is not None else fel
    factors, value, table = [], None, None
    for ch in box:
        if ch.tag == "property":
            factors.append(ch.text.strip())
        elif ch.tag == "value":
            value = float(ch.text.strip())
        elif ch.tag == "table":
            table = parse_table(ch)
    return {"name": fel.get("name"), "factors": factors, "value": value, "table": table}


class Image:
    """Flat double image: grids (deduplicated) then table bodies."""

    def __init__(self):
        self.vals = []
        self.grids = {}      # tuple -> (name, off, len)
        self.defines = []

    def grid(self, xs, hint):
        key = tuple(xs)
        for a, b in zip(xs, xs[1:]):
            assert b > a, f"breakpoints of {hint} must increase strictly"
        if key not in self.grids:
            name = f"G{len(self.grids)}_{hint}"
            self.grids[key] = (name, len(self.vals), len(xs))
            self.vals.extend(xs)
        return self.grids[key]

    def body(self, vals):
        off = len(self.vals)
        self.vals.extend(vals)
        return off


def derived_constants():
    """Constants the reference derives at start-up, computed with the same expressions in
    IEEE double and the same libm (Python's math.pow/exp/sqrt), so CPU and GPU code can use
    them as literals.  Sources: cuda_fdm/ref/jsb_const.py:6-40 (units, ISA rows),
    jsb_atmos.py:11-33 + 74-76 (lapse rates, pressure and density breakpoints),
    jsb_frames.py:9-19 (WGS84), jsb_fdm.py:19 (SLGRAVITY), jsb_propulsion.py:23 (IdleFF),
    jsb_auxiliary.py:17 (sea-level speed of sound)."""
    import math
    KTSTOFPS = 1.68781
    FTTOM = 0.3048
    KGTOSLUG = 0.06852168
    KtoDegR = 1.8
    Rstar = 8.31432 * (KGTOSLUG / (KtoDegR * FTTOM * FTTOM))
    Mair = 28.9645 * KGTOSLUG / 1000.0
    g0 = 9.80665 / FTTOM
    Reng = Rstar / Mair
    SHRatio = 1.40
    SLT, SLP = 518.67, 2116.228
    ER = 6356766.0 / FTTOM
    alts = [0.0000, 36089.2388, 65616.7979, 104986.8766, 154199.4751, 167322.8346,
            232939.6325, 278385.8268, 298556.4304]
    temps = [518.67, 389.97, 389.97, 411.57, 487.17, 487.17, 386.37, 336.5028, 336.5028]
    n = len(alts)
    lapse = [(temps[b + 1] - temps[b]) / (alts[b + 1] - alts[b]) for b in range(n - 1)]
    pbrk = [SLP] + [0.0] * (n - 1)
    for b in range(n - 1):
        Tmb, dH, L = temps[b], alts[b + 1] - alts[b], lapse[b]
        if L != 0.0:
            pbrk[b + 1] = pbrk[b] * (Tmb / (Tmb + L * dH)) ** (g0 * Mair / (Rstar * L))
        else:
            pbrk[b + 1] = pbrk[b] * math.exp(-g0 * Mair * dH / (Rstar * Tmb))
    dbrk = [pbrk[i] / (Reng * temps[i]) for i in range(n)]

    def temperature(alt):      # jsb_atmos.py:43-49
        gp = (alt * ER) / (ER + alt)
        x = gp if gp >= 0.0 else 0.0
        if x <= alts[0]:
            t = temps[0]
        elif x >= alts[-1]:
            t = temps[-1]
        else:
            r = 1
            while r < n - 1 and alts[r] < x:
                r += 1
            t = (x - alts[r - 1]) / (alts[r] - alts[r - 1])
            t = min(t, 1.0) * (temps[r] - temps[r - 1]) + temps[r - 1]
        return t if gp >= 0.0 else t + gp * lapse[0]

    # base temperature the pressure routine uses for layer b: temperature(geometric(BaseAlt))
    tmb_p = [temperature((alts[b] * ER) / (ER - alts[b])) for b in range(n - 1)]
    sem_a, sem_b = 20925646.32546, 20855486.5951
    ec = sem_b / sem_a
    return {
        "scalars": [("F16M_RSTAR", Rstar), ("F16M_MAIR", Mair), ("F16M_G0", g0),
                    ("F16M_RENG", Reng), ("F16M_EARTH_RADIUS_ISA", ER),
                    ("F16M_RHO_SL", SLP / (Reng * SLT)),
                    ("F16M_GAMMA_R", SHRatio * Reng),
                    ("F16M_STD_SL_SOUNDSPEED", math.sqrt(SHRatio * Reng * SLT)),
                    ("F16M_FPSTOKTS", 1.0 / KTSTOFPS),
                    ("F16M_SLGRAVITY", 14.0764417572E15 / (sem_a * sem_a)),
                    ("F16M_IDLEFF", 17800.0 ** 0.2 * 107.0),
                    ("F16M_WGS_EC", ec), ("F16M_WGS_E2", 1.0 - ec * ec)],
        "arrays": [("F16M_ATM_ALT", alts), ("F16M_ATM_TMP", temps), ("F16M_ATM_LAPSE", lapse),
                   ("F16M_ATM_PBRK", pbrk), ("F16M_ATM_DBRK", dbrk), ("F16M_ATM_TMB_P", tmb_p)],
    }


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--assets", default=DEFAULT_ASSETS)
    ap.add_argument("--out-dir", default=os.path.dirname(os.path.abspath(__file__)))
    args = ap.parse_args()

    ac = ET.parse(os.path.join(args.assets, "aircraft/f16/f16.xml")).getroot()
    en = ET.parse(os.path.join(args.assets, "engine/F100-PW-229.xml")).getroot()

    img = Image()
    consts = []

    # ---- metrics / reference points ----
    m = ac.find("metrics")
    sw = float(m.find("wingarea").text)
    bw = float(m.find("wingspan").text)
    cbar = float(m.find("chord").text)
    consts += [("F16M_SW", sw), ("F16M_BW", bw), ("F16M_CBAR", cbar)]
    locs = {}
    for loc in m.findall("location"):
        locs[loc.get("name")] = [float(loc.find(k).text) for k in ("x", "y", "z")]
    for nm in ("AERORP", "EYEPOINT"):
        for k, v in zip("XYZ", locs[nm]):
            consts.append((f"F16M_{nm}_{k}", v))

    # ---- mass balance ----
    mb = ac.find("mass_balance")
    for tag in ("ixx", "iyy", "izz", "ixy", "ixz", "iyz", "emptywt"):
        consts.append((f"F16M_{tag.upper()}", float(mb.find(tag).text)))
    cg = [float(mb.find("location").find(k).text) for k in ("x", "y", "z")]
    for k, v in zip("XYZ", cg):
        consts.append((f"F16M_BASECG_{k}", v))
    pm = mb.find("pointmass")
    consts.append(("F16M_PILOT_WT", float(pm.find("weight").text)))
    for k, v in zip("XYZ", [float(pm.find("location").find(c).text) for c in ("x", "y", "z")]):
        consts.append((f"F16M_PILOT_{k}", v))
    tanks = ac.find("propulsion").findall("tank")
    for ti in (0, 1):   # the two internal tanks carry all fuel (external tanks are empty)
        loc = tanks[ti].find("location")
        for k, c in zip("XYZ", ("x", "y", "z")):
            consts.append((f"F16M_TANK{ti}_{k}", float(loc.find(c).text)))
        consts.append((f"F16M_TANK{ti}_CAP", float(tanks[ti].find("capacity").text)))

    # ---- engine ----
    for tag in ("milthrust", "maxthrust", "bypassratio", "tsfc", "atsfc", "idlen1", "idlen2",
                "maxn1", "maxn2"):
        consts.append((f"F16M_ENG_{tag.upper()}", float(en.find(tag).text)))
    eng_tabs = {}
    for f in en.findall("function"):
        t = parse_table(f.find("table"))
        eng_tabs[f.get("name")] = t

    # ---- FCS scheduled gains ----
    fcs_tabs = {}
    for sg in ac.iter("scheduled_gain"):
        nm = sg.get("name")
        if nm in ("fcs/aileron-speed-compensated", "fcs/elevator-scheduler", "fcs/yaw-rate-norm"):
            fcs_tabs[nm] = parse_table(sg.find("table"))

    # ---- aerodynamics ----
    aero = ac.find("aerodynamics")
    top = {}
    axes = {}
    for el in aero:
        if el.tag == "function":
            f = parse_function(el)
            top[f["name"]] = f
        elif el.tag == "axis":
            axes[el.get("name")] = [parse_function(f) for f in el.findall("function")]

    hint_of = {"aero/alpha-rad": "ALPHA", "aero/beta-rad": "BETA", "fcs/elevator-pos-rad": "ELEV",
               "velocities/mach": "MACH", "aero/h_b-mac-ft": "HB", "velocities/vg-fps": "VG",
               "atmosphere/density-altitude": "DENSALT"}

    tables = []   # (name, dict with offsets)

    def add_table(tname, t):
        rec = {"kind": t["kind"], "row_var": t["row_var"]}
        rec["rg"] = img.grid(t["x"], hint_of[t["row_var"]])
        if t["kind"] == 1:
            rec["off"] = img.body(t["y"])
        else:
            rec["col_var"] = t["col_var"]
            rec["cg"] = img.grid(t["c"], hint_of[t["col_var"]])
            rec["off"] = img.body([v for row in t["d"] for v in row])
        tables.append((tname, rec))
        return rec

    dc0 = derived_constants()
    isa = dict(dc0["arrays"])
    hint_of["ISA"] = "ISA"
    add_table("ISA_TEMP", {"kind": 1, "row_var": "ISA", "x": isa["F16M_ATM_ALT"],
                           "y": isa["F16M_ATM_TMP"]})
    kclge = add_table("KCLGE", top["aero/function/kCLge"]["table"])
    fcs_ail = add_table("FCS_AIL_SPEED", fcs_tabs["fcs/aileron-speed-compensated"])
    fcs_elev = add_table("FCS_ELEV_SCHED", fcs_tabs["fcs/elevator-scheduler"])
    fcs_yaw = add_table("FCS_YAW_RATE", fcs_tabs["fcs/yaw-rate-norm"])
    e_idle = add_table("ENG_IDLE", eng_tabs["IdleThrust"])
    e_mil = add_table("ENG_MIL", eng_tabs["MilThrust"])
    e_aug = add_table("ENG_AUG", eng_tabs["AugThrust"])

    terms = []
    for ai, ax in enumerate(AXES):
        for f in axes[ax]:
            short = f["name"].split("/")[-1]
            rec = add_table("AERO_" + short, f["table"]) if f["table"] else None
            terms.append((ai, short, f, rec))
    assert len(terms) == 40, len(terms)
    # Reciprocal interval widths, one vector per grid, after every table body (the offsets
    # above are unchanged): a bracket factor is (key - x[i]) * riv[i] instead of a division by
    # x[i+1] - x[i].  The widths are differenced in IEEE double exactly as the kernel would.
    riv_off = {}
    for key, (name, _, _) in img.grids.items():
        riv_off[name] = img.body([1.0 / (b - a) for a, b in zip(key, key[1:])])
    # ISA layer constants, 8 per layer, so the atmosphere reads its layer's numbers with one
    # indexed load each (jsb_atmos.py:52-111 written as exp/log):
    #   pressure layer b:  [0] base altitude, [1] base pressure, [2] lapse / base temperature,
    #                      [3] exponent (-g0 M / (R* lapse), or -g0 M / (R* T) when isothermal);
    #                      P = pb * exp(e * log(1 + k dH)), or pb * exp(e * dH);
    #   density layer d:   [4] base altitude, [5] 1 / base density, [6] density exponent
    #                      (-1 / (1 + g0 M / (R* lapse)), 0 when isothermal), [7] T / lapse
    #                      (or -R* T / (g0 M)); da = base + c (exp(x log(rho/rb)) - 1), or
    #                      base + c log(rho/rb).
    atm = dict(dc0["arrays"])
    sca = dict(dc0["scalars"])
    g0m = sca["F16M_G0"] * sca["F16M_MAIR"]
    rst = sca["F16M_RSTAR"]
    layer = []
    for i in range(8):
        lap, tmb, tmp = atm["F16M_ATM_LAPSE"][i], atm["F16M_ATM_TMB_P"][i], atm["F16M_ATM_TMP"][i]
        iso = lap == 0.0
        layer += [atm["F16M_ATM_ALT"][i], atm["F16M_ATM_PBRK"][i],
                  0.0 if iso else lap / tmb,
                  -(g0m / (rst * tmb)) if iso else -(g0m / (rst * lap)),
                  atm["F16M_ATM_ALT"][i], 1.0 / atm["F16M_ATM_DBRK"][i],
                  0.0 if iso else -1.0 / (1.0 + g0m / (rst * lap)),
                  -(rst * tmp) / g0m if iso else tmp / lap]
    atm_layer_off = img.body(layer)

    # ------------------------------------------------------------------ header
    out = []
    w = out.append
    w("/* f16_model_gen.h -- GENERATED by gen_f16_model.py from f16.xml and F100-PW-229.xml.")
    w(" * Do not edit: rerun the generator.  Plain C: shared by the CPU oracle and the HIP kernels.")
    w(" * Layout: F16M_IMAGE = [grids (each distinct breakpoint vector once) | table bodies];")
    w(" * 2-D bodies are row-major [row][col]. */")
    w("#ifndef F16_MODEL_GEN_H")
    w("#define F16_MODEL_GEN_H")
    w("")
    w("/* ---- model constants ---- */")
    for n, v in consts:
        w(f"#define {n} ({fnum(v)})")
    w("")
    w("/* ---- derived start-up constants (same expressions/libm as the reference) ---- */")
    dc = derived_constants()
    for n, v in dc["scalars"]:
        w(f"#define {n} ({fnum(v)})")
    for n, vals in dc["arrays"]:
        w(f"#define {n}_INIT {{ " + ", ".join(fnum(v) for v in vals) + " }")
    w("")
    w("/* ---- breakpoint grids: offset / length in F16M_IMAGE ---- */")
    for key, (name, off, ln) in img.grids.items():
        w(f"#define F16M_{name}_OFF {off}")
        w(f"#define F16M_{name}_LEN {ln}")
        w(f"#define F16M_{name}_RIV {riv_off[name]}")
    w("")
    w("/* ---- tables: body offset, grids ---- */")
    for tname, rec in tables:
        w(f"#define F16M_T_{tname}_OFF {rec['off']}")
        w(f"#define F16M_TG_{tname}_R {rec['rg'][0]}")
        if rec["kind"] == 2:
            w(f"#define F16M_TG_{tname}_C {rec['cg'][0]}")
        w(f"#define F16M_T_{tname}_RG {rec['rg'][1]}")
        w(f"#define F16M_T_{tname}_NR {rec['rg'][2]}")
        if rec["kind"] == 2:
            w(f"#define F16M_T_{tname}_CG {rec['cg'][1]}")
            w(f"#define F16M_T_{tname}_NC {rec['cg'][2]}")
    w("")
    w(f"#define F16M_ATM_LAYER_OFF {atm_layer_off}")
    w("#define F16M_ATM_LAYER_STRIDE 8")
    w(f"#define F16M_IMAGE_LEN {len(img.vals)}")
    w("#define F16M_IMAGE_INIT { \\")
    for i in range(0, len(img.vals), 6):
        chunk = ", ".join(fnum(v) for v in img.vals[i:i + 6])
        w(f"  {chunk}, \\")
    w("}")
    w("")
    w("/* ---- aero coefficient functions (XML order within each axis) ---- */")
    w("enum f16m_aero_var {")
    for p, e, _ in AERO_VARS:
        w(f"  F16M_V_{e}, /* {p} */")
    w("  F16M_NVAR };")
    w("enum f16m_axis { " + ", ".join(f"F16M_AX_{a}" for a in AXES) + " };")
    w("typedef struct {")
    w("  int axis, nfac, fac[6];")
    w("  int has_value; double value;")
    w("  int kind;            /* 0 none, 1 one-D, 2 two-D */")
    w("  int row_var, col_var; /* enum f16m_aero_var */")
    w("  int rg, nr, cg, nc, off;")
    w("} f16m_aero_term;")
    w("#define F16M_NAERO 40")
    w("#define F16M_AERO_TERMS_INIT { \\")
    for ai, short, f, rec in terms:
        facs = [VAR_INDEX[p] for p in f["factors"]]
        assert len(facs) <= 6
        fa = "{" + ", ".join(str(x) for x in facs + [0] * (6 - len(facs))) + "}"
        hv = 1 if f["value"] is not None else 0
        val = fnum(f["value"] if hv else 0.0)
        if rec is None:
            tpart = "0, -1, -1, 0, 0, 0, 0, 0"
        elif rec["kind"] == 1:
            tpart = (f"1, {VAR_INDEX[rec['row_var']]}, -1, {rec['rg'][1]}, {rec['rg'][2]}, 0, 0, "
                     f"{rec['off']}")
        else:
            tpart = (f"2, {VAR_INDEX[rec['row_var']]}, {VAR_INDEX[rec['col_var']]}, "
                     f"{rec['rg'][1]}, {rec['rg'][2]}, {rec['cg'][1]}, {rec['cg'][2]}, {rec['off']}")
        w(f"  {{ {ai}, {len(facs)}, {fa}, {hv}, {val}, {tpart} }}, /* {short} */ \\")
    w("}")
    w("")
    w("#endif /* F16_MODEL_GEN_H */")
    with open(os.path.join(args.out_dir, "f16_model_gen.h"), "w") as fh:
        fh.write("\n".join(out) + "\n")

    # ------------------------------------------------------- device aero code
    # Every grid used by an aero table gets one bracket; 1-D tables take the clamp-to-end
    # bracket, 2-D axes the clamped-factor bracket.  Factor products keep the oracle's
    # left-to-right order so the per-term results are bit-identical.
    const_of = {"metrics/Sw-sqft": sw, "metrics/bw-ft": bw, "metrics/cbarw-ft": cbar}
    var_expr = {p: ex for p, _, ex in AERO_VARS if ex}
    used1, used2 = {}, {}
    for _, short, f, rec in terms:
        if rec is None:
            continue
        if rec["kind"] == 1:
            used1[rec["rg"]] = rec["row_var"]
        else:
            used2[rec["rg"]] = rec["row_var"]
            used2[rec["cg"]] = rec["col_var"]
    # per-grid upper-bracket index: r = 1 + #{ i in [1, n-2] : x[i] < key }, i.e. the first
    # i >= 1 with x[i] >= key (clamped to n-1), which is where the reference's forward scan
    # stops (jsb_tables.py:32-33, 59-61).  Literal breakpoints keep the compares in registers.
    g = []
    gw = g.append
    gw("// f16_grid_gen.inc -- GENERATED by gen_f16_model.py; do not edit.")
    gw("// Upper-bracket index per breakpoint grid, with the breakpoints as literals.")
    for key, (name, off, ln) in img.grids.items():
        cmps = " + ".join(f"(int)({fnum(x)} < key)" for x in key[1:-1]) or "0"
        gw(f"F16_HD int f16m_upper_{name}(double key) {{ return 1 + {cmps}; }}")
        gw(f"#define F16M_{name}_X0 ({fnum(key[0])})")
        gw(f"#define F16M_{name}_XN ({fnum(key[-1])})")
    with open(os.path.join(args.out_dir, "f16_grid_gen.inc"), "w") as fh:
        fh.write("\n".join(g) + "\n")

    # The speedbrake is never driven (its position is identically +0), so the four terms with
    # that factor are exactly +-0 for every finite state and are omitted.
    # The build-up is emitted in three layers so that callers can evaluate it piecewise as its
    # inputs become available and still get the same bits:
    #   brackets  (one per shared grid), grouped by key: alpha/beta, mach, elevator;
    #   lookups   lk_<term> = the term's table value, grouped by the brackets they need;
    #   sums      per axis, FREE = terms with no control-surface position (as a factor or a
    #             table variable), CTL = the others; each a left-to-right sum from 0 in XML
    #             order of the term's factors times its lookup; axis = FREE + CTL.
    CTL = {"fcs/aileron-pos-rad", "fcs/elevator-pos-rad", "fcs/rudder-pos-rad",
           "fcs/lef-pos-rad", "fcs/flaperon-mix-rad"}
    SB = "fcs/speedbrake-pos-rad"
    KEYGRP = {"aero/alpha-rad": "AB", "aero/beta-rad": "AB", "velocities/mach": "MACH",
              "fcs/elevator-pos-rad": "ELEV"}
    d = []
    dw = d.append

    def macro(name, stmts):
        dw(f"#define {name} \\")
        for i, st in enumerate(stmts):
            dw(f"  {st}" + ("; \\" if i + 1 < len(stmts) else ""))
        if not stmts:
            dw("  do {} while (0)")

    dw("// f16_aero_gen.inc -- GENERATED by gen_f16_model.py; do not edit.")
    dw("// The 40-function F-16 aero build-up in three layers over names in scope (`T`, the model")
    dw("// image; qbar alpha beta bi2vel ci2vel mach kclge p q r ail elev rud lef flap gear):")
    dw("//   F16_AERO_BRACKETS_{AB,MACH,ELEV}: one bracket per shared grid (b1_<grid>, b2_<grid>),")
    dw("//     keyed on alpha/beta, mach, elevator position;")
    dw("//   F16_AERO_LOOKUPS_{AB,MACH,ELEV}: lk_<term> = the term's table value, by the brackets")
    dw("//     it needs;")
    dw("//   F16_AERO_<AXIS>_FREE / _CTL: the terms without / with a control-surface position, each")
    dw("//     a left-to-right sum from 0 in XML order; the axis is FREE + CTL;")
    dw("//   F16_AERO_<AXIS>_SCALE, _EARLY, _LATE: the axis as SCALE * (EARLY + LATE), SCALE the")
    dw("//     factors every term starts with, EARLY the rest of the alpha/beta-only terms, LATE the")
    dw("//     terms that need mach or the elevator position (each a sum in XML order).")
    dw("// Terms with the speedbrake factor (identically 0) are omitted.")
    brk = {"AB": [], "MACH": [], "ELEV": []}
    for gr, var in sorted(used1.items(), key=lambda kv: kv[0][1]):
        brk[KEYGRP[var]].append(f"const F16Br1 b1_{gr[0]} = F16_BR1({gr[0]}, {var_expr[var]})")
    for gr, var in sorted(used2.items(), key=lambda kv: kv[0][1]):
        brk[KEYGRP[var]].append(f"const F16Br2 b2_{gr[0]} = F16_BR2({gr[0]}, {var_expr[var]})")
    lks = {"AB": [], "MACH": [], "ELEV": []}
    sums = {}
    # Every term of an axis starts with the same factors -- qbar, the wing area and, for the
    # moments, the span or chord -- so the axis is also evaluated as SCALE * (EARLY + LATE):
    # EARLY sums the rest of each term whose table is keyed on alpha/beta only and whose factors
    # are all known once the air-relative geometry, the body rates and the aileron/rudder/LEF/
    # flaperon positions are (XML order), LATE the terms that need mach or the elevator.  Callers
    # that split the substep evaluate EARLY before the mach and elevator exist.
    PREFIX_OK = {"aero/qbar-psf", "metrics/Sw-sqft", "metrics/bw-ft", "metrics/cbarw-ft"}
    LATE_VARS = {"velocities/mach", "fcs/elevator-pos-rad"}
    split = {}
    for ai, ax in enumerate(AXES):
        prefix = None
        early, late = [], []
        for aj, short, f, rec in terms:
            if aj != ai or SB in f["factors"]:
                continue
            fs = list(f["factors"])
            npre = 0
            while npre < len(fs) and fs[npre] in PREFIX_OK:
                npre += 1
            pre = tuple(fs[:npre])
            if prefix is None:
                prefix = pre
            if pre != prefix:
                raise SystemExit(f"{ax}: term {short} does not share the axis prefix {prefix}")
            rest = [fnum(const_of[pp]) if pp in const_of else var_expr[pp] for pp in fs[npre:]]
            if f["value"] is not None:
                rest.append(fnum(f["value"]))
            keys = []
            if rec is not None:
                keys = [rec["row_var"]] + ([rec["col_var"]] if rec["kind"] == 2 else [])
                rest.append(f"lk_{short}")
            is_late = bool(LATE_VARS & (set(fs) | set(keys)))
            (late if is_late else early).append((short, " * ".join(rest) if rest else "1.0"))
        scale = " * ".join(fnum(const_of[pp]) if pp in const_of else var_expr[pp] for pp in prefix)
        split[ax] = (scale, early, late)
    for ai, ax in enumerate(AXES):
        parts_of = {"FREE": [], "CTL": []}
        for aj, short, f, rec in terms:
            if aj != ai:
                continue
            if SB in f["factors"]:
                dw(f"// {ax.lower()}: {short} omitted (speedbrake factor)")
                continue
            parts = []
            for pp in f["factors"]:
                parts.append(fnum(const_of[pp]) if pp in const_of else var_expr[pp])
            if f["value"] is not None:
                parts.append(fnum(f["value"]))
            uses = set(f["factors"])
            if rec is not None:
                keys = [rec["row_var"]] + ([rec["col_var"]] if rec["kind"] == 2 else [])
                uses |= set(keys)
                grp = "ELEV" if "ELEV" in {KEYGRP[k] for k in keys} else (
                    "MACH" if "MACH" in {KEYGRP[k] for k in keys} else "AB")
                if rec["kind"] == 1:
                    lk = f"f16_lerp1(T, F16M_T_AERO_{short}_OFF, b1_{rec['rg'][0]})"
                else:
                    lk = (f"f16_lerp2(T, F16M_T_AERO_{short}_OFF, F16M_T_AERO_{short}_NC, "
                          f"b2_{rec['rg'][0]}, b2_{rec['cg'][0]})")
                lks[grp].append(f"const double lk_{short} = {lk}")
                parts.append(f"lk_{short}")
            kind = "CTL" if CTL & uses else "FREE"
            parts_of[kind].append((short, " * ".join(parts)))
        sums[ax] = parts_of
    for grp in ("AB", "MACH", "ELEV"):
        macro(f"F16_AERO_BRACKETS_{grp}", brk[grp])
    dw("#define F16_AERO_BRACKETS F16_AERO_BRACKETS_AB; F16_AERO_BRACKETS_MACH; F16_AERO_BRACKETS_ELEV")
    for grp in ("AB", "MACH", "ELEV"):
        macro(f"F16_AERO_LOOKUPS_{grp}", lks[grp])
    dw("#define F16_AERO_LOOKUPS F16_AERO_LOOKUPS_AB; F16_AERO_LOOKUPS_MACH; F16_AERO_LOOKUPS_ELEV")
    for ax in AXES:
        for kind in ("FREE", "CTL"):
            dw(f"#define F16_AERO_{ax}_{kind} ( \\")
            dw("  0.0 \\")
            for short, expr in sums[ax][kind]:
                dw(f"  + {expr} /* {short} */ \\")
            dw("  )")
    for ax in AXES:
        scale, early, late = split[ax]
        dw(f"#define F16_AERO_{ax}_SCALE ({scale})")
        for kind, lst in (("EARLY", early), ("LATE", late)):
            dw(f"#define F16_AERO_{ax}_{kind} ( \\")
            dw("  0.0 \\")
            for short, expr in lst:
                dw(f"  + {expr} /* {short} */ \\")
            dw("  )")
    with open(os.path.join(args.out_dir, "f16_aero_gen.inc"), "w") as fh:
        fh.write("\n".join(d) + "\n")
    print(f"image {len(img.vals)} doubles, {len(img.grids)} grids, {len(tables)} tables")


if __name__ == "__main__":
    main()
