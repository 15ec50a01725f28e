#!/usr/bin/env python3
"""Write the IC-seeding golden vectors (tests/golden/seed_golden.npz) from the reference.

Why an import is used here: the reference's seeding (cuda_fdm/ic.py:117-138 build_seed_vector,
which runs cuda_fdm/ref/jsb_fdm.py:142-210 FDM.seed with a throwaway force path) has no
host-compilable C counterpart, no golden file of its own and no closed form, so nothing else
pins it.  This script imports it from a reference checkout IN THE BUILD CONTAINER ONLY and
stores inputs and outputs as plain arrays; the reference never travels with the repository.

Two lineages: the root package (FCS component dt 1/120) and the 184-D runtime copy under
research/competition_36500/runtime (FCS dt 1/60).  Each is imported in its own subprocess
because both are named ``cuda_fdm``.

IC row layout (matches oracle orc_build_seed and the HIP seed kernel):
    [lat_deg, lon_deg, alt_ft, vt_fps, phi_deg, theta_deg, psi_deg, alpha_deg, beta_deg, fuel_lbs]
Usage:  python tests/golden/make_fdm_golden.py [--ref /root/reference]
"""
import argparse
import json
import os
import subprocess
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
LINEAGES = {120: "", 60: "research/competition_36500/runtime"}


def ic_rows(n=48, seed=20261201):
    rng = np.random.default_rng(seed)
    rows = []
    heads = [0.0, 90.0, 180.0, 270.0]
    for i in range(n):
        lat = 37.240778 + rng.uniform(-0.05, 0.05)
        lon = 131.869556 + rng.uniform(-0.05, 0.05)
        alt = rng.uniform(2000.0, 33000.0)
        vt = rng.uniform(150.0, 350.0) / 0.3048
        if i < 16:      # contest-like: level, wings level, cardinal headings
            phi = th = al = be = 0.0
            psi = heads[i % 4]
        else:
            phi = rng.uniform(-60.0, 60.0)
            th = rng.uniform(-20.0, 20.0)
            psi = rng.uniform(0.0, 360.0)
            al = rng.uniform(-4.0, 12.0)
            be = rng.uniform(-4.0, 4.0)
        fuel = [6000.0, 3000.0, 6972.0][i % 3]
        rows.append([lat, lon, alt, vt, phi, th, psi, al, be, fuel])
    # a supersonic and a very slow case exercise the pitot iteration and the FCS triggers
    rows.append([37.24, 131.87, 36000.0, 1.6 * 968.0, 0.0, 0.0, 45.0, 1.0, 0.0, 6000.0])
    rows.append([37.24, 131.87, 3000.0, 160.0, 0.0, 5.0, 10.0, 8.0, 0.0, 6000.0])
    return np.array(rows, dtype=np.float64)


def child(ref_root, sub, rows_json):
    sys.path.insert(0, os.path.join(ref_root, sub) if sub else ref_root)
    from cuda_fdm.ic import build_seed_vector  # noqa: E402  (reference, build container only)
    rows = json.loads(rows_json)
    out = []
    for r in rows:
        out.append(build_seed_vector(lat_deg=r[0], lon_deg=r[1], alt_ft=r[2], vt_fps=r[3],
                                     phi_deg=r[4], theta_deg=r[5], psi_deg=r[6], alpha_deg=r[7],
                                     beta_deg=r[8], fuel_lbs=r[9]))
    print(json.dumps([[float.hex(float(v)) for v in row] for row in out]))


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--ref", default="/root/reference")
    ap.add_argument("--child", nargs=2)
    a = ap.parse_args()
    if a.child:
        child(a.ref, a.child[0], sys.stdin.read())
        return
    rows = ic_rows()
    res = {"ic": rows}
    for rate, sub in LINEAGES.items():
        p = subprocess.run([sys.executable, __file__, "--ref", a.ref, "--child", sub or "", "x"],
                           input=json.dumps(rows.tolist()), capture_output=True, text=True, check=True)
        seeds = np.array([[float.fromhex(v) for v in row] for row in json.loads(p.stdout)])
        assert seeds.shape == (len(rows), 101)
        res[f"seed_{rate}"] = seeds
    np.savez_compressed(os.path.join(HERE, "seed_golden.npz"), **res)
    print("wrote seed_golden.npz", {k: v.shape for k, v in res.items()})


if __name__ == "__main__":
    main()
