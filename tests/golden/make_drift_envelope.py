#!/usr/bin/env python3
"""Write tests/golden/drift_envelope.npz: how far the reference's own two implementations of
the flight model drift apart on BASELINE C1, decision by decision.

The two implementations are the reference's C model (research/competition_36500/runtime/
cuda_fdm/gen/fdm.cuh, the code its GPU kernel runs, compiled for the host into
oracle/_ref/libf16ref_120.so by oracle/Makefile) and the CPU restatement of its Python model
(cuda_fdm/ref, oracle/liborc.so).  Both start from the same seeded states and fly the same
actions: 8 replicas of C1 (seeds 0-7; each 64 head-on engagements, 600 decisions of i.i.d.
21-bin actions, FCS at 120 Hz) = 1,024 aircraft.  They differ only where fdm.cuh rounds
differently from the Python model (x**3.5 vs x^3 sqrt x, (1-n)**3 vs (1-n)(1-n)(1-n),
/mass vs *(1/mass)); random full-deflection manoeuvring amplifies those last-ulp differences
exponentially.

Stored per decision d (0-based, after decision d+1): over the aircraft still above the 304.8 m
hard deck in the restatement's run (a cumulative mask), the 0.5 / 0.75 / 0.9 / 1.0 quantiles
of |ECI position difference| in feet, and the number of such aircraft.

Usage (build container, needs oracle/_ref):  python tests/golden/make_drift_envelope.py
"""
import importlib
import os
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(os.path.dirname(HERE))
sys.path.insert(0, os.path.join(ROOT, "tests"))
sys.path.insert(0, ROOT)



def main():
    import oracle_lib as O
    icm = importlib.import_module("2026_ai_pilot_challenge-1st_solution_amd.ic")
    orc, ref = O.load(), O.load_ref(120)
    if ref is None:
        raise SystemExit("oracle/_ref/libf16ref_120.so is missing: run make -C oracle")
    ic, acts = O.c1_replicas(icm)
    a = orc.seed(ic, 120)
    b = a.copy()
    alive = np.ones(len(a), bool)
    q = np.zeros((O.DRIFT_NDEC, len(O.DRIFT_QUANTILES)))
    count = np.zeros(O.DRIFT_NDEC, np.int64)
    for d in range(O.DRIFT_NDEC):
        orc.step(a, acts[d], 6, want_obs=False)
        ref.step(b, acts[d], 6)
        alive &= O.altitude_m(a) > 304.8
        q[d] = O.drift_quantiles(a, b, alive)
        count[d] = alive.sum()
    np.savez_compressed(os.path.join(HERE, "drift_envelope.npz"),
                        quantiles=np.array(O.DRIFT_QUANTILES), pos_ft=q, alive=count)
    print("wrote drift_envelope.npz; alive at 600:", count[-1])


if __name__ == "__main__":
    main()
