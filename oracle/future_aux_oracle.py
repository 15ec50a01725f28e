"""CPU restatement of the reference's future-aux labels (research/competition_36500/runtime/
cuda_fdm/future_aux.py:29-55, build_future_labels).  TEST INFRASTRUCTURE ONLY (imported by
tests/).  Plain loops over (t, engagement) in float64, the label rounded to float32 once.

episode id(t) = number of episode starts in [0, t] (future_aux.py:46, cumsum over time); the
horizon h label of step t exists when t + h < T and id(t + h) == id(t):
    residual = pos(t + h) - pos(t) - vel(t) * (h * dt)
    label    = R(t) @ residual / 100        (R(t) = own NED->body rotation, row-major)
slot 0: the partner (positions 6:9, velocities 9:12), h = 5; slot 1: own (0:3, 3:6), h = 10."""
import numpy as np

SLOTS = ((0, 5, 6, 9), (1, 10, 0, 3))


def future_labels(features, starts, dt):
    f = np.asarray(features, np.float64)
    st = np.asarray(starts)
    T, nenv = f.shape[:2]
    labels = np.zeros((T, nenv, 6), np.float32)
    mask = np.zeros((T, nenv, 2), bool)
    eid = np.cumsum(st.astype(np.int64), axis=0)
    for e in range(nenv):
        for t in range(T):
            for slot, h, pos, vel in SLOTS:
                if t + h >= T or eid[t + h, e] != eid[t, e]:
                    continue
                res = [(f[t + h, e, pos + i] - f[t, e, pos + i]) - f[t, e, vel + i] * (h * dt)
                       for i in range(3)]
                R = f[t, e, 12:21].reshape(3, 3)
                for i in range(3):
                    labels[t, e, 3 * slot + i] = np.float32(
                        (R[i, 0] * res[0] + R[i, 1] * res[1] + R[i, 2] * res[2]) / 100.0)
                mask[t, e, slot] = True
    return labels, mask
