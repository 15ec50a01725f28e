"""CPU restatement of the reference learner's GAE (research/competition_36500/runtime/cuda_fdm/
ppo_gpu.py:1979-1995).  TEST INFRASTRUCTURE ONLY (imported by tests/ and bench.py's CPU leg).

Two forms:
  gae_f32  -- the reference's float32 operation order, element by element (numpy float32
              scalars round after every operation, as torch's eager elementwise kernels do);
  gae_f64  -- the textbook recurrence in float64 (ppo_gpu_val.py:_ref_gae, CleanRL convention).
Buffers are time-major (T, ncol); `done` is (T, nenv) shared by nagents columns per engagement;
done[t] is the done flag entering step t."""
import numpy as np


def _expand(done, nagents):
    return np.repeat(np.asarray(done), nagents, axis=-1)


def gae_f32(rew, val, done, last_val, next_done, gamma, lam, nagents=1):
    rew = np.asarray(rew, np.float32); val = np.asarray(val, np.float32)
    d = _expand(np.asarray(done, np.float32), nagents)
    nd = _expand(np.asarray(next_done, np.float32), nagents)
    T = rew.shape[0]
    g = np.float32(gamma)
    gl = np.float32(float(gamma) * float(lam))
    one = np.float32(1.0)
    adv = np.zeros_like(rew)
    last = np.zeros(rew.shape[1], np.float32)
    for t in reversed(range(T)):
        if t == T - 1:
            nnt = one - nd
            nv = np.asarray(last_val, np.float32)
        else:
            nnt = one - d[t + 1]
            nv = val[t + 1]
        delta = (rew[t] + (g * nv) * nnt) - val[t]
        last = delta + (gl * nnt) * last
        adv[t] = last
    return adv, adv + val


def gae_f64(rew, val, done, last_val, next_done, gamma, lam, nagents=1):
    rew = np.asarray(rew, np.float64); val = np.asarray(val, np.float64)
    d = _expand(np.asarray(done, np.float64), nagents)
    nd = _expand(np.asarray(next_done, np.float64), nagents)
    T = rew.shape[0]
    adv = np.zeros_like(rew)
    last = np.zeros(rew.shape[1])
    for t in reversed(range(T)):
        nnt = 1.0 - (nd if t == T - 1 else d[t + 1])
        nv = np.asarray(last_val, np.float64) if t == T - 1 else val[t + 1]
        delta = rew[t] + gamma * nv * nnt - val[t]
        last = delta + gamma * lam * nnt * last
        adv[t] = last
    return adv, adv + val
