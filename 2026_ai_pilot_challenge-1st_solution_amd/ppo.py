"""Rollout-side learner pieces on the GPU: GAE over the rollout buffer.

``gae`` replaces the Python reverse loop of PPOGPUTrainer.collect_rollout
(research/competition_36500/runtime/cuda_fdm/ppo_gpu.py:1979-1995) with one kernel launch
(f16_gae, one lane per (engagement, agent) column).  Same masking contract: ``done[t]`` is the
done flag entering step t (``b_done[t] = _next_done``), the last step uses ``next_done`` and the
bootstrap ``last_val``, and completed matches (termination or the 200 s timeout) are not
bootstrapped.
"""
import torch

from . import _lib


def gae(rew, val, done, last_val, next_done, gamma=0.997, lam=0.95):
    """rew, val: (T, nenv) or (T, nenv, nagents) float32; done: (T, nenv); last_val: (nenv,) or
    (nenv, nagents); next_done: (nenv,).  Returns (adv, ret) shaped like rew."""
    if rew.dtype != torch.float32 or val.dtype != torch.float32:
        raise TypeError("rewards and values must be float32 (the reference's buffers)")
    shape = rew.shape
    if rew.ndim == 2:
        T, nenv = shape
        nag = 1
    elif rew.ndim == 3:
        T, nenv, nag = shape
    else:
        raise ValueError("rew must be (T, nenv) or (T, nenv, nagents)")
    if val.shape != shape or tuple(done.shape) != (T, nenv):
        raise ValueError("val must match rew; done must be (T, nenv)")
    if last_val.numel() != nenv * nag or next_done.numel() != nenv:
        raise ValueError("last_val must hold nenv*nagents values, next_done nenv")
    dev = rew.device
    f = lambda x: x.to(device=dev, dtype=torch.float32).contiguous()
    rew, val, done, last_val, next_done = (f(x) for x in (rew, val, done, last_val, next_done))
    adv = torch.empty_like(rew)
    ret = torch.empty_like(rew)
    # gamma*lambda is formed in double then rounded once, as the reference's Python scalars are
    gl = float(torch.tensor(float(gamma) * float(lam), dtype=torch.float32))
    g = float(torch.tensor(float(gamma), dtype=torch.float32))
    rc = _lib.lib().f16_gae(_lib.ptr(rew), _lib.ptr(val), _lib.ptr(done), _lib.ptr(last_val),
                            _lib.ptr(next_done), T, nenv, nag, _lib.ctypes.c_float(g),
                            _lib.ctypes.c_float(gl), _lib.ptr(adv), _lib.ptr(ret),
                            _lib.stream_handle(dev))
    _lib.check(rc, "f16_gae")
    return adv, ret
