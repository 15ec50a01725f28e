"""Rollout-side learner pieces on the GPU: the self-play rollout collector and GAE over the
rollout buffer.

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


# algorithmic MLP work of one policy row (actor + critic, unpadded): 2 x MACs
POLICY_FLOP_PER_ROW = {d: 2 * (2 * 256 * d + 2 * 256 * 256 + 84 * 256 + 256) for d in (184, 214)}


class SelfPlayRollout:
    """Rollout collection with one policy on both aircraft of every engagement (BASELINE C4):
    the per-step sequence of PPOGPUTrainer.collect_rollout (research/competition_36500/runtime/
    cuda_fdm/ppo_gpu.py:1856-1932) -- RunningNorm.update, normalised observations into b_obs,
    actor draw + log-probability + critic value, action_to_env, env.step, reward and done into
    the buffers -- then the bootstrap value of the last observations and GAE
    (ppo_gpu.py:1971-1995) over (T, nenv, 2).  The learner's rows are both planes here, so every
    buffer carries nac = 2 nenv rows per step.

    Per step: f16_norm_update (3 small launches), f16_policy_step, the FDM decision and
    f16_env_post_step (which writes the float32 rewards and done flags straight into the
    buffers and draws autoreset pool rows itself); no host synchronisation.  stats=True adds the
    reference's episode-return bookkeeping (a few small torch launches per step)."""

    def __init__(self, env, net, T=64, gamma=0.99, lam=0.95, seed=0, update_norm=True,
                 stats=True):
        from .policy import PolicyStep, RunningNorm
        self.env, self.net, self.T = env, net, int(T)
        self.gamma, self.lam = float(gamma), float(lam)
        self.update_norm, self.want_stats = bool(update_norm), bool(stats)
        D, nac, ne, dev = env.OBS_SIZE, env.nac, env.nenv, env.device
        self.D, self.nac, self.nenv, self.device = D, nac, ne, dev
        self.norm = RunningNorm(D, dev)
        self.policy = PolicyStep(D, dev, seed)
        f32 = torch.float32
        self.b_obs = torch.empty(self.T, nac, D, dtype=f32, device=dev)
        self.b_act = torch.empty(self.T, nac, 4, dtype=torch.int64, device=dev)
        self.b_logp = torch.empty(self.T, nac, dtype=f32, device=dev)
        self.b_rew = torch.empty(self.T, nac, dtype=f32, device=dev)
        self.b_val = torch.empty(self.T, nac, dtype=f32, device=dev)
        self.b_done = torch.empty(self.T, ne, dtype=f32, device=dev)
        self.last_val = torch.empty(nac, dtype=f32, device=dev)
        self.next_obs = None
        self.next_done = torch.zeros(ne, dtype=f32, device=dev)
        self.ep_ret = torch.zeros(nac, dtype=f32, device=dev)
        self.ep_len = torch.zeros(ne, dtype=f32, device=dev)
        self.finite_acc = torch.ones(ne, dtype=torch.uint8, device=dev)
        self.global_step = 0
        # When set to a list, collect() appends (start, end) events around each policy launch.
        self.policy_events = None

    def reset(self, **kw):
        obs = self.env.reset(**kw)
        self.next_obs = obs.reshape(self.nac, self.D)
        self.next_done.zero_()
        return obs

    def _policy(self, obs, **out):
        ev = self.policy_events
        if ev is not None:
            e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            e0.record()
        self.policy(obs, [(self.net, 0, self.nac)], norm=self.norm, step=self.global_step, **out)
        if ev is not None:
            e1.record()
            ev.append((e0, e1))

    def collect(self):
        """One rollout of T steps; returns (adv, ret) as (T, nenv, 2) and a stats dict."""
        if self.next_obs is None:
            raise RuntimeError("call reset() first")
        env, T = self.env, self.T
        dev = self.device
        self.finite_acc.fill_(1)
        self.b_done[0].copy_(self.next_done)
        if self.want_stats:
            ret_sum = torch.zeros((), device=dev)
            ep_count = torch.zeros((), device=dev)
        for t in range(T):
            obs = self.next_obs
            if self.update_norm:
                self.norm.update(obs)
            self._policy(obs, nobs_out=self.b_obs[t], act_idx=self.b_act[t], logp=self.b_logp[t],
                         value=self.b_val[t], env_actions=env.sim.actions)
            done_t = self.b_done[t + 1] if t + 1 < T else self.next_done
            self.next_obs = env.step_rollout(self.b_rew[t], done_t, self.finite_acc)
            if self.want_stats:
                d2 = done_t.repeat_interleave(2)
                self.ep_ret += self.b_rew[t]
                ret_sum += (self.ep_ret * d2).sum()
                ep_count += done_t.sum()
                self.ep_ret *= 1.0 - d2
            self.global_step += 1
        self._policy(self.next_obs, value=self.last_val)
        shape = (T, self.nenv, 2)
        adv, ret = gae(self.b_rew.view(shape), self.b_val.view(shape), self.b_done,
                       self.last_val.view(self.nenv, 2), self.next_done, self.gamma, self.lam)
        stats = {"trajectory_finite": self.finite_acc.all()}
        if self.want_stats:
            stats.update(ret_sum=ret_sum, ep_count=ep_count)
        return adv, ret, stats
