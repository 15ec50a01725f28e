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
    stream, h = _lib.launch_stream(dev)
    rc = _lib.lib().f16_gae(_lib.ptr(rew), _lib.ptr(val), _lib.ptr(done), _lib.ptr(last_val),
                            _lib.ptr(next_done), T, nenv, nag, _lib.ctypes.c_float(g),
                            _lib.ctypes.c_float(gl), _lib.ptr(adv), _lib.ptr(ret), h)
    _lib.record(stream, (rew, val, done, last_val, next_done))
    _lib.check(rc, "f16_gae")
    return adv, ret


# algorithmic MLP work of one policy row (actor + critic, unpadded): 2 x MACs
POLICY_FLOP_PER_ROW = {d: 2 * (2 * 256 * d + 2 * 256 * 256 + 84 * 256 + 256) for d in (184, 214)}


class _RolloutGraph:
    """Records a collector's _run() once as a HIP graph (torch.cuda.CUDAGraph) and replays it.

    The env's and the collector's draw counters become device int32 scalars that the recorded
    launches read (step_base) and that the graph itself advances by T at its end.  Before every
    replay they are refilled from the host counters (collector.global_step, env._post_steps), so
    env steps taken outside the graph between two replays (an evaluation on the same env) move
    the next replay's draws on exactly as they move an eager collect's.  The first collect()
    runs eagerly so that every lazily allocated workspace exists before recording."""

    def __init__(self, owner, device):
        self.owner = owner
        self.graph = None
        self.warm = False
        self.pol_base = torch.zeros((), dtype=torch.int32, device=device)
        self.env_base = torch.zeros((), dtype=torch.int32, device=device)
        self.out = None

    def collect(self):
        o, env, T = self.owner, self.owner.env, self.owner.T
        if not self.warm:
            out = o._run()
            o.global_step += T
            self.warm = True
            return out
        for v in (o.global_step, env._post_steps):
            if not 0 <= v < 2 ** 31 - 4 * T:
                raise OverflowError("draw counters beyond the int32 device counters")
        if self.graph is None:
            p0 = env._post_steps
            torch.cuda.synchronize(self.pol_base.device)
            g = torch.cuda.CUDAGraph()
            with torch.cuda.graph(g):
                self.out = o._run(self.pol_base, self.env_base)
                self.pol_base.add_(T)
                self.env_base.add_(T)
            env._post_steps = p0            # recording ran nothing
            self.graph = g
        # small fills on the stream, outside the graph: the replay reads the host's counters
        self.pol_base.fill_(o.global_step)
        self.env_base.fill_(env._post_steps)
        self.graph.replay()
        o.global_step += T
        env._post_steps += T
        adv, ret, stats = self.out
        return adv, ret, dict(stats)


def _aux_buffers(o, env, aux):
    """aux=True: the future-aux buffers of collect_rollout (ppo_gpu.py:1194-1197) -- features of
    plane 0 per step (T, nenv, 21) float64, labels (T, nenv, 6) float32 and mask (T, nenv, 2),
    built after the rollout by f16_future_labels from the features and b_done."""
    o.b_aux_features = o.b_aux_labels = o.b_aux_mask = None
    if not aux:
        return
    env.enable_aux_capture()
    ne, dev = env.nenv, env.device
    o.b_aux_features = torch.zeros(o.T, ne, 21, dtype=torch.float64, device=dev)
    o.b_aux_labels = torch.zeros(o.T, ne, 6, dtype=torch.float32, device=dev)
    o._aux_mask_u8 = torch.zeros(o.T, ne, 2, dtype=torch.uint8, device=dev)
    o.b_aux_mask = o._aux_mask_u8.view(torch.bool)


def _aux_labels(o):
    if o.b_aux_features is not None:            # ppo_gpu.py:1996-1999
        from .future_aux import labels_into
        labels_into(o.b_aux_features, o.b_done, o.env.obr.dt, o.b_aux_labels, o._aux_mask_u8)


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
    reference's episode-return bookkeeping (a few small torch launches per step).

    graph=True records the whole rollout (T steps, bootstrap value, GAE) once as a HIP graph
    and replays it: the first collect() runs eagerly (it allocates every workspace), the second
    records and replays, later ones replay.  The draws' step counters then live on the device
    and advance inside the graph, so the results equal the eager collector's bit for bit.  The
    returned adv/ret are overwritten by the next collect(); weights refreshed with
    net.pack() are picked up by the next replay.  (stats=False only.)"""

    def __init__(self, env, net, T=64, gamma=0.99, lam=0.95, seed=0, update_norm=True,
                 stats=True, graph=False, aux=False, fuse_norm=True):
        from .policy import PolicyStep, RunningNorm
        self.env, self.net, self.T = env, net, int(T)
        self.gamma, self.lam = float(gamma), float(lam)
        self.update_norm, self.want_stats = bool(update_norm), bool(stats)
        # the post-physics launch of step t also forms the RunningNorm partial sums of the rows
        # step t + 1 normalises, which then needs only the merge (identical statistics)
        self.fuse_norm = bool(fuse_norm) and self.update_norm and env.norm_fusable()
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
        self._graph_mode = bool(graph)
        if self._graph_mode and self.want_stats:
            raise ValueError("graph=True needs stats=False")
        self._graphs = _RolloutGraph(self, dev) if self._graph_mode else None
        _aux_buffers(self, env, aux)

    def reset(self, **kw):
        obs = self.env.reset(**kw)
        self.next_obs = obs.reshape(self.nac, self.D)
        self.next_done.zero_()
        return obs

    def _policy(self, obs, step, step_base, **out):
        ev = self.policy_events
        if ev is not None:
            e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            e0.record()
        self.policy(obs, [(self.net, 0, self.nac)], norm=self.norm, step=step,
                    step_base=step_base, **out)
        if ev is not None:
            e1.record()
            ev.append((e0, e1))

    def _run(self, pol_base=None, env_base=None):
        """The rollout's launches.  With the bases (device counters) the draws' step counters
        are base + t instead of the host counters."""
        env, T = self.env, self.T
        dev = self.device
        g0 = 0 if pol_base is not None else self.global_step
        self.finite_acc.fill_(1)
        self.b_done[0].copy_(self.next_done)
        if self.want_stats:
            ret_sum = torch.zeros((), device=dev)
            ep_count = torch.zeros((), device=dev)
        for t in range(T):
            obs = self.next_obs
            if self.b_aux_features is not None:       # features of s_t (ppo_gpu.py:1876-1879)
                self.b_aux_features[t].copy_(env.obr.aux_features)
            if self.update_norm:
                if self.fuse_norm and t > 0:
                    self.norm.merge(self.nac)     # partials from step t - 1's post-physics launch
                else:
                    self.norm.update(obs)
            self._policy(obs, g0 + t, pol_base, nobs_out=self.b_obs[t], act_idx=self.b_act[t],
                         logp=self.b_logp[t], value=self.b_val[t], env_actions=env.sim.actions)
            done_t = self.b_done[t + 1] if t + 1 < T else self.next_done
            fused = self.norm if (self.fuse_norm and t + 1 < T) else None
            self.next_obs = env.step_rollout(self.b_rew[t], done_t, self.finite_acc,
                                             step_base=env_base, step=t, norm=fused)
            if self.want_stats:
                d2 = done_t.repeat_interleave(2)
                self.ep_ret += self.b_rew[t]
                ret_sum += (self.ep_ret * d2).sum()
                ep_count += done_t.sum()
                self.ep_ret *= 1.0 - d2
        self._policy(self.next_obs, g0 + T, pol_base, value=self.last_val)
        _aux_labels(self)
        shape = (T, self.nenv, 2)
        adv, ret = gae(self.b_rew.view(shape), self.b_val.view(shape), self.b_done,
                       self.last_val.view(self.nenv, 2), self.next_done, self.gamma, self.lam)
        stats = {}
        if self.want_stats:
            stats.update(ret_sum=ret_sum, ep_count=ep_count)
        return adv, ret, stats

    def collect(self):
        """One rollout of T steps; returns (adv, ret) as (T, nenv, 2) and a stats dict."""
        if self.next_obs is None:
            raise RuntimeError("call reset() first")
        if self._graph_mode:
            adv, ret, stats = self._graphs.collect()
        else:
            adv, ret, stats = self._run()
            self.global_step += self.T
        stats["trajectory_finite"] = self.finite_acc.all()
        return adv, ret, stats


def zipf_weights(n, s=1.1):
    """Opponent weights proportional to k^-s, k = 1..n (BASELINE league: Zipf(1.1) over 8)."""
    w = [float(k) ** -float(s) for k in range(1, int(n) + 1)]
    tot = sum(w)
    return [x / tot for x in w]


class LeagueRollout:
    """League-scale collection (BASELINE C5): the learner on plane 0 of every engagement and
    frozen opponent networks on plane 1, each engagement's opponent drawn from categorical
    weights (Zipf(1.1) by default) and redrawn when the engagement autoresets -- the
    ``opp_kind="pool"`` branch of PPOGPUTrainer.collect_rollout (research/competition_36500/
    runtime/cuda_fdm/ppo_gpu.py:1876-1908, 536-592), with the opponents evaluated as one grouped
    launch over rows sorted by opponent on the device (no host synchronisation, no per-opponent
    loop).  Buffers are per engagement (the learner's plane); GAE over (T, nenv).

    Per step: f16_norm_update over the learner's rows, f16_policy_step for the learner,
    f16_group_rows + one grouped f16_policy_step for all opponents, the FDM decision,
    f16_env_post_step (rewards, termination incl. optional fuel exhaustion, autoreset and the
    opponent redraw), and a strided copy of the learner's rewards.

    graph=True records the rollout as a HIP graph as SelfPlayRollout does (same results bit for
    bit; adv/ret overwritten by the next collect()).

    stats=True (eager only) adds collect_rollout's episode and match bookkeeping
    (ppo_gpu.py:1940-1969): returns, lengths and completed episodes of the learner; wins,
    losses and altitude losses from the terminal HP and altitude of both aircraft; and the
    per-opponent win / loss / episode counts, each finished match credited to the opponent that
    played it (the kernel redraws an autoreset engagement's opponent inside the step)."""

    def __init__(self, env, net, opponents, T=128, gamma=0.99, lam=0.95, seed=0,
                 update_norm=True, opp_weights=None, opp_norms=None, graph=False, aux=False,
                 stats=False, opp_deterministic=False):
        from .policy import PolicyStep, RunningNorm
        if len(opponents) < 1 or len(opponents) > 16:
            raise ValueError("1..16 opponent networks")
        self.env, self.net, self.opponents, self.T = env, net, list(opponents), int(T)
        self.gamma, self.lam, self.update_norm = float(gamma), float(lam), bool(update_norm)
        D, ne, nac, dev = env.OBS_SIZE, env.nenv, env.nac, env.device
        self.D, self.nenv, self.nac, self.device = D, ne, nac, dev
        self.seed = int(seed)
        self.norm = RunningNorm(D, dev)
        self.opp_norms = list(opp_norms) if opp_norms is not None else \
            [RunningNorm(D, dev) for _ in self.opponents]
        self.policy = PolicyStep(D, dev, seed)
        w = opp_weights if opp_weights is not None else zipf_weights(len(self.opponents))
        cdf, acc = [], 0.0
        for x in w:
            acc += float(x)
            cdf.append(acc)
        cdf = [c / acc for c in cdf]
        cdf[-1] = 1.0
        self.opp_weights = [float(x) / acc for x in w]
        env.opp_cdf = torch.tensor(cdf, dtype=torch.float32, device=dev)
        env.opp_assign = torch.zeros(ne, dtype=torch.int32, device=dev)
        self.main_rows = torch.arange(0, nac, 2, dtype=torch.int32, device=dev)
        self.opp_rows = torch.empty(ne, dtype=torch.int32, device=dev)
        self.opp_offsets = torch.empty(len(self.opponents) + 1, dtype=torch.int32, device=dev)
        self._group_work = torch.empty(max(8, _lib.lib().f16_group_workspace_bytes(ne)),
                                       dtype=torch.uint8, device=dev)
        f32 = torch.float32
        self.b_obs = torch.empty(self.T, ne, D, dtype=f32, device=dev)
        self.b_act = torch.empty(self.T, ne, 4, dtype=torch.int64, device=dev)
        self.b_logp = torch.empty(self.T, ne, dtype=f32, device=dev)
        self.b_rew = torch.empty(self.T, ne, dtype=f32, device=dev)
        self.b_val = torch.empty(self.T, ne, dtype=f32, device=dev)
        self.b_done = torch.empty(self.T, ne, dtype=f32, device=dev)
        self.last_val = torch.empty(ne, dtype=f32, device=dev)
        self.next_obs = None
        self.next_done = torch.zeros(ne, dtype=f32, device=dev)
        self.finite_acc = torch.ones(ne, dtype=torch.uint8, device=dev)
        self.global_step = 0
        self._lib = _lib.lib()
        # When set to lists, collect() appends (start, end) events around the policy launches.
        self.policy_events = None
        self.opp_events = None
        self._graph_mode = bool(graph)
        self.want_stats = bool(stats)
        self.opp_deterministic = bool(opp_deterministic)   # PPOGPUConfig.opp_sample = False
        if self._graph_mode and self.want_stats:
            raise ValueError("graph=True needs stats=False")
        self._graphs = _RolloutGraph(self, dev) if self._graph_mode else None
        if self.want_stats:
            self.min_alt = float(getattr(env, "min_altitude_m", 304.8))
            self.ep_ret = torch.zeros(ne, dtype=f32, device=dev)
            self.ep_len = torch.zeros(ne, dtype=f32, device=dev)
            self._thp = torch.empty(nac, dtype=torch.float64, device=dev)
            self._talt = torch.empty(nac, dtype=torch.float64, device=dev)
        # the opponents' grouping and launch run on a second stream (default priority) beside
        # the learner's normalisation and launch; both join before the env step
        self._side = None
        _aux_buffers(self, env, aux)

    def reset(self, **kw):
        """Reset the env and draw every engagement's opponent from the weights (seeded)."""
        import numpy as np
        obs = self.env.reset(**kw)
        rng = np.random.default_rng(self.seed + 7919)
        ids = rng.choice(len(self.opponents), size=self.nenv, p=np.asarray(self.opp_weights))
        self.env.opp_assign.copy_(torch.as_tensor(ids, dtype=torch.int32))
        self.next_obs = obs.reshape(self.nac, self.D)
        self.next_done.zero_()
        if self.want_stats:
            self.ep_ret.zero_()
            self.ep_len.zero_()
        return obs

    def _timed(self, events, fn):
        if events is None:
            return fn()
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record()
        out = fn()
        e1.record()
        events.append((e0, e1))
        return out

    def _opponents(self, obs, step, step_base):
        stream, h = _lib.launch_stream(self.device)
        rc = self._lib.f16_group_rows(_lib.ptr(self.env.opp_assign), self.nenv,
                                      len(self.opponents), 2, 1, _lib.ptr(self.opp_rows),
                                      _lib.ptr(self.opp_offsets), _lib.ptr(self._group_work), h)
        _lib.record_owned(self, stream, (self.env.opp_assign, self.opp_rows, self.opp_offsets,
                                         self._group_work))
        _lib.check(rc, "f16_group_rows")
        groups = [(net, None, None, nrm) for net, nrm in zip(self.opponents, self.opp_norms)]
        self.policy(obs, groups, rows=self.opp_rows, group_offsets=self.opp_offsets,
                    max_group_rows=self.nenv, nphys=self.nac, step=step, salt=1,
                    deterministic=self.opp_deterministic, env_actions=self.env.sim.actions,
                    step_base=step_base)

    def _run(self, pol_base=None, env_base=None):
        """The rollout's launches (see SelfPlayRollout._run for the device counters)."""
        env, T = self.env, self.T
        g0 = 0 if pol_base is not None else self.global_step
        self.finite_acc.fill_(1)
        self.b_done[0].copy_(self.next_done)
        main = torch.cuda.current_stream(self.device)
        if self._side is None:
            self._side = torch.cuda.Stream(device=self.device)
        st = self._stats_begin() if self.want_stats else None
        for t in range(T):
            obs = self.next_obs
            if self.b_aux_features is not None:
                self.b_aux_features[t].copy_(env.obr.aux_features)
            # plane 1 (grouping + the opponents' launch) beside plane 0 (normalisation + the
            # learner's launch): they share only reads of obs and write disjoint action rows
            self._side.wait_stream(main)
            with torch.cuda.stream(self._side):
                self._timed(self.opp_events, lambda: self._opponents(obs, g0 + t, pol_base))
            if self.update_norm:
                # plane 0's rows as a strided view (every second row), the same rows in the same
                # order as rows=main_rows, without the row-index loads
                self.norm.update(obs[0::2])
            self._timed(self.policy_events, lambda: self.policy(
                obs, [(self.net, 0, self.nenv)], norm=self.norm, rows=self.main_rows,
                nphys=self.nac, step=g0 + t, salt=0, nobs_out=self.b_obs[t],
                act_idx=self.b_act[t], logp=self.b_logp[t], value=self.b_val[t],
                env_actions=env.sim.actions, step_base=pol_base))
            main.wait_stream(self._side)
            done_t = self.b_done[t + 1] if t + 1 < T else self.next_done
            assign_t = env.opp_assign.clone() if st is not None else None
            self.next_obs = env.step_rollout(
                None, done_t, self.finite_acc, step_base=env_base, step=t,
                reward0_f32=self.b_rew[t], terminal_hp=self._thp if st is not None else None,
                terminal_alt_m=self._talt if st is not None else None)
            if st is not None:
                self._stats_step(st, self.b_rew[t], done_t, assign_t)
        self.policy(self.next_obs, [(self.net, 0, self.nenv)], norm=self.norm,
                    rows=self.main_rows, nphys=self.nac, step=g0 + T, value=self.last_val,
                    step_base=pol_base)
        _aux_labels(self)
        adv, ret = gae(self.b_rew, self.b_val, self.b_done, self.last_val, self.next_done,
                       self.gamma, self.lam)
        return adv, ret, (st if st is not None else {})

    def _stats_begin(self):
        dev, P = self.device, len(self.opponents)
        z = lambda: torch.zeros((), device=dev)
        return {"ret_sum": z(), "len_sum": z(), "ep_count": z(), "win_sum": z(),
                "loss_sum": z(), "alt_loss_sum": z(), "opponent_alt_loss_sum": z(),
                "opponent_ids": torch.arange(P, device=dev),
                "win_by_opp": torch.zeros(P, device=dev), "loss_by_opp": torch.zeros(P, device=dev),
                "ep_by_opp": torch.zeros(P, device=dev)}

    def _stats_step(self, st, rew, done, assign):
        """One step of collect_rollout's bookkeeping (ppo_gpu.py:1940-1969) from the learner's
        reward, the done flags, the terminal HP / altitude rows and the step's assignment."""
        self.ep_ret += rew
        self.ep_len += 1.0
        st["ret_sum"] += (self.ep_ret * done).sum()
        st["len_sum"] += (self.ep_len * done).sum()
        st["ep_count"] += done.sum()
        keep = 1.0 - done
        self.ep_ret.mul_(keep)
        self.ep_len.mul_(keep)
        th = self._thp.view(self.nenv, 2)
        ta = self._talt.view(self.nenv, 2)
        own_alt_dead = ta[:, 0] < self.min_alt
        own_dead = (th[:, 0] <= 0.0) | own_alt_dead
        opp_dead = (th[:, 1] <= 0.0) | (ta[:, 1] < self.min_alt)
        both_alive = ~own_dead & ~opp_dead
        win = (opp_dead & ~own_dead) | (both_alive & (th[:, 0] > th[:, 1] + 1e-9))
        loss = (own_dead & ~opp_dead) | (both_alive & (th[:, 0] < th[:, 1] - 1e-9))
        done_b = done.bool()
        dwin, dloss = (win & done_b).float(), (loss & done_b).float()
        st["win_sum"] += dwin.sum()
        st["loss_sum"] += dloss.sum()
        st["alt_loss_sum"] += (loss & own_alt_dead & done_b).float().sum()
        st["opponent_alt_loss_sum"] += (win & (ta[:, 1] < self.min_alt) & done_b).float().sum()
        rows = assign.long()
        st["win_by_opp"].scatter_add_(0, rows, dwin)
        st["loss_by_opp"].scatter_add_(0, rows, dloss)
        st["ep_by_opp"].scatter_add_(0, rows, done_b.float())

    def collect(self):
        """One rollout of T steps; returns (adv, ret) as (T, nenv) and a stats dict."""
        if self.next_obs is None:
            raise RuntimeError("call reset() first")
        if self._graph_mode:
            adv, ret, stats = self._graphs.collect()
        else:
            adv, ret, stats = self._run()
            self.global_step += self.T
        stats["trajectory_finite"] = self.finite_acc.all()
        return adv, ret, stats
