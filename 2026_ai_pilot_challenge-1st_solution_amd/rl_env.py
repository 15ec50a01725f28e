"""GpuDogfightVecEnv: batched 1v1 engagements (physics + observation + reward) on one GPU.

Mirror of the reference's ``GpuDogfightVecEnv`` (research/competition_36500/runtime/cuda_fdm/
rl_env.py:175-592): same constructor, attributes, reset / reset_evaluation / step / state9
contract and ``info`` keys.  The post-physics half of ``step`` (advance, reward, termination,
terminal observation, autoreset from the GPU initial-condition pool, re-anchoring and the new
observation) is one kernel launch (f16_env_post_step) instead of three kernels and about ten
torch operations; nothing inside ``step`` synchronises with the host.
"""
import numpy as np
import torch

from . import _lib
from . import ic as icm
from .gpu_env import GpuDogfight, STATE_N
from .obs_reward import (MY_REWARD_CONFIG, OBS_SIZE, OBS_SIZE_EXT, BatchObsReward,
                         reward_cfg_struct, validate_reward_mode)

FT2M = 0.3048
SEA_LEVEL_RADIUS_FT = 20925646.32546
HARD_DECK_M = 1000.0 * FT2M
NEUTRAL_ACTION = (0.0, 0.0, 0.0, 1.0)


class GpuDogfightVecEnv:
    """nenv engagements x 2 aircraft.  obs_dim 184 (default) or 214 (with NED accelerations)."""

    def __init__(self, nenv, substeps=6, precision="fp64", block=128, seed=None, device="cuda",
                 min_altitude_m=304.8, max_engage_time_s=200.0, reward_cfg=None, reward_mode=0,
                 alt_hunt_coef=5.0, scenario="mixed", headon_distance_m=5539.0, fcs_rate=60,
                 obs_dim=OBS_SIZE, ic_pool_size=4096, fuel_exhaustion=False, fuel_lbs_range=None):
        if precision != "fp64":
            raise ValueError("GpuDogfightVecEnv supports precision='fp64' only")
        if obs_dim not in (OBS_SIZE, OBS_SIZE_EXT):
            raise ValueError("obs_dim must be 184 or 214")
        self.sim = GpuDogfight(nenv, substeps=substeps, planes_per_env=2, precision=precision,
                               block=block, fcs_rate=fcs_rate, device=device)
        self.nenv = int(nenv)
        self.nac = self.sim.nac
        self.substeps = int(substeps)
        self.device = torch.device(device)
        self.seed = 0 if seed is None else int(seed)
        self.rng = np.random.default_rng(seed)
        # device-side draws (warm-up actions, autoreset pool picks) come from the env's own
        # generator rather than torch's global one, so an env is reproducible from its seed
        self.torch_gen = torch.Generator(device=self.device).manual_seed(self.seed)
        self.scenario = scenario
        self.headon_distance_m = float(headon_distance_m)
        self.scenario_b_prob = 0.0
        self.min_altitude_m = float(min_altitude_m)
        self.max_engage_time_s = float(max_engage_time_s)
        self.reward_cfg = dict(MY_REWARD_CONFIG if reward_cfg is None else reward_cfg)
        self.reward_mode = validate_reward_mode(reward_mode, alt_hunt_coef)
        self.alt_hunt_coef = float(alt_hunt_coef)
        self.fuel_exhaustion = bool(fuel_exhaustion)
        self.fuel_lbs_range = None if fuel_lbs_range is None else tuple(map(float, fuel_lbs_range))
        self.OBS_SIZE = int(obs_dim)
        # league: per-engagement opponent ids redrawn at autoreset from this CDF (set by the
        # league collector; None otherwise)
        self.opp_assign = None
        self.opp_cdf = None
        self.obr = BatchObsReward(nenv, device=device)
        if self.OBS_SIZE == OBS_SIZE_EXT:
            self.obr.enable_external_observations()
        self.ic_pool = None
        self.ic_pool_size = int(ic_pool_size)
        self._evaluation_seed_bank = None
        self._evaluation_seed_bank_key = None
        self._evaluation_seed_metadata = None
        n, ne, dev = self.nac, self.nenv, self.device
        self._obs = torch.zeros(n, self.OBS_SIZE, dtype=torch.float32, device=dev)
        self._neutral = torch.tensor([NEUTRAL_ACTION], dtype=torch.float64,
                                     device=dev).expand(n, 4).contiguous()
        # When set to a list, step() appends (start, end) events around its post-physics launch.
        self.kernel_events = None
        self._rec = self.obr._recon()
        self._cfg, self._cfg_key = None, None
        self._post_steps = 0
        # per-aircraft "all 101 state values finite" flags, written by the physics launch from
        # registers and read by the post-physics launch instead of the state (rl_env.py:545);
        # fused_finite=False makes the post-physics launch read the state and test it itself
        self._state_fin = torch.empty(n, dtype=torch.uint8, device=dev)
        self.fused_finite = True
        # physics and post-physics in one launch (f16_env_step) where the finite flags are on;
        # fused_step=False issues sim.step and f16_env_post_step as two launches
        self.fused_step = True
        # wavefronts per 64 aircraft in the one-launch step: 4 (f16_env_step) or 2
        # (f16_env_step_tworole); the same results
        self.step_roles = 4
        # per pool row, what an autoreset from it produces (observation, reward anchors, aux
        # features), so the post-physics launch copies instead of rebuilding; pool_tables=False
        # makes it rebuild them
        self.pool_tables = True
        self._pool_key = None
        self._pool_src = None
        self._capture_terminal_obs = True     # step's default (step_training clears it)
        self._pool_buf = None
        self._call_tensors = ()

    def enable_aux_capture(self):
        """Turn on the future-aux features (BatchObsReward.enable_aux_capture): every step and
        reset then also writes obr.aux_features (nenv, 21) for the returned observations."""
        self.obr.enable_aux_capture()
        self._rec = self.obr._recon()

    # ---- initial conditions (rl_env.py:218-375) ----
    def _sample_pairs(self, npairs):
        return icm.contest_rows(self.rng, npairs, self.scenario_b_prob, self.fuel_lbs_range)

    def _initialize_physical_seeds(self, rows):
        """(2P, 10) IC rows -> (P, 2, 101) float64 states after the neutral tick."""
        count = rows.shape[0]
        init = GpuDogfight(count // 2, precision=self.sim.precision, fcs_rate=self.sim.fcs_rate,
                           device=self.device)
        init.seed_rows(torch.as_tensor(rows, dtype=torch.float64, device=self.device))
        init.step(torch.tensor([NEUTRAL_ACTION] * count, dtype=torch.float64, device=self.device),
                  substeps=1, want_obs=False)
        return init.states.reshape(count // 2, 2, STATE_N).contiguous()

    def _ensure_ic_pool(self):
        if self.ic_pool is None:
            self.ic_pool = self._initialize_physical_seeds(self._sample_pairs(self.ic_pool_size))

    # ---- reset (rl_env.py:362-434) ----
    def reset(self, stagger=True, max_stagger_steps=256, warmup_action_fn=None):
        """Fresh contest ICs for every engagement; with stagger, each engagement is advanced a
        random number of valid decisions so episode phases are spread.  Returns obs (nenv,2,D)."""
        seeds = self._initialize_physical_seeds(self._sample_pairs(self.nenv))
        if not bool(torch.isfinite(seeds).all()):
            raise FloatingPointError("non-finite initial physical states")
        self.sim.load_seed(seeds)
        self.obr.reset_all()
        self.obr.kernel_init_reward_state(self.sim.states)
        if stagger and max_stagger_steps > 0:
            finite = self._staggered_warmup(max_stagger_steps, warmup_action_fn)
            if not bool(finite):               # the warm-up's one host check
                raise FloatingPointError("non-finite physical trajectory during staggered initialization")
        return self._build_obs_all()

    def _build_obs_all(self, env_mask=None):
        out = self.obr._build(self.sim.states, env_mask, self.OBS_SIZE, self._obs)
        return out.view(self.nenv, 2, self.OBS_SIZE)

    def _random_actions(self):
        a = torch.empty(self.nac, 4, dtype=torch.float64, device=self.device)
        a[:, 0:3].uniform_(-0.2, 0.2, generator=self.torch_gen)
        a[:, 3].uniform_(0.6, 0.9, generator=self.torch_gen)
        return a

    def _staggered_warmup(self, max_steps, action_fn):
        """rl_env.py:386-434 on the device: engagement e is advanced p_e ~ U[0, max_steps) valid
        decisions; an engagement that departs (below 100 m or non-finite) before its phase is
        re-seeded from the initial-condition pool (f16_env_reseed: pool row, reconstructor reset,
        re-anchored reward) and counts again; at its phase its physics and reconstructor are
        captured.  Nothing inside the loop synchronises with the host: every branch of the
        reference's loop is a masked device update and the loop runs its max_steps bound.
        Returns the device flag "every uncaptured trajectory stayed finite"."""
        self._ensure_ic_pool()
        ne, dev = self.nenv, self.device
        targ = torch.as_tensor(self.rng.integers(0, max_steps, size=ne)).pin_memory()
        targ = targ.to(dev, non_blocking=True)
        age = torch.zeros(ne, dtype=torch.long, device=dev)
        captured_mask = targ == 0
        captured = self.sim.states.clone()
        obr_buf = self.obr.clone_state()
        warm_finite = torch.ones((), dtype=torch.bool, device=dev)
        mask_u8 = torch.empty(ne, dtype=torch.uint8, device=dev)
        for k in range(max_steps):
            if action_fn is None:
                a = self._random_actions()
            else:
                a = action_fn(self._build_obs_all().reshape(self.nac, self.OBS_SIZE))
                a = torch.as_tensor(a, dtype=torch.float64, device=self.device).reshape(self.nac, 4)
            self.sim.step(a, substeps=self.substeps, want_obs=False)
            fin = torch.isfinite(self.sim.states).reshape(ne, -1).all(dim=1)
            warm_finite.logical_and_((fin | captured_mask).all())
            # push + advance (the kernel's reward side effects are re-anchored after capture)
            self.obr.kernel_advance(self.sim.states, a, cfg=self.reward_cfg,
                                    min_alt=self.min_altitude_m, max_time=self.max_engage_time_s,
                                    reward_mode=self.reward_mode, alt_hunt_coef=self.alt_hunt_coef)
            dep = self._departed_envs(self.state9_flat()) & (~captured_mask)
            mask_u8.copy_(dep)
            self._reseed(mask_u8, 0x80000000 | k)
            age = torch.where(dep, torch.zeros_like(age), age) + (~captured_mask).long()
            hit = (~captured_mask) & (age == targ)
            captured = torch.where(hit.repeat_interleave(2)[:, None], self.sim.states, captured)
            self.obr.capture_where(obr_buf, hit)
            captured_mask = captured_mask | hit
        rest = ~captured_mask                      # departed too late to reach their phase
        mask_u8.copy_(rest)
        self._reseed(mask_u8, 0x80000000 | max_steps)
        captured = torch.where(rest.repeat_interleave(2)[:, None], self.sim.states, captured)
        self.obr.capture_where(obr_buf, rest)
        self.sim.states.copy_(captured)
        self.obr.restore(obr_buf)
        self.obr.kernel_init_reward_state(self.sim.states)
        return warm_finite

    def _reseed(self, mask_u8, step):
        """f16_env_reseed over the engagements with mask_u8 set (pool draws keyed by `step`)."""
        io = self._io(None)
        io.step = step & 0xffffffff
        io.opp_assign = None
        stream, h = _lib.launch_stream(self.device)
        rc = self.obr._lib.f16_env_reseed(_lib.ctypes.byref(io), _lib.ctypes.byref(self._rec),
                                          mask_u8.data_ptr(), h)
        self._record(stream, (mask_u8,))
        _lib.check(rc, "f16_env_reseed")

    def _buffers(self):
        """The env's own device buffers a step or reseed launch may touch (the simulator's and
        the reconstructor's are recorded by their owners)."""
        pb = self._pool_buf or {}
        return (self._obs, self._state_fin, self.ic_pool, pb.get("obs"), pb.get("prev_x"),
                pb.get("alt"), pb.get("aux"), self.opp_assign, self.opp_cdf)

    def _record(self, stream, per_call):
        """Mark every tensor a launch of this env touches as used on the launch stream
        (cuda_fdm/tests/cuda_rt.py:134-136): the persistent buffers once per stream, `per_call`
        (the caller's actions, picks and output buffers) on each call.  Outputs this env
        allocates per call on the launch stream itself need no record."""
        _lib.record_owned(self.sim, stream, self.sim._buffers())
        _lib.record_owned(self.obr, stream, self.obr._recon_tensors())
        _lib.record_owned(self, stream, self._buffers())
        _lib.record(stream, per_call)

    def _departed_envs(self, s9_flat=None, floor_m=100.0):
        s9 = (self.state9() if s9_flat is None else s9_flat.view(self.nenv, 2, 9))
        alt = -s9[:, :, 2]
        bad = (alt < floor_m) | (~torch.isfinite(s9).all(dim=2))
        return bad.any(dim=1)

    def reset_evaluation(self, *, paired=False, seed_block=0):
        """Deterministic stratified contest bank, no warm-up (rl_env.py:260-327, 343-356)."""
        key = (bool(paired), int(seed_block))
        if self._evaluation_seed_bank is None or self._evaluation_seed_bank_key != key:
            self._evaluation_seed_bank = self._build_evaluation_seed_bank(paired, seed_block)
            self._evaluation_seed_bank_key = key
        self.sim.load_seed(self._evaluation_seed_bank)
        self.obr.reset_all()
        self.obr.kernel_init_reward_state(self.sim.states)
        return self._build_obs_all()

    def _build_evaluation_seed_bank(self, paired, seed_block):
        if paired and self.nenv % 8:
            raise ValueError("mirrored 3:1 evaluation requires nenv divisible by 8")
        base = self.nenv // 2 if paired else self.nenv
        rng = np.random.default_rng((self.seed + 19_870_331 + int(seed_block) * 1_000_003)
                                    % (2 ** 63 - 1))
        alt_order, spd_order = rng.permutation(base), rng.permutation(base)
        lo_a, hi_a = icm.CONTEST_ALT_FT
        lo_s, hi_s = icm.CONTEST_SPEED_MPS
        rows = np.zeros((self.nac, 10))
        counts = {str(int(d)): 0 for d in icm.CONTEST_DIST_A_FT}
        for e in range(base):
            alt = lo_a + (alt_order[e] + 0.5) / base * (hi_a - lo_a)
            spd = lo_s + (spd_order[e] + 0.5) / base * (hi_s - lo_s)
            dist = icm.CONTEST_DIST_A_FT[e % len(icm.CONTEST_DIST_A_FT)]
            counts[str(int(dist))] += 1
            rows[2 * e:2 * e + 2] = icm.contest_pair(
                self.rng, alt_ft=alt, speed=spd, side_swap=(e % 2) == 1, scenario_b=False,
                head_swap=((e // 2) % 2) == 1, dist_ft=dist)
        if paired:
            rows[2 * base:] = rows[:2 * base]
        self._evaluation_seed_metadata = {
            "paired": bool(paired), "seed_block": int(seed_block), "base_count": int(base),
            "three_nine": int(base), "headon": 0, "three_nine_distance_counts": counts}
        return self._initialize_physical_seeds(rows)

    # ---- step (rl_env.py:529-580) ----
    def _to_nac4(self, actions):
        a = torch.as_tensor(actions, dtype=torch.float64, device=self.device)
        return a.reshape(self.nac, 4)

    def _pool_table_ptrs(self):
        """Device tables of what an autoreset from each pool row produces: the observation
        (2 rows), the re-anchored geometry advantage and log altitude, plane 0's aux features.
        Built by the reference's own reset sequence on the pool's states (reset_envs ->
        init_reward -> build_obs, rl_env.py:559-577) through the same kernels, so a copied row
        equals a rebuilt one bit for bit; rebuilt when the pool tensor, its contents (torch's
        version counter), the observation width or aux capture change.  The tensor the tables
        were built from is held (_pool_src) and compared by identity: a replaced pool
        (`env.ic_pool = None` then a redraw, or a restored one) is a different object even
        where the allocator gives it the old pool's address.  The tables live in persistent
        buffers, so a recorded HIP graph keeps reading the current ones."""
        pool = self.ic_pool
        aux = self.obr.aux_features is not None
        key = (tuple(pool.shape), pool._version, self.OBS_SIZE, aux)
        if self._pool_src is not pool or self._pool_key != key:
            P, D = pool.shape[0], self.OBS_SIZE
            t = BatchObsReward(P, device=self.device)
            if D == OBS_SIZE_EXT:
                t.enable_external_observations()
            if aux:
                t.enable_aux_capture()
            states = pool.reshape(2 * P, STATE_N)
            t.kernel_init_reward_state(states)
            buf = self._pool_buf
            if buf is None or buf["obs"].shape != (2 * P, D):
                buf = {"obs": torch.empty(2 * P, D, dtype=torch.float32, device=self.device),
                       "prev_x": torch.empty(2 * P, dtype=torch.float64, device=self.device),
                       "alt": torch.empty(2 * P, dtype=torch.float64, device=self.device),
                       "aux": torch.zeros(P, 21, dtype=torch.float64, device=self.device)}
                self._pool_buf = buf
            t._build(states, None, D, buf["obs"])
            buf["prev_x"].copy_(t.prev_x)
            buf["alt"].copy_(t.prev_alt_log)
            if aux:
                buf["aux"].copy_(t.aux_features)
            self._pool_key, self._pool_src = key, pool
        b = self._pool_buf
        return (b["obs"].data_ptr(), b["prev_x"].data_ptr(), b["alt"].data_ptr(),
                b["aux"].data_ptr())

    def _io(self, pick):
        """F16EnvStepIO with the env's persistent pointers; per-call outputs set by the caller."""
        io = _lib.F16EnvStepIO()
        io.states, io.ld = self.sim._state_soa.data_ptr(), self.nac
        io.actions = self.sim.actions.data_ptr()
        io.ic_pool, io.pool_size = self.ic_pool.data_ptr(), self.ic_pool.shape[0]
        io.pick = pick.data_ptr() if pick is not None else None
        io.seed, io.step = self.seed, self._post_steps & 0xffffffff
        io.obs_dim, io.obs = self.OBS_SIZE, self._obs.data_ptr()
        if self.opp_assign is not None:
            io.opp_assign, io.opp_cdf = self.opp_assign.data_ptr(), self.opp_cdf.data_ptr()
            io.n_opp = self.opp_cdf.numel()
        if self.pool_tables:
            io.pool_obs, io.pool_prev_x, io.pool_prev_alt_log, io.pool_aux = \
                self._pool_table_ptrs()
        return io

    def _advance(self, io, actions, state_fin):
        """The physics step of `actions` and the post-physics step `io` describes: one
        f16_env_step launch with fused_step and the finite flags (state_fin) on (where the
        batch exceeds what the full-row tile keeps resident it issues the two launches itself),
        else sim.step and f16_env_post_step.  kernel_events, when a list, gets the one launch's
        (start, end)."""
        if not (self.fused_step and state_fin is not None):
            self.sim.step(actions, substeps=self.substeps, want_obs=False, finite_out=state_fin)
            io.state_finite = state_fin.data_ptr() if state_fin is not None else None
            self._post(io)
            return
        a = self.sim.action_source(actions)
        io.state_finite = state_fin.data_ptr()
        c = self._cfg_struct()
        ev = self.kernel_events
        if ev is not None:
            e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            e0.record()
        fn = (self.obr._lib.f16_env_step_tworole if self.step_roles == 2 else
              self.obr._lib.f16_env_step)
        stream, h = _lib.launch_stream(self.device)
        rc = fn(_lib.ctypes.byref(io), _lib.ctypes.byref(self._rec), _lib.ctypes.byref(c),
                a.data_ptr(), self.substeps, self.sim.fcs_rate, state_fin.data_ptr(), h)
        if ev is not None:
            e1.record()
            ev.append((e0, e1))
        self._record(stream, self._call_tensors + (a,))
        _lib.check(rc, "f16_env_step")
        self._post_steps += 1

    def _post(self, io):
        c = self._cfg_struct()
        ev = self.kernel_events
        if ev is not None:
            e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            e0.record()
        stream, h = _lib.launch_stream(self.device)
        rc = self.obr._lib.f16_env_post_step(_lib.ctypes.byref(io), _lib.ctypes.byref(self._rec),
                                             _lib.ctypes.byref(c), h)
        if ev is not None:
            e1.record()
            ev.append((e0, e1))
        self._record(stream, self._call_tensors)
        _lib.check(rc, "f16_env_post_step")
        self._post_steps += 1

    def _cfg_struct(self):
        key = (tuple(sorted(self.reward_cfg.items())), self.min_altitude_m, self.max_engage_time_s,
               self.reward_mode, self.alt_hunt_coef, self.fuel_exhaustion)
        if self._cfg_key != key:
            self._cfg = reward_cfg_struct(self.reward_cfg, self.min_altitude_m,
                                          self.max_engage_time_s, self.reward_mode,
                                          self.alt_hunt_coef, self.fuel_exhaustion)
            self._cfg_key = key
        return self._cfg

    def step_training(self, actions):
        """The root lineage's training-consumer step (cuda_fdm/rl_env.py:518-527): step() with
        the terminal-observation copy turned off for this call (info["terminal_obs"] is None);
        the instance default is restored even if the step raises."""
        previous = getattr(self, "_capture_terminal_obs", True)
        self._capture_terminal_obs = False
        try:
            return self.step(actions)
        finally:
            self._capture_terminal_obs = previous

    def step(self, actions, *, reset_indices=None, terminal_obs=None, capture_terminal_obs=None):
        """actions (nenv,2,4) or (nac,4) [aileron, elevator, rudder, throttle].
        Returns (obs (nenv,2,D) f32, reward (nenv,2) f64, done (nenv,) bool, info).
        capture_terminal_obs=False (root lineage, cuda_fdm/rl_env.py:529; `terminal_obs` is the
        same switch) skips the terminal-observation copy: info["terminal_obs"] is None.  Unset,
        the instance default `_capture_terminal_obs` (True) applies.  reset_indices: the 184-D
        lineage's explicit pool rows per engagement (R/cuda_fdm/rl_env.py:499)."""
        if capture_terminal_obs is None:
            capture_terminal_obs = terminal_obs
        if capture_terminal_obs is None:
            capture_terminal_obs = getattr(self, "_capture_terminal_obs", True)
        terminal_obs = bool(capture_terminal_obs)
        a = self._to_nac4(actions)
        self._ensure_ic_pool()
        state_fin = self._state_fin if self.fused_finite and self.substeps >= 1 else None
        if reset_indices is None:
            # the pool row of each finished engagement is drawn inside the post-physics launch
            # (uniform over the pool: Philox keyed by the env seed, the step count and the
            # engagement), the reference's torch.randint draw (R/cuda_fdm/rl_env.py:534-535) without
            # a launch of its own
            pick = None
        else:
            if (reset_indices.shape != (self.nenv,) or reset_indices.dtype != torch.long
                    or reset_indices.device != self.sim.states.device):
                raise ValueError("reset indices must be one device int64 index per environment")
            pick = reset_indices.contiguous()
        n, ne, dev = self.nac, self.nenv, self.device
        reward = torch.empty(n, dtype=torch.float64, device=dev)
        tobs = (torch.empty(n, self.OBS_SIZE, dtype=torch.float32, device=dev) if terminal_obs
                else None)
        terminal_hp = torch.empty(n, dtype=torch.float64, device=dev)
        terminal_alt = torch.empty(n, dtype=torch.float64, device=dev)
        term, trunc, done, fin = (torch.empty(ne, dtype=torch.bool, device=dev) for _ in range(4))
        io = self._io(pick)
        self._call_tensors = (pick,)
        p = lambda t: t.data_ptr() if t is not None else None
        io.terminal_obs, io.reward = p(tobs), p(reward)
        io.term, io.trunc, io.done, io.terminal_finite = p(term), p(trunc), p(done), p(fin)
        io.terminal_hp, io.terminal_alt_m = p(terminal_hp), p(terminal_alt)
        self._advance(io, a, state_fin)
        info = {"terminated": term, "truncated": trunc,
                "terminal_obs": tobs.view(ne, 2, self.OBS_SIZE) if tobs is not None else None,
                "terminal_hp": terminal_hp.view(ne, 2),
                "terminal_alt_m": terminal_alt.view(ne, 2), "done": done,
                "terminal_state_finite": fin}
        return self._obs.view(ne, 2, self.OBS_SIZE), reward.view(ne, 2), done, info

    def norm_fusable(self):
        """Whether step_rollout can also form the RunningNorm partial sums of its new rows."""
        return bool(self.obr._lib.f16_env_post_step_norm_fusable(self.nenv, self.OBS_SIZE))

    def step_rollout(self, reward_f32, done_f32, finite_acc, step_base=None, step=0, norm=None,
                     reward0_f32=None, terminal_hp=None, terminal_alt_m=None):
        """The rollout collector's step: the controls already sit in sim.actions (written by the
        policy kernel); the physics and the post-physics step (one launch, _advance) write the
        float32 rewards (nac,) and done flags (nenv,) straight into the caller's buffers and clear
        finite_acc (nenv,) bytes of engagements whose state went non-finite.  Autoreset pool rows
        are drawn inside the kernel (Philox keyed by the env seed and a per-env step counter).
        step_base (device int32 scalar) + step replaces the env's host step counter in the
        kernel's draws: a rollout recorded in a HIP graph advances step_base on the device.
        norm (a RunningNorm, only where norm_fusable()): the launch also writes the partial sums
        of the new observation rows into its workspace, for norm.merge(nac).  reward_f32 may be
        None when reward0_f32 (nenv,) is given: the launch then writes only each engagement's
        first aircraft's reward, straight into a learner-side buffer.  terminal_hp and
        terminal_alt_m (float64 (nac,), optional) receive step()'s info["terminal_hp"] and
        info["terminal_alt_m"] rows."""
        self._ensure_ic_pool()
        state_fin = self._state_fin if self.fused_finite and self.substeps >= 1 else None
        io = self._io(None)
        if step_base is not None:
            io.step, io.step_base = int(step) & 0xffffffff, step_base.data_ptr()
        if reward_f32 is None and reward0_f32 is None:
            raise ValueError("step_rollout needs reward_f32 or reward0_f32")
        io.reward_f32 = reward_f32.data_ptr() if reward_f32 is not None else None
        io.reward0_f32 = reward0_f32.data_ptr() if reward0_f32 is not None else None
        io.done_f32 = done_f32.data_ptr()
        io.finite_acc = finite_acc.data_ptr()
        for t in (terminal_hp, terminal_alt_m):
            if t is not None and (t.dtype != torch.float64 or t.numel() != self.nac or
                                  not t.is_contiguous() or t.device != self._obs.device):
                raise ValueError("terminal_hp / terminal_alt_m: contiguous float64 (nac,) on the "
                                 "env's device")
        if terminal_hp is not None:
            io.terminal_hp = terminal_hp.data_ptr()
        if terminal_alt_m is not None:
            io.terminal_alt_m = terminal_alt_m.data_ptr()
        if norm is not None:
            norm.fused_partials(io, self.nac)
        self._call_tensors = (reward_f32, reward0_f32, done_f32, finite_acc, step_base,
                              terminal_hp, terminal_alt_m) + (
            (norm._work, norm.count) if norm is not None else ())
        self._advance(io, self.sim.actions, state_fin)
        return self._obs.view(self.nac, self.OBS_SIZE)

    # ---- state export (rl_env.py:583-592) ----
    def state9_flat(self):
        out = torch.empty(self.nac, 9, dtype=torch.float64, device=self.device)
        stream, h = _lib.launch_stream(self.device)
        rc = self.obr._lib.f16_state9(_lib.ptr(self.sim._state_soa), self.nac, self.nac,
                                      _lib.ptr(out), h)
        _lib.record_owned(self.sim, stream, self.sim._buffers())
        _lib.check(rc, "f16_state9")
        return out

    def state9(self):
        return self.state9_flat().view(self.nenv, 2, 9)
