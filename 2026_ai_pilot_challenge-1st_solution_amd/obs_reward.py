"""BatchObsReward: observation / reward / termination reconstructor on the GPU.

Mirror of the reference's kernel path of ``BatchObsReward``
(research/competition_36500/runtime/cuda_fdm/obs_reward.py:319-569): same constructor, tensor
attributes, kernel_* methods, masked resets and snapshot/restore.  The kernels are the gfx950
ones in libf16hip.so (include/f16_obs.h), launched on the caller's current stream.

Differences in mechanism, not contract:
  * per-aircraft vectors (prev_att, pqr, act_hist, and the 214-D prev-velocity/acceleration)
    live structure-of-arrays; the public attributes are (nac, 3) / (nac, 5, 4) views of them;
  * ``states`` may be the simulator's structure-of-arrays view (GpuDogfight.states) or any
    (nac, 101) float64 CUDA tensor;
  * there is no torch fallback: the s9-input torch methods (advance, build_obs,
    compute_reward) of the reference are its CPU audit path and are not mirrored.
"""
import math

import torch

from . import _lib
from .future_aux import AUX_FEATURE_DIM

OBS_SIZE = 184
OBS_SIZE_EXT = 214
ACT_LEN, ACT_DIM = 5, 4
DT_PER_STEP = 6.0 / 60.0

# MY_REWARD_CONFIG scalars read by the kernels (claude_code/my_reward.py:45-103)
MY_REWARD_CONFIG = {
    "win_reward": 5.0, "loss_reward": -5.0,
    "timeout_win_reward": 5.0, "timeout_loss_reward": -5.0, "timeout_draw_reward": -4.0,
    "damage_scale": 10.0, "own_damage_weight": 1.0, "shaping_reward_scale": 0.0001,
}
STANDARD_REWARD, ALTITUDE_HUNT_REWARD, ATTACK_REWARD, DEFENSE_REWARD = 0, 1, 2, 3


def validate_reward_mode(mode, coefficient=5.0):
    """cuda_fdm/reward_modes.py validate_reward_mode."""
    if mode not in (STANDARD_REWARD, ALTITUDE_HUNT_REWARD, ATTACK_REWARD, DEFENSE_REWARD):
        raise ValueError(f"unknown reward mode: {mode!r}")
    if not math.isfinite(coefficient) or coefficient < 0:
        raise ValueError("altitude-hunt coefficient must be finite and nonnegative")
    return int(mode)


def reward_cfg_struct(cfg, min_alt, max_time, mode, alt_hunt_coef, fuel_exhaustion=False):
    c = _lib.F16RewardCfg()
    c.own_damage_weight = float(cfg.get("own_damage_weight", 0.5))
    for key in ("damage_scale", "shaping_reward_scale", "win_reward", "loss_reward",
                "timeout_win_reward", "timeout_loss_reward", "timeout_draw_reward"):
        setattr(c, key, float(cfg[key]))
    c.min_alt_m, c.max_time_s = float(min_alt), float(max_time)
    c.alt_hunt_coef = float(alt_hunt_coef)
    c.mode = int(mode)
    c.fuel_exhaustion = int(bool(fuel_exhaustion))
    return c


def soa_states(states, nac):
    """(pointer tensor, ld) for a (nac, 101) float64 CUDA tensor: the structure-of-arrays buffer
    behind a transposed view is used in place, anything else is transposed into a copy."""
    if not torch.is_tensor(states) or states.dtype != torch.float64:
        raise TypeError("FDM states kernel requires dtype torch.float64; no implicit pointer cast")
    if tuple(states.shape) != (nac, 101):
        raise ValueError(f"FDM states shape {tuple(states.shape)} != {(nac, 101)}")
    if states.device.type != "cuda":
        raise ValueError("FDM states must be on a CUDA (HIP) device")
    if states.stride(0) == 1 and states.stride(1) >= nac:
        return states, states.stride(1)
    soa = states.t().contiguous()
    return soa, nac


class BatchObsReward:
    """nac = 2*nenv aircraft; aircraft a of engagement e is 2e (plane 0) or 2e+1 (plane 1)."""

    _AC_KEYS = ("hp", "fuel", "prev_att", "prev_valid", "pqr", "last_dmg_dealt",
                "last_dmg_taken", "hp_loss", "act_hist", "prev_x", "prev_x_valid",
                "prev_alt_log")
    _ENV_KEYS = ("t_sec",)

    def __init__(self, nenv, device="cuda", dtype=torch.float64, enable_kernel=True):
        if dtype != torch.float64:
            raise ValueError("the observation/reward kernels run in float64 only")
        if not enable_kernel:
            raise ValueError("BatchObsReward on MI355X is the HIP kernel path only")
        self.nenv = int(nenv)
        self.nac = 2 * self.nenv
        self.device = torch.device(device)
        self.dtype = dtype
        self.dt = DT_PER_STEP
        self._lib = _lib.lib()
        idx = torch.arange(self.nac, device=self.device)
        self.partner = idx ^ 1
        self.env_of = idx // 2
        self._alloc()
        self.reset_all()
        self.block = 256
        n, ne, dev = self.nac, self.nenv, self.device
        self.obs_buf = torch.zeros(n, OBS_SIZE, dtype=torch.float32, device=dev)
        self.reward_buf = torch.zeros(n, dtype=torch.float64, device=dev)
        self.term_buf = torch.zeros(ne, dtype=torch.uint8, device=dev)
        self.trunc_buf = torch.zeros(ne, dtype=torch.uint8, device=dev)
        self.aux_features = None
        self.kernel_ready = True

    def _alloc(self):
        n, ne, dev, dt = self.nac, self.nenv, self.device, self.dtype
        self.hp = torch.ones(n, device=dev, dtype=dt)
        self.fuel = torch.ones(n, device=dev, dtype=dt)
        self.t_sec = torch.zeros(ne, device=dev, dtype=dt)
        self._att_soa = torch.zeros(3, n, device=dev, dtype=dt)
        self.prev_att = self._att_soa.t()
        self.prev_valid = torch.zeros(n, device=dev, dtype=torch.bool)
        self._pqr_soa = torch.zeros(3, n, device=dev, dtype=dt)
        self.pqr = self._pqr_soa.t()
        self.last_dmg_dealt = torch.zeros(n, device=dev, dtype=dt)
        self.last_dmg_taken = torch.zeros(n, device=dev, dtype=dt)
        self.hp_loss = torch.zeros(n, device=dev, dtype=dt)
        self._hist_soa = torch.zeros(ACT_LEN * ACT_DIM, n, device=dev, dtype=dt)
        self.act_hist = self._hist_soa.t().view(n, ACT_LEN, ACT_DIM)
        self.prev_x = torch.zeros(n, device=dev, dtype=dt)
        self.prev_x_valid = torch.zeros(n, device=dev, dtype=torch.bool)
        self.prev_alt_log = torch.zeros(n, device=dev, dtype=dt)
        self._vel_soa = None
        self._acc_soa = None

    def _recon(self):
        r = _lib.F16Recon()
        p = lambda t: t.data_ptr() if t is not None else None
        r.hp, r.fuel, r.t_sec = p(self.hp), p(self.fuel), p(self.t_sec)
        r.prev_att, r.prev_valid, r.pqr = p(self._att_soa), p(self.prev_valid), p(self._pqr_soa)
        r.dealt, r.taken, r.hp_loss = p(self.last_dmg_dealt), p(self.last_dmg_taken), p(self.hp_loss)
        r.act_hist, r.prev_x, r.prev_x_valid = p(self._hist_soa), p(self.prev_x), p(self.prev_x_valid)
        r.prev_alt_log = p(self.prev_alt_log)
        r.prev_vel_ned, r.accel = p(self._vel_soa), p(self._acc_soa)
        r.ld, r.nenv = self.nac, self.nenv
        r.aux = p(self.aux_features)
        return r

    def enable_aux_capture(self):
        """Future-aux features (obs_reward.py:355-358): every observation launch also writes the
        (nenv, 21) float64 features of plane 0 (training labels only, never observations)."""
        if self.aux_features is None:
            self.aux_features = torch.zeros(self.nenv, AUX_FEATURE_DIM, dtype=torch.float64,
                                            device=self.device)

    def _check(self, t, shape, dtypes, label):
        """Validate the raw-pointer ABI before a launch can read memory (obs_reward.py:391-401)."""
        if not torch.is_tensor(t) or t.dtype not in dtypes:
            raise TypeError(f"{label} kernel requires dtype {dtypes}; no implicit pointer cast")
        if tuple(t.shape) != tuple(shape):
            raise ValueError(f"{label} shape {tuple(t.shape)} != {tuple(shape)}")
        if t.device != self.hp.device:
            raise ValueError(f"{label} must be on the reconstructor's CUDA device")
        return t.contiguous()

    def _mask(self, mask):
        if mask is None:
            return None
        return self._check(mask, (self.nenv,), (torch.bool, torch.uint8), "environment mask")

    def _recon_tensors(self):
        """The reconstructor buffers an F16Recon points at (for the launch-stream record)."""
        return (self.hp, self.fuel, self.t_sec, self._att_soa, self.prev_valid, self._pqr_soa,
                self.last_dmg_dealt, self.last_dmg_taken, self.hp_loss, self._hist_soa,
                self.prev_x, self.prev_x_valid, self.prev_alt_log, self._vel_soa, self._acc_soa,
                self.aux_features, self.obs_buf, self.reward_buf, self.term_buf, self.trunc_buf)

    # ---- kernels (obs_reward.py:410-469) ----
    def kernel_advance(self, states, actions, cfg=None, min_alt=304.8, max_time=200.0,
                       reward_mode=0, alt_hunt_coef=5.0):
        """Push actions, advance HP/fuel/rates/time, terminate, reward (after sim.step).
        Returns (reward (nac,) f64, term (nenv,) u8, trunc (nenv,) u8) buffers."""
        cfg = MY_REWARD_CONFIG if cfg is None else cfg
        mode = validate_reward_mode(reward_mode, alt_hunt_coef)
        st, ld = soa_states(states, self.nac)
        ac = self._check(actions, (self.nac, 4), (torch.float64,), "actions")
        c = reward_cfg_struct(cfg, min_alt, max_time, mode, alt_hunt_coef)
        rec = self._recon()
        stream, h = _lib.launch_stream(self.device)
        rc = self._lib.f16_obr_advance(_lib.ptr(st), ld, _lib.ptr(ac), _lib.ctypes.byref(rec),
                                       _lib.ctypes.byref(c), _lib.ptr(self.reward_buf),
                                       _lib.ptr(self.term_buf), _lib.ptr(self.trunc_buf), h)
        _lib.record(stream, (st, ac))
        _lib.record_owned(self, stream, self._recon_tensors())
        _lib.check(rc, "f16_obr_advance")
        return self.reward_buf, self.term_buf, self.trunc_buf

    def kernel_init_reward_state(self, states, env_mask=None):
        """Re-anchor geometry advantage and log altitude from the current states."""
        st, ld = soa_states(states, self.nac)
        m = self._mask(env_mask)
        rec = self._recon()
        stream, h = _lib.launch_stream(self.device)
        rc = self._lib.f16_obr_init_reward(_lib.ptr(st), ld, _lib.ptr(m), _lib.ctypes.byref(rec),
                                           h)
        _lib.record(stream, (st, m))
        _lib.record_owned(self, stream, self._recon_tensors())
        _lib.check(rc, "f16_obr_init_reward")

    def kernel_build_obs(self, states, env_mask=None):
        """states + reconstructor -> obs_buf (nac, 184) float32 (masked rows only)."""
        return self._build(states, env_mask, OBS_SIZE, self.obs_buf)

    def _build(self, states, env_mask, dim, out):
        st, ld = soa_states(states, self.nac)
        m = self._mask(env_mask)
        rec = self._recon()
        stream, h = _lib.launch_stream(self.device)
        rc = self._lib.f16_obr_build_obs(_lib.ptr(st), ld, _lib.ptr(m), _lib.ctypes.byref(rec),
                                         dim, _lib.ptr(out), h)
        _lib.record(stream, (st, m, out))
        _lib.record_owned(self, stream, self._recon_tensors())
        _lib.check(rc, "f16_obr_build_obs")
        return out

    # ---- 214-D variant (obs_reward.py:471-496, external_observation.cu) ----
    def enable_external_observations(self):
        if self._acc_soa is not None:
            return
        dev, dt = self.device, self.dtype
        self._vel_soa = torch.zeros(3, self.nac, device=dev, dtype=dt)
        self._acc_soa = torch.zeros(3, self.nac, device=dev, dtype=dt)
        self.external_previous_velocity = self._vel_soa.t()
        self.external_accel = self._acc_soa.t()
        self.external_obs = torch.zeros(self.nac, OBS_SIZE_EXT, device=dev, dtype=torch.float32)
        self._AC_KEYS = self._AC_KEYS + ("external_previous_velocity", "external_accel")

    def build_external_obs(self, states):
        """(nac, 214) float32: the 184-D layout with own/partner NED acceleration in 5 frames
        spliced in before the action history."""
        self.enable_external_observations()
        return self._build(states, None, OBS_SIZE_EXT, self.external_obs)

    # ---- resets (obs_reward.py:498-534) ----
    def reset_all(self):
        self.hp.fill_(1.0); self.fuel.fill_(1.0); self.t_sec.zero_()
        self._att_soa.zero_(); self.prev_valid.zero_(); self._pqr_soa.zero_()
        self.last_dmg_dealt.zero_(); self.last_dmg_taken.zero_(); self.hp_loss.zero_()
        self._hist_soa.zero_(); self.prev_x.zero_(); self.prev_x_valid.zero_()
        self.prev_alt_log.zero_()
        if self._acc_soa is not None:
            self._acc_soa.zero_(); self._vel_soa.zero_()

    def reset_envs(self, env_mask):
        """In-place masked reset of the engagements selected by env_mask (nenv,) bool; no host
        synchronisation, buffer addresses unchanged."""
        ac = env_mask.repeat_interleave(2)
        ac1 = ac.unsqueeze(1)
        if self._acc_soa is not None:
            self.external_accel.masked_fill_(ac1, 0.0)
            self.external_previous_velocity.masked_fill_(ac1, 0.0)
        self.hp.masked_fill_(ac, 1.0)
        self.fuel.masked_fill_(ac, 1.0)
        self.t_sec.masked_fill_(env_mask, 0.0)
        self.prev_att.masked_fill_(ac1, 0.0)
        self.prev_valid.masked_fill_(ac, False)
        self.pqr.masked_fill_(ac1, 0.0)
        self.last_dmg_dealt.masked_fill_(ac, 0.0)
        self.last_dmg_taken.masked_fill_(ac, 0.0)
        self.hp_loss.masked_fill_(ac, 0.0)
        self.act_hist.masked_fill_(ac.view(-1, 1, 1), 0.0)
        self.prev_x.masked_fill_(ac, 0.0)
        self.prev_x_valid.masked_fill_(ac, False)
        self.prev_alt_log.masked_fill_(ac, 0.0)

    # ---- snapshot / capture / restore (obs_reward.py:536-556) ----
    def clone_state(self):
        buf = {k: getattr(self, k).clone() for k in self._AC_KEYS + self._ENV_KEYS}
        if self.aux_features is not None:
            buf["aux_features"] = self.aux_features.clone()
        return buf

    def capture_into(self, buf, env_mask):
        ac = env_mask.repeat_interleave(2)
        for k in self._AC_KEYS:
            buf[k][ac] = getattr(self, k)[ac]
        for k in self._ENV_KEYS:
            buf[k][env_mask] = getattr(self, k)[env_mask]
        if self.aux_features is not None:
            buf["aux_features"][env_mask] = self.aux_features[env_mask]

    def capture_where(self, buf, env_mask):
        """capture_into without host synchronisation: masked device copies (torch.where)."""
        ac = env_mask.repeat_interleave(2)
        keys = [(k, ac) for k in self._AC_KEYS] + [(k, env_mask) for k in self._ENV_KEYS]
        if self.aux_features is not None:
            keys.append(("aux_features", env_mask))
        for k, mask in keys:
            cur, dst = getattr(self, k), buf[k]
            torch.where(mask.view(-1, *([1] * (cur.dim() - 1))), cur, dst, out=dst)

    def restore(self, buf):
        for k in self._AC_KEYS + self._ENV_KEYS:
            getattr(self, k).copy_(buf[k])
        if self.aux_features is not None:
            self.aux_features.copy_(buf["aux_features"])

    def push_actions(self, actions_nac4):
        """Roll the action history by one decision, newest first (obs_reward.py:559-563)."""
        a = self._check(actions_nac4.to(self.dtype), (self.nac, 4), (torch.float64,), "actions")
        self._hist_soa[4:].copy_(self._hist_soa[:-4].clone())
        self._hist_soa[:4].copy_(a.t())
