"""GpuDogfight: batched F-16 flight dynamics on one MI355X.

Mirror of the reference's ``cuda_fdm/gpu_env.py:25-112`` (same constructor, attributes and
methods).  Differences in mechanism, not in contract:
  * the state lives structure-of-arrays in a (101, nac) float64 buffer; ``states`` is its
    (nac, 101) transposed view, so row indexing, ``copy_`` and ``torch.where`` work as before
    while the kernel reads and writes coalesced columns;
  * the kernel is precompiled gfx950 code in libf16hip.so, launched through the C ABI on the
    caller's current stream (no JIT, no register-cap option);
  * ``reset_ic`` seeds on the device (f16_seed_batch) instead of in host Python;
  * precision="fp32" runs f16_fdm_step_batch_f32, the same model generated in single precision
    at build time (as the reference generates its fp32 kernel from the fp64 source); seeds are
    computed in fp64 and rounded, as the reference's load_seed does.
"""
import math

import numpy as np
import torch

from . import _lib

STATE_N = 101
OBS_N = 17
# output columns (cuda_fdm/gpu_env.py:19-22)
OBS = dict(eci_pos=slice(0, 3), eci_vel=slice(3, 6), euler=slice(6, 9),
           vUVW=slice(9, 12), alpha=12, beta=13, mach=14, Vt=15, alt_asl=16)

IC_KEYS = ("lat_deg", "lon_deg", "alt_ft", "vt_fps", "phi_deg", "theta_deg", "psi_deg",
           "alpha_deg", "beta_deg", "fuel_lbs")


def ic_rows(ic_list):
    """IC dicts (cuda_fdm/ic.py:117 build_seed_vector kwargs) -> (n, 10) float64 rows."""
    rows = []
    for ic in ic_list:
        if ic.get("lat_type", "geodetic") != "geodetic":
            raise ValueError("only geodetic IC latitude is supported")
        rows.append([float(ic.get(k, 0.0 if k != "fuel_lbs" else 6000.0)) for k in IC_KEYS])
    return np.asarray(rows, dtype=np.float64).reshape(-1, len(IC_KEYS))


class GpuDogfight:
    """nenv engagements x planes_per_env aircraft; a = ppe*e + plane."""

    def __init__(self, nenv, substeps=1, planes_per_env=2, block=128, precision="fp64",
                 max_registers="auto", fcs_rate=120, device="cuda"):
        if precision not in ("fp64", "fp32"):
            raise ValueError("precision must be 'fp64' or 'fp32'")
        if not torch.cuda.is_available():
            raise RuntimeError("GpuDogfight needs a HIP device")
        if fcs_rate not in (120, 60):
            raise ValueError("fcs_rate must be 120 (root lineage) or 60 (184-D lineage)")
        self.device = torch.device(device)
        self.nenv = int(nenv)
        self.ppe = int(planes_per_env)
        self.nac = self.nenv * self.ppe
        self.substeps = int(substeps)
        self.block = block                  # accepted for compatibility; the kernel fixes 256
        self.precision = precision
        self.max_registers = max_registers  # accepted for compatibility (no JIT register cap)
        self.fcs_rate = int(fcs_rate)
        self.dtype = torch.float32 if precision == "fp32" else torch.float64
        self._lib = _lib.lib()
        self._state_soa = torch.zeros(STATE_N, self.nac, dtype=self.dtype, device=self.device)
        self._obs_soa = torch.zeros(OBS_N, self.nac, dtype=self.dtype, device=self.device)
        self.states = self._state_soa.t()      # (nac, 101) view of the SoA buffer
        self.obs = self._obs_soa.t()           # (nac, 17) view
        self.actions = torch.zeros(self.nac, 4, dtype=self.dtype, device=self.device)
        # When set to a list, every launch appends a (start, end) pair of timing events
        # recorded on the launch stream immediately around the kernel (bench/profiling).
        self.kernel_events = None

    @property
    def kern(self):
        """Footprint {regs, lds, scratch, max_threads} of the kernel `step` launches (reference
        attribute: the kernel object, cuda_fdm/gpu_env.py:49-55)."""
        return self.kernel_info(onelane=False)

    def kernel_info(self, onelane=False):
        """Footprint of the four-wave kernel `step` launches (default) or of the one-lane kernel;
        with precision="fp32", of the single-precision four-wave kernel (`onelane` ignored)."""
        out = (_lib.ctypes.c_int * 4)()
        if self.precision == "fp32":
            fn = self._lib.f16_fdm_kernel_info_f32
        else:
            fn = self._lib.f16_fdm_kernel_info_onelane if onelane else self._lib.f16_fdm_kernel_info
        _lib.check(fn(self.fcs_rate, out), "f16_fdm_kernel_info")
        return dict(regs=out[0], lds=out[1], scratch=out[2], max_threads=out[3])

    def _buffers(self):
        """The device buffers every launch of this simulator touches."""
        return (self._state_soa, self.actions, self._obs_soa)

    # ---- reset (cuda_fdm/gpu_env.py:64-92) ----
    def load_seed(self, seed):
        """seed: (101,), (ppe,101), (nac,101) or (nenv,ppe,101); numpy or torch."""
        t = torch.as_tensor(seed, dtype=torch.float64)
        if t.ndim == 1:
            t = t.unsqueeze(0).expand(self.nac, -1)
        elif t.ndim == 3:
            t = t.reshape(self.nac, STATE_N)
        elif t.shape[0] != self.nac:
            t = t.unsqueeze(0).expand(self.nenv, -1, -1).reshape(self.nac, STATE_N)
        self.states.copy_(t.to(self.device))

    def reset_ic(self, ic_list):
        """nac IC dicts (or (nenv,) lists of ppe dicts) -> device-side seeding."""
        flat = []
        for item in ic_list:
            if isinstance(item, dict):
                flat.append(item)
            else:
                flat.extend(item)
        if len(flat) != self.nac:
            raise ValueError(f"{len(flat)} ICs != nac {self.nac}")
        self.seed_rows(torch.as_tensor(ic_rows(flat), device=self.device))

    def seed_rows(self, ic, rows=None):
        """Seed aircraft from an (n, 10) float64 device tensor of IC rows (IC_KEYS order).
        rows: optional (n,) int64 device tensor of target aircraft indices."""
        ic = ic.to(device=self.device, dtype=torch.float64).contiguous()
        if ic.ndim != 2 or ic.shape[1] != len(IC_KEYS):
            raise ValueError("ic must be (n, 10)")
        n = ic.shape[0]
        if rows is not None:
            rows = rows.to(device=self.device, dtype=torch.int64).contiguous()
            if rows.shape != (n,):
                raise ValueError("rows must be (n,)")
            if n and not bool(((rows >= 0) & (rows < self.nac)).all()):   # one host sync
                raise IndexError(f"rows must lie in [0, {self.nac})")
        elif n != self.nac:
            raise ValueError("without rows, n must equal nac")
        # fp32: seed an fp64 copy of the state (rows not seeded keep their values exactly) and
        # round it back
        soa = self._state_soa if self.precision == "fp64" else self._state_soa.double()
        stream, h = _lib.launch_stream(self.device)
        rc = self._lib.f16_seed_batch(_lib.ptr(ic), n, self.fcs_rate, _lib.ptr(soa),
                                      self.nac, _lib.ptr(rows), h)
        _lib.record(stream, (ic, rows, soa))
        _lib.record_owned(self, stream, self._buffers())
        _lib.check(rc, "f16_seed_batch")
        if soa is not self._state_soa:
            self._state_soa.copy_(soa)

    # ---- step (cuda_fdm/gpu_env.py:95-106) ----
    def action_source(self, actions):
        """The (nac, 4) device tensor (self.dtype) a step launch reads its controls from.  The
        reference copies the actions into self.actions before its launch; a separate contiguous
        device tensor is returned as is (the launch reads it and writes the copy itself),
        anything else is copied into self.actions here and self.actions is returned."""
        a = torch.as_tensor(actions, dtype=self.dtype, device=self.device).reshape(self.nac, 4)
        if self.precision == "fp64" and (a.is_contiguous() and a.untyped_storage().data_ptr()
                != self.actions.untyped_storage().data_ptr()):
            return a
        if a.data_ptr() != self.actions.data_ptr():
            self.actions.copy_(a)
        return self.actions

    def step(self, actions, substeps=None, want_obs=True, finite_out=None):
        """actions (nac,4) or (nenv,ppe,4) [aileron, elevator, rudder, throttle] -> obs view
        (nenv, ppe, 17).  want_obs=False skips the 17-value output write.  finite_out: an
        optional (nac,) uint8/bool device tensor that receives, per aircraft, whether all 101
        state values after the step are finite (f16_fdm_step_batch_finite; substeps >= 1; fp64
        only)."""
        ss = self.substeps if substeps is None else int(substeps)
        if finite_out is not None and self.precision != "fp64":
            raise ValueError("finite_out is available with precision='fp64' only")
        if finite_out is not None:
            if (finite_out.dtype not in (torch.uint8, torch.bool) or finite_out.numel() != self.nac
                    or not finite_out.is_contiguous() or finite_out.device != self.states.device):
                raise ValueError("finite_out must be a contiguous (nac,) uint8/bool device tensor")
            if ss < 1:
                raise ValueError("finite_out needs substeps >= 1")
        a = self.action_source(actions)
        keep = a.data_ptr() != self.actions.data_ptr()
        ev = self.kernel_events
        if ev is not None:
            e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            e0.record()
        obs_p = _lib.ptr(self._obs_soa) if want_obs else None
        stream, h = _lib.launch_stream(self.device)
        if self.precision == "fp32":
            rc = self._lib.f16_fdm_step_batch_f32(
                _lib.ptr(self._state_soa), self.nac, _lib.ptr(self.actions), self.nac, ss,
                self.fcs_rate, obs_p, self.nac, h)
        elif keep:
            rc = self._lib.f16_fdm_step_batch_keep(
                _lib.ptr(self._state_soa), self.nac, _lib.ptr(a), _lib.ptr(self.actions),
                self.nac, ss, self.fcs_rate, obs_p, self.nac,
                _lib.ptr(finite_out) if finite_out is not None else None, h)
        elif finite_out is None:
            rc = self._lib.f16_fdm_step_batch(
                _lib.ptr(self._state_soa), self.nac, _lib.ptr(self.actions), self.nac, ss,
                self.fcs_rate, obs_p, self.nac, h)
        else:
            rc = self._lib.f16_fdm_step_batch_finite(
                _lib.ptr(self._state_soa), self.nac, _lib.ptr(self.actions), self.nac, ss,
                self.fcs_rate, obs_p, self.nac, _lib.ptr(finite_out), h)
        if ev is not None:
            e1.record()
            ev.append((e0, e1))
        _lib.record_owned(self, stream, self._buffers())
        _lib.record(stream, (a if keep else None, finite_out))
        _lib.check(rc, "f16_fdm_step_batch")
        return self.obs.view(self.nenv, self.ppe, OBS_N)

    def get_state(self):
        return self.states.view(self.nenv, self.ppe, STATE_N)

    def get_obs(self):
        return self.obs.view(self.nenv, self.ppe, OBS_N)
