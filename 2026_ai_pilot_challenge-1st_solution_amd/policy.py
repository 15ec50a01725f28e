"""Rollout-side policy on the GPU: the discrete actor-critic MLP, observation running
normalisation, and the fused policy step.

Mirrors the reference's pieces of this path:
  * ``MLPActorCritic`` -- claude_code/model.py:162-241 MLPDiscreteActorCritic (separate actor and
    critic MLPs, tanh, per-channel 21-bin categorical over 4 channels) with the same parameter
    names (``actor_logits.<i>.weight`` / ``critic.<i>.weight``);
  * ``RunningNorm`` -- research/competition_36500/runtime/cuda_fdm/ppo_gpu.py:183-227;
  * ``make_action_grid`` / ``action_to_env`` -- ppo_gpu.py:178-181, 361-370.
The forward pass runs in one gfx950 kernel (f16_policy_step: bf16 weights and activations on
MFMA with fp32 accumulation, fp32 normalisation, softmax, draw and log-probability); the torch
parameters are the fp32 master copy that ``pack`` rounds to bf16 for the kernel.
"""
import ctypes

import numpy as np
import torch

from . import _lib

ACTION_BINS = 21
ACT_DIM = 4
HIDDEN = 256
NF = 1377
LOGITS_PAD = 96


def make_action_grid(num_bins=ACTION_BINS, device="cpu"):
    """linspace(-1, 1, num_bins) in float32 (ppo_gpu.py:178-181)."""
    return torch.linspace(-1.0, 1.0, int(num_bins), device=device)


def action_to_env(idx, num_bins=ACTION_BINS, grid=None):
    """(N, 4) bins -> (N, 4) float32 controls; throttle 0.5 z + 0.5 (ppo_gpu.py:361-370)."""
    if grid is None:
        grid = make_action_grid(num_bins, device=idx.device)
    ctrl = grid[idx.long()].clone()
    ctrl[:, 3] = 0.5 * ctrl[:, 3] + 0.5
    return ctrl


def kpad(obs_dim):
    return (int(obs_dim) + 31) // 32 * 32


def frag_major(w):
    """(N, K) matrix -> the kernels' fragment-major order (N % 32 == 0, K % 16 == 0): one 512-element
    block per (32-row tile, 16-column slice), element (n, k) of a block at lane
    32 ((k % 16) // 8) + n % 32, position k % 8 -- the bf16x8 operand lane l of a
    32x32x16 MFMA reads, so each wavefront's load of one block is 1 KB contiguous."""
    N, K = w.shape
    return w.reshape(N // 32, 32, K // 16, 2, 8).permute(0, 2, 3, 1, 4).reshape(-1)


def frag_unmajor(v, N, K):
    """Inverse of frag_major: flat blocks -> (N, K)."""
    return v.reshape(N // 32, K // 16, 2, 32, 8).permute(0, 3, 1, 2, 4).reshape(N, K)


def _mlp(in_dim, hidden, out_dim):
    layers, last = [], in_dim
    for h in hidden:
        layers += [torch.nn.Linear(last, h), torch.nn.Tanh()]
        last = h
    layers.append(torch.nn.Linear(last, out_dim))
    return torch.nn.Sequential(*layers)


class MLPActorCritic(torch.nn.Module):
    """Separate actor (obs -> 256 -> 256 -> 4 x 21 logits) and critic (obs -> 256 -> 256 -> 1)."""

    def __init__(self, obs_dim, act_dim=ACT_DIM, num_bins=ACTION_BINS, hidden=(HIDDEN, HIDDEN),
                 activation="tanh", init="orthogonal", init_std=0.02, generator=None):
        super().__init__()
        if tuple(hidden) != (HIDDEN, HIDDEN) or activation != "tanh":
            raise ValueError("the fused kernel implements hidden=(256, 256) with tanh")
        if act_dim != ACT_DIM or num_bins != ACTION_BINS:
            raise ValueError("the fused kernel implements 4 channels x 21 bins")
        if obs_dim not in (184, 214):
            raise ValueError("obs_dim must be 184 or 214")
        self.obs_dim, self.act_dim, self.num_bins = int(obs_dim), act_dim, num_bins
        self.hidden = list(hidden)
        self.activation = activation
        self.actor_logits = _mlp(obs_dim, hidden, act_dim * num_bins)
        self.critic = _mlp(obs_dim, hidden, 1)
        with torch.no_grad():
            for mod in self.modules():
                if isinstance(mod, torch.nn.Linear):
                    if init == "orthogonal":       # model.py:86-90 _init_weights
                        torch.nn.init.orthogonal_(mod.weight, gain=float(np.sqrt(2)),
                                                  generator=generator)
                    elif init == "normal":         # BASELINE C4/C5: N(0, 0.02)
                        mod.weight.normal_(0.0, float(init_std), generator=generator)
                    else:
                        raise ValueError(f"unknown init {init!r}")
                    mod.bias.zero_()
        self._packed = None

    def forward_reference(self, obs):
        """fp32 torch forward (logits (N,4,21), value (N,)) -- for checks, not the rollout."""
        return (self.actor_logits(obs).view(-1, self.act_dim, self.num_bins),
                self.critic(obs).squeeze(-1))

    @torch.no_grad()
    def pack(self, device=None):
        """Round the parameters to the kernel's blobs: (bf16 weights, f32 biases/heads)."""
        device = device or next(self.parameters()).device
        kp = kpad(self.obs_dim)
        a, c = self.actor_logits, self.critic
        w1 = torch.zeros(2 * HIDDEN, kp)
        w1[:HIDDEN, :self.obs_dim] = a[0].weight.float().cpu()
        w1[HIDDEN:, :self.obs_dim] = c[0].weight.float().cpu()
        w3 = torch.zeros(LOGITS_PAD, HIDDEN)
        w3[:self.act_dim * self.num_bins] = a[4].weight.float().cpu()
        wbf = torch.cat([frag_major(w1), frag_major(a[2].weight.float().cpu()),
                         frag_major(c[2].weight.float().cpu()), frag_major(w3)]).to(torch.bfloat16)
        b3 = torch.zeros(LOGITS_PAD)
        b3[:self.act_dim * self.num_bins] = a[4].bias.float().cpu()
        wf = torch.cat([a[0].bias.float().cpu(), c[0].bias.float().cpu(), a[2].bias.float().cpu(),
                        c[2].bias.float().cpu(), b3, c[4].weight.float().cpu().flatten(),
                        c[4].bias.float().cpu()])
        assert wf.numel() == NF
        old = self._packed
        if old is not None and old[0].device == torch.device(device) and old[0].shape == wbf.shape:
            # refresh in place: launches recorded in a HIP graph keep pointing at these blobs
            old[0].copy_(wbf)
            old[1].copy_(wf)
        else:
            self._packed = (wbf.to(device).contiguous(), wf.to(device).contiguous())
        return self._packed

    def packed(self):
        return self._packed if self._packed is not None else self.pack()


class RunningNorm:
    """Observation running mean/variance with a clipped normalisation (ppo_gpu.py:183-227).
    ``update`` runs on the device (f16_norm_update); ``normalize`` is fused into the policy
    step and also available standalone."""

    def __init__(self, dim, device, clip=10.0, eps=1e-8):
        self.dim = int(dim)
        self.device = torch.device(device)
        self.mean = torch.zeros(dim, device=device, dtype=torch.float32)
        self.var = torch.ones(dim, device=device, dtype=torch.float32)
        self.count = torch.zeros((), device=device, dtype=torch.float32) + 1e-4
        self.clip = float(clip)
        self.eps = float(eps)
        self._work = None

    def _workspace(self, n):
        need = _lib.lib().f16_norm_workspace_bytes(n, self.dim)
        if self._work is None or self._work.numel() < need:
            self._work = torch.empty(max(need, 8), dtype=torch.uint8, device=self.device)
        return self._work

    def fused_partials(self, io, n):
        """Point an F16EnvStepIO's norm fields at this normaliser's workspace, so the
        post-physics step writes the partial sums of its n new observation rows; `merge(n)`
        then completes update() of those rows."""
        w = self._workspace(n)
        nb = (n + 127) // 128
        io.norm_partial = w.data_ptr()
        io.norm_count = self.count.data_ptr()
        io.norm_count_snap = w.data_ptr() + nb * 2 * self.dim * 8   # the workspace's last slot

    @torch.no_grad()
    def merge(self, n):
        """The second half of update(): fold the partial sums already in the workspace (written
        by a post-physics step with fused_partials) into mean/var."""
        L = _lib.lib()
        stream, h = _lib.launch_stream(self.device)
        rc = L.f16_norm_merge(n, self.dim, _lib.ptr(self.mean), _lib.ptr(self.var),
                              _lib.ptr(self._workspace(n)), h)
        _lib.record_owned(self, stream, (self.mean, self.var, self.count, self._work))
        _lib.check(rc, "f16_norm_merge")

    @torch.no_grad()
    def update(self, x, rows=None):
        """x: (N, dim) float32 CUDA rows (or the rows listed in `rows`, int32)."""
        if x.dtype != torch.float32 or x.dim() != 2 or x.shape[1] != self.dim:
            raise ValueError("RunningNorm.update needs (N, dim) float32")
        if x.stride(1) != 1:
            x = x.contiguous()
        n = x.shape[0] if rows is None else rows.numel()
        L = _lib.lib()
        self._workspace(n)
        stream, h = _lib.launch_stream(self.device)
        rc = L.f16_norm_update(_lib.ptr(x), x.stride(0), _lib.ptr(rows), n, self.dim,
                               _lib.ptr(self.mean), _lib.ptr(self.var), _lib.ptr(self.count),
                               _lib.ptr(self._work), h)
        _lib.record_owned(self, stream, (self.mean, self.var, self.count, self._work))
        _lib.record(stream, (x, rows))
        _lib.check(rc, "f16_norm_update")

    @torch.no_grad()
    def normalize(self, x):
        n = (x - self.mean) / torch.sqrt(self.var + self.eps)
        return n.clamp_(-self.clip, self.clip)

    def state_dict(self):
        return {"mean": self.mean.clone(), "var": self.var.clone(), "count": self.count.clone()}

    def load_state_dict(self, sd):
        self.mean.copy_(sd["mean"]); self.var.copy_(sd["var"]); self.count.copy_(sd["count"])

    def clone(self):
        c = RunningNorm(self.dim, self.device, self.clip, self.eps)
        c.load_state_dict(self.state_dict())
        return c


class PolicyStep:
    """One fused launch: [normalise] -> actor/critic -> draw -> log-prob -> controls.

    groups: list of (MLPActorCritic, row_begin, row_end) over logical rows; rows: optional int32
    logical -> physical row map (None = identity)."""

    def __init__(self, obs_dim, device="cuda", seed=0):
        self.obs_dim = int(obs_dim)
        self.device = torch.device(device)
        self.seed = int(seed)
        self.grid = make_action_grid(ACTION_BINS, device=self.device).contiguous()
        self._lib = _lib.lib()

    def __call__(self, obs, groups, *, norm=None, rows=None, step=0, salt=0, deterministic=False,
                 nobs_out=None, act_idx=None, logp=None, value=None, env_actions=None,
                 logits_out=None, group_offsets=None, max_group_rows=None, nphys=None,
                 step_base=None, packed=True):
        """groups: (net, row_begin, row_end) or (net, row_begin, row_end, norm) -- a per-network
        RunningNorm overrides `norm` for that network.  group_offsets: device int32 (ngroups+1)
        row boundaries computed on the device (f16_group_rows); then row_begin/row_end are
        ignored, max_group_rows bounds any group's size and nphys bounds the physical rows;
        packed=True launches about len(rows) / 64 + ngroups workgroups, each taking the next
        64-row tile of the groups in order, instead of ngroups x max_group_rows / 64 (same
        results).
        step_base: optional device int32 scalar added to `step` in the kernel (rollouts recorded
        in a HIP graph advance it on the device between replays).
        nphys given with a row map skips the (host-synchronising) row-map validation: the caller
        guarantees 0 <= rows < nphys."""
        if obs.dtype != torch.float32 or obs.dim() != 2 or obs.shape[1] != self.obs_dim:
            raise ValueError(f"obs must be (N, {self.obs_dim}) float32")
        if obs.stride(1) != 1:
            raise ValueError("obs rows must be contiguous")
        if len(groups) > 16:
            raise ValueError("at most 16 networks per launch")
        groups = [tuple(g) + (None,) * (4 - len(g)) for g in groups]
        if group_offsets is not None:
            # device-side ranges: the caller bounds them (rows, outputs sized for every row)
            if rows is None or max_group_rows is None or nphys is None:
                raise ValueError("group_offsets needs rows, max_group_rows and nphys")
            if group_offsets.dtype != torch.int32 or group_offsets.numel() < len(groups) + 1:
                raise ValueError("group_offsets must be int32 with ngroups + 1 entries")
            nlog = rows.numel()
        else:
            nlog = max([int(g[2]) for g in groups] + [0])
            if any(int(g[1]) < 0 or int(g[2]) < int(g[1]) for g in groups):
                raise ValueError("group row ranges must satisfy 0 <= begin <= end")
        if rows is not None:
            if rows.dtype != torch.int32 or rows.dim() != 1 or not rows.is_contiguous():
                raise ValueError("rows must be a contiguous int32 vector")
            if rows.numel() < nlog:
                raise ValueError("rows shorter than the groups' logical range")
            if group_offsets is None and nphys is None:     # validate (host synchronisation)
                nphys = int(rows[:nlog].max().item()) + 1 if nlog else 0
                if nlog and int(rows[:nlog].min().item()) < 0:
                    raise ValueError("negative physical row")
        else:
            nphys = nlog
        if obs.shape[0] < nphys:
            raise ValueError("obs has fewer rows than the rows addressed")
        for t, rows_needed, w in ((nobs_out, nlog, self.obs_dim), (act_idx, nlog, 4),
                                  (logp, nlog, 1), (value, nlog, 1), (env_actions, nphys, 4),
                                  (logits_out, nlog, 84)):
            if t is None:
                continue
            if not t.is_contiguous() and t is not nobs_out:
                raise ValueError("output buffers must be contiguous")
            if t.shape[0] < rows_needed or (t.dim() > 1 and t.shape[1] < w):
                raise ValueError("output buffer too small for the rows addressed")
        dtypes = ((act_idx, torch.int64), (logp, torch.float32), (value, torch.float32),
                  (env_actions, torch.float64), (logits_out, torch.float32),
                  (nobs_out, torch.float32))
        if any(t is not None and t.dtype != d for t, d in dtypes):
            raise ValueError("output buffer dtype mismatch")
        a = _lib.F16PolicyArgs()
        a.obs, a.obs_ld, a.obs_dim = obs.data_ptr(), obs.stride(0), self.obs_dim
        if norm is not None:
            a.mean, a.var = norm.mean.data_ptr(), norm.var.data_ptr()
            a.clip, a.eps = norm.clip, norm.eps
        else:
            per = [g[3] for g in groups if len(g) > 3 and g[3] is not None]
            a.clip, a.eps = (per[0].clip, per[0].eps) if per else (10.0, 1e-8)
        a.rows = rows.data_ptr() if rows is not None else None
        a.ngroups = len(groups)
        keep = []
        for i, (net, b, e, gnorm) in enumerate(groups):
            if net.obs_dim != self.obs_dim:
                raise ValueError("network obs_dim differs from the step's")
            wbf, wf = net.packed()
            keep.append((wbf, wf))
            a.group[i].wbf, a.group[i].wf = wbf.data_ptr(), wf.data_ptr()
            if gnorm is not None:
                a.group[i].mean, a.group[i].var = gnorm.mean.data_ptr(), gnorm.var.data_ptr()
            a.group[i].row_begin, a.group[i].row_end = int(b or 0), int(e or 0)
        if group_offsets is not None:
            a.group_offsets, a.max_group_rows = group_offsets.data_ptr(), int(max_group_rows)
            a.total_group_rows = nlog if packed else 0
        a.seed, a.step, a.salt = self.seed, int(step) & 0xffffffff, int(salt) & 0xffffffff
        a.deterministic = int(bool(deterministic))
        a.grid = self.grid.data_ptr()
        if nobs_out is not None:
            a.nobs_out, a.nobs_ld = nobs_out.data_ptr(), nobs_out.stride(0)
        p = lambda t: t.data_ptr() if t is not None else None
        a.act_idx, a.logp, a.value = p(act_idx), p(logp), p(value)
        if step_base is not None:
            if step_base.dtype != torch.int32 or not step_base.is_cuda:
                raise ValueError("step_base must be a device int32 scalar")
            a.step_base = step_base.data_ptr()
        a.env_actions, a.logits_out = p(env_actions), p(logits_out)
        stream, h = _lib.launch_stream(self.device)
        rc = self._lib.f16_policy_step(ctypes.byref(a), h)
        _lib.record(stream, (obs, rows, group_offsets, nobs_out, act_idx, logp, value,
                             env_actions, logits_out, step_base, self.grid)
                    + (() if norm is None else (norm.mean, norm.var))
                    + tuple(t for wb in keep for t in wb)
                    + tuple(t for g in groups if g[3] is not None for t in (g[3].mean, g[3].var)))
        _lib.check(rc, "f16_policy_step")
        return keep
