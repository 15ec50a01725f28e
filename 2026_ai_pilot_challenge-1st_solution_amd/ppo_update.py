"""The PPO update on the GPU: PPOGPUTrainer.update (research/competition_36500/runtime/cuda_fdm/
ppo_gpu.py:2019-2145) for the discrete actor-critic MLP, in the reference's configuration
(PPOConfig, ppo_gpu.py:955-978: clip 0.2, 4 epochs x 8 minibatches, Adam lr 3e-4 eps 1e-5 per
network, max grad norm 0.5, target KL 0.03, per-minibatch advantage normalisation).

Per minibatch two C-ABI calls:
  * f16_ppo_grad: gathered rows -> forward of both networks -> log-softmax, entropy, ratio,
    clipped surrogate and value error -> every parameter gradient (bf16 MFMA, fp32 accumulation,
    deterministic reductions) and the minibatch statistics;
  * f16_ppo_adam_step: clip_grad_norm_ of each network, torch.optim.Adam's update of the fp32
    master parameters, and the repack of the bf16 blobs the rollout kernel reads -- the next
    rollout (eager or a replayed HIP graph) sees the new weights with no host work.
Each epoch's shuffle is f16_permutation (a keyed Feistel permutation drawn on the device) in
place of torch.randperm's sort of random keys, and the finite check before the update reads each
buffer once (f16_all_finite), on a second stream beside the first minibatch's gradient and tested
before its optimizer step.  One host synchronisation per epoch (the KL early-stop test, as the
reference's ``float(last_kl)``) and one for the finite check.

The master parameters are one flat fp32 buffer (actor_parameters() then critic_parameters());
the network's torch parameters become views into it, so state_dict() keeps the reference's
names and shapes.
"""
import ctypes
import math
from dataclasses import dataclass
from typing import Optional

import torch

from . import _lib

NSTATS = 8
STAT_PL, STAT_VL, STAT_ENT, STAT_KL, STAT_CF, STAT_ADV_MEAN, STAT_ADV_STD, STAT_BAD = range(8)
WT_ELEMS = 256 * 96 + 2 * 256 * 256


@dataclass
class UpdateConfig:
    """The update's fields of PPOConfig (ppo_gpu.py:955-978), same defaults."""
    clip_coef: float = 0.2
    update_epochs: int = 4
    num_minibatches: int = 8
    lr: float = 3e-4
    critic_lr: Optional[float] = None
    ent_coef: float = 0.0
    vf_coef: float = 0.5
    max_grad_norm: float = 0.5
    target_kl: Optional[float] = 0.03
    norm_adv: bool = True


def finite_flag(floats, flags=()):
    """One device byte, 1 when every element of the float32/float64 tensors `floats` is finite
    and every element of the uint8/bool tensors `flags` is nonzero, else 0: the reference's
    torch.stack([...isfinite(x).all()...]).all() before an update (ppo_gpu.py:2000-2009) as one
    read of each buffer (f16_all_finite), no host synchronisation."""
    spans, keep = [], []
    for xs, kinds in ((floats, (torch.float32, torch.float64)), (flags, (torch.uint8, torch.bool))):
        for x in xs:
            if x.dtype not in kinds:
                raise TypeError(f"finite_flag: unsupported dtype {x.dtype}")
            if not x.is_cuda:
                raise ValueError("finite_flag: device tensors only")
            x = x.contiguous()
            keep.append(x)
            spans.append((x.data_ptr(), x.numel(), x.element_size()))
    if not keep:
        raise ValueError("finite_flag: nothing to check")
    if len(spans) > 16:
        raise ValueError("finite_flag: at most 16 tensors")
    dev = keep[0].device
    if any(x.device != dev for x in keep):
        raise ValueError("finite_flag: tensors on different devices")
    arr = (_lib.F16FiniteSpan * len(spans))(*[_lib.F16FiniteSpan(p, n, e) for p, n, e in spans])
    out = torch.empty(1, dtype=torch.uint8, device=dev)
    stream, h = _lib.launch_stream(dev)
    rc = _lib.lib().f16_all_finite(arr, len(spans), _lib.ptr(out), h)
    _lib.record(stream, keep + [out])
    _lib.check(rc, "f16_all_finite")
    return out


def param_counts(obs_dim):
    out = (ctypes.c_long * 2)()
    _lib.check(_lib.lib().f16_ppo_param_counts(int(obs_dim), out), "f16_ppo_param_counts")
    return int(out[0]), int(out[1])


def net_parameters(net):
    """The network's parameters in the flat order (model.py:179-185)."""
    a, c = net.actor_logits, net.critic
    return [a[0].weight, a[0].bias, a[2].weight, a[2].bias, a[4].weight, a[4].bias,
            c[0].weight, c[0].bias, c[2].weight, c[2].bias, c[4].weight, c[4].bias]


class PPOUpdater:
    """Owns the learner's master parameters, the Adam state and the update workspace.

    ``update(rollout, adv, ret)`` takes a collector's buffers (SelfPlayRollout or LeagueRollout:
    b_obs normalised observations, b_act bins, b_logp, b_val) and its GAE output, and returns the
    reference's result dict (pl, vl, ent, kl, cf, ev, epochs, early, actor_grad_norm,
    critic_grad_norm, optimizer_steps) with tensors where the reference keeps tensors."""

    def __init__(self, net, cfg=None, seed=0, device=None):
        self.cfg = cfg or UpdateConfig()
        dev = torch.device(device) if device is not None else next(net.parameters()).device
        if dev.type != "cuda":
            raise ValueError("the update runs on the GPU (HIP); there is no CPU path")
        self.net, self.device, self.D = net, dev, int(net.obs_dim)
        self._L = _lib.lib()
        self.na, self.nc = param_counts(self.D)
        params = net_parameters(net)
        if sum(p.numel() for p in params) != self.na + self.nc:
            raise ValueError("network shape does not match the flat layout")
        with torch.no_grad():
            flat = torch.cat([p.detach().reshape(-1).float().to(dev) for p in params])
        self.flat = flat.contiguous()
        off = 0
        for p in params:
            n = p.numel()
            p.data = self.flat[off:off + n].view(p.shape)
            off += n
        self.exp_avg = torch.zeros_like(self.flat)
        self.exp_avg_sq = torch.zeros_like(self.flat)
        self.grad = torch.zeros_like(self.flat)
        self.grad_norms = torch.zeros(2, dtype=torch.float32, device=dev)
        self.wT = torch.empty(WT_ELEMS, dtype=torch.bfloat16, device=dev)
        self.wbf, self.wf = net.pack(dev)
        self.pack()
        self.steps = 0
        self.gen = torch.Generator(device=dev)
        self.gen.manual_seed(int(seed))
        self._work = None
        self._work_rows = 0
        self._adv_work = None
        self._side = None                                  # the finite check's stream
        self.stats = torch.zeros(1, NSTATS, dtype=torch.float32, device=dev)

    # ---- blobs
    def pack(self):
        """Rewrite the rollout blobs and the transposed blob from the master parameters."""
        stream, h = _lib.launch_stream(self.device)
        rc = self._L.f16_ppo_pack(_lib.ptr(self.flat), self.D, _lib.ptr(self.wbf),
                                  _lib.ptr(self.wf), _lib.ptr(self.wT), h)
        _lib.record_owned(self, stream, self._buffers())
        _lib.check(rc, "f16_ppo_pack")

    def _buffers(self):
        """The updater's device buffers (master parameters, moments, gradients, blobs,
        workspace, statistics) for the launch-stream record."""
        return (self.flat, self.exp_avg, self.exp_avg_sq, self.grad, self.grad_norms, self.wT,
                self.wbf, self.wf, getattr(self, "_work", None), getattr(self, "stats", None))

    def _workspace(self, mb_rows):
        if self._work is None or mb_rows > self._work_rows:
            nbytes = self._L.f16_ppo_workspace_bytes(self.D, int(mb_rows))
            if nbytes < 0:
                raise ValueError("bad minibatch size")
            self._work = torch.empty(nbytes, dtype=torch.uint8, device=self.device)
            self._work_rows = int(mb_rows)
        return self._work

    # ---- one minibatch
    def minibatch_grad(self, obs, act, old_logp, adv, ret, idx, stats_row=None, adv_stats=None):
        """Loss gradients of the minibatch idx (int64 device indices into the flattened buffers)
        into self.grad; statistics into stats_row (8 floats).  adv_stats: the minibatch's
        advantage mean and std (2 device floats, from epoch_adv_stats), or None to form them."""
        cfg = self.cfg
        n = int(idx.numel())
        if stats_row is None:
            stats_row = self.stats[0]
        a = _lib.F16PPOArgs()
        a.obs, a.obs_ld, a.obs_dim = _lib.ptr(obs), obs.stride(0), self.D
        a.act, a.old_logp, a.adv, a.ret = (_lib.ptr(x) for x in (act, old_logp, adv, ret))
        a.count = obs.shape[0]
        a.idx, a.mb_rows = _lib.ptr(idx), n
        a.clip_coef, a.ent_coef, a.vf_coef = cfg.clip_coef, cfg.ent_coef, cfg.vf_coef
        a.norm_adv = 1 if cfg.norm_adv else 0
        a.wbf, a.wf, a.wT = _lib.ptr(self.wbf), _lib.ptr(self.wf), _lib.ptr(self.wT)
        a.grad, a.stats, a.work = _lib.ptr(self.grad), _lib.ptr(stats_row), \
            _lib.ptr(self._workspace(n))
        a.adv_stats = _lib.ptr(adv_stats)
        stream, h = _lib.launch_stream(self.device)
        rc = self._L.f16_ppo_grad(ctypes.byref(a), h)
        _lib.record_owned(self, stream, self._buffers())
        _lib.record(stream, (obs, act, old_logp, adv, ret, idx, stats_row, adv_stats))
        _lib.check(rc, "f16_ppo_grad")

    def epoch_adv_stats(self, adv, perm, mb_rows):
        """(nmb, 2) device floats: every minibatch's advantage mean and sample std for the
        epoch's permutation cut into mb_rows slices (f16_ppo_adv_stats: two launches per epoch
        instead of two per minibatch; the same values f16_ppo_grad forms per minibatch)."""
        total = int(perm.numel())
        nmb = (total + mb_rows - 1) // mb_rows
        nbytes = self._L.f16_ppo_adv_work_bytes(int(mb_rows), nmb)
        if nbytes < 0:
            raise ValueError("bad minibatch size")
        if self._adv_work is None or self._adv_work.numel() < nbytes:
            self._adv_work = torch.empty(nbytes, dtype=torch.uint8, device=self.device)
        out = torch.empty(nmb, 2, dtype=torch.float32, device=self.device)
        stream, h = _lib.launch_stream(self.device)
        rc = self._L.f16_ppo_adv_stats(_lib.ptr(adv), _lib.ptr(perm), total, int(adv.numel()),
                                       int(mb_rows), nmb, _lib.ptr(out),
                                       _lib.ptr(self._adv_work), h)
        _lib.record(stream, (adv, perm, out, self._adv_work))
        _lib.check(rc, "f16_ppo_adv_stats")
        return out

    def optimizer_step(self):
        """clip_grad_norm_ + Adam on both networks, then the blobs (ppo_gpu.py:2088-2105)."""
        cfg = self.cfg
        self.steps += 1
        a = _lib.F16AdamArgs()
        a.obs_dim = self.D
        a.param, a.exp_avg, a.exp_avg_sq, a.grad = (_lib.ptr(x) for x in (
            self.flat, self.exp_avg, self.exp_avg_sq, self.grad))
        a.max_grad_norm = cfg.max_grad_norm
        a.actor_lr = float(cfg.lr)
        a.critic_lr = float(cfg.lr if cfg.critic_lr is None else cfg.critic_lr)
        a.beta1, a.beta2, a.eps = 0.9, 0.999, 1e-5
        a.step = self.steps
        a.grad_norms = _lib.ptr(self.grad_norms)
        a.wbf, a.wf, a.wT = _lib.ptr(self.wbf), _lib.ptr(self.wf), _lib.ptr(self.wT)
        a.work = _lib.ptr(self._workspace(max(1, self._work_rows)))
        stream, h = _lib.launch_stream(self.device)
        rc = self._L.f16_ppo_adam_step(ctypes.byref(a), h)
        _lib.record_owned(self, stream, self._buffers())
        _lib.check(rc, "f16_ppo_adam_step")

    def permutation(self, count):
        """The epoch's shuffle, torch.randperm(count)'s role (ppo_gpu.py:2055): f16_permutation
        keyed by a 62-bit word drawn on the device from the updater's generator, so the draw
        needs no host synchronisation and a restored generator repeats it."""
        key = torch.randint(0, 2 ** 62, (1,), dtype=torch.int64, device=self.device,
                            generator=self.gen)
        perm = torch.empty(int(count), dtype=torch.int64, device=self.device)
        stream, h = _lib.launch_stream(self.device)
        rc = self._L.f16_permutation(_lib.ptr(perm), int(count), _lib.ptr(key), h)
        _lib.record(stream, (perm, key))
        _lib.check(rc, "f16_permutation")
        return perm

    # ---- the update (ppo_gpu.py:2019-2145)
    def update(self, rollout, adv, ret, perms=None):
        cfg, dev = self.cfg, self.device
        obs = rollout.b_obs.flatten(0, 1)
        act = rollout.b_act.flatten(0, 1)
        old_logp = rollout.b_logp.flatten()
        b_val = rollout.b_val.reshape(-1)
        advantages, returns = adv.reshape(-1), ret.reshape(-1)
        count = int(obs.shape[0])
        if count == 0 or cfg.update_epochs < 1 or cfg.num_minibatches < 1:
            raise ValueError("MLP PPO requires nonempty rollout, positive epochs and minibatches")
        if advantages.numel() != b_val.numel() or returns.numel() != b_val.numel():
            raise ValueError("advantage/return shape must match the rollout values")
        if obs.shape[1] != self.D:
            raise ValueError("observation width does not match the network")
        # one aggregate finite check before any optimizer step (ppo_gpu.py:2000-2009): read on
        # a second stream beside the first minibatch's gradient launches, its flag copied to the
        # host on that stream and tested before the first Adam step, so the parameters and the
        # optimizer state are untouched when the update is refused
        cur = torch.cuda.current_stream(dev)
        if self._side is None:
            self._side = torch.cuda.Stream(device=dev)   # default priority
        self._side.wait_stream(cur)
        with torch.cuda.stream(self._side):
            ok = finite_flag((obs, rollout.b_rew, b_val, old_logp, advantages, returns))
        checked = False
        obs, act = obs.contiguous(), act.contiguous()
        old_logp, advantages, returns = (x.contiguous().float() for x in
                                         (old_logp, advantages, returns))
        mb_size = (count + cfg.num_minibatches - 1) // cfg.num_minibatches
        nmb = (count + mb_size - 1) // mb_size
        self._workspace(mb_size)
        if self.stats.shape[0] < nmb:
            self.stats = torch.zeros(nmb, NSTATS, dtype=torch.float32, device=dev)
        early, epoch, steps = False, 0, 0
        last_kl = torch.zeros((), device=dev)
        for epoch in range(cfg.update_epochs):
            if perms is not None:
                perm = perms[epoch].to(dev, torch.int64)
            else:
                perm = self.permutation(count)
            adv_stats = self.epoch_adv_stats(advantages, perm, mb_size)
            for j, s in enumerate(range(0, count, mb_size)):
                mb = perm[s:s + mb_size]
                self.minibatch_grad(obs, act, old_logp, advantages, returns, mb, self.stats[j],
                                    adv_stats=adv_stats[j])
                if not checked:
                    with torch.cuda.stream(self._side):
                        finite = bool(ok.cpu())           # waits for the side stream only
                    if not finite:
                        raise FloatingPointError(
                            "non-finite physical trajectory or PPO rollout; update refused")
                    checked = True
                self.optimizer_step()
                steps += 1
            last_kl = self.stats[:nmb, STAT_KL].mean()
            if cfg.target_kl is not None and float(last_kl) > cfg.target_kl:
                early = True
                break
        last = self.stats[nmb - 1]
        count_f = b_val.numel()
        var_y = returns.var() if count_f > 1 else torch.zeros((), device=dev)
        ev = torch.where(var_y == 0, torch.zeros((), device=dev),
                         1.0 - (returns - b_val).var(correction=1 if count_f > 1 else 0) /
                         (var_y + 1e-8))
        return {"pl": last[STAT_PL].clone(), "vl": last[STAT_VL].clone(),
                "ent": last[STAT_ENT].clone(), "kl": last_kl, "cf": last[STAT_CF].clone(),
                "ev": ev, "epochs": epoch + 1, "early": early,
                "actor_grad_norm": self.grad_norms[0].clone(),
                "critic_grad_norm": self.grad_norms[1].clone(),
                "optimizer_steps": steps}


# algorithmic matrix work of one transition in the update (2 x MACs): forward of both networks,
# the backward through the hidden layers, and every weight gradient
def update_flop_per_row(D):
    fwd = 2 * (2 * 256 * D + 2 * 256 * 256 + 84 * 256 + 256)
    bwd_x = 2 * (84 * 256 + 2 * 256 * 256 + 256)
    wgrad = 2 * (2 * 256 * D + 2 * 256 * 256 + 84 * 256 + 256)
    return fwd + bwd_x + wgrad
