"""The PPO-update oracle (oracle/ppo_oracle.py) pinned on the CPU: its hand-written backward
equals torch autograd through the reference's loss; autograd's gradient equals central finite
differences of the loss in float64; the loss reduces to its closed forms in special cases; the
optimizer's first step has Adam's closed form with the clipped gradient."""
import importlib.util
import math
import os

import numpy as np
import pytest
import torch

from conftest import ROOT

_spec = importlib.util.spec_from_file_location("ppo_oracle", os.path.join(ROOT, "oracle", "ppo_oracle.py"))
P = importlib.util.module_from_spec(_spec)
_spec.loader.exec_module(P)


def make_params(D, seed=0, std=0.08, dtype=torch.float32):
    g = torch.Generator().manual_seed(seed)
    na, nc = P.counts(D)
    flat = torch.randn(na + nc, generator=g, dtype=torch.float64) * std
    pa, pc = P.unflatten(flat, D)
    for d in (pa, pc):                                   # biases a little smaller
        d["b1"].mul_(0.5); d["b2"].mul_(0.5); d["b3"].mul_(0.5)
    return flat.to(dtype)


def make_batch(flat, D, M, seed=1, logp_noise=0.15, dtype=torch.float32):
    g = torch.Generator().manual_seed(seed)
    obs = (torch.randn(M, D, generator=g, dtype=torch.float64) * 1.5).clamp(-10, 10).to(dtype)
    act = torch.randint(0, P.BINS, (M, P.CH), generator=g)
    pa, _ = P.unflatten(flat.to(dtype), D)
    with torch.no_grad():
        lg = P._mlp(pa, obs).view(-1, P.CH, P.BINS)
        lp = torch.distributions.Categorical(logits=lg).log_prob(act).sum(-1)
    old = (lp + logp_noise * torch.randn(M, generator=g, dtype=torch.float64).to(dtype)).to(dtype)
    adv = torch.randn(M, generator=g, dtype=torch.float64).to(dtype)
    ret = torch.randn(M, generator=g, dtype=torch.float64).to(dtype)
    return obs, act, old, adv, ret


@pytest.mark.parametrize("D", [184, 214])
@pytest.mark.parametrize("ent_coef,norm_adv", [(0.0, True), (0.01, True), (0.01, False)])
def test_mirror_backward_equals_autograd(D, ent_coef, norm_adv):
    flat = make_params(D)
    b = make_batch(flat, D, 37)
    ga, sa = P.reference_minibatch(flat, D, *b, ent_coef=ent_coef, norm_adv=norm_adv)
    gm, sm = P.mirror_minibatch(flat, D, *b, ent_coef=ent_coef, norm_adv=norm_adv, bf16=False)
    scale = ga.abs().max()
    assert scale > 0
    assert torch.allclose(gm, ga, rtol=1e-4, atol=2e-6 * float(scale)), \
        float((gm - ga).abs().max() / scale)
    for k in ("pl", "vl", "ent", "kl", "cf"):
        assert math.isclose(sm[k], sa[k], rel_tol=1e-5, abs_tol=1e-6), k
    # some ratios are clipped on each side, so both branches of the surrogate are exercised
    r = sa["ratio"]
    assert ((r < 0.8) | (r > 1.2)).any() and ((r > 0.8) & (r < 1.2)).any()


def test_autograd_equals_finite_differences():
    D = 184
    flat = make_params(D, dtype=torch.float64)
    b = make_batch(flat, D, 9, logp_noise=0.05, dtype=torch.float64)
    g, _ = P.reference_minibatch(flat, D, *b, ent_coef=0.02)
    rng = np.random.default_rng(3)
    na, nc = P.counts(D)
    # coordinates in every parameter tensor of both networks
    offs, off = [], 0
    for _, shp in P.shapes(D)[0] + P.shapes(D)[1]:
        n = math.prod(shp)
        offs += [off + int(x) for x in rng.integers(0, n, 3)]
        off += n
    h = 1e-6
    for i in offs:
        fp, fm = flat.clone(), flat.clone()
        fp[i] += h
        fm[i] -= h
        lp = P.reference_minibatch(fp, D, *b, ent_coef=0.02)[1]["loss"]
        lm = P.reference_minibatch(fm, D, *b, ent_coef=0.02)[1]["loss"]
        fd = (lp - lm) / (2 * h)
        assert abs(fd - float(g[i])) <= 1e-6 + 1e-5 * abs(fd), (i, fd, float(g[i]))


def test_loss_special_cases():
    D = 184
    flat = make_params(D)
    pa, pc = P.unflatten(flat, D)
    pa["W3"].zero_(); pa["b3"].zero_()                  # uniform policy over 21 bins
    obs, act, _, adv, _ = make_batch(flat, D, 64)
    with torch.no_grad():
        lp = torch.full((64,), 4 * math.log(1 / 21))
        v = P._mlp(pc, obs).squeeze(-1)
    _, st = P.reference_minibatch(flat, D, obs, act, lp, adv, v.clone(), ent_coef=0.0)
    assert abs(st["kl"]) < 1e-6 and st["cf"] == 0.0     # ratio 1
    assert abs(st["pl"]) < 1e-6                           # -mean of normalised advantages
    assert math.isclose(st["ent"], 4 * math.log(21), rel_tol=1e-6)
    assert st["vl"] < 1e-12                               # returns equal to the values


def test_optimizer_first_step_closed_form():
    D = 184
    flat = make_params(D)
    na, nc = P.counts(D)
    g = torch.randn(na + nc, generator=torch.Generator().manual_seed(5)) * 1e-3
    g[:na] *= 50.0                                        # the actor's gradient gets clipped
    opt = P.ReferenceOptim(flat, D, lr=3e-4, max_grad_norm=0.5)
    na_n, nc_n = opt.step(g)
    for sl, norm in ((slice(0, na), na_n), (slice(na, na + nc), nc_n)):
        gg = g[sl].double()
        tn = float(gg.norm())
        assert math.isclose(norm, tn, rel_tol=1e-5)
        gc = gg * min(1.0, 0.5 / (tn + 1e-6))
        want = flat[sl].double() - 3e-4 * gc / (gc.abs() + 1e-5)   # m^ = g, v^ = g^2 at step 1
        assert torch.allclose(opt.params()[sl].double(), want, rtol=2.5e-7, atol=1e-9)   # fp32
    assert na_n > 0.5 > nc_n
