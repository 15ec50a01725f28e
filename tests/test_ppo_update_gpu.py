"""PPO update on the GPU (f16_ppo_grad / f16_ppo_adam_step / f16_ppo_pack through the C ABI)
against the CPU oracle (oracle/ppo_oracle.py): minibatch gradients and statistics against the
bf16-mirrored restatement, the optimizer against torch.optim.Adam + clip_grad_norm_, whole
updates against the reference's epoch/minibatch loop, the repacked blobs against policy.pack, and
the first minibatch of a real rollout at ratio 1."""
import importlib.util
import math
import os
from types import SimpleNamespace

import numpy as np
import pytest
import torch

from conftest import ROOT, import_pkg

_spec = importlib.util.spec_from_file_location("ppo_oracle", os.path.join(ROOT, "oracle", "ppo_oracle.py"))
P = importlib.util.module_from_spec(_spec)
_spec.loader.exec_module(P)

pytestmark = pytest.mark.gpu


def make_net(D, seed=0):
    pol = import_pkg("policy")
    torch.manual_seed(seed)
    return pol.MLPActorCritic(D)                 # orthogonal(sqrt 2) init, model.py:86-90


def flat_of(net):
    U = import_pkg("ppo_update")
    return torch.cat([p.detach().reshape(-1).float().cpu() for p in U.net_parameters(net)])


def fake_rollout(flat, D, T, rows, seed=1, logp_noise=0.15):
    """Rollout-shaped buffers: normalised observations, drawn bins, collection log-probabilities
    near the current policy's (bf16-mirrored forward) so ratios straddle the clip range."""
    g = torch.Generator().manual_seed(seed)
    M = T * rows
    obs = (torch.randn(M, D, generator=g) * 1.3).clamp(-10, 10)
    act = torch.randint(0, P.BINS, (M, P.CH), generator=g)
    _, st = P.mirror_minibatch(flat, D, obs, act, torch.zeros(M), torch.zeros(M), torch.zeros(M),
                               norm_adv=False, bf16=True)
    logp = st["new_logp"] + logp_noise * torch.randn(M, generator=g)
    adv = torch.randn(M, generator=g) * 2.0 + 0.3
    ret = torch.randn(M, generator=g)
    val = torch.randn(M, generator=g)
    rew = torch.randn(M, generator=g)
    ro = SimpleNamespace(b_obs=obs.view(T, rows, D), b_act=act.view(T, rows, 4),
                         b_logp=logp.view(T, rows), b_val=val.view(T, rows),
                         b_rew=rew.view(T, rows))
    return ro, adv.view(T, rows), ret.view(T, rows)


def to_dev(ro, dev):
    return SimpleNamespace(**{k: v.to(dev).contiguous() for k, v in vars(ro).items()})


def rel_err(a, b):
    return float((a - b).norm() / max(float(b.norm()), 1e-30))


def check_grads(g_gpu, g_ref, D, tol):
    """Per parameter tensor: relative 2-norm error below tol."""
    ga, gc = P.unflatten(g_gpu, D)
    ra, rc = P.unflatten(g_ref, D)
    worst = 0.0
    for tag, x, y in (("actor", ga, ra), ("critic", gc, rc)):
        for k in x:
            e = rel_err(x[k], y[k])
            worst = max(worst, e)
            assert e < tol, (tag, k, e)
    print(f"  worst per-tensor relative gradient error {worst:.2e}", flush=True)


def test_pack_matches_policy_pack(gpu):
    U = import_pkg("ppo_update")
    for D in (184, 214):
        net = make_net(D, seed=3).to(gpu)
        wbf_ref, wf_ref = (t.clone() for t in net.pack(gpu))
        up = U.PPOUpdater(net)                   # packs from the flat master copy
        assert torch.equal(up.wbf, wbf_ref) and torch.equal(up.wf, wf_ref)
        a, c = net.actor_logits, net.critic
        pol = import_pkg("policy")
        wT = up.wT.float().cpu()
        W3T = pol.frag_unmajor(wT[:256 * 96], 256, 96)
        assert torch.equal(W3T[:, :84], a[4].weight.detach().cpu().t().to(torch.bfloat16).float())
        assert (W3T[:, 84:] == 0).all()
        W2aT = pol.frag_unmajor(wT[256 * 96:256 * 96 + 65536], 256, 256)
        W2cT = pol.frag_unmajor(wT[256 * 96 + 65536:], 256, 256)
        assert torch.equal(W2aT, a[2].weight.detach().cpu().t().to(torch.bfloat16).float())
        assert torch.equal(W2cT, c[2].weight.detach().cpu().t().to(torch.bfloat16).float())


@pytest.mark.parametrize("D,mb,ent_coef,norm_adv", [(184, 300, 0.0, True), (214, 300, 0.01, True),
                                                    (184, 64, 0.01, False), (214, 1, 0.0, True),
                                                    (184, 2500, 0.0, True)])
def test_minibatch_grad_matches_oracle(gpu, D, mb, ent_coef, norm_adv):
    U = import_pkg("ppo_update")
    print(f"minibatch grad D={D} mb={mb} ent={ent_coef} norm_adv={norm_adv}", flush=True)
    net = make_net(D, seed=D + mb)
    flat = flat_of(net)
    T, rows = 5, 600
    ro, adv, ret = fake_rollout(flat, D, T, rows, seed=mb)
    up = U.PPOUpdater(net.to(gpu), U.UpdateConfig(ent_coef=ent_coef, norm_adv=norm_adv))
    idx = torch.randperm(T * rows, generator=torch.Generator().manual_seed(7))[:mb]
    d = to_dev(ro, gpu)
    obs, act, logp = d.b_obs.flatten(0, 1), d.b_act.flatten(0, 1), d.b_logp.flatten()
    advd, retd = adv.reshape(-1).to(gpu), ret.reshape(-1).to(gpu)
    up.minibatch_grad(obs, act, logp, advd, retd, idx.to(gpu))
    stats = up.stats[0].cpu()
    g_gpu = up.grad.cpu()
    o = ro.b_obs.flatten(0, 1)[idx]
    g_ref, st = P.mirror_minibatch(flat, D, o, ro.b_act.flatten(0, 1)[idx],
                                   ro.b_logp.flatten()[idx], adv.reshape(-1)[idx],
                                   ret.reshape(-1)[idx], ent_coef=ent_coef, norm_adv=norm_adv)
    assert torch.isfinite(g_gpu).all()
    check_grads(g_gpu, g_ref, D, tol=3e-3)
    U_ = U
    for k, j in (("pl", U_.STAT_PL), ("vl", U_.STAT_VL), ("ent", U_.STAT_ENT), ("kl", U_.STAT_KL)):
        assert math.isclose(float(stats[j]), st[k], rel_tol=2e-3, abs_tol=2e-5), (k, float(stats[j]), st[k])
    # the clip fraction counts rows: at most a few rows at the clip edge may flip
    assert abs(float(stats[U_.STAT_CF]) - st["cf"]) <= 2.0 / mb + 1e-7
    a_sel = adv.reshape(-1)[idx].double()
    assert math.isclose(float(stats[U_.STAT_ADV_MEAN]), float(a_sel.mean()), rel_tol=1e-5, abs_tol=1e-6)
    if mb > 1:
        assert math.isclose(float(stats[U_.STAT_ADV_STD]), float(a_sel.std()), rel_tol=1e-5)
    assert float(stats[U_.STAT_BAD]) == 0.0


def test_out_of_range_indices_are_counted_not_read(gpu):
    U = import_pkg("ppo_update")
    D = 184
    net = make_net(D, seed=11)
    flat = flat_of(net)
    ro, adv, ret = fake_rollout(flat, D, 2, 100, seed=4)
    up = U.PPOUpdater(net.to(gpu))
    d = to_dev(ro, gpu)
    idx = torch.tensor([3, -5, 17, 200, 250, 199], dtype=torch.int64, device=gpu)   # count 200
    up.minibatch_grad(d.b_obs.flatten(0, 1), d.b_act.flatten(0, 1), d.b_logp.flatten(),
                      adv.reshape(-1).to(gpu), ret.reshape(-1).to(gpu), idx)
    assert float(up.stats[0, U.STAT_BAD]) == 3.0
    assert torch.isfinite(up.grad).all()


def test_optimizer_step_matches_torch_adam(gpu):
    U = import_pkg("ppo_update")
    D = 214
    net = make_net(D, seed=5)
    flat = flat_of(net)
    up = U.PPOUpdater(net.to(gpu), U.UpdateConfig(lr=3e-4, critic_lr=1e-3))
    ref = P.ReferenceOptim(flat, D, lr=3e-4, critic_lr=1e-3, max_grad_norm=0.5)
    gen = torch.Generator().manual_seed(9)
    for step in range(4):
        g = torch.randn(flat.numel(), generator=gen) * (1e-3 if step % 2 else 3e-2)
        up.grad.copy_(g.to(gpu))
        up.optimizer_step()
        na, nc = ref.step(g)
        p_gpu = up.flat.cpu()
        p_ref = ref.params()
        assert torch.allclose(p_gpu, p_ref, rtol=1e-6, atol=1e-8), float((p_gpu - p_ref).abs().max())
        gn = up.grad_norms.cpu()
        assert math.isclose(float(gn[0]), na, rel_tol=1e-5)
        assert math.isclose(float(gn[1]), nc, rel_tol=1e-5)
    # the rollout blobs follow the master parameters
    wbf, wf = up.wbf.clone(), up.wf.clone()
    net.pack(gpu)
    assert torch.equal(net.packed()[0], wbf) and torch.equal(net.packed()[1], wf)


def test_update_matches_reference_loop(gpu):
    """Two epochs of four minibatches (ragged last) with fixed permutations: final parameters,
    statistics and norms against the reference loop with the mirrored gradients."""
    U = import_pkg("ppo_update")
    D = 184
    net = make_net(D, seed=21)
    flat = flat_of(net)
    T, rows = 4, 130
    ro, adv, ret = fake_rollout(flat, D, T, rows, seed=22, logp_noise=0.05)
    count = T * rows
    gen = torch.Generator().manual_seed(23)
    perms = [torch.randperm(count, generator=gen) for _ in range(2)]
    cfg = U.UpdateConfig(update_epochs=2, num_minibatches=4, target_kl=None)
    up = U.PPOUpdater(net.to(gpu), cfg)
    res = up.update(to_dev(ro, gpu), adv.to(gpu), ret.to(gpu), perms=perms)
    mb = (count + 3) // 4
    p_ref, rr = P.reference_update(flat, D, ro.b_obs.flatten(0, 1), ro.b_act.flatten(0, 1),
                                   ro.b_logp.flatten(), adv.reshape(-1), ret.reshape(-1), perms,
                                   mb, target_kl=None)
    assert res["optimizer_steps"] == rr["optimizer_steps"] == 8
    assert res["epochs"] == 2 and not res["early"]
    p_gpu = up.flat.cpu()
    diff = (p_gpu - p_ref).abs()
    moved = (p_ref - flat).abs()
    print("update: max |dp| %.3g, median %.3g; mean step %.3g" %
          (float(diff.max()), float(diff.median()), float(moved.mean())), flush=True)
    # Adam makes each coordinate's step the ratio of its moments, so a coordinate-wise relative
    # gradient difference e (bf16 rounding flips and accumulation order, ~1e-3) moves it by about
    # e * lr per step, and an element near zero can change sign: bound the worst by the steps'
    # total, the typical coordinate by 1 % of one step, and the far tail by its share
    lr, steps = cfg.lr, 8
    far = float((diff > 0.05 * lr).float().mean())
    print("  share of coordinates off by more than 5 %% of a step: %.2e" % far, flush=True)
    assert float(diff.max()) <= 2 * lr * steps
    assert far < 2e-3
    assert float(diff.median()) < 1e-2 * lr
    for k in ("pl", "vl", "ent"):
        assert math.isclose(float(res[k]), rr[k], rel_tol=5e-3, abs_tol=5e-5), k
    assert math.isclose(float(res["kl"]), rr["kl"], rel_tol=5e-2, abs_tol=2e-5)
    assert math.isclose(float(res["actor_grad_norm"]), rr["actor_grad_norm"], rel_tol=5e-3)
    assert math.isclose(float(res["critic_grad_norm"]), rr["critic_grad_norm"], rel_tol=5e-3)


def test_early_stop_and_refusals(gpu):
    U = import_pkg("ppo_update")
    D = 184
    net = make_net(D, seed=31)
    flat = flat_of(net)
    ro, adv, ret = fake_rollout(flat, D, 2, 64, seed=32, logp_noise=0.5)
    up = U.PPOUpdater(net.to(gpu), U.UpdateConfig(target_kl=1e-6, num_minibatches=2))
    res = up.update(to_dev(ro, gpu), adv.to(gpu), ret.to(gpu))
    assert res["early"] and res["epochs"] == 1 and res["optimizer_steps"] == 2
    bad = to_dev(ro, gpu)
    bad.b_obs[0, 3, 5] = float("nan")
    before = [t.clone() for t in (up.flat, up.exp_avg, up.exp_avg_sq)]
    steps = up.steps
    with pytest.raises(FloatingPointError):
        up.update(bad, adv.to(gpu), ret.to(gpu))
    # refused before any optimizer step: parameters, moments and the step count untouched
    torch.cuda.synchronize()
    assert all(torch.equal(x, y) for x, y in zip(before, (up.flat, up.exp_avg, up.exp_avg_sq)))
    assert up.steps == steps
    with pytest.raises(ValueError):
        up.update(to_dev(ro, gpu), adv[:1].to(gpu), ret.to(gpu))


def test_first_minibatch_of_a_rollout_has_ratio_one(gpu):
    """At the collection weights the update's log-probability equals the rollout kernel's bit
    for bit: every ratio is exactly 1, so the approximate KL and the clip fraction are 0."""
    ppo = import_pkg("ppo")
    U = import_pkg("ppo_update")
    rl = import_pkg("rl_env")
    env = rl.GpuDogfightVecEnv(64, seed=0, ic_pool_size=64)
    net = make_net(184, seed=41).to(gpu)
    ro = ppo.SelfPlayRollout(env, net, T=8, seed=3, stats=False)
    ro.reset(stagger=True, max_stagger_steps=8)
    adv, ret, _ = ro.collect()
    up = U.PPOUpdater(net)
    count = ro.b_obs.shape[0] * ro.b_obs.shape[1]
    idx = torch.arange(count, device=gpu)
    up.minibatch_grad(ro.b_obs.flatten(0, 1), ro.b_act.flatten(0, 1), ro.b_logp.flatten(),
                      adv.reshape(-1), ret.reshape(-1), idx)
    st = up.stats[0].cpu()
    assert float(st[U.STAT_KL]) == 0.0 and float(st[U.STAT_CF]) == 0.0
    # a full update then trains: the next rollout runs on the new weights
    res = up.update(ro, adv, ret)
    assert res["optimizer_steps"] >= 8
    adv2, ret2, _ = ro.collect()
    assert torch.isfinite(adv2).all()


def _isfinite_all(floats, flags=()):
    ok = all(bool(torch.isfinite(x.cpu()).all()) for x in floats)
    return ok and all(bool((x.cpu() != 0).all()) for x in flags)


def test_finite_flag_matches_isfinite(gpu):
    """f16_all_finite against torch.isfinite(x).all() / (flags != 0).all(): float32, float64 and
    uint8/bool spans of sizes 0..several chunks, views starting off the 16-byte grid, one inf,
    -inf or NaN (or one zero flag) planted at the head, in the 16-byte body or at the tail, and
    the largest finite and subnormal values (finite)."""
    U = import_pkg("ppo_update")
    g = torch.Generator().manual_seed(3)
    cases = 0
    for dtype in (torch.float32, torch.float64, torch.uint8, torch.bool):
        is_flag = dtype in (torch.uint8, torch.bool)
        for n in (0, 1, 3, 5, 16, 17, 63, 1000, 4099, 1 << 20):
            for off in (0, 1, 3):
                if n == 0 and off:
                    continue
                if is_flag:
                    base = torch.randint(1, 256, (n + off + 8,), generator=g).to(torch.uint8)
                    base = base.bool() if dtype == torch.bool else base
                else:
                    base = torch.randn(n + off + 8, generator=g, dtype=torch.float64).to(dtype)
                    if n > 2:
                        fi = torch.finfo(dtype)
                        base[off] = fi.max
                        base[off + n - 1] = -fi.tiny / 4          # subnormal
                base[off + n:] = 0 if is_flag else float("nan")  # outside the span
                dev = base.cuda()
                view = dev[off:off + n]
                fl, fa = ((), (view,)) if is_flag else ((view,), ())
                if n > 0:
                    fl_extra = (torch.ones(7, device="cuda"),)
                    assert _isfinite_all(fl, fa)
                    assert bool(U.finite_flag(fl + fl_extra, fa)), (dtype, n, off)
                cases += 1
                for pos in sorted({0, n // 2, n - 1}) if n > 0 else ():
                    for bad in ((0,) if is_flag else (float("inf"), -float("inf"), float("nan"))):
                        planted = dev.clone()
                        planted[off + pos] = bad
                        pv = planted[off:off + n]
                        fl2, fa2 = ((), (pv,)) if is_flag else ((pv,), ())
                        got = bool(U.finite_flag(fl2 + (torch.ones(5, device="cuda"),), fa2))
                        assert got is False and _isfinite_all(fl2, fa2) is False, (dtype, n, off, pos, bad)
                        cases += 1
    assert cases > 300
    # several spans at once: the flag is the AND of all of them
    a = torch.randn(1000, device="cuda")
    b = torch.randn(333, device="cuda", dtype=torch.float64)
    c = torch.ones(77, dtype=torch.uint8, device="cuda")
    assert bool(U.finite_flag((a, b), (c,)))
    b[200] = float("nan")
    assert not bool(U.finite_flag((a, b), (c,)))


def test_finite_flag_argument_checks(gpu):
    """Refused before any launch: more than 16 spans, an element size other than 1, 4, 8, a
    pointer off its element alignment, a negative count, no flag; and the Python wrapper's dtype,
    device and count checks."""
    U, L = import_pkg("ppo_update"), import_pkg("_lib")
    lib = L.lib()
    x = torch.zeros(64, device="cuda")
    flag = torch.zeros(1, dtype=torch.uint8, device="cuda")
    h = L.stream_handle()
    S = L.F16FiniteSpan

    def call(spans, flag_ptr=L.ptr(flag)):
        arr = (S * max(1, len(spans)))(*spans)
        return lib.f16_all_finite(arr, len(spans), flag_ptr, h)

    ok = S(x.data_ptr(), 64, 4)
    assert call([ok]) == 0
    torch.cuda.synchronize()
    assert int(flag.item()) == 1
    assert call([ok] * 17) == L.F16_EINVAL
    assert call([S(x.data_ptr(), 64, 2)]) == L.F16_EINVAL
    assert call([S(x.data_ptr() + 2, 8, 4)]) == L.F16_EINVAL
    assert call([S(x.data_ptr() + 4, 8, 8)]) == L.F16_EINVAL
    assert call([S(x.data_ptr(), -1, 4)]) == L.F16_EINVAL
    assert call([ok], flag_ptr=None) == L.F16_EINVAL
    with pytest.raises(TypeError):
        U.finite_flag((torch.zeros(4, dtype=torch.float16, device="cuda"),))
    with pytest.raises(ValueError):
        U.finite_flag((torch.zeros(4),))
    with pytest.raises(ValueError):
        U.finite_flag([x] * 17)
    with pytest.raises(ValueError):
        U.finite_flag(())


def test_permutation_is_a_uniform_shuffle(gpu):
    """f16_permutation: a permutation of 0..n-1 for n from 1 through non-powers of four and past
    2^21; another key, another permutation; where each element of five lands over 2,000 keys is
    uniform, and so is where each element of 17 lands (chi-square below the 0.1 % point
    for n - 1 degrees of freedom; the same network with four rounds fails it); at 2^21 + 3
    elements the mean displacement |perm[i] - i| / n is 1/3 and i and perm[i] are uncorrelated,
    as for a uniformly random permutation."""
    L = import_pkg("_lib")
    lib = L.lib()
    h = L.stream_handle()

    def perm_of(n, key):
        k = torch.tensor([key], dtype=torch.int64, device="cuda")
        p = torch.empty(n, dtype=torch.int64, device="cuda")
        assert lib.f16_permutation(L.ptr(p), n, L.ptr(k), h) == 0
        return p

    for n in (1, 2, 3, 4, 5, 16, 17, 1000, 65537, 1 << 21, (1 << 21) + 3):
        p = perm_of(n, 12345 + n)
        assert torch.equal(torch.sort(p).values, torch.arange(n, device="cuda")), n
    assert not torch.equal(perm_of(1000, 1), perm_of(1000, 2))
    assert torch.equal(perm_of(1000, 7), perm_of(1000, 7))
    K = 2000
    for n, bound in ((5, 18.47), (17, 39.25)):      # chi-square 0.1 % points, n - 1 dof
        draws = torch.stack([perm_of(n, 1000 + k) for k in range(K)]).cpu()
        for e in range(n):
            pos = (draws == e).nonzero()[:, 1]
            cnt = torch.bincount(pos, minlength=n).double()
            chi2 = float(((cnt - K / n) ** 2 / (K / n)).sum())
            assert chi2 < bound, (n, e, cnt.tolist())
    # the unequal-halves network above 2^15 elements: where positions 0, 777 and n - 1 send
    # their element over 400 keys, in 16 bins of the range (chi-square, 15 dof, 0.1 % point)
    n = (1 << 16) + 3
    draws = torch.stack([perm_of(n, 1000 + k)[[0, 777, n - 1]] for k in range(400)]).cpu()
    for c in range(3):
        cnt = torch.bincount(draws[:, c] * 16 // n, minlength=16).double()
        assert float(((cnt - 25.0) ** 2 / 25.0).sum()) < 37.7, cnt.tolist()
    n = (1 << 21) + 3
    p = perm_of(n, 99).double()
    i = torch.arange(n, device="cuda", dtype=torch.float64)
    assert abs(float((p - i).abs().mean()) / n - 1 / 3) < 2e-3
    corr = float(((p - p.mean()) * (i - i.mean())).mean() / (p.std() * i.std()))
    assert abs(corr) < 3e-3
    # argument checks (nothing launched)
    k = torch.zeros(1, dtype=torch.int64, device="cuda")
    out = torch.empty(4, dtype=torch.int64, device="cuda")
    assert lib.f16_permutation(L.ptr(out), 0, L.ptr(k), h) == L.F16_EINVAL
    assert lib.f16_permutation(L.ptr(out), (1 << 31) + 1, L.ptr(k), h) == L.F16_EINVAL
    assert lib.f16_permutation(None, 4, L.ptr(k), h) == L.F16_EINVAL
    assert lib.f16_permutation(L.ptr(out), 4, None, h) == L.F16_EINVAL


def test_epoch_advantage_stats_equal_per_minibatch(gpu):
    """f16_ppo_adv_stats forms every minibatch's advantage mean and std of an epoch in two
    launches: equal bit for bit to what f16_ppo_grad forms for each minibatch alone (a ragged
    last minibatch, sizes across the 2,048-row partial blocks), and a minibatch gradient fed the
    precomputed pair equals the one that forms it; the argument checks refuse a bad cut."""
    U, L = import_pkg("ppo_update"), import_pkg("_lib")
    D = 184
    net = make_net(D, seed=11)
    flat = flat_of(net)
    T, rows = 7, 1000
    ro, adv, ret = fake_rollout(flat, D, T, rows, seed=3)
    up = U.PPOUpdater(net.to(gpu), U.UpdateConfig())
    d = to_dev(ro, gpu)
    obs, act, logp = d.b_obs.flatten(0, 1), d.b_act.flatten(0, 1), d.b_logp.flatten()
    advd, retd = adv.reshape(-1).to(gpu), ret.reshape(-1).to(gpu)
    count = T * rows
    for mb in (2048, 2049, 1000, 333, count):
        perm = torch.randperm(count, generator=torch.Generator().manual_seed(mb)).to(gpu)
        st = up.epoch_adv_stats(advd, perm, mb)
        nmb = (count + mb - 1) // mb
        assert st.shape == (nmb, 2)
        for j in sorted({0, nmb - 1}):
            idx = perm[j * mb:(j + 1) * mb]
            up.minibatch_grad(obs, act, logp, advd, retd, idx)
            own = up.stats[0].clone()
            g_own = up.grad.clone()
            assert float(own[U.STAT_ADV_MEAN]) == float(st[j, 0]), (mb, j)
            assert float(own[U.STAT_ADV_STD]) == float(st[j, 1]), (mb, j)
            up.minibatch_grad(obs, act, logp, advd, retd, idx, adv_stats=st[j])
            assert torch.equal(up.grad, g_own), (mb, j)
            assert torch.equal(up.stats[0], own), (mb, j)
    lib, h = L.lib(), L.stream_handle()
    perm = torch.arange(count, device=gpu)
    out = torch.empty(16, dtype=torch.float32, device=gpu)
    work = torch.empty(1 << 20, dtype=torch.uint8, device=gpu)
    args = lambda total, mb, nmb: lib.f16_ppo_adv_stats(L.ptr(advd), L.ptr(perm), total, count,
                                                        mb, nmb, L.ptr(out), L.ptr(work), h)
    assert args(count, 1000, 7) == 0
    torch.cuda.synchronize()
    assert args(count, 1000, 6) == L.F16_EINVAL      # too few minibatches for the cut
    assert args(count, 1000, 8) == L.F16_EINVAL      # one minibatch past the end
    assert args(0, 1000, 1) == L.F16_EINVAL
    assert lib.f16_ppo_adv_work_bytes(0, 1) == -1
