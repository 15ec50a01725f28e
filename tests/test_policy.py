"""Policy step: the fused normalise -> actor/critic MLP -> categorical draw -> controls kernel
(include/f16_policy.h) and the RunningNorm update.

CPU part: the draw's checker (oracle/policy_oracle.c) is pinned by Philox4x32-10's published
known-answer vectors, its IEEE-only exp by libm, and its inverse-CDF draw by the distribution it
must produce; the library's struct layout by its own sizeof.
GPU part (tolerances): normalised observations within 1 float32 ulp of the reference formula
(ppo_gpu.py:210-214); logits and values within 5e-3 x max(1, their standard deviation) of a
float64 evaluation of the same bf16-rounded weights and activations, 99% of them within 1e-4 x
that scale (differences: fp32 accumulation order, and hidden activations whose tanh lands on a
bf16 rounding boundary -- one such flip moves a value by ~2^-8 |w| per unit it feeds); sampled bins bit-exact against the checker fed
the kernel's logits, log-probabilities within 1e-5; controls exact against action_to_env."""
import ctypes

import numpy as np
import pytest

import oracle_lib
from conftest import import_pkg

U32 = ctypes.c_uint32


def _orc_lib(orc):
    L = orc.L
    L.orc_philox4x32_10.argtypes = [ctypes.POINTER(U32), U32, U32]
    L.orc_exp_nonpos.argtypes = [ctypes.c_float]
    L.orc_exp_nonpos.restype = ctypes.c_float
    L.orc_policy_sample.argtypes = [ctypes.c_void_p, ctypes.c_void_p, ctypes.c_long,
                                    ctypes.c_uint64, U32, U32, ctypes.c_int, ctypes.c_void_p,
                                    ctypes.c_void_p]
    return L


def philox(orc, ctr, key):
    c = (U32 * 4)(*ctr)
    _orc_lib(orc).orc_philox4x32_10(c, key[0], key[1])
    return [c[i] for i in range(4)]


def oracle_sample(orc, logits, rows, seed, step, salt=0, deterministic=False):
    L = _orc_lib(orc)
    logits = np.ascontiguousarray(logits, np.float32)
    rows = np.ascontiguousarray(rows, np.int64)
    n = logits.shape[0]
    idx = np.zeros((n, 4), np.int64)
    lp = np.zeros(n, np.float32)
    L.orc_policy_sample(logits.ctypes.data, rows.ctypes.data, n, seed, step, salt,
                        int(deterministic), idx.ctypes.data, lp.ctypes.data)
    return idx, lp


# ------------------------------------------------------------------------ CPU: checker pins
def test_philox_known_answers(orc):
    """Random123 kat_vectors, philox4x32 with 10 rounds."""
    assert philox(orc, [0, 0, 0, 0], [0, 0]) == [0x6627e8d5, 0xe169c58d, 0xbc57ac4c, 0x9b00dbd8]
    assert philox(orc, [0xffffffff] * 4, [0xffffffff, 0xffffffff]) == \
        [0x408f276d, 0x41c83b0e, 0xa20bc7c6, 0x6d5451fd]
    assert philox(orc, [0x243f6a88, 0x85a308d3, 0x13198a2e, 0x03707344],
                  [0xa4093822, 0x299f31d0]) == [0xd16cfe09, 0x94fdcceb, 0x5001e420, 0x24126ea1]


def test_exp_nonpos_accuracy(orc):
    L = _orc_lib(orc)
    xs = np.concatenate([-np.logspace(-8, np.log10(86.9), 4000), [0.0, -1e-30, -86.99]])
    got = np.array([L.orc_exp_nonpos(float(x)) for x in xs.astype(np.float32)], np.float64)
    ref = np.exp(xs.astype(np.float32).astype(np.float64))
    assert (np.abs(got - ref) <= 4e-7 * ref + 1e-44).all()
    assert L.orc_exp_nonpos(-100.0) == 0.0 and L.orc_exp_nonpos(0.0) == 1.0


def test_sampler_distribution(orc):
    """The inverse-CDF draw follows softmax(logits): 20k rows x 4 channels per logit vector."""
    rng = np.random.default_rng(0)
    lg = rng.normal(0, 1.5, 84).astype(np.float32)
    n = 20000
    idx, lp = oracle_sample(orc, np.tile(lg, (n, 1)), np.arange(n), seed=0, step=3)
    for ch in range(4):
        l = lg[21 * ch:21 * ch + 21].astype(np.float64)
        p = np.exp(l - l.max()); p /= p.sum()
        freq = np.bincount(idx[:, ch], minlength=21) / n
        sd = np.sqrt(p * (1 - p) / n)
        assert (np.abs(freq - p) <= 5 * sd + 1e-12).all(), ch
    # log-probability of the drawn bins
    ref = sum(np.log(np.exp(lg[21 * c:21 * c + 21].astype(np.float64) - lg[21 * c:21 * c + 21].max())
                     / np.exp(lg[21 * c:21 * c + 21].astype(np.float64) -
                              lg[21 * c:21 * c + 21].max()).sum())[idx[:, c]] for c in range(4))
    assert np.abs(lp - ref).max() < 2e-5


def test_sampler_closed_forms(orc):
    lg = np.zeros((3, 84), np.float32)
    lg[0, 7] = 60.0                              # channel 0 certain
    lg[1] = -np.arange(84, dtype=np.float32)     # deterministic argmax: bin 0 everywhere
    idx, _ = oracle_sample(orc, lg, [0, 1, 2], seed=5, step=0)
    assert idx[0, 0] == 7
    idx_d, lp_d = oracle_sample(orc, lg, [0, 1, 2], seed=5, step=0, deterministic=True)
    assert (idx_d[1] == 0).all() and idx_d[0, 0] == 7
    # uniform logits: the bin is floor(21 u) up to float rounding at the cell edges
    c = philox(orc, [2, 0, 1, 0], [5, 0])
    u = (c[0] >> 8) * 2.0 ** -24
    assert idx[2, 1] == min(20, int(np.floor(21 * u)))
    np.testing.assert_allclose(lp_d[2], 4 * np.log(1 / 21), rtol=1e-6)


def test_library_struct_layout(pkg):
    L = import_pkg("_lib")
    out = (ctypes.c_long * 4)()
    L.check(L.lib().f16_abi_struct_sizes(out, 4), "f16_abi_struct_sizes")
    assert out[0] == ctypes.sizeof(L.F16PolicyGroup)
    assert out[1] == ctypes.sizeof(L.F16PolicyArgs)
    assert out[2] == ctypes.sizeof(L.F16PPOArgs)
    assert out[3] == ctypes.sizeof(L.F16AdamArgs)


def test_frag_major_blocks():
    """Block (t, s) of a fragment-major matrix holds, at lane l, row 32t + l%32 and columns
    16s + 8(l/32) .. +8: the 32x32x16 MFMA operand of lane l."""
    import torch
    P = import_pkg("policy")
    N, K = 64, 48
    w = torch.arange(N * K, dtype=torch.float64).view(N, K)
    f = P.frag_major(w)
    assert torch.equal(P.frag_unmajor(f, N, K), w)
    t, s = 1, 2
    blk = f[(t * (K // 16) + s) * 512:(t * (K // 16) + s + 1) * 512].view(64, 8)
    for l in (0, 5, 31, 32, 63):
        assert torch.equal(blk[l], w[32 * t + l % 32, 16 * s + 8 * (l // 32):16 * s + 8 * (l // 32) + 8])


def test_pack_layout():
    import torch
    P = import_pkg("policy")
    net = P.MLPActorCritic(184, init="normal", generator=torch.Generator().manual_seed(0))
    wbf, wf = net.pack(device="cpu")
    kp = 192
    w = wbf.float()
    W1 = P.frag_unmajor(w[:512 * kp], 512, kp)
    a, c = net.actor_logits, net.critic
    assert torch.equal(W1[:256, :184], a[0].weight.to(torch.bfloat16).float())
    assert torch.equal(W1[256:, :184], c[0].weight.to(torch.bfloat16).float())
    assert (W1[:, 184:] == 0).all()
    off = 512 * kp + 2 * 256 * 256
    assert torch.equal(P.frag_unmajor(w[512 * kp:512 * kp + 65536], 256, 256),
                       a[2].weight.to(torch.bfloat16).float())
    W3 = P.frag_unmajor(w[off:off + 96 * 256], 96, 256)
    assert torch.equal(W3[:84], a[4].weight.to(torch.bfloat16).float()) and (W3[84:] == 0).all()
    assert wf.numel() == 1377 and torch.equal(wf[1120:1376], c[4].weight.flatten())


@pytest.mark.parametrize("init", ["normal", "orthogonal"])
def test_init_draws_only_from_the_generator(init):
    """A seeded generator fixes every weight, whatever the global RNG did before (parity
    tests build their networks this way, so their inputs must not depend on test order)."""
    import torch
    P = import_pkg("policy")
    nets = []
    for glob in (1, 2):
        torch.manual_seed(glob)
        nets.append(P.MLPActorCritic(184, init=init, generator=torch.Generator().manual_seed(5)))
    for p, q in zip(nets[0].parameters(), nets[1].parameters()):
        assert torch.equal(p, q)
    if init == "orthogonal":                       # gain sqrt(2): W W^T = 2 I on the short side
        w = nets[0].actor_logits[2].weight.double()
        assert torch.allclose(w @ w.T, 2 * torch.eye(256, dtype=torch.float64), atol=1e-5)


# ------------------------------------------------------------------------ GPU
def _bf(x):
    import torch
    return torch.as_tensor(x).to(torch.bfloat16).to(torch.float64).numpy()


def _ref_forward(net, nobs):
    """float64 evaluation with the kernel's bf16 roundings of weights and activations."""
    a, c = net.actor_logits, net.critic
    W = lambda m: _bf(m.weight.detach().float().cpu())
    B = lambda m: m.bias.detach().double().cpu().numpy()
    x = _bf(nobs)
    h1 = _bf(np.tanh(x @ W(a[0]).T + B(a[0])))
    c1 = _bf(np.tanh(x @ W(c[0]).T + B(c[0])))
    h2 = _bf(np.tanh(h1 @ W(a[2]).T + B(a[2])))
    c2 = _bf(np.tanh(c1 @ W(c[2]).T + B(c[2])))
    logits = h2 @ W(a[4]).T + B(a[4])
    value = c2 @ c[4].weight.detach().double().cpu().numpy().ravel() + B(c[4])
    return logits, value


def _setup(gpu, obs_dim, n, seed, init="normal"):
    import torch
    P = import_pkg("policy")
    g = torch.Generator().manual_seed(seed)
    net = P.MLPActorCritic(obs_dim, init=init, generator=g).to(gpu)
    rng = np.random.default_rng(seed)
    obs = rng.normal(0.3, 2.0, (n, obs_dim)).astype(np.float32)
    obs[rng.random((n, obs_dim)) < 0.01] *= 40.0            # some values beyond the clip
    norm = P.RunningNorm(obs_dim, gpu)
    norm.mean.copy_(torch.as_tensor(rng.normal(0, 0.5, obs_dim).astype(np.float32)))
    norm.var.copy_(torch.as_tensor(rng.uniform(0.2, 3.0, obs_dim).astype(np.float32)))
    return P, net, torch.as_tensor(obs, device=gpu), norm


@pytest.mark.gpu
@pytest.mark.parametrize("obs_dim,init", [(184, "normal"), (184, "orthogonal"), (214, "normal")])
def test_policy_step_matches_reference(gpu, orc, obs_dim, init, worst):
    import torch
    n = 4096 + 37                                            # a ragged last tile
    P, net, obs, norm = _setup(gpu, obs_dim, n, 1, init)
    step = P.PolicyStep(obs_dim, device=gpu, seed=0)
    nobs = torch.empty(n, obs_dim, dtype=torch.float32, device=gpu)
    idx = torch.empty(n, 4, dtype=torch.int64, device=gpu)
    logp = torch.empty(n, dtype=torch.float32, device=gpu)
    val = torch.empty(n, dtype=torch.float32, device=gpu)
    acts = torch.full((n, 4), 9.0, dtype=torch.float64, device=gpu)
    logits = torch.empty(n, 84, dtype=torch.float32, device=gpu)
    step(obs, [(net, 0, n)], norm=norm, step=7, nobs_out=nobs, act_idx=idx, logp=logp, value=val,
         env_actions=acts, logits_out=logits)
    torch.cuda.synchronize()
    # normalisation: the reference's float32 expression
    o, mu, var = obs.cpu().numpy(), norm.mean.cpu().numpy(), norm.var.cpu().numpy()
    ref_n = np.clip((o - mu) / np.sqrt(var + np.float32(1e-8)), -10, 10).astype(np.float32)
    got_n = nobs.cpu().numpy()
    assert (np.abs(got_n - ref_n) <= np.spacing(np.abs(ref_n))).all()
    # MLP
    ref_l, ref_v = _ref_forward(net.cpu(), got_n)
    got_l, got_v = logits.cpu().numpy(), val.cpu().numpy()
    # one bf16 flip of a hidden activation moves a logit by ~2^-8 |w|: scale by the spread
    for name, got, ref in (("logits", got_l, ref_l), ("values", got_v, ref_v)):
        scale = max(1.0, float(np.std(ref)))
        err = np.abs(got - ref)
        worst(f"policy {name} |err| / max(1, std) ({obs_dim})", err.max() / scale, 5e-3)
        worst(f"policy {name} 99% quantile / max(1, std) ({obs_dim})",
              np.quantile(err, 0.99) / scale, 1e-4)
        assert err.max() < 5e-3 * scale
        assert np.quantile(err, 0.99) < 1e-4 * scale
    # draw: exact against the checker on the kernel's logits
    r_idx, r_lp = oracle_sample(orc, got_l, np.arange(n), seed=0, step=7)
    np.testing.assert_array_equal(idx.cpu().numpy(), r_idx)
    assert np.abs(logp.cpu().numpy() - r_lp).max() < 1e-5
    # controls: action_to_env of the drawn bins, float32 -> float64
    ref_a = P.action_to_env(idx.cpu(), 21).double().numpy()
    np.testing.assert_array_equal(acts.cpu().numpy(), ref_a)


@pytest.mark.gpu
def test_policy_groups_and_row_maps(gpu, orc):
    """Several networks in one launch over gathered rows equal one launch per network."""
    import torch
    n = 3000
    P, net0, obs, norm = _setup(gpu, 184, n, 2)
    net1 = P.MLPActorCritic(184, init="normal", generator=torch.Generator().manual_seed(3)).to(gpu)
    net2 = P.MLPActorCritic(184, init="orthogonal",
                            generator=torch.Generator().manual_seed(4)).to(gpu)
    perm = np.random.default_rng(4).permutation(n).astype(np.int32)
    rows = torch.as_tensor(perm, device=gpu)
    bounds = [(net0, 0, 1000), (net1, 1000, 1001), (net2, 1001, n)]
    step = P.PolicyStep(184, device=gpu, seed=11)
    out = {k: torch.empty(n, *s, dtype=d, device=gpu) for k, s, d in
           [("idx", (4,), torch.int64), ("lp", (), torch.float32), ("v", (), torch.float32),
            ("lg", (84,), torch.float32)]}
    acts = torch.zeros(n, 4, dtype=torch.float64, device=gpu)
    step(obs, bounds, norm=norm, rows=rows, step=2, salt=1, act_idx=out["idx"], logp=out["lp"],
         value=out["v"], env_actions=acts, logits_out=out["lg"])
    for net, b, e in bounds:
        sub = obs[rows[b:e].long()].contiguous()
        lg = torch.empty(e - b, 84, dtype=torch.float32, device=gpu)
        v = torch.empty(e - b, dtype=torch.float32, device=gpu)
        step(sub, [(net, 0, e - b)], norm=norm, logits_out=lg, value=v)
        torch.testing.assert_close(out["lg"][b:e], lg, rtol=0, atol=0)
        torch.testing.assert_close(out["v"][b:e], v, rtol=0, atol=0)
    # draws use the physical row in the counter
    r_idx, _ = oracle_sample(orc, out["lg"].cpu().numpy(), perm.astype(np.int64), seed=11, step=2,
                             salt=1)
    np.testing.assert_array_equal(out["idx"].cpu().numpy(), r_idx)
    ref_a = np.zeros((n, 4))
    ref_a[perm] = P.action_to_env(out["idx"].cpu(), 21).double().numpy()
    np.testing.assert_array_equal(acts.cpu().numpy(), ref_a)


@pytest.mark.gpu
def test_running_norm_update_matches_reference(gpu):
    """Three batch updates against the reference's float32 merge (ppo_gpu.py:194-207)."""
    import torch
    P = import_pkg("policy")
    norm = P.RunningNorm(184, gpu)
    mean = np.zeros(184, np.float32); var = np.ones(184, np.float32)
    count = np.float32(0) + np.float32(1e-4)
    rng = np.random.default_rng(5)
    for k in range(3):
        x = rng.normal(rng.normal(0, 2, 184), rng.uniform(0.1, 3, 184), (5000 + 999 * k, 184))
        x = x.astype(np.float32)
        norm.update(torch.as_tensor(x, device=gpu))
        bm = x.astype(np.float64).mean(0).astype(np.float32)
        bv = x.astype(np.float64).var(0).astype(np.float32)
        bc = np.float32(x.shape[0])
        delta = bm - mean
        tot = count + bc
        mean = mean + delta * (bc / tot)
        M2 = var * count + bv * bc + (delta * delta) * (count * bc / tot)
        var = M2 / tot
        count = tot
    np.testing.assert_allclose(norm.mean.cpu().numpy(), mean, rtol=2e-6, atol=1e-6)
    np.testing.assert_allclose(norm.var.cpu().numpy(), var, rtol=2e-6)
    assert float(norm.count) == float(count)
    # row-mapped update equals the update over the gathered rows
    n2 = P.RunningNorm(184, gpu)
    n3 = P.RunningNorm(184, gpu)
    X = torch.as_tensor(rng.normal(0, 1, (3000, 184)).astype(np.float32), device=gpu)
    rows = torch.arange(0, 3000, 2, dtype=torch.int32, device=gpu)
    n2.update(X, rows=rows)
    n3.update(X[0::2].contiguous())
    assert torch.equal(n2.mean, n3.mean) and torch.equal(n2.var, n3.var)


@pytest.mark.gpu
def test_policy_argument_errors(gpu):
    import torch
    P, net, obs, norm = _setup(gpu, 184, 64, 6)
    step = P.PolicyStep(184, device=gpu)
    with pytest.raises(ValueError):
        step(obs.double(), [(net, 0, 64)])
    with pytest.raises(ValueError):
        step(obs[:, :100], [(net, 0, 64)])
    with pytest.raises(ValueError):
        step(obs, [(net, 0, 64)] * 17)
    out = torch.empty(64, dtype=torch.float32, device=gpu)
    step(obs, [(net, 0, 0)], value=out)                       # empty range: no launch, no error
