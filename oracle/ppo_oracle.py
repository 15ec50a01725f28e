"""CPU restatement of the reference learner's MLP PPO update (research/competition_36500/runtime/
cuda_fdm/ppo_gpu.py:2019-2145, PPOGPUTrainer.update) for the discrete actor-critic of
claude_code/model.py:162-241.  TEST INFRASTRUCTURE ONLY (imported by tests/ and bench.py's CPU
leg); torch on the CPU in float32.

Three pieces:
  reference_minibatch  -- one minibatch as the reference computes it: torch autograd through
                          Categorical(logits).log_prob/entropy, the clipped surrogate, the value
                          loss (ppo_gpu.py:2059-2109), in float32;
  mirror_minibatch     -- the same gradients by hand (log-softmax, tanh and linear-layer backward
                          formulas), optionally rounding to bfloat16 exactly where the GPU kernels
                          do (layer inputs, weights, hidden activations, the logits' and hidden
                          layers' gradients).  With rounding off it must equal reference_minibatch
                          (that pins the hand-written backward on autograd); with rounding on it is
                          the checker of f16_ppo_grad;
  reference_update     -- the epoch/minibatch loop with clip_grad_norm_ and torch.optim.Adam
                          (eps 1e-5, separate actor and critic optimizers, KL early stop at epoch
                          end, ppo_gpu.py:2054-2118) over given permutations.
Flat parameter layout (the reference's actor_parameters() then critic_parameters() order):
  actor  W1 [256][D] b1 [256] W2 [256][256] b2 [256] W3 [84][256] b3 [84]
  critic W1 [256][D] b1 [256] W2 [256][256] b2 [256] w3 [1][256] b3 [1]
"""
import math

import torch

H = 256
NL = 84
BINS = 21
CH = 4


def shapes(D):
    a = [("W1", (H, D)), ("b1", (H,)), ("W2", (H, H)), ("b2", (H,)), ("W3", (NL, H)), ("b3", (NL,))]
    c = [("W1", (H, D)), ("b1", (H,)), ("W2", (H, H)), ("b2", (H,)), ("W3", (1, H)), ("b3", (1,))]
    return a, c


def counts(D):
    a, c = shapes(D)
    return (sum(math.prod(s) for _, s in a), sum(math.prod(s) for _, s in c))


def unflatten(flat, D):
    """flat (n_actor + n_critic) -> (actor dict, critic dict) of views."""
    a, c = shapes(D)
    out, off = [], 0
    for group in (a, c):
        d = {}
        for name, s in group:
            n = math.prod(s)
            d[name] = flat[off:off + n].view(s)
            off += n
        out.append(d)
    return out[0], out[1]


def _mlp(p, x, out_act=False):
    h1 = torch.tanh(x @ p["W1"].T + p["b1"])
    h2 = torch.tanh(h1 @ p["W2"].T + p["b2"])
    return h2 @ p["W3"].T + p["b3"]


def _adv(adv, norm_adv):
    # ppo_gpu.py:2074-2078: sample std; a singleton is not normalised
    if norm_adv and adv.numel() > 1:
        return (adv - adv.mean()) / (adv.std() + 1e-8)
    return adv


def reference_minibatch(flat, D, obs, act, old_logp, adv, ret, clip=0.2, ent_coef=0.0,
                        vf_coef=0.5, norm_adv=True):
    """Autograd gradients (flat) and statistics of one minibatch, float32 (ppo_gpu.py:2059-2109)."""
    flat = flat.detach().clone().requires_grad_(True)
    pa, pc = unflatten(flat, D)
    logits = _mlp(pa, obs).view(-1, CH, BINS)
    dist = torch.distributions.Categorical(logits=logits)
    new_logp = dist.log_prob(act.long()).sum(-1)
    entropy = dist.entropy().sum(-1)
    log_ratio = new_logp - old_logp
    ratio = log_ratio.exp()
    A = _adv(adv, norm_adv)
    pg1 = -A * ratio
    pg2 = -A * torch.clamp(ratio, 1 - clip, 1 + clip)
    policy_loss = torch.max(pg1, pg2).mean()
    ent = entropy.mean()
    actor_loss = policy_loss - ent_coef * ent
    new_value = _mlp(pc, obs).squeeze(-1)
    value_loss = 0.5 * ((new_value - ret) ** 2).mean()
    critic_loss = vf_coef * value_loss
    (actor_loss + critic_loss).backward()     # the two networks share no parameter
    with torch.no_grad():
        stats = {"loss": float(actor_loss + critic_loss),
                 "pl": float(policy_loss), "vl": float(value_loss), "ent": float(ent),
                 "kl": float(((ratio - 1.0) - log_ratio).mean()),
                 "cf": float(((ratio - 1.0).abs() > clip).float().mean()),
                 "ratio": ratio.detach().clone(), "new_logp": new_logp.detach().clone()}
    return flat.grad.detach().clone(), stats


def _bf(x, on):
    return x.to(torch.bfloat16).to(torch.float32) if on else x


def mirror_minibatch(flat, D, obs, act, old_logp, adv, ret, clip=0.2, ent_coef=0.0, vf_coef=0.5,
                     norm_adv=True, bf16=True):
    """Hand-written forward/backward of one minibatch.  Returns (flat gradient, stats)."""
    with torch.no_grad():
        pa, pc = unflatten(flat.detach().float(), D)
        M = obs.shape[0]
        x = _bf(obs.float(), bf16)
        out = torch.zeros_like(flat, dtype=torch.float32)
        ga, gc = unflatten(out, D)
        # ---- actor
        W1, W2, W3 = (_bf(pa[k], bf16) for k in ("W1", "W2", "W3"))
        h1 = _bf(torch.tanh(x @ W1.T + pa["b1"]), bf16)
        h2 = _bf(torch.tanh(h1 @ W2.T + pa["b2"]), bf16)
        z = (h2 @ W3.T + pa["b3"]).view(M, CH, BINS)
        lsm = z - torch.logsumexp(z, dim=-1, keepdim=True)
        p = lsm.exp()
        a = act.long()
        new_logp = lsm.gather(-1, a.unsqueeze(-1)).squeeze(-1).sum(-1)
        hc = -(p * lsm).sum(-1)                                   # per-channel entropy
        entropy = hc.sum(-1)
        log_ratio = new_logp - old_logp
        ratio = log_ratio.exp()
        A = _adv(adv.float(), norm_adv)
        lo, hi = 1 - clip, 1 + clip
        rc = torch.clamp(ratio, lo, hi)
        pg1, pg2 = -A * ratio, -A * rc
        inr = ((ratio >= lo) & (ratio <= hi)).float()
        dr = torch.where(pg1 > pg2, -A, torch.where(pg1 < pg2, -A * inr, 0.5 * -A + 0.5 * (-A * inr)))
        gcoef = dr * ratio / M                                   # d loss / d new_logp
        onehot = torch.nn.functional.one_hot(a, BINS).float()
        dz = gcoef[:, None, None] * (onehot - p) + (ent_coef / M) * p * (lsm + hc[..., None])
        dz = _bf(dz.reshape(M, NL), bf16)
        dh2 = _bf((dz @ W3) * (1 - h2 * h2), bf16)
        dh1 = _bf((dh2 @ W2) * (1 - h1 * h1), bf16)
        ga["W3"].copy_(dz.T @ h2); ga["b3"].copy_(dz.sum(0))
        ga["W2"].copy_(dh2.T @ h1); ga["b2"].copy_(dh2.sum(0))
        ga["W1"].copy_(dh1.T @ x); ga["b1"].copy_(dh1.sum(0))
        # ---- critic (its head stays float32 in the kernels' f32 blob)
        C1, C2 = _bf(pc["W1"], bf16), _bf(pc["W2"], bf16)
        c1 = _bf(torch.tanh(x @ C1.T + pc["b1"]), bf16)
        c2 = _bf(torch.tanh(c1 @ C2.T + pc["b2"]), bf16)
        v = (c2 @ pc["W3"].T + pc["b3"]).squeeze(-1)
        err = v - ret.float()
        dv = vf_coef * err / M
        gc["W3"].copy_((dv @ c2)[None]); gc["b3"].copy_(dv.sum()[None])
        dc2 = _bf(dv[:, None] * pc["W3"][0][None] * (1 - c2 * c2), bf16)
        dc1 = _bf((dc2 @ C2) * (1 - c1 * c1), bf16)
        gc["W2"].copy_(dc2.T @ c1); gc["b2"].copy_(dc2.sum(0))
        gc["W1"].copy_(dc1.T @ x); gc["b1"].copy_(dc1.sum(0))
        stats = {"pl": float(torch.max(pg1, pg2).mean()), "vl": float(0.5 * (err * err).mean()),
                 "ent": float(entropy.mean()), "kl": float(((ratio - 1) - log_ratio).mean()),
                 "cf": float(((ratio - 1).abs() > clip).float().mean()), "ratio": ratio,
                 "new_logp": new_logp}
    return out, stats


class ReferenceOptim:
    """clip_grad_norm_ + torch.optim.Adam(eps=1e-5) per network, as ppo_gpu.py:1303-1304,
    2088-2090, 2103-2105 apply them."""

    def __init__(self, flat, D, lr=3e-4, critic_lr=None, max_grad_norm=0.5):
        self.D = D
        self.flat = flat.detach().clone().float()
        na, _ = counts(D)
        self.na = na
        self.pa = torch.nn.Parameter(self.flat[:na].clone())
        self.pc = torch.nn.Parameter(self.flat[na:].clone())
        self.oa = torch.optim.Adam([self.pa], lr=lr, eps=1e-5)
        self.oc = torch.optim.Adam([self.pc], lr=critic_lr if critic_lr is not None else lr,
                                   eps=1e-5)
        self.max_grad_norm = max_grad_norm

    def params(self):
        return torch.cat([self.pa.detach(), self.pc.detach()])

    def step(self, grad):
        """One optimizer step of each network from the flat gradient; returns the two norms."""
        na = self.na
        self.oa.zero_grad(set_to_none=True)
        self.pa.grad = grad[:na].clone()
        ga = torch.nn.utils.clip_grad_norm_([self.pa], self.max_grad_norm)
        self.oa.step()
        self.oc.zero_grad(set_to_none=True)
        self.pc.grad = grad[na:].clone()
        gc = torch.nn.utils.clip_grad_norm_([self.pc], self.max_grad_norm)
        self.oc.step()
        return float(ga), float(gc)


def reference_update(flat, D, obs, act, logp, adv, ret, perms, mb_size, clip=0.2, ent_coef=0.0,
                     vf_coef=0.5, norm_adv=True, lr=3e-4, critic_lr=None, max_grad_norm=0.5,
                     target_kl=0.03, bf16=True):
    """The update loop over given per-epoch permutations (ppo_gpu.py:2054-2118) with the mirrored
    minibatch gradients.  Returns (final flat params, result dict)."""
    opt = ReferenceOptim(flat, D, lr, critic_lr, max_grad_norm)
    count = obs.shape[0]
    epoch, early, steps, last, norms = 0, False, 0, None, (0.0, 0.0)
    last_kl = 0.0
    for epoch, perm in enumerate(perms):
        kls = []
        for s in range(0, count, mb_size):
            mb = perm[s:s + mb_size]
            g, st = mirror_minibatch(opt.params(), D, obs[mb], act[mb], logp[mb], adv[mb], ret[mb],
                                     clip, ent_coef, vf_coef, norm_adv, bf16)
            norms = opt.step(g)
            steps += 1
            kls.append(st["kl"])
            last = st
        last_kl = float(torch.tensor(kls, dtype=torch.float32).mean())
        if target_kl is not None and last_kl > target_kl:
            early = True
            break
    res = {"pl": last["pl"], "vl": last["vl"], "ent": last["ent"], "kl": last_kl, "cf": last["cf"],
           "epochs": epoch + 1, "early": early, "optimizer_steps": steps,
           "actor_grad_norm": norms[0], "critic_grad_norm": norms[1]}
    return opt.params(), res
