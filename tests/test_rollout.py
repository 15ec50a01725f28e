"""GPU: the self-play rollout collector (BASELINE C4 sequence) end to end.

The pieces are each checked against the reference elsewhere (physics, observation/reward, policy
step, GAE); here the wiring: every buffer row is what the step that wrote it consumed.
  * b_act / b_logp are the draws of the policy evaluated on b_obs[t] at counter step t
    (re-evaluated from the stored normalised observations, draws checked by the CPU checker);
  * the controls sent to the physics are action_to_env of the last draws;
  * b_done[t] is the done flag entering step t; adv/ret are GAE of the buffers (float32 checker);
  * two collectors from the same seeds produce identical buffers.
"""
import importlib.util
import os

import numpy as np
import pytest
import torch

from conftest import ROOT, import_pkg
from test_policy import oracle_sample

_spec = importlib.util.spec_from_file_location("gae_oracle", os.path.join(ROOT, "oracle", "gae_oracle.py"))
GO = importlib.util.module_from_spec(_spec)
_spec.loader.exec_module(GO)

pytestmark = pytest.mark.gpu


def _collector(gpu, nenv=256, T=12, seed=3):
    E = import_pkg("rl_env").GpuDogfightVecEnv
    P = import_pkg("policy")
    R = import_pkg("ppo")
    env = E(nenv, seed=seed, ic_pool_size=64)
    net = P.MLPActorCritic(184, init="normal", generator=torch.Generator().manual_seed(seed)).to(gpu)
    ro = R.SelfPlayRollout(env, net, T=T, gamma=0.99, lam=0.95, seed=0)
    ro.reset(stagger=True, max_stagger_steps=8)
    return ro


def test_rollout_buffers_consistent(gpu, orc):
    ro = _collector(gpu)
    T, nac, nenv = ro.T, ro.nac, ro.nenv
    g0 = ro.global_step
    adv, ret, stats = ro.collect()
    torch.cuda.synchronize()
    assert bool(stats["trajectory_finite"])
    P = import_pkg("policy")
    step = P.PolicyStep(184, device=gpu, seed=0)
    for t in range(T):
        lg = torch.empty(nac, 84, dtype=torch.float32, device=gpu)
        v = torch.empty(nac, dtype=torch.float32, device=gpu)
        step(ro.b_obs[t], [(ro.net, 0, nac)], norm=None, logits_out=lg, value=v)
        assert torch.equal(v, ro.b_val[t]), t
        idx, lp = oracle_sample(orc, lg.cpu().numpy(), np.arange(nac), seed=0, step=g0 + t)
        np.testing.assert_array_equal(ro.b_act[t].cpu().numpy(), idx)
        assert np.abs(ro.b_logp[t].cpu().numpy() - lp).max() < 1e-5
    last = P.action_to_env(ro.b_act[T - 1].cpu(), 21).double()
    np.testing.assert_array_equal(ro.env.sim.actions.cpu().numpy(), last.numpy())
    # normalised observations are clipped to +-10
    assert float(ro.b_obs.abs().max()) <= 10.0
    # GAE of the buffers, (T, nac) columns with the done flag shared by the 2 planes
    ref_adv, ref_ret = GO.gae_f32(ro.b_rew.cpu().numpy(), ro.b_val.cpu().numpy(),
                                  ro.b_done.cpu().numpy(), ro.last_val.cpu().numpy(),
                                  ro.next_done.cpu().numpy(), 0.99, 0.95, nagents=2)
    np.testing.assert_array_equal(adv.reshape(T, nac).cpu().numpy(), ref_adv)
    np.testing.assert_array_equal(ret.reshape(T, nac).cpu().numpy(), ref_ret)


def test_rollout_deterministic(gpu):
    a, b = _collector(gpu, nenv=128, T=6), _collector(gpu, nenv=128, T=6)
    ra, rb = a.collect(), b.collect()
    for name in ("b_obs", "b_act", "b_logp", "b_rew", "b_val", "b_done"):
        assert torch.equal(getattr(a, name), getattr(b, name)), name
    assert torch.equal(ra[0], rb[0]) and torch.equal(ra[1], rb[1])
