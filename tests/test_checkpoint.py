"""Checkpoint and bundle formats (R/cuda_fdm/ppo_gpu.py:2815-2962 save/load,
claude_code/model.py:599-691 save_bundle/load_bundle, R/cuda_fdm/gpu_ckpt_to_bundle.py).

The bundle metadata is pinned by a golden written with the reference's own save_bundle
(tests/golden/make_bundle_golden.py); the weights file is the reference's gzip pickle of the
state_dict; the loader unpickles tensors only.  GPU: a checkpoint round-trips the updater's
parameters, Adam moments and step count, and its optimizer states load into torch.optim.Adam,
which then takes the same step as the updater."""
import gzip
import json
import os
import pickle

import numpy as np
import pytest
import torch

from conftest import ROOT, import_pkg

GOLDEN = os.path.join(ROOT, "tests", "golden")


def golden_inputs():
    g = np.load(os.path.join(GOLDEN, "bundle_norm_golden.npz"))
    obs_norm = {"mean": g["mean"].tolist(), "var": g["var"].tolist(), "count": float(g["count"])}
    meta = json.load(open(os.path.join(GOLDEN, "bundle_metadata_golden.json"), encoding="utf-8"))
    extra = {k: meta[k] for k in ("reward_module", "observation_module", "observation_mode",
                                  "selected_iteration", "source", "trainer",
                                  "observation_contract", "policy_hz", "action_repeat",
                                  "training_protocol", "auxiliary_trained",
                                  "auxiliary_contract")}
    return obs_norm, extra, meta


def test_bundle_metadata_matches_reference_writer(tmp_path):
    C, P = import_pkg("checkpoint"), import_pkg("policy")
    obs_norm, extra, meta = golden_inputs()
    net = P.MLPActorCritic(184)
    C.save_bundle(net, tmp_path, obs_norm=obs_norm, extra_metadata=extra)
    ours = json.loads((tmp_path / C.METADATA_FILENAME).read_text(encoding="utf-8"))
    assert ours == meta
    assert list(ours) == list(meta)                      # same key order as the reference


def test_bundle_weights_round_trip(tmp_path):
    C, P = import_pkg("checkpoint"), import_pkg("policy")
    torch.manual_seed(3)
    net = P.MLPActorCritic(184)
    C.save_bundle(net, tmp_path)
    with gzip.open(tmp_path / C.WEIGHTS_FILENAME, "rb") as fh:   # the reference's own reader
        plain = pickle.load(fh)
    sd = net.state_dict()
    assert list(plain) == list(sd)
    assert all(torch.equal(plain[k], sd[k]) for k in sd)
    net2, meta = C.load_bundle(tmp_path)
    assert all(torch.equal(net2.state_dict()[k], sd[k]) for k in sd)
    assert meta["model"]["type"] == "mlp_discrete_actor_critic"


def test_bundle_export_drops_the_aux_heads(tmp_path):
    """checkpoint_to_bundle on a checkpoint trained with the auxiliary heads (cfg aux_pred):
    the bundle holds the policy's tensors only, equal to the checkpoint's, and says it was
    trained with them; the same checkpoint claiming no aux training is refused."""
    C, P, F = import_pkg("checkpoint"), import_pkg("policy"), import_pkg("future_aux")
    torch.manual_seed(4)
    sd = P.MLPActorCritic(184).state_dict()
    heads = {"actor_aux_head.weight": torch.randn(6, 256), "actor_aux_head.bias": torch.randn(6),
             "critic_aux_head.weight": torch.randn(6, 256), "critic_aux_head.bias": torch.randn(6)}
    assert set(heads) == F.AUX_STATE_KEYS
    ck = {"model": {**sd, **heads}, "cfg": {"aux_pred": True, "num_bins": 21},
          "auxiliary_contract": F.AUX_CONTRACT, "iteration": 7}
    torch.save(ck, tmp_path / "aux.pt")
    C.checkpoint_to_bundle(tmp_path / "aux.pt", tmp_path / "bundle")
    net, meta = C.load_bundle(tmp_path / "bundle")
    assert list(net.state_dict()) == list(sd)
    assert all(torch.equal(net.state_dict()[k], sd[k]) for k in sd)
    assert meta["auxiliary_trained"] is True and meta["auxiliary_contract"] == F.AUX_CONTRACT
    ck["cfg"]["aux_pred"] = False
    torch.save(ck, tmp_path / "bad.pt")
    with pytest.raises(ValueError, match="auxiliary"):
        C.checkpoint_to_bundle(tmp_path / "bad.pt", tmp_path / "bundle2")


def test_bundle_loader_refuses_code(tmp_path):
    C, P = import_pkg("checkpoint"), import_pkg("policy")
    C.save_bundle(P.MLPActorCritic(184), tmp_path)

    class Evil:
        def __reduce__(self):
            return (os.getenv, ("HOME",))          # any callable outside the allow-list
    with gzip.open(tmp_path / C.WEIGHTS_FILENAME, "wb") as fh:
        pickle.dump({"actor_logits.0.weight": Evil()}, fh)
    with pytest.raises(pickle.UnpicklingError):
        C.load_bundle(tmp_path)


def test_adam_state_dict_helpers_cpu():
    """The exported optimizer state is torch's own Adam layout: loading it into a torch Adam and
    stepping equals stepping the original."""
    C = import_pkg("checkpoint")
    torch.manual_seed(0)
    ps = [torch.nn.Parameter(torch.randn(5, 3)), torch.nn.Parameter(torch.randn(3))]
    opt = torch.optim.Adam(ps, lr=3e-4, eps=1e-5)
    for _ in range(3):
        for p in ps:
            p.grad = torch.randn_like(p)
        opt.step()
    flat_m = torch.cat([opt.state[p]["exp_avg"].reshape(-1) for p in ps])
    flat_v = torch.cat([opt.state[p]["exp_avg_sq"].reshape(-1) for p in ps])
    sd = C._adam_state_dict(ps, flat_m, flat_v, 3, 3e-4)
    m2, v2 = torch.zeros_like(flat_m), torch.zeros_like(flat_v)
    assert C._load_adam_state_dict(sd, ps, m2, v2) == 3
    assert torch.equal(m2, flat_m) and torch.equal(v2, flat_v)
    ps2 = [torch.nn.Parameter(p.detach().clone()) for p in ps]
    opt2 = torch.optim.Adam(ps2, lr=3e-4, eps=1e-5)
    opt2.load_state_dict(sd)
    g = [torch.randn_like(p) for p in ps]
    for p, q, gg in zip(ps, ps2, g):
        p.grad, q.grad = gg.clone(), gg.clone()
    opt.step()
    opt2.step()
    assert all(torch.equal(p, q) for p, q in zip(ps, ps2))


@pytest.mark.gpu
def test_checkpoint_round_trip_and_torch_adam_resume(gpu, tmp_path):
    C, P, U = import_pkg("checkpoint"), import_pkg("policy"), import_pkg("ppo_update")
    torch.manual_seed(4)
    net = P.MLPActorCritic(184).to(gpu)
    up = U.PPOUpdater(net, U.UpdateConfig(lr=3e-4, critic_lr=1e-3))
    norm = P.RunningNorm(184, gpu)
    norm.mean.normal_(); norm.var.uniform_(0.5, 2.0); norm.count.fill_(777.0)
    gen = torch.Generator().manual_seed(1)
    for _ in range(3):
        up.grad.copy_((torch.randn(up.flat.numel(), generator=gen) * 1e-3).to(gpu))
        up.optimizer_step()
    path = C.save_checkpoint(tmp_path / "ck.pt", up, norm, global_step=123, iteration=4)
    net2 = P.MLPActorCritic(184).to(gpu)
    up2 = U.PPOUpdater(net2, U.UpdateConfig(lr=3e-4, critic_lr=1e-3))
    norm2 = P.RunningNorm(184, gpu)
    ck = C.load_checkpoint(path, up2, norm2)
    assert ck["global_step"] == 123 and ck["iteration"] == 4 and up2.steps == 3
    assert torch.equal(up2.flat, up.flat)
    assert torch.equal(up2.exp_avg, up.exp_avg) and torch.equal(up2.exp_avg_sq, up.exp_avg_sq)
    assert torch.equal(up2.wbf, up.wbf) and torch.equal(up2.wT, up.wT)
    assert torch.equal(norm2.mean, norm.mean) and float(norm2.count) == 777.0
    # the reference's optimizer resumes from the exported state and takes the updater's step
    na = up.na
    ref_ps = [torch.nn.Parameter(p.detach().cpu().clone()) for p in U.net_parameters(net)[:6]]
    ref = torch.optim.Adam(ref_ps, lr=3e-4, eps=1e-5)
    ref.load_state_dict(ck["actor_opt"])
    g = (torch.randn(up.flat.numel(), generator=gen) * 1e-4)
    up.grad.copy_(g.to(gpu))
    up.optimizer_step()                                     # small gradient: clip is 1
    off = 0
    for p in ref_ps:
        p.grad = g[off:off + p.numel()].view(p.shape).clone()
        off += p.numel()
    ref.step()
    got = up.flat[:na].cpu()
    want = torch.cat([p.detach().reshape(-1) for p in ref_ps])
    assert torch.allclose(got, want, rtol=1e-6, atol=1e-8)
    # checkpoint -> bundle (gpu_ckpt_to_bundle)
    b = C.checkpoint_to_bundle(path, tmp_path / "bundle")
    meta = json.loads((b / C.METADATA_FILENAME).read_text(encoding="utf-8"))
    assert meta["selected_iteration"] == 4 and meta["source"] == "gpu_ckpt_to_bundle:ck.pt"
    assert meta["obs_normalization"]["count"] == 777.0
    net3, _ = C.load_bundle(b)
    assert all(torch.equal(net3.state_dict()[k], v.cpu()) for k, v in ck["model"].items())


def _collector(gpu, kind, env_seed, graph):
    """A small collector of `kind` ("selfplay": BASELINE C4's shape; "league": C5's with the
    214-D observation, fuel exhaustion and three frozen opponents) whose env and learner are
    seeded by env_seed (the opponents are the league's fixed pool)."""
    E, P, R = import_pkg("rl_env").GpuDogfightVecEnv, import_pkg("policy"), import_pkg("ppo")
    mk = lambda d, s: P.MLPActorCritic(d, init="normal", init_std=0.05,
                                        generator=torch.Generator().manual_seed(s)).to(gpu)
    if kind == "selfplay":
        env = E(200, seed=env_seed, ic_pool_size=64, max_engage_time_s=2.0)
        return R.SelfPlayRollout(env, mk(184, env_seed), T=8, seed=0, stats=False, graph=graph)
    env = E(200, seed=env_seed, ic_pool_size=64, max_engage_time_s=2.0, obs_dim=214,
            fuel_exhaustion=True, fuel_lbs_range=(30.0, 3000.0))
    return R.LeagueRollout(env, mk(214, env_seed), [mk(214, 90 + k) for k in range(3)], T=8,
                           seed=0, graph=graph)


def _bits(t):
    return t.contiguous().view(torch.int32 if t.element_size() == 4 else
                               torch.int64 if t.element_size() == 8 else torch.uint8)


@pytest.mark.gpu
@pytest.mark.parametrize("kind,graph", [("selfplay", False), ("selfplay", True),
                                        ("league", False)])
def test_runtime_resume_is_bit_identical(gpu, tmp_path, kind, graph):
    """The checkpoint's runtime half (R/cuda_fdm/ppo_gpu.py:2859-2921): a run saved after two
    collect + update iterations and resumed into a fresh env, network, updater and collector --
    built with other seeds, so every value has to come from the file -- collects the next
    rollout bit for bit as the uninterrupted run does: observations, actions, log-probabilities,
    rewards, values, done flags, advantages, returns, and the simulator and reconstructor state
    after it (autoresets from the restored IC pool and its rebuilt tables, fuel exhaustion and
    opponent redraws included)."""
    C, U = import_pkg("checkpoint"), import_pkg("ppo_update")
    ro = _collector(gpu, kind, 5, graph)
    up = U.PPOUpdater(ro.net, U.UpdateConfig(target_kl=None, update_epochs=1), seed=3)
    ro.reset(stagger=True, max_stagger_steps=20)
    for _ in range(2):
        adv, ret, _ = ro.collect()
        up.update(ro, adv, ret)
    path = C.save_checkpoint(tmp_path / "run.pt", up, ro.norm, global_step=ro.global_step,
                             iteration=2, runtime=ro)
    adv, ret, _ = ro.collect()
    want = {n: getattr(ro, n).clone() for n in ("b_obs", "b_act", "b_logp", "b_rew", "b_val",
                                                "b_done", "next_done")}
    want.update(adv=adv.clone(), ret=ret.clone(), states=ro.env.sim.states.clone(),
                **{"obr_" + k: v for k, v in ro.env.obr.clone_state().items()})
    done = float(want["b_done"].sum())

    ro2 = _collector(gpu, kind, 17, graph)                  # other seeds everywhere
    up2 = U.PPOUpdater(ro2.net, U.UpdateConfig(target_kl=None, update_epochs=1), seed=11)
    ck = C.load_checkpoint(path, up2, ro2.norm, runtime=ro2)
    assert ck["global_step"] == ro2.global_step == ro.global_step - ro.T
    adv2, ret2, _ = ro2.collect()
    got = {n: getattr(ro2, n) for n in ("b_obs", "b_act", "b_logp", "b_rew", "b_val", "b_done",
                                        "next_done")}
    got.update(adv=adv2, ret=ret2, states=ro2.env.sim.states,
               **{"obr_" + k: v for k, v in ro2.env.obr.clone_state().items()})
    assert set(got) == set(want)
    for name in want:
        assert torch.equal(_bits(got[name]), _bits(want[name])), name
    assert done > 0                                          # autoresets inside the window
    # the restored updater draws the same minibatch permutation
    assert torch.equal(up2.permutation(64), up.permutation(64))


def test_runtime_state_round_trips_through_weights_only_load(tmp_path):
    """The runtime state is plain data: tensors, ints, floats, strings, dicts and lists only, so
    torch.load(weights_only=True) reads it back (numpy's generator state included)."""
    import numpy as np
    C = import_pkg("checkpoint")
    np.random.seed(12)
    saved = C._rng_np_to_saved(np.random.get_state())
    torch.save({"numpy_rng": saved}, tmp_path / "r.pt")
    back = torch.load(tmp_path / "r.pt", weights_only=True)["numpy_rng"]
    a = np.random.random(5)
    np.random.set_state(C._rng_np_from_saved(back))
    assert np.array_equal(np.random.random(5), a)
