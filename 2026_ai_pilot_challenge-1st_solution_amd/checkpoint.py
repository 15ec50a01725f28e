"""Checkpoints and submission bundles in the reference's formats.

* ``save_checkpoint`` / ``load_checkpoint``: the learner's part of PPOGPUTrainer.save / load
  (R/cuda_fdm/ppo_gpu.py:2815-2862, 2922-2962) -- ``model`` (the MLP's state_dict under the
  reference's parameter names), ``actor_opt`` / ``critic_opt`` (torch.optim.Adam state_dicts,
  built by a real torch Adam so the reference's trainer can load them), ``norm`` (RunningNorm
  mean/var/count), ``global_step``, ``iteration``, ``cfg``.  Written atomically (temp + rename)
  after a finite check, as the reference does; read with ``torch.load(weights_only=True)``.
* ``save_bundle`` / ``load_bundle``: the two-file bundle of claude_code/model.py:599-691
  (``metadata.json`` + gzip-pickled CPU state_dict ``policy_weights.pkl.gz``).  ``load_bundle``
  unpickles through an allow-list (plain containers and torch tensors only), never arbitrary
  code.
* ``checkpoint_to_bundle``: R/cuda_fdm/gpu_ckpt_to_bundle.py for the 184-D MLP checkpoint.
* ``runtime_state`` / ``restore_runtime``: the trainer's runtime half of the checkpoint
  (R/cuda_fdm/ppo_gpu.py:2859-2921 ``_runtime_state`` / ``_restore_runtime``): simulator states,
  actions and 17-value output, the reconstructor, the IC pool, the env's generators and draw
  counter, the collector's next observation/done, step counter and episode bookkeeping, the
  league's opponent assignment, the updater's minibatch generator, and the process RNGs, so
  that a run resumed from the checkpoint collects exactly what the uninterrupted run does.
  ``save_checkpoint(..., runtime=collector)`` stores it under ``runtime``;
  ``load_checkpoint(..., runtime=collector)`` restores it.
"""
import gzip
import io
import json
import math
import os
import pickle
from pathlib import Path

import numpy as np
import torch

from . import future_aux as _future_aux
from . import policy as _policy

WEIGHTS_FILENAME = "policy_weights.pkl.gz"
METADATA_FILENAME = "metadata.json"
# the observation contract string the reference's bundles carry (claude_code/
# observation_contract.py:14): the submission provider rebuilds observations by it
CUDA_OBSERVATION_CONTRACT = "cuda_claude164r_command_poststep_v1"
ACTION_LOW = [-1.0, -1.0, -1.0, 0.0]     # claude_code/model.py:566-567 SIM_ACTION_LOW/HIGH
ACTION_HIGH = [1.0, 1.0, 1.0, 1.0]


def _require_finite(obj, what):
    """Every tensor / float inside `obj` finite (cuda_fdm/finite_checks.py require_finite)."""
    def walk(x, path):
        if torch.is_tensor(x):
            if x.is_floating_point() and not bool(torch.isfinite(x).all()):
                raise FloatingPointError(f"{what}: non-finite values in {path}")
        elif isinstance(x, float):
            if not math.isfinite(x):
                raise FloatingPointError(f"{what}: non-finite value at {path}")
        elif isinstance(x, dict):
            for k, v in x.items():
                walk(v, f"{path}.{k}")
        elif isinstance(x, (list, tuple)):
            for i, v in enumerate(x):
                walk(v, f"{path}[{i}]")
    walk(obj, what)


# ---- torch.optim.Adam state_dicts <-> the updater's flat moments
def _adam_state_dict(params, m, v, steps, lr):
    """A real torch.optim.Adam over CPU copies of `params`, its moments set from the flat views:
    the state_dict has exactly this torch's Adam layout (param_groups + per-parameter state)."""
    cpu = [torch.nn.Parameter(p.detach().cpu().clone()) for p in params]
    opt = torch.optim.Adam(cpu, lr=lr, eps=1e-5)
    if steps > 0:
        off = 0
        for p in cpu:
            n = p.numel()
            opt.state[p] = {"step": torch.tensor(float(steps)),
                            "exp_avg": m[off:off + n].detach().cpu().view(p.shape).clone(),
                            "exp_avg_sq": v[off:off + n].detach().cpu().view(p.shape).clone()}
            off += n
    return opt.state_dict()


def _load_adam_state_dict(sd, params, m, v):
    """Moments of a torch.optim.Adam state_dict into the flat views; returns its step count."""
    cpu = [torch.nn.Parameter(p.detach().cpu().clone()) for p in params]
    opt = torch.optim.Adam(cpu, lr=1e-3, eps=1e-5)
    opt.load_state_dict(sd)
    steps, off = 0, 0
    for p in cpu:
        n = p.numel()
        st = opt.state.get(p, {})
        if st:
            m[off:off + n].copy_(st["exp_avg"].reshape(-1).to(m.device))
            v[off:off + n].copy_(st["exp_avg_sq"].reshape(-1).to(v.device))
            steps = int(float(st["step"]))
        else:
            m[off:off + n].zero_()
            v[off:off + n].zero_()
        off += n
    return steps


def _split_params(updater):
    from .ppo_update import net_parameters
    ps = net_parameters(updater.net)
    return ps[:6], ps[6:]


# ---- runtime state (R/cuda_fdm/ppo_gpu.py:2859-2921)
def _rng_np_to_saved(state):
    """np.random.get_state() as plain data (torch.load(weights_only=True) reads no numpy)."""
    name, keys, pos, has_gauss, cached = state
    return {"name": name, "keys": torch.as_tensor(np.asarray(keys, dtype=np.int64)),
            "pos": int(pos), "has_gauss": int(has_gauss), "cached_gaussian": float(cached)}


def _rng_np_from_saved(d):
    return (d["name"], d["keys"].numpy().astype(np.uint32), int(d["pos"]), int(d["has_gauss"]),
            float(d["cached_gaussian"]))


def runtime_state(collector, updater=None):
    """Everything a collector (SelfPlayRollout / LeagueRollout) and its env carry from one
    rollout to the next, as plain CPU tensors and Python data (the reference's _runtime_state
    plus what this build's device-side draws key on: the env's post-physics step counter and
    the collector's step counter)."""
    env, sim, obr = collector.env, collector.env.sim, collector.env.obr
    cpu = lambda t: t.detach().cpu().clone()
    st = {
        "sim": {"states": cpu(sim.states), "obs": cpu(sim.obs), "actions": cpu(sim.actions)},
        "obr": {k: cpu(v) for k, v in obr.clone_state().items()},
        "env": {"obs": cpu(env._obs), "ic_pool": None if env.ic_pool is None else cpu(env.ic_pool),
                "post_steps": int(env._post_steps), "seed": int(env.seed),
                "rng": env.rng.bit_generator.state,
                "torch_gen": env.torch_gen.get_state().cpu().clone(),
                "reward_mode": int(env.reward_mode), "alt_hunt_coef": float(env.alt_hunt_coef),
                "opp_assign": None if env.opp_assign is None else cpu(env.opp_assign),
                "opp_cdf": None if env.opp_cdf is None else cpu(env.opp_cdf),
                "obs_dim": int(env.OBS_SIZE), "nenv": int(env.nenv)},
        "trainer": {"next_done": cpu(collector.next_done),
                    "global_step": int(collector.global_step),
                    "has_next_obs": collector.next_obs is not None,
                    "norm": {k: cpu(v) for k, v in collector.norm.state_dict().items()}},
        "numpy_rng": _rng_np_to_saved(np.random.get_state()),
        "torch_rng": torch.get_rng_state(),
        "cuda_rng": (torch.cuda.get_rng_state(env.device) if env.device.type == "cuda"
                     else None)}
    for name in ("ep_ret", "ep_len"):
        if hasattr(collector, name):
            st["trainer"][name] = cpu(getattr(collector, name))
    if hasattr(collector, "opp_norms"):
        st["trainer"]["opp_norms"] = [{k: cpu(v) for k, v in n.state_dict().items()}
                                      for n in collector.opp_norms]
    if updater is not None:
        st["updater_gen"] = updater.gen.get_state().cpu().clone()
    _require_finite({"sim": st["sim"], "obr": st["obr"]}, "runtime state")
    return st


def restore_runtime(collector, state, updater=None):
    """Restore a runtime_state into a collector built with the same sizes (the reference's
    _restore_runtime): every buffer is written in place, so launches recorded in a HIP graph
    keep their addresses; the IC pool is replaced, which rebuilds its autoreset tables."""
    env, sim, obr = collector.env, collector.env.sim, collector.env.obr
    e = state["env"]
    if e["nenv"] != env.nenv or e["obs_dim"] != env.OBS_SIZE:
        raise ValueError("runtime environment count or observation width mismatch")
    _require_finite({"sim": state["sim"], "obr": state["obr"]}, "restored runtime")
    dev = env.device
    sim.states.copy_(state["sim"]["states"])
    sim.obs.copy_(state["sim"]["obs"])
    sim.actions.copy_(state["sim"]["actions"])
    if "external_accel" in state["obr"]:
        obr.enable_external_observations()
    if "aux_features" in state["obr"]:
        env.enable_aux_capture()
    obr.restore({k: v.to(dev) for k, v in state["obr"].items()})
    env._obs.copy_(e["obs"])
    env.ic_pool = None if e["ic_pool"] is None else e["ic_pool"].to(dev).contiguous()
    env._post_steps = int(e["post_steps"])
    env.seed = int(e["seed"])
    env.rng.bit_generator.state = e["rng"]
    env.torch_gen.set_state(e["torch_gen"])
    from .obs_reward import validate_reward_mode
    env.reward_mode = validate_reward_mode(e["reward_mode"], e["alt_hunt_coef"])
    env.alt_hunt_coef = float(e["alt_hunt_coef"])
    if e["opp_assign"] is not None:
        if env.opp_assign is None or env.opp_assign.shape != e["opp_assign"].shape:
            raise ValueError("runtime league assignment does not match the collector")
        env.opp_assign.copy_(e["opp_assign"])
        env.opp_cdf.copy_(e["opp_cdf"])
    t = state["trainer"]
    collector.next_done.copy_(t["next_done"])
    collector.global_step = int(t["global_step"])
    collector.next_obs = env._obs.view(env.nac, env.OBS_SIZE) if t["has_next_obs"] else None
    collector.norm.load_state_dict({k: v.to(dev) for k, v in t["norm"].items()})
    for name in ("ep_ret", "ep_len"):
        if name in t and hasattr(collector, name):
            getattr(collector, name).copy_(t[name])
    if "opp_norms" in t and hasattr(collector, "opp_norms"):
        for n, sd in zip(collector.opp_norms, t["opp_norms"]):
            n.load_state_dict({k: v.to(dev) for k, v in sd.items()})
    if updater is not None and "updater_gen" in state:
        updater.gen.set_state(state["updater_gen"])
    np.random.set_state(_rng_np_from_saved(state["numpy_rng"]))
    torch.set_rng_state(state["torch_rng"])
    if state.get("cuda_rng") is not None and env.device.type == "cuda":
        torch.cuda.set_rng_state(state["cuda_rng"], env.device)


def save_checkpoint(path, updater, norm=None, global_step=0, iteration=0, extra=None,
                    runtime=None):
    """The learner's checkpoint (model, both Adam states, norm, counters, cfg); with
    `runtime` (a collector), also its runtime state under "runtime" (ppo_gpu.py:2845-2846)."""
    from dataclasses import asdict
    actor, critic = _split_params(updater)
    na = updater.na
    cfg = asdict(updater.cfg)
    ckpt = {"model": {k: v.detach().cpu().clone() for k, v in updater.net.state_dict().items()},
            "actor_opt": _adam_state_dict(actor, updater.exp_avg[:na], updater.exp_avg_sq[:na],
                                          updater.steps, updater.cfg.lr),
            "critic_opt": _adam_state_dict(critic, updater.exp_avg[na:], updater.exp_avg_sq[na:],
                                           updater.steps,
                                           updater.cfg.lr if updater.cfg.critic_lr is None
                                           else updater.cfg.critic_lr),
            "norm": ({k: v.detach().cpu().clone() for k, v in norm.state_dict().items()}
                     if norm is not None else None),
            "global_step": int(global_step), "iteration": int(iteration), "cfg": cfg}
    if extra:
        ckpt.update(extra)
    if runtime is not None:
        ckpt["runtime"] = runtime_state(runtime, updater)
    _require_finite({k: ckpt[k] for k in ("model", "actor_opt", "critic_opt", "norm")},
                    "checkpoint learner")
    path = Path(path)
    path.parent.mkdir(parents=True, exist_ok=True)
    temp = path.with_suffix(path.suffix + ".tmp")
    torch.save(ckpt, temp)
    os.replace(temp, path)
    return path


def load_checkpoint(path, updater, norm=None, runtime=None):
    """Restore a checkpoint written by save_checkpoint (or the reference's, when its extra entries
    are plain data): parameters (through the flat master copy), Adam moments and step count,
    RunningNorm; with `runtime` (a collector of the same sizes) and a stored runtime state, the
    collector, its env and the RNGs too.  Returns the checkpoint dict."""
    ckpt = torch.load(path, map_location="cpu", weights_only=True)
    _require_finite({k: ckpt.get(k) for k in ("model", "actor_opt", "critic_opt", "norm")},
                    "loaded checkpoint")
    with torch.no_grad():
        updater.net.load_state_dict(ckpt["model"])        # copies into the flat master buffer
    actor, critic = _split_params(updater)
    na = updater.na
    sa = _load_adam_state_dict(ckpt["actor_opt"], actor, updater.exp_avg[:na],
                               updater.exp_avg_sq[:na])
    sc = _load_adam_state_dict(ckpt["critic_opt"], critic, updater.exp_avg[na:],
                               updater.exp_avg_sq[na:])
    if sa != sc:
        raise ValueError("actor and critic optimizers have different step counts")
    updater.steps = sa
    updater.pack()
    if norm is not None and ckpt.get("norm") is not None:
        norm.load_state_dict({k: v.to(norm.device) for k, v in ckpt["norm"].items()})
    if runtime is not None:
        if ckpt.get("runtime") is None:
            raise ValueError("checkpoint holds no runtime state")
        restore_runtime(runtime, ckpt["runtime"], updater)
    return ckpt


# ---- bundles (claude_code/model.py:599-691)
def save_bundle(net, output_dir, obs_norm=None, extra_metadata=None):
    """metadata.json + policy_weights.pkl.gz for the discrete MLP actor-critic."""
    out = Path(output_dir)
    out.mkdir(parents=True, exist_ok=True)
    metadata = {
        "framework": "claude_code_ppo",
        "algorithm": "PPO",
        "observation_mode": "tactical16",
        "observation_size": int(net.obs_dim),
        "action_size": int(net.act_dim),
        "recurrent": False,
        "recurrent_type": None,
        "model": {"type": "mlp_discrete_actor_critic", "hidden": list(net.hidden),
                  "activation": net.activation, "critic_hidden": list(net.hidden),
                  "critic_activation": net.activation, "num_bins": int(net.num_bins)},
        "throttle_remap": "(a+1)/2",
        "action_clip": {"low": list(ACTION_LOW), "high": list(ACTION_HIGH)},
        "obs_normalization": obs_norm,
    }
    if extra_metadata:
        metadata.update(extra_metadata)
    (out / METADATA_FILENAME).write_text(json.dumps(metadata, indent=2, ensure_ascii=False),
                                         encoding="utf-8")
    state = {k: v.detach().cpu() for k, v in net.state_dict().items()}
    with gzip.open(out / WEIGHTS_FILENAME, "wb") as fh:
        pickle.dump(state, fh, protocol=pickle.HIGHEST_PROTOCOL)
    return out


def _storage_from_bytes(b):
    return torch.load(io.BytesIO(b), weights_only=True)


class _TensorUnpickler(pickle.Unpickler):
    """Unpickles dicts/lists of torch tensors and nothing else: find_class resolves only the
    tensor-rebuilding entry points (storages re-read with weights_only=True)."""
    _ALLOWED = {("collections", "OrderedDict"), ("torch._utils", "_rebuild_tensor_v2"),
                ("torch._utils", "_rebuild_parameter"), ("torch", "Size")}

    def find_class(self, module, name):
        if (module, name) == ("torch.storage", "_load_from_bytes"):
            return _storage_from_bytes
        if (module, name) in self._ALLOWED:
            return super().find_class(module, name)
        if module == "torch" and name.endswith("Storage"):
            return super().find_class(module, name)
        raise pickle.UnpicklingError(f"bundle weights may hold only tensors, not {module}.{name}")


def load_bundle(bundle_dir, device="cpu"):
    """(MLPActorCritic, metadata) from a bundle directory (claude_code/model.py:655-691)."""
    bundle = Path(bundle_dir)
    metadata = json.loads((bundle / METADATA_FILENAME).read_text(encoding="utf-8"))
    with gzip.open(bundle / WEIGHTS_FILENAME, "rb") as fh:
        state = _TensorUnpickler(fh).load()
    mm = metadata.get("model", {})
    if mm.get("type") != "mlp_discrete_actor_critic":
        raise ValueError(f"unsupported bundle model type {mm.get('type')!r}")
    net = _policy.MLPActorCritic(int(metadata.get("observation_size", 184)),
                                 act_dim=int(metadata.get("action_size", 4)),
                                 num_bins=int(mm.get("num_bins", 21)),
                                 hidden=tuple(mm.get("hidden", (256, 256))),
                                 activation=mm.get("activation", "tanh"))
    net.load_state_dict(state)
    return net.to(device).eval(), metadata


def obs_norm_from_checkpoint(norm):
    """RunningNorm state -> the bundle's obs_normalization (gpu_ckpt_to_bundle.py:77-91)."""
    if not norm:
        return None
    f = lambda x: x.detach().cpu().double() if torch.is_tensor(x) else torch.as_tensor(x).double()
    return {"mean": f(norm["mean"]).tolist(), "var": f(norm["var"]).tolist(),
            "count": float(f(norm["count"]))}


def checkpoint_to_bundle(ckpt_path, output_dir, observation_module="claude_code.my_observation",
                         reward_module="claude_code.my_reward"):
    """gpu_ckpt_to_bundle.py:110-192 for this build's 184-D MLP checkpoints."""
    ckpt_path = Path(ckpt_path)
    ckpt = torch.load(ckpt_path, map_location="cpu", weights_only=True)
    if "model" not in ckpt:
        raise KeyError(f"{ckpt_path} is not a PPO trainer checkpoint (no 'model' key)")
    _require_finite(ckpt["model"], "export.model")
    if ckpt.get("norm") is not None:
        _require_finite(ckpt["norm"], "export.normalization")
    cfg = ckpt.get("cfg") or {}
    # the auxiliary prediction heads teach the trunk and are never deployed: exactly their four
    # tensors are dropped (gpu_ckpt_to_bundle.py:129-131); other unexpected keys still fail the
    # strict load below
    sd = _future_aux.inference_state_dict(ckpt["model"], enabled=bool(cfg.get("aux_pred", False)))
    if observation_module != "claude_code.my_observation":
        raise ValueError("bundle export supports only the 184D training observation contract")
    obs_dim = int(sd["actor_logits.0.weight"].shape[1])
    head = sd["actor_logits.4.weight"]
    num_bins = int(cfg.get("num_bins", head.shape[0] // 4))
    act_dim = head.shape[0] // num_bins
    if obs_dim != 184 or act_dim != 4:
        raise ValueError("the submission contract requires 184 observations and 4 controls")
    net = _policy.MLPActorCritic(obs_dim)
    net.load_state_dict(sd, strict=True)
    return save_bundle(net, output_dir, obs_norm=obs_norm_from_checkpoint(ckpt.get("norm")),
                       extra_metadata={
                           "reward_module": reward_module,
                           "observation_module": observation_module,
                           "observation_mode": "claude164r",
                           "selected_iteration": int(ckpt.get("iteration", -1)),
                           "source": f"gpu_ckpt_to_bundle:{ckpt_path.name}",
                           "trainer": "cuda_fdm.PPOGPUTrainer",
                           "observation_contract": CUDA_OBSERVATION_CONTRACT,
                           "policy_hz": 10,
                           "action_repeat": 6,
                           "training_protocol": ckpt.get("training_protocol",
                                                         "legacy_mid_episode_pool_v1"),
                           "auxiliary_trained": bool(cfg.get("aux_pred", False)),
                           "auxiliary_contract": ckpt.get("auxiliary_contract"),
                       })
