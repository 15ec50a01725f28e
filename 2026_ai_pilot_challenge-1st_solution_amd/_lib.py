"""ctypes binding of libf16hip.so (C ABI declared in include/f16_fdm.h, include/f16_obs.h,
include/f16_policy.h and include/f16_ppo.h).

torch is imported first so that the process's HIP runtime is torch's; the library then binds
to that same runtime (libamdhip64.so.7) and launches on torch's streams.  There is no CPU
fallback: if the library is missing or fails to load, every call raises.

Stream contract (cuda_fdm/tests/cuda_rt.py:107-139): each launch goes to the caller's current
stream with no synchronisation; data readiness across streams is the caller's (wait_stream), and
the tensors a launch touches are marked with `record` so their memory outlives the launch.
"""
import ctypes
import os

import torch  # noqa: F401  (loads the HIP runtime the library binds to)

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "libf16hip.so")

F16_EINVAL = -1
F16_ERATE = -2
F16_ETOOBIG = -3

_vp, _i, _l, _d = ctypes.c_void_p, ctypes.c_int, ctypes.c_long, ctypes.c_double


class F16Recon(ctypes.Structure):
    """include/f16_obs.h F16Recon: device pointers of the reconstructor buffers."""
    _fields_ = [("hp", _vp), ("fuel", _vp), ("t_sec", _vp), ("prev_att", _vp),
                ("prev_valid", _vp), ("pqr", _vp), ("dealt", _vp), ("taken", _vp),
                ("hp_loss", _vp), ("act_hist", _vp), ("prev_x", _vp), ("prev_x_valid", _vp),
                ("prev_alt_log", _vp), ("prev_vel_ned", _vp), ("accel", _vp), ("ld", _l),
                ("nenv", _i), ("aux", _vp)]


class F16RewardCfg(ctypes.Structure):
    """include/f16_obs.h F16RewardCfg."""
    _fields_ = [("own_damage_weight", _d), ("damage_scale", _d), ("shaping_reward_scale", _d),
                ("win_reward", _d), ("loss_reward", _d), ("timeout_win_reward", _d),
                ("timeout_loss_reward", _d), ("timeout_draw_reward", _d), ("min_alt_m", _d),
                ("max_time_s", _d), ("alt_hunt_coef", _d), ("mode", _i),
                ("fuel_exhaustion", _i)]


class F16EnvStepIO(ctypes.Structure):
    """include/f16_obs.h F16EnvStepIO."""
    _fields_ = [("states", _vp), ("ld", _l), ("actions", _vp), ("ic_pool", _vp),
                ("pool_size", _l), ("pick", _vp), ("seed", ctypes.c_ulonglong),
                ("step", ctypes.c_uint), ("obs_dim", _i), ("obs", _vp), ("terminal_obs", _vp),
                ("reward", _vp), ("reward_f32", _vp), ("term", _vp), ("trunc", _vp),
                ("done", _vp), ("done_f32", _vp), ("terminal_hp", _vp),
                ("terminal_alt_m", _vp), ("terminal_finite", _vp), ("finite_acc", _vp),
                ("opp_assign", _vp), ("opp_cdf", _vp), ("n_opp", _i), ("step_base", _vp),
                ("norm_partial", _vp), ("norm_count", _vp), ("norm_count_snap", _vp),
                ("state_finite", _vp), ("pool_obs", _vp), ("pool_prev_x", _vp),
                ("pool_prev_alt_log", _vp), ("pool_aux", _vp), ("reward0_f32", _vp)]


class F16FiniteSpan(ctypes.Structure):
    """include/f16_ppo.h F16FiniteSpan."""
    _fields_ = [("ptr", _vp), ("n", _l), ("elem_bytes", _i)]


class F16PolicyGroup(ctypes.Structure):
    """include/f16_policy.h F16PolicyGroup."""
    _fields_ = [("wbf", _vp), ("wf", _vp), ("mean", _vp), ("var", _vp), ("row_begin", _i),
                ("row_end", _i)]


class F16PolicyArgs(ctypes.Structure):
    """include/f16_policy.h F16PolicyArgs."""
    _fields_ = [("obs", _vp), ("obs_ld", _l), ("obs_dim", _i), ("mean", _vp), ("var", _vp),
                ("clip", ctypes.c_float), ("eps", ctypes.c_float), ("rows", _vp),
                ("ngroups", _i), ("group", F16PolicyGroup * 16), ("group_offsets", _vp),
                ("max_group_rows", _i), ("total_group_rows", _i), ("seed", ctypes.c_ulonglong),
                ("step", ctypes.c_uint), ("salt", ctypes.c_uint), ("deterministic", _i),
                ("grid", _vp), ("nobs_out", _vp), ("nobs_ld", _l), ("act_idx", _vp),
                ("logp", _vp), ("value", _vp), ("env_actions", _vp), ("logits_out", _vp),
                ("step_base", _vp)]


class F16PPOArgs(ctypes.Structure):
    """include/f16_ppo.h F16PPOArgs."""
    _fields_ = [("obs", _vp), ("obs_ld", _l), ("obs_dim", _i), ("act", _vp), ("old_logp", _vp),
                ("adv", _vp), ("ret", _vp), ("count", _l), ("idx", _vp), ("mb_rows", _i),
                ("clip_coef", ctypes.c_float), ("ent_coef", ctypes.c_float),
                ("vf_coef", ctypes.c_float), ("norm_adv", _i), ("wbf", _vp), ("wf", _vp),
                ("wT", _vp), ("grad", _vp), ("stats", _vp), ("work", _vp), ("adv_stats", _vp)]


class F16AdamArgs(ctypes.Structure):
    """include/f16_ppo.h F16AdamArgs."""
    _fields_ = [("obs_dim", _i), ("param", _vp), ("exp_avg", _vp), ("exp_avg_sq", _vp),
                ("grad", _vp), ("max_grad_norm", ctypes.c_float), ("actor_lr", _d),
                ("critic_lr", _d), ("beta1", _d), ("beta2", _d), ("eps", _d), ("step", _i),
                ("grad_norms", _vp), ("wbf", _vp), ("wf", _vp), ("wT", _vp), ("work", _vp)]


_RP, _CP = ctypes.POINTER(F16Recon), ctypes.POINTER(F16RewardCfg)
_SIGNATURES = {
    "f16_fdm_step_batch": (_i, [_vp, _l, _vp, _i, _i, _i, _vp, _l, _vp]),
    "f16_fdm_step_batch_finite": (_i, [_vp, _l, _vp, _i, _i, _i, _vp, _l, _vp, _vp]),
    "f16_fdm_step_batch_keep": (_i, [_vp, _l, _vp, _vp, _i, _i, _i, _vp, _l, _vp, _vp]),
    "f16_fdm_step_batch_onelane": (_i, [_vp, _l, _vp, _i, _i, _i, _vp, _l, _vp]),
    "f16_fdm_step_batch_split": (_i, [_vp, _l, _vp, _i, _i, _i, _vp, _l, _vp]),
    "f16_seed_batch": (_i, [_vp, _i, _i, _vp, _l, _vp, _vp]),
    "f16_fdm_kernel_info": (_i, [_i, ctypes.POINTER(_i)]),
    "f16_fdm_kernel_info_onelane": (_i, [_i, ctypes.POINTER(_i)]),
    "f16_fdm_step_batch_f32": (_i, [_vp, _l, _vp, _i, _i, _i, _vp, _l, _vp]),
    "f16_fdm_kernel_info_f32": (_i, [_i, ctypes.POINTER(_i)]),
    "f16_gae": (_i, [_vp, _vp, _vp, _vp, _vp, _i, _i, _i, ctypes.c_float, ctypes.c_float, _vp,
                     _vp, _vp]),
    "f16_obr_advance": (_i, [_vp, _l, _vp, _RP, _CP, _vp, _vp, _vp, _vp]),
    "f16_obr_init_reward": (_i, [_vp, _l, _vp, _RP, _vp]),
    "f16_obr_build_obs": (_i, [_vp, _l, _vp, _RP, _i, _vp, _vp]),
    "f16_env_post_step": (_i, [ctypes.POINTER(F16EnvStepIO), _RP, _CP, _vp]),
    "f16_env_post_step_onewave": (_i, [ctypes.POINTER(F16EnvStepIO), _RP, _CP, _vp]),
    "f16_env_step": (_i, [ctypes.POINTER(F16EnvStepIO), _RP, _CP, _vp, _i, _i, _vp, _vp]),
    "f16_env_step_tworole": (_i, [ctypes.POINTER(F16EnvStepIO), _RP, _CP, _vp, _i, _i, _vp, _vp]),
    "f16_env_post_step_norm_fusable": (_i, [_i, _i]),
    "f16_env_reseed": (_i, [ctypes.POINTER(F16EnvStepIO), _RP, _vp, _vp]),
    "f16_state9": (_i, [_vp, _l, _i, _vp, _vp]),
    "f16_future_labels": (_i, [_vp, _vp, _i, _i, _d, _vp, _vp, _vp]),
    "f16_policy_step": (_i, [ctypes.POINTER(F16PolicyArgs), _vp]),
    "f16_norm_workspace_bytes": (_l, [_i, _i]),
    "f16_abi_struct_sizes": (_i, [ctypes.POINTER(_l), _i]),
    "f16_group_rows": (_i, [_vp, _i, _i, _i, _i, _vp, _vp, _vp, _vp]),
    "f16_group_workspace_bytes": (_l, [_i]),
    "f16_norm_update": (_i, [_vp, _l, _vp, _i, _i, _vp, _vp, _vp, _vp, _vp]),
    "f16_norm_merge": (_i, [_i, _i, _vp, _vp, _vp, _vp]),
    "f16_norm_noalloc_max_bytes": (_l, []),
    "f16_norm_update_noalloc": (_i, [_vp, _l, _vp, _i, _i, _vp, _vp, _vp, _vp]),
    "f16_ppo_param_counts": (_i, [_i, ctypes.POINTER(_l)]),
    "f16_ppo_workspace_bytes": (_l, [_i, _i]),
    "f16_ppo_grad": (_i, [ctypes.POINTER(F16PPOArgs), _vp]),
    "f16_ppo_adam_step": (_i, [ctypes.POINTER(F16AdamArgs), _vp]),
    "f16_ppo_pack": (_i, [_vp, _i, _vp, _vp, _vp, _vp]),
    "f16_all_finite": (_i, [ctypes.POINTER(F16FiniteSpan), _i, _vp, _vp]),
    "f16_permutation": (_i, [_vp, _l, _vp, _vp]),
    "f16_ppo_adv_work_bytes": (_l, [_i, _i]),
    "f16_ppo_adv_stats": (_i, [_vp, _vp, _l, _l, _i, _i, _vp, _vp, _vp]),
}

_lib = None


def lib():
    """Load (once) and return the library; raise if it is not built."""
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise RuntimeError(
                f"{LIB_PATH} is missing: build it with __graft_entry__.build() or "
                "python -m <package>.build; there is no CPU fallback")
        L = ctypes.CDLL(LIB_PATH)
        for name, (res, args) in _SIGNATURES.items():
            fn = getattr(L, name)
            fn.restype = res
            fn.argtypes = args
        _lib = L
    return _lib


def exported_symbols():
    return sorted(_SIGNATURES)


def check(rc, what):
    """Map a C-ABI return code to the reference's error classes (cuda_rt.py:36-44)."""
    if rc == 0:
        return
    if rc == F16_EINVAL:
        raise ValueError(f"{what}: invalid size, stride or pointer")
    if rc == F16_ERATE:
        raise ValueError(f"{what}: unsupported FCS rate (120 or 60 Hz)")
    if rc == F16_ETOOBIG:
        raise ValueError(f"{what}: size exceeds the entry point's limit")
    raise RuntimeError(f"HIP error {-(rc + 1000)} in {what}")


def ptr(t):
    return ctypes.c_void_p(t.data_ptr()) if t is not None else None


def stream_handle(device=None):
    return ctypes.c_void_p(torch.cuda.current_stream(device).cuda_stream)


def launch_stream(device=None):
    """(stream, C handle) of the caller's current stream on `device`: every launch of this
    library goes there, and `record` marks its tensors as used on the same stream."""
    s = torch.cuda.current_stream(device)
    return s, ctypes.c_void_p(s.cuda_stream)


def record(stream, tensors):
    """The reference's lifetime contract (cuda_fdm/tests/cuda_rt.py:134-136): every tensor a
    launch reads or writes, temporaries included, is marked as used on the launch's stream
    (Tensor.record_stream), so torch's caching allocator does not hand its memory to another
    stream's allocation before that stream has passed the launch -- the case of a tensor
    allocated on one stream, handed to a launch on another and then dropped by its owner.

    The allocator keeps a block's recorded streams until the block is freed, so a record is
    made once per (tensor object, storage address, stream): a persistent buffer is recorded on
    its first launch on a stream, a fresh tensor on each call.  torch itself ignores a record
    on the stream the tensor was allocated on."""
    key = stream.cuda_stream
    for t in tensors:
        if t is None:
            continue
        tag = (key, t.data_ptr())
        seen = getattr(t, "_f16_streams", None)
        if seen is None:
            seen = set()
            t._f16_streams = seen
        elif tag in seen:
            continue
        t.record_stream(stream)
        seen.add(tag)


def record_owned(owner, stream, tensors):
    """record() for the buffers an object holds across launches (a simulator's state, a
    reconstructor's vectors): skipped while the stream and every buffer object are those of the
    owner's previous record.  The owner keeps these objects alive, and the allocator keeps a
    block's recorded streams until the block is freed, so the earlier record still holds; a
    replaced buffer (a new object) or another stream records again."""
    prev = owner.__dict__.get("_f16_owned")
    key = stream.cuda_stream
    if (prev is not None and prev[0] == key and len(prev[1]) == len(tensors)
            and all(a is b for a, b in zip(prev[1], tensors))):
        return
    record(stream, tensors)
    owner._f16_owned = (key, tensors)
