"""Future-aux training labels (R/cuda_fdm/future_aux.py): short-horizon position residuals of the
two aircraft, never policy observations.

Features (float64, plane 0's perspective, written by the observation kernels when
``BatchObsReward.enable_aux_capture()`` is on): own NED position [m] and NED velocity [m/s], the
partner's, own NED-to-body rotation row-major.  Labels: the partner 5 steps ahead and own 10
steps ahead, minus the constant-velocity prediction, in the current own body frame, / 100 m;
masked across episode starts and past the rollout's end (``f16_future_labels``, one lane per
engagement).
"""
import torch

from . import _lib

AUX_FEATURE_DIM = 21
AUX_DIM = 6
AUX_OPP_H = 5
AUX_SELF_H = 10
AUX_POS_SCALE_M = 100.0
# checkpoint metadata identifying this label construction (R/cuda_fdm/future_aux.py:16-17)
AUX_PROTOCOL = "cuda_mlp_flat_finite_horizon_future_aux_diverse_h3_reset_v8"
AUX_CONTRACT = "main_body_cv_residual_opp5_self10_scale100_v1"
# the auxiliary prediction heads' tensors: trained, never deployed (R/cuda_fdm/future_aux.py:18-19)
AUX_STATE_KEYS = frozenset(("actor_aux_head.weight", "actor_aux_head.bias",
                            "critic_aux_head.weight", "critic_aux_head.bias"))


def auxiliary_error(prediction, target, mask):
    """Masked mean squared error of (rows, 6) predictions against the labels, with the (rows, 2)
    per-horizon mask (R/cuda_fdm/future_aux.py:58-67): returns (mse, sse, count), sse and count
    the per-horizon sums of squared errors and of masked elements (3 per unmasked horizon).
    Non-finite predictions are not filtered: a NaN under a masked label still reaches the loss,
    so a finite check downstream catches it."""
    err = (prediction - target).reshape(-1, 2, 3)
    per_h = (err * err).sum(-1)                     # (rows, 2) squared error per horizon
    sse = (per_h * mask).sum(0)
    count = mask.sum(0).to(sse.dtype) * 3.0
    return sse.sum() / torch.clamp(count.sum(), min=1.0), sse, count


def inference_state_dict(state_dict, enabled=False):
    """The state_dict without the auxiliary heads (R/cuda_fdm/future_aux.py:70-75): with
    `enabled` (the checkpoint was trained with them) exactly AUX_STATE_KEYS must be present, else
    none of the heads' keys may be; any other combination raises ValueError."""
    heads = {k for k in state_dict if k.startswith(("actor_aux_head.", "critic_aux_head."))}
    if heads != (AUX_STATE_KEYS if enabled else frozenset()):
        raise ValueError("checkpoint auxiliary metadata and prediction-head keys disagree")
    return {k: v for k, v in state_dict.items() if k not in AUX_STATE_KEYS}


@torch.no_grad()
def build_future_labels(features, episode_starts, dt):
    """features (T, nenv, 21) float64 device tensor; episode_starts (T, nenv) (the done flag
    entering each step); dt the decision interval [s].  Returns labels (T, nenv, 6) float32 and
    mask (T, nenv, 2) bool, as future_aux.py:29-55."""
    if features.dim() != 3 or features.shape[-1] != AUX_FEATURE_DIM:
        raise ValueError("auxiliary features must have shape (T, environments, 21)")
    if tuple(episode_starts.shape) != tuple(features.shape[:2]) or not (float(dt) > 0.0):
        raise ValueError("invalid auxiliary episode shape or control interval")
    T, nenv = features.shape[:2]
    dev = features.device
    labels = torch.empty(T, nenv, AUX_DIM, dtype=torch.float32, device=dev)
    mask = torch.empty(T, nenv, 2, dtype=torch.uint8, device=dev)
    labels_into(features, episode_starts, dt, labels, mask)
    return labels, mask.bool()


def labels_into(features, episode_starts, dt, labels, mask_u8):
    """build_future_labels into given buffers (labels float32 (T, nenv, 6), mask uint8
    (T, nenv, 2)); no allocation when the inputs are already float64 / float32 contiguous."""
    dev = features.device
    f = features if features.dtype == torch.float64 and features.is_contiguous() else \
        features.to(torch.float64).contiguous()
    starts = episode_starts if (episode_starts.dtype == torch.float32 and
                                episode_starts.is_contiguous()) else \
        episode_starts.to(device=dev, dtype=torch.float32).contiguous()
    T, nenv = f.shape[:2]
    stream, h = _lib.launch_stream(dev)
    rc = _lib.lib().f16_future_labels(_lib.ptr(f), _lib.ptr(starts), T, nenv, float(dt),
                                      _lib.ptr(labels), _lib.ptr(mask_u8), h)
    _lib.record(stream, (f, starts, labels, mask_u8))
    _lib.check(rc, "f16_future_labels")
