"""Future-aux features and labels (R/cuda_fdm/future_aux.py; obs_kernel.cu:348-355).

CPU: the label oracle (oracle/future_aux_oracle.py) against closed forms -- a constant-velocity
trajectory has zero residual, a known extra displacement d gives R d / 100, episode starts
inside the horizon mask the label, a start at t itself does not.  GPU: f16_future_labels equals
the oracle; the observation kernels' features equal the state9 rows of both aircraft and satisfy
R R^T = I, det R = 1 and R v_ned = (u, v, w); the collectors record them per step."""
import importlib.util
import math
import os

import numpy as np
import pytest

from conftest import ROOT, import_pkg

_spec = importlib.util.spec_from_file_location("future_aux_oracle",
                                               os.path.join(ROOT, "oracle", "future_aux_oracle.py"))
FA = importlib.util.module_from_spec(_spec)
_spec.loader.exec_module(FA)


def rot(yaw, pitch, roll):
    cy, sy, cp, sp, cr, sr = (math.cos(yaw), math.sin(yaw), math.cos(pitch), math.sin(pitch),
                              math.cos(roll), math.sin(roll))
    return np.array([[cp * cy, cp * sy, -sp],
                     [sr * sp * cy - cr * sy, sr * sp * sy + cr * cy, sr * cp],
                     [cr * sp * cy + sr * sy, cr * sp * sy - sr * cy, cr * cp]])


def trajectory(T, nenv, dt, rng):
    """Constant-velocity straight flight for both aircraft, random attitude per step."""
    f = np.zeros((T, nenv, 21))
    for e in range(nenv):
        p0, v0 = rng.normal(0, 1000, 3), rng.normal(0, 200, 3)
        q0, w0 = rng.normal(0, 1000, 3), rng.normal(0, 200, 3)
        for t in range(T):
            f[t, e, 0:3], f[t, e, 3:6] = p0 + v0 * t * dt, v0
            f[t, e, 6:9], f[t, e, 9:12] = q0 + w0 * t * dt, w0
            f[t, e, 12:21] = rot(*rng.uniform(-3, 3, 3)).ravel()
    return f


def test_auxiliary_error_known_case():
    """Two rows, horizons (opponent, self): row 0 errs by (1, 2, 2) on the opponent horizon
    (squared 9) and by 1 on one self component (1), row 1 by 3 on every component (27 each);
    row 1's self horizon is masked.  sse = (9 + 27, 1), count = (6, 3), mse = 37 / 9.  A NaN
    prediction under a masked label still poisons the mean."""
    import torch
    F = import_pkg("future_aux")
    target = torch.zeros(2, 6, dtype=torch.float64)
    pred = torch.tensor([[1.0, 2.0, 2.0, 0.0, 1.0, 0.0], [3.0] * 6], dtype=torch.float64)
    mask = torch.tensor([[1.0, 1.0], [1.0, 0.0]], dtype=torch.float64)
    mse, sse, count = F.auxiliary_error(pred, target, mask)
    assert sse.tolist() == [36.0, 1.0] and count.tolist() == [6.0, 3.0]
    assert float(mse) == 37.0 / 9.0
    pred[1, 4] = float("nan")
    assert math.isnan(float(F.auxiliary_error(pred, target, mask)[0]))
    zero = F.auxiliary_error(pred[:0], target[:0], mask[:0])[0]
    assert float(zero) == 0.0                   # no unmasked element: divided by 1, not 0


def test_inference_state_dict_strips_exactly_the_aux_heads():
    """The four auxiliary-head tensors are dropped when the checkpoint says it trained them;
    present without that, absent with it, or one more head key all raise."""
    import torch
    F, P = import_pkg("future_aux"), import_pkg("policy")
    base = P.MLPActorCritic(184).state_dict()
    heads = {k: torch.zeros(1) for k in F.AUX_STATE_KEYS}
    out = F.inference_state_dict({**base, **heads}, enabled=True)
    assert list(out) == list(base)
    assert F.inference_state_dict(base).keys() == base.keys()
    for sd, enabled in (({**base, **heads}, False), (base, True),
                        ({**base, **heads, "actor_aux_head.scale": torch.zeros(1)}, True)):
        with pytest.raises(ValueError, match="auxiliary"):
            F.inference_state_dict(sd, enabled=enabled)


def test_oracle_closed_forms():
    rng = np.random.default_rng(0)
    T, nenv, dt = 24, 3, 0.1
    f = trajectory(T, nenv, dt, rng)
    starts = np.zeros((T, nenv))
    lab, mask = FA.future_labels(f, starts, dt)
    assert mask[:T - 5, :, 0].all() and not mask[T - 5:, :, 0].any()
    assert mask[:T - 10, :, 1].all() and not mask[T - 10:, :, 1].any()
    assert np.abs(lab).max() < 1e-6            # straight flight: nothing to predict
    # an extra displacement d of the partner at t = 12 shows in the label of t = 7 as R(7) d / 100
    d = np.array([30.0, -40.0, 50.0])
    g = f.copy()
    g[12, 1, 6:9] += d
    lab2, _ = FA.future_labels(g, starts, dt)
    want = g[7, 1, 12:21].reshape(3, 3) @ d / 100.0
    np.testing.assert_allclose(lab2[7, 1, 0:3], want, rtol=1e-6, atol=1e-6)
    # own displacement at t = 15 -> slot 1 of t = 5
    g = f.copy()
    g[15, 2, 0:3] += d
    lab3, _ = FA.future_labels(g, starts, dt)
    np.testing.assert_allclose(lab3[5, 2, 3:6], g[5, 2, 12:21].reshape(3, 3) @ d / 100.0,
                               rtol=1e-6, atol=1e-6)
    # episode starts: a start at s masks t in [s - h, s - 1]; a start at t itself does not
    starts[9, 0] = 1
    lab4, mask4 = FA.future_labels(f, starts, dt)
    assert not mask4[4:9, 0, 0].any() and mask4[3, 0, 0] and mask4[9, 0, 0]
    assert not mask4[0:9, 0, 1].any() and mask4[9, 0, 1]
    assert (lab4[~mask4.repeat(3, axis=-1)] == 0).all()


@pytest.mark.gpu
def test_labels_kernel_matches_oracle(gpu):
    import torch
    FX = import_pkg("future_aux")
    rng = np.random.default_rng(1)
    T, nenv, dt = 40, 37, 0.1
    f = trajectory(T, nenv, dt, rng) + rng.normal(0, 5, (T, nenv, 21)) * \
        np.r_[np.ones(12), np.zeros(9)]
    starts = (rng.random((T, nenv)) < 0.08).astype(np.float32)
    lab, mask = FX.build_future_labels(torch.as_tensor(f, device=gpu),
                                       torch.as_tensor(starts, device=gpu), dt)
    rl, rm = FA.future_labels(f, starts, dt)
    np.testing.assert_array_equal(mask.cpu().numpy(), rm)
    np.testing.assert_allclose(lab.cpu().numpy(), rl, rtol=1e-6, atol=1e-7)


@pytest.mark.gpu
def test_env_features_match_state9(gpu):
    import torch
    E = import_pkg("rl_env")
    env = E.GpuDogfightVecEnv(64, seed=3, ic_pool_size=64)
    env.enable_aux_capture()
    env.reset(stagger=True, max_stagger_steps=6)
    g = torch.Generator(device="cuda").manual_seed(0)
    for k in range(12):
        acts = torch.rand(env.nac, 4, generator=g, device=gpu, dtype=torch.float64) * 2 - 1
        acts[:, 3] = (acts[:, 3] + 1) / 2
        env.step(acts)
        torch.cuda.synchronize()
        aux = env.obr.aux_features.cpu().numpy()
        s9 = env.state9().cpu().numpy()                       # (nenv, 2, 9)
        np.testing.assert_array_equal(aux[:, 0:3], s9[:, 0, 0:3])
        np.testing.assert_array_equal(aux[:, 6:9], s9[:, 1, 0:3])
        R = aux[:, 12:21].reshape(-1, 3, 3)
        np.testing.assert_allclose(R @ R.transpose(0, 2, 1), np.broadcast_to(np.eye(3), R.shape),
                                   atol=1e-12)
        np.testing.assert_allclose(np.linalg.det(R), 1.0, atol=1e-12)
        uvw = np.einsum("eij,ej->ei", R, aux[:, 3:6])
        np.testing.assert_allclose(uvw, s9[:, 0, 6:9], rtol=1e-9, atol=1e-9)


@pytest.mark.gpu
def test_rollout_records_features_and_labels(gpu):
    import torch
    E, P, R = import_pkg("rl_env"), import_pkg("policy"), import_pkg("ppo")
    env = E.GpuDogfightVecEnv(64, seed=5, ic_pool_size=64)
    net = P.MLPActorCritic(184, init="normal", generator=torch.Generator().manual_seed(1)).to(gpu)
    ro = R.SelfPlayRollout(env, net, T=24, seed=0, stats=False, aux=True)
    ro.reset(stagger=True, max_stagger_steps=8)
    feats0 = env.obr.aux_features.clone()
    ro.collect()
    torch.cuda.synchronize()
    f = ro.b_aux_features.cpu().numpy()
    assert np.array_equal(f[0], feats0.cpu().numpy())
    rl, rm = FA.future_labels(f, ro.b_done.cpu().numpy(), env.obr.dt)
    np.testing.assert_array_equal(ro.b_aux_mask.cpu().numpy(), rm)
    np.testing.assert_allclose(ro.b_aux_labels.cpu().numpy(), rl, rtol=1e-6, atol=1e-7)
