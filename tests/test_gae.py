"""GAE: the CPU restatement (oracle/gae_oracle.py) pinned by the reference's known answers and
the closed form; the GPU kernel (f16_gae through the C ABI) bit-exact against it."""
import importlib.util
import os

import numpy as np
import pytest

from conftest import ROOT, import_pkg

_spec = importlib.util.spec_from_file_location("gae_oracle", os.path.join(ROOT, "oracle", "gae_oracle.py"))
G = importlib.util.module_from_spec(_spec)
_spec.loader.exec_module(G)


def boundary_case():
    """cuda_fdm/tests/time_limit_value_audit.py:26-92 BoundaryEnv with a critic that returns
    obs[:,0]: one step, lanes 0-2 end by timeout, lane 3 by destruction, lane 4 lives on."""
    rew = np.array([[5.0, -5.0, -4.0, 5.0, 1.0]], np.float32)
    val = np.full((1, 5), 2.0, np.float32)          # reset observation 2.0
    done = np.zeros((1, 5), np.float32)             # nothing done entering step 0
    last_val = np.array([100.0, 100.0, 100.0, 100.0, 10.0], np.float32)
    next_done = np.array([1, 1, 1, 1, 0], np.float32)
    return rew, val, done, last_val, next_done


def test_boundary_known_answer():
    adv, ret = G.gae_f32(*boundary_case(), gamma=0.997, lam=0.95)
    assert np.allclose(ret[0], [5.0, -5.0, -4.0, 5.0, 10.97], atol=2e-6)


def test_closed_form_small():
    """A_t = sum_k (gamma*lambda)^k (prod of nonterminal masks) delta_{t+k}, by brute force."""
    rng = np.random.default_rng(0)
    T, B, g, l = 7, 5, 0.99, 0.95
    rew = rng.normal(size=(T, B)); val = rng.normal(size=(T, B))
    done = (rng.random((T, B)) < 0.25).astype(np.float64); done[0] = 0
    lv = rng.normal(size=B); nd = (rng.random(B) < 0.3).astype(np.float64)
    vnext = np.vstack([val[1:], lv[None]]); nnt = 1.0 - np.vstack([done[1:], nd[None]])
    delta = rew + g * vnext * nnt - val
    want = np.zeros((T, B))
    for t in range(T):
        acc, w = 0.0, np.ones(B)
        for k in range(t, T):
            acc = acc + w * delta[k]
            w = w * g * l * nnt[k]
        want[t] = acc
    adv, ret = G.gae_f64(rew, val, done, lv, nd, g, l)
    assert np.allclose(adv, want, atol=1e-12)
    a32, _ = G.gae_f32(rew, val, done, lv, nd, g, l)
    assert np.allclose(a32, want, atol=1e-5)


@pytest.mark.gpu
def test_gpu_boundary_known_answer(gpu):
    import torch
    ppo = import_pkg("ppo")
    t = [torch.as_tensor(x, device=gpu) for x in boundary_case()]
    adv, ret = ppo.gae(*t, gamma=0.997, lam=0.95)
    assert np.allclose(ret.cpu().numpy()[0], [5.0, -5.0, -4.0, 5.0, 10.97], atol=2e-6)


@pytest.mark.gpu
@pytest.mark.parametrize("T,nenv,nag", [(64, 16384, 2), (13, 1000, 1), (1, 7, 2), (9, 33, 3),
                                         (16, 100, 2), (17, 65, 2), (128, 4096, 2),
                                         (256, 300, 2), (257, 70, 2), (300, 129, 1),
                                         (20, 32768, 2)])
def test_gpu_bit_exact(gpu, T, nenv, nag):
    """BASELINE C4 shape [64, 16384] x 2 agents plus ragged shapes (partial segments and
    column blocks, one to sixteen 16-step segments; past 256 steps or from 65,536 columns on,
    the chunked kernel);
    bit-exact vs the fp32 restatement, within 1e-5 of the float64 recurrence."""
    import torch
    ppo = import_pkg("ppo")
    rng = np.random.default_rng(T * 7 + nenv)
    rew = rng.normal(size=(T, nenv, nag)).astype(np.float32)
    val = rng.normal(size=(T, nenv, nag)).astype(np.float32)
    done = (rng.random((T, nenv)) < 0.05).astype(np.float32)
    lv = rng.normal(size=(nenv, nag)).astype(np.float32)
    nd = (rng.random(nenv) < 0.05).astype(np.float32)
    dev = lambda x: torch.as_tensor(x, device=gpu)
    adv, ret = ppo.gae(dev(rew), dev(val), dev(done), dev(lv), dev(nd), gamma=0.99, lam=0.95)
    a_ref, r_ref = G.gae_f32(rew.reshape(T, -1), val.reshape(T, -1), done, lv.reshape(-1), nd,
                             0.99, 0.95, nagents=nag)
    assert np.array_equal(adv.cpu().numpy().reshape(T, -1), a_ref)
    assert np.array_equal(ret.cpu().numpy().reshape(T, -1), r_ref)
    a64, _ = G.gae_f64(rew.reshape(T, -1), val.reshape(T, -1), done, lv.reshape(-1), nd,
                       0.99, 0.95, nagents=nag)
    scale = np.maximum(1.0, np.abs(a64))
    assert (np.abs(adv.cpu().numpy().reshape(T, -1) - a64) / scale).max() < 1e-5


@pytest.mark.gpu
def test_gpu_empty_and_errors(gpu):
    import torch
    ppo = import_pkg("ppo")
    z = torch.zeros(0, 4, dtype=torch.float32, device=gpu)
    adv, ret = ppo.gae(z, z, torch.zeros(0, 4, device=gpu), torch.zeros(4, device=gpu),
                       torch.zeros(4, device=gpu))
    assert adv.shape == (0, 4)
    with pytest.raises(TypeError):
        ppo.gae(z.double(), z, z, torch.zeros(4, device=gpu), torch.zeros(4, device=gpu))
