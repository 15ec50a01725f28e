"""GPU: f16_norm_update_noalloc (the RunningNorm update with its workspace in the library's
fixed device array) against f16_norm_update (caller workspace), through the C ABI.

Two calls in a row, the second with a smaller batch and a row list, so the second call runs on
an array that still holds the first call's partial sums: the statistics must equal the
workspace entry point's bit for bit after each call.  A batch beyond the array is rejected with
F16_ETOOBIG before anything runs.
"""
import numpy as np
import pytest
import torch

from conftest import import_pkg

pytestmark = pytest.mark.gpu


def _state(gpu, dim, seed):
    g = torch.Generator().manual_seed(seed)
    mean = (torch.randn(dim, generator=g) * 0.5).to(gpu)
    var = (torch.rand(dim, generator=g) + 0.5).to(gpu)
    count = torch.tensor([1234.0], device=gpu)
    return mean, var, count


@pytest.mark.parametrize("dim", [184, 214])
def test_norm_update_noalloc_equals_workspace_entry(gpu, dim):
    L = import_pkg("_lib")
    lib = L.lib()
    g = torch.Generator().manual_seed(dim)
    x1 = (torch.randn(40000, dim, generator=g) * 3.0 + 1.0).to(gpu)
    x2 = (torch.randn(5000, dim + 6, generator=g) * 0.7 - 2.0).to(gpu)     # row stride > dim
    rows2 = torch.randperm(5000, generator=g)[:3001].to(torch.int32).to(gpu)
    a = _state(gpu, dim, 1)
    b = tuple(t.clone() for t in a)
    work = torch.empty(lib.f16_norm_workspace_bytes(40000, dim), dtype=torch.uint8, device=gpu)
    s = L.stream_handle(gpu)
    for x, rows, n in ((x1, None, 40000), (x2, rows2, 3001)):
        rc = lib.f16_norm_update(L.ptr(x), x.stride(0), L.ptr(rows), n, dim, L.ptr(a[0]),
                                 L.ptr(a[1]), L.ptr(a[2]), L.ptr(work), s)
        L.check(rc, "f16_norm_update")
        rc = lib.f16_norm_update_noalloc(L.ptr(x), x.stride(0), L.ptr(rows), n, dim,
                                         L.ptr(b[0]), L.ptr(b[1]), L.ptr(b[2]), s)
        L.check(rc, "f16_norm_update_noalloc")
        torch.cuda.synchronize()
        for u, v in zip(a, b):
            assert torch.equal(u, v), n
    # the statistics moved (the update did something) and follow the batch moments
    assert float(b[2]) == 1234.0 + 40000 + 3001


def test_norm_update_noalloc_rejects_beyond_its_array(gpu):
    L = import_pkg("_lib")
    lib = L.lib()
    cap = lib.f16_norm_noalloc_max_bytes()
    assert cap == 8 << 20
    dim = 214
    n_ok = 262144
    assert lib.f16_norm_workspace_bytes(n_ok, dim) <= cap
    n_big = n_ok * 2
    assert lib.f16_norm_workspace_bytes(n_big, dim) > cap
    mean, var, count = _state(gpu, dim, 3)
    keep = mean.clone()
    x = torch.zeros(1, dim, device=gpu)          # never read: the size check comes first
    rc = lib.f16_norm_update_noalloc(L.ptr(x), dim, None, n_big, dim, L.ptr(mean), L.ptr(var),
                                     L.ptr(count), L.stream_handle(gpu))
    assert rc == L.F16_ETOOBIG
    with pytest.raises(ValueError):
        L.check(rc, "f16_norm_update_noalloc")
    torch.cuda.synchronize()
    assert torch.equal(mean, keep) and float(count) == 1234.0
