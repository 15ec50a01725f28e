"""The reference's stream and lifetime contract at the C ABI (cuda_fdm/tests/cuda_rt.py:107-139,
tested by cuda_fdm/tests/kernel_stream_val.py:46-71 and :147-186).

Every launch goes to the caller's current stream with no synchronisation, and every tensor a
launch reads or writes is marked as used on that stream (Tensor.record_stream), so torch's
caching allocator cannot hand its memory to another stream's allocation while the launch may
still read it.  The CPU tests check the record bookkeeping of _lib with stand-in tensors; the
GPU test runs the reference's three cases:
  1. a 64-step environment trace (a subset killed at step 3, another truncated at step 7) on a
     non-default stream equals the default-stream trace exactly;
  2. 20 times: a default-stream allocation borrowed by an observation launch on a delayed side
     stream, its Python owner deleted and the allocator pressed with same-size allocations
     filled with -12345 before the launch runs -- the observations equal the expected ones;
  3. a strided (nac, 101) input (its contiguous copy is made inside the wrapper) gives the same
     observations.
"""
from types import SimpleNamespace

import pytest

from conftest import import_pkg


class _FakeTensor:
    """Stand-in for a device tensor: counts record_stream calls (no GPU needed)."""

    def __init__(self, ptr):
        self.ptr, self.records = ptr, []

    def data_ptr(self):
        return self.ptr

    def record_stream(self, stream):
        self.records.append(stream.cuda_stream)


def test_record_marks_each_tensor_once_per_stream():
    L = import_pkg("_lib")
    s1, s2 = SimpleNamespace(cuda_stream=123456), SimpleNamespace(cuda_stream=654321)
    a, b = _FakeTensor(0x1000), _FakeTensor(0x2000)
    L.record(s1, (a, None, b))
    assert a.records == [123456] and b.records == [123456]
    L.record(s1, (a, b))                       # already recorded on this stream
    assert a.records == [123456] and b.records == [123456]
    L.record(s2, (a,))                         # another stream records again
    assert a.records == [123456, 654321] and b.records == [123456]
    a.ptr = 0x3000                             # new storage behind the same object
    L.record(s1, (a,))
    assert a.records == [123456, 654321, 123456]


def test_record_owned_follows_stream_and_buffer_objects():
    L = import_pkg("_lib")
    owner = SimpleNamespace()
    s1, s2 = SimpleNamespace(cuda_stream=1), SimpleNamespace(cuda_stream=2)
    x, y = _FakeTensor(0x10), _FakeTensor(0x20)
    L.record_owned(owner, s1, (x, y))
    L.record_owned(owner, s1, (x, y))
    assert x.records == [1] and y.records == [1]
    L.record_owned(owner, s2, (x, y))
    assert x.records == [1, 2] and y.records == [1, 2]
    z = _FakeTensor(0x30)                      # a replaced buffer is recorded
    L.record_owned(owner, s2, (x, z))
    assert z.records == [2] and x.records == [1, 2]


def _trace(env, initial, controls):
    """The reference's run_trace (kernel_stream_val.py:82-113): forced endings at steps 3 and
    7, every output, the states and the reconstructor per step."""
    import torch
    _restore(env, initial)
    rows = []
    for i, commands in enumerate(controls):
        if i == 3:
            env.obr.hp[::8] = 0.0                      # a subset dies, others continue
        if i == 7:
            env.obr.t_sec[1::8] = 201.0                # a distinct subset truncates
        obs, reward, done, info = env.step(commands)
        vals = [obs.reshape(-1).double(), reward.reshape(-1), done.double(),
                info["terminal_obs"].reshape(-1).double(), info["terminal_hp"].reshape(-1),
                info["terminal_state_finite"].double(), env.sim.states.reshape(-1)]
        vals += [v.reshape(-1).double() for v in env.obr.clone_state().values()]
        rows.append(torch.cat(vals))
    return torch.stack(rows)


def _snapshot(env):
    return dict(states=env.sim.states.clone(), obr=env.obr.clone_state(), obs=env._obs.clone(),
                post_steps=env._post_steps)


def _restore(env, snap):
    env.sim.states.copy_(snap["states"])
    env.obr.restore(snap["obr"])
    env._obs.copy_(snap["obs"])
    env._post_steps = snap["post_steps"]       # the in-kernel autoreset draws' counter


def _max_abs(a, b):
    """Largest |a - b| over finite entries; positions where either side is not finite must
    agree in their non-finite value class (the reference's finite_max_abs_error)."""
    import torch
    fa, fb = torch.isfinite(a), torch.isfinite(b)
    assert torch.equal(fa, fb)
    assert torch.equal(torch.isnan(a), torch.isnan(b))
    assert torch.equal(a[~fa & ~torch.isnan(a)], b[~fb & ~torch.isnan(b)])
    return float((a[fa] - b[fb]).abs().max()) if bool(fa.any()) else 0.0


@pytest.mark.gpu
def test_stream_and_lifetime_contract(gpu):
    import torch
    E = import_pkg("rl_env").GpuDogfightVecEnv
    env = E(32, seed=271, ic_pool_size=128)
    env.reset(stagger=False)
    env._ensure_ic_pool()
    g = torch.Generator(device=gpu).manual_seed(81)
    controls = torch.rand(64, env.nac, 4, device=gpu, dtype=torch.float64, generator=g)
    controls[:, :, :3] = (controls[:, :, :3] - 0.5) * 0.2
    controls[:, :, 3] = 0.6 + 0.2 * controls[:, :, 3]
    initial = _snapshot(env)
    print("stream contract: default-stream trace, 32 engagements x 64 steps", flush=True)
    reference = _trace(env, initial, controls)
    torch.cuda.synchronize()
    done_steps = int(reference[:, 2 * 32 * 184 + 64:2 * 32 * 184 + 96].sum())
    assert done_steps > 0                              # the forced endings happened

    # 1. the same trace on a non-default stream
    print("stream contract: side-stream trace", flush=True)
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        side_trace = _trace(env, initial, controls)
    side.synchronize()
    assert _max_abs(reference, side_trace) == 0.0

    # 2. a default-stream allocation borrowed on a delayed side stream, its owner deleted,
    #    the allocator pressed before the launch runs
    print("stream contract: borrowed allocation under allocator pressure x 20", flush=True)
    _restore(env, initial)
    expected = env.obr.kernel_build_obs(env.sim.states).clone()
    default = torch.cuda.current_stream()
    pressure = None
    for rep in range(20):
        borrowed = env.sim.states.clone()
        assert borrowed.stride() == env.sim.states.stride()   # used in place by the launch
        side.wait_stream(default)
        with torch.cuda.stream(side):
            torch.cuda._sleep(1000000)
            actual = env.obr.kernel_build_obs(borrowed).clone()
        del borrowed
        for _ in range(4):
            pressure = torch.empty_like(env.sim.states).fill_(-12345.0)
        side.synchronize()
        assert _max_abs(actual, expected) == 0.0, rep
    del pressure

    # 3. a strided input: the wrapper's contiguous copy stays alive until the launch ran
    print("stream contract: strided input", flush=True)
    wide = torch.empty(env.nac, 202, device=gpu, dtype=torch.float64)
    wide[:, ::2] = env.sim.states
    strided = env.obr.kernel_build_obs(wide[:, ::2]).clone()
    assert _max_abs(strided, expected) == 0.0
