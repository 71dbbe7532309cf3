"""GPU test of lx_ReduceSum_noalloc, the allocation-free variant of lx_ReduceSum: through the C ABI, on
two calls in a row (the second with a smaller input), its output equals lx_ReduceSum's bit for bit (the
same kernels in the same order; only the partials and intermediates live in the static scratch array),
and reductions whose intermediates exceed the array fail before launching anything."""
import ctypes

import numpy as np
import pytest

from onnx_amd import DeviceTensor, HipExecutionProvider as HIP, OpStatus
from onnx_amd import _lib as L

pytestmark = pytest.mark.gpu


def noalloc(x, axes, keepdims, out):
    a = np.asarray(axes if axes is not None else [], np.int64)
    arr = (ctypes.c_int64 * max(1, a.size))(*a.tolist())
    n = -1 if axes is None else int(a.size)
    return L.lib().lx_ReduceSum_noalloc(ctypes.byref(x.h), arr, n, keepdims, -1, ctypes.byref(out.h))


def reference(x, axes, keepdims):
    r = HIP.ReduceSum(x, axes, keepdims)
    assert r.Status == OpStatus.Success, r.Message
    return r.Outputs[0].to_numpy()


def make(rng, shape, dt):
    if np.issubdtype(dt, np.integer):
        return rng.integers(-(2**20), 2**20, shape).astype(dt)
    return rng.uniform(-1, 1, shape).astype(dt)


# (dtype, axes, keepdims, first shape, second (smaller) shape)
CASES = [
    (np.float32, [1], 1, (64, 2048, 256), (8, 512, 256)),     # strided axis, split partials (1 MiB)
    (np.float32, None, 1, (1 << 22,), (1 << 18,)),            # whole tensor: long-row split
    (np.float32, [-1], 0, (4096, 768), (100, 768)),           # last axis, one wave per row (no scratch)
    (np.int64, [1, 3], 1, (6, 40, 33, 8), (3, 10, 7, 4)),     # two passes: an intermediate in a scratch slot
    (np.int32, [0, 2], 0, (16, 300, 64), (5, 17, 16)),        # two passes, wrapping int32
    (np.float64, [1], 1, (32, 5000, 6), (2, 3, 6)),           # double, odd inner
    # few column tiles split over many row slices: the planner caps the partials at the scratch's 2 MiB
    (np.float32, [1], 1, (255, 1024, 256), (3, 64, 256)),
    (np.float32, [1], 1, (200, 2048, 256), (7, 100, 256)),
    (np.float32, [1], 1, (300, 512, 255), (5, 40, 255)),      # unaligned rows: single-element tiles
]


@pytest.mark.parametrize("dt,axes,keep,big,small", CASES)
def test_noalloc_equals_reduce_sum_twice(hip, dt, axes, keep, big, small):
    rng = np.random.default_rng(11)
    for shape in (big, small):
        x = DeviceTensor.from_numpy(make(rng, shape, dt))
        want = reference(x, axes, keep)
        out = DeviceTensor.empty(want.shape, dt)
        print(f"noalloc {np.dtype(dt).name} {shape} axes {axes}", flush=True)
        st = noalloc(x, axes, keep, out)
        assert st == L.OK, L.last_error()
        got = out.to_numpy()
        assert got.shape == want.shape
        assert np.array_equal(got.view(np.uint8), want.view(np.uint8)), (shape, np.abs(got - want).max())


def test_noalloc_rejects_what_does_not_fit(hip):
    rng = np.random.default_rng(12)
    # first pass (axis 2) leaves a [2, 2^19] float intermediate: 4 MiB, beyond a 1 MiB scratch slot
    x = DeviceTensor.from_numpy(make(rng, (2, 1 << 19, 2), np.float32))
    out = DeviceTensor.from_numpy(np.full((1, 1 << 19, 1), 7.0, np.float32))
    assert noalloc(x, [0, 2], 1, out) == L.ERR_NOT_SUPPORTED
    assert "scratch" in L.last_error()
    assert np.all(out.to_numpy() == 7.0)   # nothing was launched
    # no caller storage: refused (the variant never allocates an output)
    empty = L.LxTensor()
    a = (ctypes.c_int64 * 1)(1)
    assert L.lib().lx_ReduceSum_noalloc(ctypes.byref(x.h), a, 1, 1, -1, ctypes.byref(empty)) == L.ERR_INVALID_ARGUMENT
    # too small caller storage (the [2, 1, 2] output needs 16 bytes): the ordinary capacity error
    tiny = DeviceTensor.empty((3,), np.float32)
    assert noalloc(x, [1], 1, tiny) == L.ERR_BUFFER_TOO_SMALL
    # and a call that fits still works afterwards
    y = DeviceTensor.from_numpy(make(rng, (4, 1000, 8), np.float32))
    want = reference(y, [1], 1)
    o = DeviceTensor.empty(want.shape, np.float32)
    assert noalloc(y, [1], 1, o) == L.OK
    assert np.array_equal(o.to_numpy(), want)


def test_noalloc_makes_no_pool_allocation(hip):
    """The pool's live bytes do not change across allocation-free calls (every block they use is the
    caller's or the static array)."""
    rng = np.random.default_rng(13)
    x = DeviceTensor.from_numpy(make(rng, (6, 40, 33, 8), np.int64))
    want = reference(x, [1, 3], 1)
    out = DeviceTensor.empty(want.shape, np.int64)
    live0, cached0 = ctypes.c_int64(), ctypes.c_int64()
    L.lib().lx_pool_stats(ctypes.byref(live0), ctypes.byref(cached0))
    for _ in range(3):
        assert noalloc(x, [1, 3], 1, out) == L.OK
    live1, cached1 = ctypes.c_int64(), ctypes.c_int64()
    L.lib().lx_pool_stats(ctypes.byref(live1), ctypes.byref(cached1))
    assert (live1.value, cached1.value) == (live0.value, cached0.value)
    assert np.array_equal(out.to_numpy(), want)
