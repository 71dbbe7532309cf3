"""GPU parity of the data-movement operators (lx_Transpose, lx_Concat,
lx_Gather, lx_Slice) against the oracle's restatement of Tensor<T>.Transpose /
Concat / Gather / Slice (TensorOps.cs:1358-1531, SliceIndex.cs:271-324).

Bar: bit-exact for every dtype (the operators only move elements), and the
reference's failures (status code and message) for invalid arguments."""
import itertools

import numpy as np
import pytest

from onnx_amd import DeviceTensor, HipExecutionProvider as HIP, OpStatus
from onnx_amd import _lib as L
from oracle import graph_oracle as GO
from oracle import oracle as O

import onnx_writer as W
from onnx_amd.graph import Model

pytestmark = pytest.mark.gpu

DTYPES = [np.float32, np.float64, np.int64, np.int32, np.int16, np.uint8, np.bool_]


def dev(a):
    return DeviceTensor.from_numpy(np.asarray(a))


def ok(r):
    assert r.Status == OpStatus.Success, r.Message
    return r.Outputs[0].to_numpy()


def bits(a, b):
    return a.shape == b.shape and a.dtype == b.dtype and np.array_equal(
        np.ascontiguousarray(a).view(np.uint8), np.ascontiguousarray(b).view(np.uint8))


def sample(shape, dt, seed):
    rng = np.random.default_rng(seed)
    if dt == np.bool_:
        return rng.integers(0, 2, shape).astype(np.bool_)
    if np.issubdtype(dt, np.integer):
        info = np.iinfo(dt)
        return rng.integers(info.min, info.max, shape, dtype=dt, endpoint=True)
    return rng.standard_normal(shape).astype(dt)


# ---- Transpose -------------------------------------------------------------------
@pytest.mark.parametrize("dt", DTYPES)
def test_transpose_all_perms(hip, dt):
    """test_backend.py:222-248: every permutation of a [2,3,4] tensor, and the default (reversed) one."""
    x = sample((2, 3, 4), dt, 1)
    for p in itertools.permutations(range(3)):
        assert bits(ok(HIP.Transpose(dev(x), list(p))), O.transpose(x, p))
    assert bits(ok(HIP.Transpose(dev(x))), O.transpose(x))
    assert bits(ok(HIP.Transpose(dev(x), [0, -1, -2])), O.transpose(x, [0, -1, -2]))


@pytest.mark.parametrize("shape,perm", [((8, 512, 12, 64), (0, 2, 1, 3)), ((8, 12, 512, 64), (0, 2, 1, 3)),
                                        ((8, 512, 12, 64), (0, 2, 3, 1)), ((768, 3072), (1, 0)),
                                        ((37, 129, 65), (0, 2, 1)), ((3, 5, 7, 11, 13), (4, 2, 0, 3, 1)),
                                        ((1, 1, 1000), (2, 0, 1)), ((300, 1, 257), (2, 1, 0)),
                                        ((2, 3, 4, 5, 6, 7, 2, 3), (7, 6, 5, 4, 3, 2, 1, 0))])
def test_transpose_shapes(hip, shape, perm):
    x = sample(shape, np.float32, 2)
    assert bits(ok(HIP.Transpose(dev(x), list(perm))), O.transpose(x, perm))


@pytest.mark.parametrize("dt", [np.float32, np.float64, np.uint8, np.int16, np.bool_])
@pytest.mark.parametrize("shape", [(3, 100, 70), (3, 100, 68), (2, 132, 260)])
def test_transpose_tiled_dtypes(hip, dt, shape):
    """Transposes that move the innermost axis: 64x64 four-wide tiles when the plane divides by 4
    (with partial edge tiles), 32x32 scalar tiles otherwise."""
    x = sample(shape, dt, 3)
    assert bits(ok(HIP.Transpose(dev(x), [0, 2, 1])), O.transpose(x, [0, 2, 1]))
    assert bits(ok(HIP.Transpose(dev(x), [2, 1, 0])), O.transpose(x, [2, 1, 0]))
    assert bits(ok(HIP.Transpose(dev(x), [1, 2, 0])), O.transpose(x, [1, 2, 0]))


def test_transpose_rank1_and_empty(hip):
    v = np.arange(7, dtype=np.float32)
    assert bits(ok(HIP.Transpose(dev(v))), v)
    s = np.array(3.5, np.float32)
    assert bits(ok(HIP.Transpose(dev(s))), s)
    # an empty input of rank >= 2 fails as the reference's copy loop does (it visits index [0, ..., 0])
    r = HIP.Transpose(dev(np.zeros((3, 0, 2), np.float32)), [2, 0, 1])
    assert r.Code == L.ERR_INVALID_ARGUMENT and r.Message == "Index was outside the bounds of the array."
    assert ok(HIP.Transpose(dev(np.zeros((0,), np.float32)))).shape == (0,)


def test_transpose_errors(hip):
    x = dev(np.ones((2, 3, 4), np.float32))
    r = HIP.Transpose(x, [0, 1])
    assert r.Code == L.ERR_INVALID_ARGUMENT
    assert r.Message == "The size of the permutation array must be the rank of the tensor: 3. (Parameter 'perm')"
    r = HIP.Transpose(x, [0, 1, 3])
    assert r.Message == "The permuted dimension 3 exceeds the number of dimensions in the tensor. (Parameter 'perm')"
    r = HIP.Transpose(x, [0, 0, 1])
    assert r.Message == "The permutation array has a repeated dimension. (Parameter 'perm')"


# ---- Concat ----------------------------------------------------------------------
@pytest.mark.parametrize("dt", DTYPES)
def test_concat_reference_cases(hip, dt):
    """test_backend.py:296-342."""
    for axis in range(3):
        a, b = sample((10, 20, 5), dt, 4), sample((10, 20, 5), dt, 5)
        assert bits(ok(HIP.Concat([dev(a), dev(b)], axis)), O.concat([a, b], axis))
    for v in [([1, 2], [3, 4]), ([[1, 2], [3, 4]], [[5, 6], [7, 8]]),
              ([[[1, 2], [3, 4]], [[5, 6], [7, 8]]], [[[9, 10], [11, 12]], [[13, 14], [15, 16]]])]:
        vals = [np.asarray(t).astype(dt) for t in v]
        for axis in range(-vals[0].ndim, vals[0].ndim):
            assert bits(ok(HIP.Concat([dev(t) for t in vals], axis)), O.concat(vals, axis))


@pytest.mark.parametrize("shapes,axis", [([(8, 512, 768)] * 3, -1), ([(8, 12, 512, 64), (8, 12, 5, 64)], 2),
                                         ([(4, 1, 33), (4, 0, 33), (4, 7, 33), (4, 2, 33)], 1),
                                         ([(1,), (1000,), (3,)], 0), ([(5, 3), (5, 1), (5, 2)], 1),
                                         ([(3, 4, 5)] * 9, 0), ([(2, 3, 8)] * 17, -1), ([(6, 2, 4), (6, 3, 4)], 1)])
def test_concat_ragged(hip, shapes, axis):
    xs = [sample(s, np.float32, 6 + i) for i, s in enumerate(shapes)]
    assert bits(ok(HIP.Concat([dev(t) for t in xs], axis)), O.concat(xs, axis))


def test_concat_errors(hip):
    a = dev(np.ones((2, 3), np.float32))
    r = HIP.Concat([a], 0)
    assert r.Code == L.ERR_INVALID_ARGUMENT
    assert r.Message == "At least two tensors must be specified for the concat operation. (Parameter 'inputs')"
    r = HIP.Concat([a, dev(np.ones((2, 4), np.float32))], 0)
    assert r.Message == ("The dimensions of each tensor in a concat operation must be the same, with the exception "
                         "of the axis dimension. (Parameter 'inputs')")
    r = HIP.Concat([a, dev(np.ones((2, 3, 1), np.float32))], 0)
    assert r.Message == "Each input tensor in a concat operation must be of the same rank. (Parameter 'inputs')"
    r = HIP.Concat([a, dev(np.ones((2, 3), np.int32))], 0)
    assert r.Code == L.ERR_WRONG_INPUT_TYPE
    z = dev(np.zeros((2, 0), np.float32))
    r = HIP.Concat([z, z, a], 1)   # the first pair concatenates to nothing: fails as in the reference
    assert r.Code == L.ERR_INVALID_ARGUMENT and r.Message == "Index was outside the bounds of the array."
    assert bits(ok(HIP.Concat([z, a, z], 1)), np.ones((2, 3), np.float32))


# ---- Gather ----------------------------------------------------------------------
def test_gather_reference_cases(hip):
    """test_backend.py:379-444, SliceTests.cs CanGather."""
    rng = np.random.default_rng(7)
    x = rng.random((10, 10)).astype(np.float32)
    for idx in ([[0, 1], [1, 2]], [[-10, -9], [1, -8]]):
        for it in (np.int64, np.int32):
            i = np.array(idx, it)
            assert bits(ok(HIP.Gather(dev(x), dev(i))), O.gather(x, i))
    d = rng.standard_normal((5, 4, 3, 2)).astype(np.float32)
    for axis in (0, 1, -1, -4):
        i = np.array([0, 1, -1], np.int64)
        assert bits(ok(HIP.Gather(dev(d), dev(i), axis)), O.gather(d, i, axis))
    d2 = rng.standard_normal((3, 3)).astype(np.float32)
    assert bits(ok(HIP.Gather(dev(d2), dev(np.array([[0, 2]], np.int64)), 1)), O.gather(d2, np.array([[0, 2]]), 1))
    a = np.arange(10).astype(np.float32)
    assert bits(ok(HIP.Gather(dev(a), dev(np.array([0, -9, -10], np.int64)), 0)),
                O.gather(a, np.array([0, -9, -10]), 0))
    s = ok(HIP.Gather(dev(a), dev(np.array(1, np.int64)), 0))
    assert bits(s, O.gather(a, np.array(1), 0))
    g = ok(HIP.Gather(dev(np.array([[1.0, 1.2], [2.3, 3.4], [4.5, 5.7]])), dev(np.array([[0, 1], [1, 2]], np.int32))))
    assert g.shape == (2, 2, 2) and g[1, 1, 1] == 5.7


@pytest.mark.parametrize("dt", DTYPES)
def test_gather_dtypes(hip, dt):
    d = sample((6, 33, 5), dt, 8)
    i = np.random.default_rng(9).integers(-5, 5, (4, 7)).astype(np.int64)
    for axis in (0, 2):
        assert bits(ok(HIP.Gather(dev(d), dev(i), axis)), O.gather(d, i, axis))


def test_gather_embedding_lookup(hip):
    """BERT-base word embedding: table [30522, 768], ids [8, 512]."""
    rng = np.random.default_rng(10)
    table = rng.standard_normal((30522, 768)).astype(np.float32)
    ids = rng.integers(0, 30522, (8, 512)).astype(np.int64)
    assert bits(ok(HIP.Gather(dev(table), dev(ids), 0)), O.gather(table, ids, 0))
    ids32 = ids.astype(np.int32)
    assert bits(ok(HIP.Gather(dev(table), dev(ids32), 0)), O.gather(table, ids32, 0))


def test_gather_empty_and_errors(hip):
    a = dev(np.arange(10, dtype=np.float32))
    for d, i in ((a, np.zeros((0,), np.int64)), (dev(np.zeros((3, 0), np.float32)), np.array([1], np.int64))):
        r = HIP.Gather(d, dev(i), 0)   # an empty output fails as in the reference's loop
        assert r.Code == L.ERR_INVALID_ARGUMENT and r.Message == "Index was outside the bounds of the array."
    for bad in ([10], [-11], [2**40], [3, 2**31]):
        r = HIP.Gather(a, dev(np.array(bad, np.int64)), 0)
        assert r.Code == L.ERR_INVALID_ARGUMENT and r.Message == "Index was outside the bounds of the array.", bad
    r = HIP.Gather(a, dev(np.array([1], np.int64)), 1)
    assert r.Message == "The specified axis 1 exceeds the number of dimensions in the tensor. (Parameter 'axis')"
    r = HIP.Gather(a, dev(np.zeros((1, 1), np.int64)), 0)
    assert r.Code == L.ERR_WRONG_INPUT_SHAPE
    r = HIP.Gather(a, dev(np.zeros((1,), np.float32)), 0)
    assert r.Code == L.ERR_WRONG_INPUT_TYPE
    # after a failed gather the next one is unaffected by the error record
    assert bits(ok(HIP.Gather(a, dev(np.array([9], np.int64)), 0)), np.array([9.0], np.float32))


def test_gather_indices_scanned_before_the_gather(hip):
    """An eager Gather with at most 1/16 as many indices as output elements scans its indices first and
    returns once every one lies in [-dim, dim); an index out of range at the last position (or one an Int64
    tensor holds beyond int32) fails with the reference's message, and clean calls before and after failing
    ones return the oracle's bits."""
    rng = np.random.default_rng(12)
    table = rng.standard_normal((1000, 64)).astype(np.float32)
    dtab = dev(table)
    for idt in (np.int64, np.int32):
        ids = rng.integers(-1000, 1000, (8, 512)).astype(idt)
        want = O.gather(table, ids, 0)
        assert bits(ok(HIP.Gather(dtab, dev(ids), 0)), want)
        bads = [1000, -1001] + ([2**40, -(2**33)] if idt == np.int64 else [2**31 - 1, -(2**31)])
        for bad in bads:
            b = ids.copy()
            b.flat[-1] = bad
            r = HIP.Gather(dtab, dev(b), 0)
            assert r.Code == L.ERR_INVALID_ARGUMENT and r.Message == "Index was outside the bounds of the array.", bad
            assert bits(ok(HIP.Gather(dtab, dev(ids), 0)), want)
    # along an inner axis, many outer rows: [16, 1000, 8] gathered by 40 indices on axis 1
    d3 = rng.standard_normal((16, 1000, 8)).astype(np.float32)
    i3 = rng.integers(0, 1000, (40,)).astype(np.int64)
    assert bits(ok(HIP.Gather(dev(d3), dev(i3), 1)), O.gather(d3, i3, 1))
    i3[-1] = -1001
    assert HIP.Gather(dev(d3), dev(i3), 1).Code == L.ERR_INVALID_ARGUMENT


# ---- Slice -----------------------------------------------------------------------
SLICE_CASES = [
    ((10, 10, 10), [0, 0, 0], [2, 2, 2], [0, 1, 2], [1, 1, 1]),
    ((10, 10, 10), [0, -7], [-8, 20], [0, 2], None),
    ((20, 10, 5), [0, 0], [3, 10], [0, 1], [1, 1]),
    ((20, 10, 5), [0], [-1], [1], [1]),
    ((20, 10, 5), [1000], [1000], [1], [1]),
    ((20, 10, 5), [1], [1000], [1], [1]),
    ((20, 10, 5), [0, 0, 3], [20, 10, 4], None, None),
    ((20, 10, 5), [0, 0, 3], [20, 10, 4], [0, 1, 2], None),
    ((20, 10, 5), [20, 10, 4], [0, 0, 1], [0, 1, 2], [-1, -3, -2]),
    ((20, 10, 5), [-1, 5], [-1000, 0], [0, -1], [-2, -1]),
    ((20, 10, 5), [3], [9], [1], [0]),
    ((20, 10, 5), [3, 1], [9, 4], [1, 1], [2, 1]),
    ((8, 512, 768), [0], [1], [1], None),
    ((8, 512, 2304), [768], [1536], [-1], None),
    ((7, 130, 66), [1, 2, 3], [6, 129, 65], [0, 1, 2], [2, 3, 5]),
]


@pytest.mark.parametrize("case", SLICE_CASES)
def test_slice_cases(hip, case):
    shape, s, e, a, st = case
    x = sample(shape, np.float32, 11)
    assert bits(ok(HIP.Slice(dev(x), s, e, a, st)), O.slice_(x, s, e, a, st))


@pytest.mark.parametrize("dt", DTYPES)
def test_slice_dtypes(hip, dt):
    x = sample((9, 40, 17), dt, 12)
    for s, e, a, st in [([1, 3], [8, 39], [0, 2], [2, 4]), ([-1], [-41], [1], [-3]), ([2], [5], [0], None)]:
        assert bits(ok(HIP.Slice(dev(x), s, e, a, st)), O.slice_(x, s, e, a, st))


def test_slice_reference_quirk_clamps_before_sign(hip):
    """Starts and ends are clamped to [0, dim] before SliceIndex sees them (TensorOps.cs:1521-1522), so a
    negative step whose end is below -dim stops before element 0 rather than including it."""
    x = np.arange(10, dtype=np.float32)
    got = ok(HIP.Slice(dev(x), [9], [-100], [0], [-1]))
    assert bits(got, O.slice_(x, [9], [-100], [0], [-1]))
    assert got.tolist() == list(range(9, 0, -1))


def test_slice_errors(hip):
    x = dev(np.ones((2, 3), np.float32))
    r = HIP.Slice(x, [0, 0, 0], [1, 1, 1])
    assert r.Code == L.ERR_WRONG_INPUT_SHAPE
    r = HIP.Slice(x, [0, 0], [1])
    assert r.Code == L.ERR_WRONG_INPUT_SHAPE
    r = HIP.Slice(x, [0], [1], [5])
    assert r.Code == L.ERR_INVALID_ARGUMENT and r.Message == "Index was outside the bounds of the array."
    r = HIP.Slice(dev(np.array(1.0, np.float32)), [0], [1])
    assert r.Code == L.ERR_WRONG_INPUT_SHAPE


# ---- the same operators as graph nodes -------------------------------------------
def test_movement_graph(hip):
    """Attention-head plumbing: Gather (embedding) -> Slice (fused QKV split) -> Transpose (heads) ->
    MatMul -> Concat, against the CPU restatement of the graph executor."""
    rng = np.random.default_rng(13)
    table = rng.standard_normal((1000, 96)).astype(np.float32)
    ids = rng.integers(-1000, 1000, (2, 16)).astype(np.int64)
    wqkv = rng.standard_normal((96, 288)).astype(np.float32) * 0.1
    inits = [("table", table), ("wqkv", wqkv), ("s0", np.array([0], np.int64)), ("e0", np.array([96], np.int64)),
             ("s1", np.array([96], np.int64)), ("e1", np.array([192], np.int64)), ("ax", np.array([-1], np.int64)),
             ("shape", np.array([2, 16, 4, 24], np.int64))]
    nodes = [W.node("Gather", ["table", "ids"], ["emb"], "gather", axis=0),
             W.node("MatMul", ["emb", "wqkv"], ["qkv"], "mm"),
             W.node("Slice", ["qkv", "s0", "e0", "ax"], ["q"], "sq"),
             W.node("Slice", ["qkv", "s1", "e1", "ax"], ["k"], "sk"),
             W.node("Reshape", ["q", "shape"], ["q4"], "rq"),
             W.node("Reshape", ["k", "shape"], ["k4"], "rk"),
             W.node("Transpose", ["q4"], ["qt"], "tq", perm=[0, 2, 1, 3]),
             W.node("Transpose", ["k4"], ["kt"], "tk", perm=[0, 2, 3, 1]),
             W.node("MatMul", ["qt", "kt"], ["scores"], "qk"),
             W.node("Concat", ["qt", "qt"], ["cat"], "cat", axis=-2)]
    outs = ["emb", "qkv", "q", "k", "qt", "kt", "scores", "cat"]
    model = W.model(nodes, [("ids", np.int64, ids.shape)], [(o, np.float32, ()) for o in outs], inits)
    g = Model.Load(model)
    assert g.Execute({"ids": DeviceTensor.from_numpy(ids)}, True), g.LastError
    got = {o: g.Output(o).to_numpy() for o in outs}
    from test_gpu_graph import _dict_nodes
    ref = GO.run(_dict_nodes(nodes), {"ids": ids}, dict(inits))
    assert bits(got["emb"], ref["emb"])

    def mm_close(a, b, c):
        mag = O.matmul(np.abs(a).astype(np.float64), np.abs(b).astype(np.float64))
        return np.all(np.abs(c.astype(np.float64) - O.matmul(a, b)) <= 1e-5 * mag + 1e-30)
    assert mm_close(got["emb"], wqkv, got["qkv"])
    # the movement nodes downstream of a MatMul: bit-exact on the device's own MatMul output
    assert bits(got["q"], O.slice_(got["qkv"], [0], [96], [-1]))
    assert bits(got["k"], O.slice_(got["qkv"], [96], [192], [-1]))
    assert bits(got["qt"], O.transpose(got["q"].reshape(2, 16, 4, 24), [0, 2, 1, 3]))
    assert bits(got["kt"], O.transpose(got["k"].reshape(2, 16, 4, 24), [0, 2, 3, 1]))
    assert bits(got["cat"], O.concat([got["qt"], got["qt"]], -2))
    assert mm_close(got["qt"], got["kt"], got["scores"])
    assert got["scores"].shape == ref["scores"].shape == (2, 4, 16, 16)


def test_graph_gather_out_of_range_fails_the_node(hip):
    nodes = [W.node("Gather", ["table", "ids"], ["y"], "gather")]
    model = W.model(nodes, [("ids", np.int64, (2,))], [("y", np.float32, ())],
                    [("table", np.ones((4, 3), np.float32))])
    g = Model.Load(model)
    assert not g.Execute({"ids": DeviceTensor.from_numpy(np.array([0, 4], np.int64))}, True)
    assert "Index was outside the bounds of the array." in g.LastError
    assert g.Execute({"ids": DeviceTensor.from_numpy(np.array([0, 3], np.int64))}, True), g.LastError
