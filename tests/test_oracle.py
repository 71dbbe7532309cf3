"""Pins the CPU oracle (oracle/lonnx_oracle.c) before it is trusted as the
parity reference.  CPU only.

What pins each oracle function (besides the restatement itself):
  broadcast shape      reference KATs (ShapeTests.cs, MathTests.cs, OpTests.cs,
                       test_backend.py) + numpy.broadcast_shapes on random shapes
  Add/Sub/Mul/Div f32  IEEE closed form: numpy float32 ops give the same bits;
                       reference KATs (test_backend.py:137-191)
  int Add/Sub/Mul/Div  two's-complement closed form (numpy wrap), truncating
                       division by Python integer arithmetic, x/0 and MIN/-1
                       error statuses; uint8 KAT semantics (test_backend.py:131-206)
  Pow                  reference KATs (test_backend.py:896-908); host powf
  Erf                  |erf_oracle - math.erf| <= 6e-7 (A&S 7.1.26 bound 1.5e-7
                       plus float32 rounding), Erf(0) = 0 exactly, the 2^-24
                       quantisation near 0, oddness, limits
  ReduceSum f32        bit-exact against numpy's sequential add.accumulate (the
                       reference's serial float fold); float64 truth bound
  ReduceMean           KATs (test_backend.py:677-784); float: sum/(float)r;
                       int32: per-element truncating divide first (closed form)
  ReduceMax            seed-0 semantics closed form max(0, max x), NaN skipped
  Softmax              KATs (test_backend.py:812-827) + float64 truth
  Cast                 numpy RNE conversion for int64->float32; .NET Convert
                       rules (banker's rounding, overflow window) by closed form
"""
import json
import math
import os

import numpy as np
import pytest

from oracle import oracle as O

HERE = os.path.dirname(os.path.abspath(__file__))
KATS = json.load(open(os.path.join(HERE, "golden", "reference_kats.json")))


def test_broadcast_shape_kats():
    for k in KATS["broadcast_shape"]:
        got = O.broadcast_shape(k["a"], k["b"])
        exp = tuple(k["out"]) if k["out"] is not None else None
        assert got == exp, k["src"]


def test_broadcast_shape_matches_numpy():
    rng = np.random.default_rng(1)
    for _ in range(2000):
        ra, rb = rng.integers(0, 5, 2)
        a = tuple(int(v) for v in rng.choice([1, 2, 3], ra))
        b = tuple(int(v) for v in rng.choice([1, 2, 3], rb))
        try:
            exp = np.broadcast_shapes(a, b)
        except ValueError:
            exp = None
        assert O.broadcast_shape(a, b) == exp, (a, b)


def test_add_int_kat():
    k = KATS["add_int"]
    a = np.zeros(k["shape"], np.int32)
    a[tuple(k["set_index"])] = k["set_value"]
    c = O.binary(O.ADD, a, a.copy())
    for e in k["expect"]:
        assert c[tuple(e["index"])] == e["value"]


def test_add_ones_broadcast_kat():
    k = KATS["add_ones_broadcast"]
    c = O.binary(O.ADD, np.ones(k["a"], np.float32), np.ones(k["b"], np.float32))
    assert c.shape == tuple(k["out"])
    assert c[tuple(k["index"])] == k["value"]


@pytest.mark.parametrize("name,op", [("sub_f32", O.SUB), ("mul_f32", O.MUL), ("div_f32", O.DIV)])
def test_binary_kats(name, op):
    k = KATS[name]
    z = O.binary(op, np.array(k["x"], np.float32), np.array(k["y"], np.float32))
    np.testing.assert_array_equal(z, np.array(k["z"], np.float32))


def test_pow_kats():
    for k in KATS["pow"]:
        z = O.binary(O.POW, np.array(k["x"], np.float32), np.array(k["y"], np.float32))
        np.testing.assert_array_equal(z, np.array(k["z"], np.float32))


def test_softmax_kats():
    for k in KATS["softmax"]:
        y = O.softmax(np.array(k["x"], np.float32), k["axis"])
        np.testing.assert_almost_equal(y, np.array(k["y"], np.float32), decimal=k["decimal"])


def test_reduce_kats():
    for k in KATS["reduce_sum_int"]:
        y = O.reduce(O.RSUM, np.array(k["data"], np.int32), k["axes"], bool(k["keepdims"]))
        np.testing.assert_array_equal(y, np.array(k["out"], np.int32))
    k = KATS["reduce_sum_double"]
    d = np.array(k["data"], np.float64)
    np.testing.assert_almost_equal(O.reduce(O.RSUM, d, k["axes"], True), d.sum(axis=1, keepdims=True),
                                   decimal=k["decimal"])
    for k in KATS["reduce_mean_f32"]:
        y = O.reduce(O.RMEAN, np.array(k["data"], np.float32), k["axes"], bool(k["keepdims"]))
        np.testing.assert_almost_equal(y, np.array(k["out"], np.float32), decimal=6)
    k = KATS["reduce_mean_double"]
    for c in k["cases"]:
        y = O.reduce(O.RMEAN, np.array(k["data"], np.float64), c["axes"], True)
        np.testing.assert_almost_equal(y, np.array(c["out"]))


def test_float_binary_ieee_closed_form():
    rng = np.random.default_rng(2)
    a = rng.standard_normal((7, 5, 33)).astype(np.float32)
    b = rng.standard_normal((5, 1)).astype(np.float32)
    b[b == 0] = 1
    for op, f in [(O.ADD, np.add), (O.SUB, np.subtract), (O.MUL, np.multiply), (O.DIV, np.divide)]:
        np.testing.assert_array_equal(O.binary(op, a, b), f(a, b))
        np.testing.assert_array_equal(O.binary(op, b, a), f(b, a))
    # denormals survive (no flush to zero)
    tiny = np.array([1e-40, -3e-42], np.float32)
    np.testing.assert_array_equal(O.binary(O.ADD, tiny, np.zeros(2, np.float32)), tiny)


@pytest.mark.parametrize("dt", [np.int32, np.int64])
def test_int_binary_closed_form(dt):
    rng = np.random.default_rng(3)
    info = np.iinfo(dt)
    a = rng.integers(info.min, info.max, 4000, dtype=dt)
    b = rng.integers(info.min, info.max, 4000, dtype=dt)
    b[b == 0] = 7
    with np.errstate(over="ignore"):
        np.testing.assert_array_equal(O.binary(O.ADD, a, b), a + b)
        np.testing.assert_array_equal(O.binary(O.SUB, a, b), a - b)
        np.testing.assert_array_equal(O.binary(O.MUL, a, b), a * b)
    q = O.binary(O.DIV, a, b)
    exp = np.array([int(x / y) if abs(int(x)) < 2**52 else (abs(int(x)) // abs(int(y))) * (1 if (x < 0) == (y < 0) else -1)
                    for x, y in zip(a.tolist(), b.tolist())], dtype=dt)
    np.testing.assert_array_equal(q, exp)
    # C# truncation, not numpy floor
    np.testing.assert_array_equal(O.binary(O.DIV, np.array([-7, 7, -7], dt), np.array([2, -2, -2], dt)),
                                  np.array([-3, -3, 3], dt))
    with pytest.raises(O.OracleError) as e:
        O.binary(O.DIV, np.array([1, 2], dt), np.array([1, 0], dt))
    assert e.value.status == O.ERR_DIVIDE_BY_ZERO
    with pytest.raises(O.OracleError) as e:
        O.binary(O.DIV, np.array([info.min], dt), np.array([-1], dt))
    assert e.value.status == O.ERR_OVERFLOW


def test_uint8_semantics():
    a = np.array([250, 3, 12, 200], np.uint8)
    b = np.array([10, 5, 24, 3], np.uint8)
    np.testing.assert_array_equal(O.binary(O.ADD, a, b), (a.astype(int) + b) % 256)
    np.testing.assert_array_equal(O.binary(O.SUB, a, b), (a.astype(int) - b) % 256)
    np.testing.assert_array_equal(O.binary(O.MUL, a, b), (a.astype(int) * b) % 256)
    np.testing.assert_array_equal(O.binary(O.DIV, a, b), a // b)


def test_erf_bound_and_special_values():
    xs = np.linspace(-6, 6, 20001).astype(np.float32)
    got = np.array([O.erf_f32(v) for v in xs], np.float64)
    ref = np.array([math.erf(float(v)) for v in xs])
    # A&S 7.1.26 is within 1.5e-7 of erf; ~10 float32 roundings add < 4.5e-7.
    # (The reference's own test allows rtol = atol = 1e-6, test_backend.py:208-220.)
    assert np.max(np.abs(got - ref)) <= 6e-7
    assert O.erf_f32(0.0) == 0.0
    # 1 - P is exact near 0: outputs are multiples of 2^-24
    assert O.erf_f32(1e-6) == 20 * 2.0 ** -24
    for v in [1e-3, 0.01, 0.3]:
        q = O.erf_f32(v) / 2.0 ** -24
        assert q == int(q)
    assert O.erf_f32(-0.7) == -O.erf_f32(0.7)
    assert O.erf_f32(float("inf")) == 1.0 and O.erf_f32(float("-inf")) == -1.0
    assert math.isnan(O.erf_f32(float("nan")))


def _same_or_both_nan(a, b):
    return (a.view(np.uint32) == b.view(np.uint32)) | (np.isnan(a) & np.isnan(b))


def test_gelu_chain_loop_equals_the_five_ops():
    """The oracle's single-loop GELU (the full-size C5 checker) is the five-node composite Div -> Erf -> Add ->
    Mul -> Mul of the pinned operators, bit for bit: on 10^7 inputs -- normal samples, random 32-bit patterns
    (every exponent, denormals, infinities, NaNs) and the neighbourhood of 0."""
    rng = np.random.default_rng(31)
    x = np.concatenate([rng.standard_normal(4_000_000).astype(np.float32),
                        rng.integers(0, 2**32, 5_000_000, dtype=np.uint64).astype(np.uint32).view(np.float32),
                        rng.uniform(-1e-3, 1e-3, 1_000_000).astype(np.float32),
                        np.array([0.0, -0.0, np.inf, -np.inf, np.nan, 1e-45, -1e-45, 3.4e38, -3.4e38], np.float32)])
    fast, comp = O.gelu_chain_fast(x), O.gelu_erf(x)
    assert _same_or_both_nan(fast, comp).all()


def test_sqrt_equals_ieee_square_root():
    """The oracle's Sqrt (the reference's Vector.SquareRoot / MathF.Sqrt, TensorOps.cs:315-317) is the correctly
    rounded IEEE square root: numpy's float32 sqrt, bit for bit, over random bit patterns (negative inputs and
    -inf give NaN, -0 gives -0) and float64 likewise."""
    rng = np.random.default_rng(32)
    x = rng.integers(0, 2**32, 2_000_000, dtype=np.uint64).astype(np.uint32).view(np.float32)
    x = np.concatenate([x, np.array([0.0, -0.0, np.inf, -np.inf, np.nan, 1e-45, 4.0, 2.0], np.float32)])
    with np.errstate(invalid="ignore"):
        ref = np.sqrt(x)
    got = O.unary(O.SQRT, x)
    assert _same_or_both_nan(got, ref).all()
    assert np.signbit(got[-7]) and got[-6] == np.inf and got[-2] == 2.0
    d = np.abs(rng.standard_normal(100000)) * 1e10
    assert np.array_equal(O.unary(O.SQRT, d), np.sqrt(d))


def test_serial_fold_matches_sequential_accumulate():
    rng = np.random.default_rng(4)
    x = rng.uniform(-1, 1, (64, 4096)).astype(np.float32)
    got = O.reduce(O.RSUM, x, [1], False)
    seq = np.add.accumulate(x, axis=1, dtype=np.float32)[:, -1]
    np.testing.assert_array_equal(got, seq)
    truth = x.astype(np.float64).sum(axis=1)
    assert np.all(np.abs(got - truth) <= 4096 * 2 ** -24 * np.abs(x).sum(axis=1))
    # strided axis: transpose then fold, same numbers as folding along the axis
    y = rng.uniform(-1, 1, (8, 300, 16)).astype(np.float32)
    got = O.reduce(O.RSUM, y, [1], True)
    seq = np.add.accumulate(y, axis=1, dtype=np.float32)[:, -1:, :]
    np.testing.assert_array_equal(got, seq)


def test_reduce_mean_semantics():
    x = np.array([[1, 2, 3], [-4, 5, 6]], np.int32)
    # divide each element first (truncating), then sum: 0+0+1 = 1, -1+1+2 = 2
    np.testing.assert_array_equal(O.reduce(O.RMEAN, x, [1], False), np.array([1, 2], np.int32))
    f = np.array([[1, 2, 4]], np.float32)
    assert O.reduce(O.RMEAN, f, [1], False)[0] == np.float32(7) / np.float32(3)
    d = np.array([[0.1, 0.2, 0.4]])
    assert O.reduce(O.RMEAN, d, [1], False)[0] == (0.1 / 3 + 0.2 / 3) + 0.4 / 3


def test_reduce_max_seed_zero():
    x = np.array([[-3, -1, -2], [1, np.nan, 5], [np.nan, np.nan, -1]], np.float32)
    np.testing.assert_array_equal(O.reduce(O.RMAX, x, [1], False), np.array([0, 5, 0], np.float32))


def test_multi_axis_reduce_int_exact():
    x = np.arange(4 * 5 * 6 * 3, dtype=np.int64).reshape(4, 5, 6, 3) - 100
    for axes in ([0, 2], [2, 1], [3, 0], [1], [-1, -3], []):
        exp = x.sum(axis=tuple(axes) if axes else None, keepdims=True)
        np.testing.assert_array_equal(O.reduce(O.RSUM, x, axes, True), exp)


def test_softmax_float64_truth():
    rng = np.random.default_rng(5)
    x = (rng.standard_normal((32, 512)) * 3).astype(np.float32)
    y = O.softmax(x, -1)
    xd = x.astype(np.float64)
    t = np.exp(xd - np.maximum(0, xd.max(-1, keepdims=True)))
    t /= t.sum(-1, keepdims=True)
    assert np.max(np.abs(y - t)) <= 1e-6
    # axis 0 of a 3-d tensor
    z = rng.standard_normal((5, 4, 3)).astype(np.float32)
    y0 = O.softmax(z, 0)
    zd = z.astype(np.float64)
    t0 = np.exp(zd - np.maximum(0, zd.max(0, keepdims=True)))
    t0 /= t0.sum(0, keepdims=True)
    assert np.max(np.abs(y0 - t0)) <= 1e-6


def test_cast_rules():
    big = np.array([2**24 + 1, 2**24 + 3, -(2**40) - 1, 2**62 + 2**38 + 1], np.int64)
    np.testing.assert_array_equal(O.cast(big, O.FLOAT), big.astype(np.float32))
    f = np.array([0.5, 1.5, 2.5, -0.5, -1.5, 2.4999998, 2147483647.0, -2147483648.5], np.float64)
    np.testing.assert_array_equal(O.cast(f, O.INT32), np.rint(f).astype(np.int32))
    for bad, to in [(2147483647.5, O.INT32), (float("nan"), O.INT32), (256.0, O.UINT8), (-0.6, O.UINT8),
                    (-0.5, O.UINT32), (9.3e18, O.INT64), (-1.0, O.UINT64)]:
        with pytest.raises(O.OracleError) as e:
            O.cast(np.array([bad]), to)
        assert e.value.status == O.ERR_OVERFLOW
    np.testing.assert_array_equal(O.cast(np.array([-0.4, 255.4], np.float32), O.UINT8), np.array([0, 255], np.uint8))
    np.testing.assert_array_equal(O.cast(np.array([0.0, -0.0, 2.0, np.nan], np.float32), O.BOOL),
                                  np.array([False, False, True, True]))
    with pytest.raises(O.OracleError):
        O.cast(np.array([300], np.int32), O.UINT8)
    with pytest.raises(O.OracleError):
        O.cast(np.array([-1], np.int64), O.UINT32)
    k = KATS["cast_dtypes"]
    for to in k["to"]:
        out = O.cast(np.array(k["input"], np.int64), to)
        assert out.dtype == np.dtype(O.NP_OF[to])


def test_composites_against_float64():
    rng = np.random.default_rng(6)
    x = (rng.standard_normal((16, 768)) * 2).astype(np.float32)
    g = (1 + 0.02 * rng.standard_normal(768)).astype(np.float32)
    b = (0.02 * rng.standard_normal(768)).astype(np.float32)
    y = O.layernorm_decomposed(x, g, b)
    xd = x.astype(np.float64)
    t = (xd - xd.mean(-1, keepdims=True)) / np.sqrt(xd.var(-1, keepdims=True) + 1e-12) * g + b
    assert np.max(np.abs(y - t)) <= 1e-5
    xs = rng.standard_normal(10000).astype(np.float32)
    gl = O.gelu_erf(xs)
    tg = np.array([0.5 * v * (1 + math.erf(v / math.sqrt(2))) for v in xs.astype(np.float64)])
    assert np.max(np.abs(gl - tg)) <= 1e-6


# ---- MatMul (TensorOps.cs:356-705) ----------------------------------------------
def test_matmul_reference_kats():
    """MathTests.cs:82-97 (CanMatMul) and :47-80 (CanMatMul2D)."""
    ones = lambda *s: np.ones(s, np.int32)  # noqa: E731
    assert O.matmul(ones(1, 1, 5, 6), ones(3, 6, 7)).shape == (1, 3, 5, 7)
    assert O.matmul(ones(2, 3, 5, 6), ones(3, 6, 7)).shape == (2, 3, 5, 7)
    assert O.matmul(ones(4, 1, 5, 6), ones(4, 2, 6, 7)).shape == (4, 2, 5, 7)
    a = np.arange(16, dtype=np.int32).reshape(2, 2, 4)
    b = np.arange(16, dtype=np.int32).reshape(2, 4, 2)
    assert O.matmul(a, b)[0, 1, 1] == 98
    c = O.matmul(ones(7, 4), ones(4, 3))
    assert c.shape == (7, 3) and c.size == 21 and np.all(c == 4)
    f = O.matmul(np.ones((1, 1, 5, 6), np.float32), np.ones((3, 6, 7), np.float32))
    assert f.shape == (1, 3, 5, 7) and np.all(f == 6)


def test_matmul_int32_wraps_like_unchecked_csharp():
    rng = np.random.default_rng(40)
    a = rng.integers(-2**31, 2**31, (5, 9), dtype=np.int64)
    b = rng.integers(-2**31, 2**31, (9, 4), dtype=np.int64)
    exact = [[sum(int(a[i, j]) * int(b[j, k]) for j in range(9)) for k in range(4)] for i in range(5)]
    want = ((np.array(exact, dtype=object) + 2**31) % 2**32 - 2**31).astype(np.int64)
    assert np.array_equal(O.matmul(a.astype(np.int32), b.astype(np.int32)).astype(np.int64), want)


def test_matmul_float_closed_forms_and_bound():
    rng = np.random.default_rng(41)
    # integer-valued operands: every product and partial sum is exact in float32
    a = rng.integers(-20, 20, (7, 33)).astype(np.float32)
    b = rng.integers(-20, 20, (33, 5)).astype(np.float32)
    assert np.array_equal(O.matmul(a, b), (a.astype(np.int64) @ b.astype(np.int64)).astype(np.float32))
    # identity: x @ I == x exactly
    x = rng.standard_normal((6, 10)).astype(np.float32)
    assert np.array_equal(O.matmul(x, np.eye(10, dtype=np.float32)), x)
    # random: within the serial-summation bound n*u*sum|a||b| of the float64 product
    a = rng.standard_normal((9, 300)).astype(np.float32)
    b = rng.standard_normal((300, 11)).astype(np.float32)
    truth = a.astype(np.float64) @ b.astype(np.float64)
    bound = 300 * 2.0**-24 * (np.abs(a).astype(np.float64) @ np.abs(b).astype(np.float64))
    assert np.all(np.abs(O.matmul(a, b) - truth) <= bound)
    d = O.matmul(a.astype(np.float64), b.astype(np.float64))
    assert np.allclose(d, truth, rtol=1e-12, atol=1e-12)


def test_matmul_broadcast_cases():
    rng = np.random.default_rng(42)
    a = rng.integers(-5, 5, (2, 1, 3, 4)).astype(np.int32)
    b = rng.integers(-5, 5, (5, 4, 6)).astype(np.int32)
    assert np.array_equal(O.matmul(a, b), np.matmul(a, b))
    # both rank 1: [1,n] x [n,1] with the leading axis removed -> shape [1]
    v = np.arange(5, dtype=np.int32)
    assert O.matmul(v, v).shape == (1,) and O.matmul(v, v)[0] == 30
    # one operand of rank 1 is broadcast element-wise first (the reference's rule, not ONNX's)
    m = rng.integers(-5, 5, (4, 4)).astype(np.int32)
    w = rng.integers(-5, 5, 4).astype(np.int32)
    assert np.array_equal(O.matmul(m, w), m @ np.broadcast_to(w, (4, 4)))
    with pytest.raises(O.OracleError):
        O.matmul(np.ones((3, 4), np.int32), np.ones(4, np.int32))   # [3,4] x [3,4]: 4 != 3
    with pytest.raises(O.OracleError):
        O.matmul(np.ones((2, 3), np.float32), np.ones((4, 2), np.float32))


# ---- data movement: the reference's own cases (test_backend.py:222-248, 296-342, 379-444, 446-557;
# ---- SliceTests.cs:6-80), expected values as those tests state them --------------------------
def test_transpose_reference_cases():
    import itertools
    rng = np.random.default_rng(60)
    x = rng.standard_normal(1000).astype(np.float32).reshape(10, 10, 10)
    assert np.array_equal(O.transpose(x, [0, 2, 1]), np.transpose(x, (0, 2, 1)))
    d = rng.random((2, 3, 4)).astype(np.float32)
    assert np.array_equal(O.transpose(d), np.transpose(d))
    for p in itertools.permutations(range(3)):
        assert np.array_equal(O.transpose(d, p), np.transpose(d, p))
    with pytest.raises(O.OracleError):
        O.transpose(d, [0, 1])
    with pytest.raises(O.OracleError):
        O.transpose(d, [0, 0, 1])


def test_concat_reference_cases():
    rng = np.random.default_rng(61)
    for axis in range(3):
        a, b = rng.random((10, 20, 5)).astype(np.float32), rng.random((10, 20, 5)).astype(np.float32)
        assert np.array_equal(O.concat([a, b], axis), np.concatenate((a, b), axis))
    cases = [([1, 2], [3, 4]), ([[1, 2], [3, 4]], [[5, 6], [7, 8]]),
             ([[[1, 2], [3, 4]], [[5, 6], [7, 8]]], [[[9, 10], [11, 12]], [[13, 14], [15, 16]]])]
    for v in cases:
        vals = [np.asarray(x, np.float32) for x in v]
        for axis in range(-vals[0].ndim, vals[0].ndim):
            assert np.array_equal(O.concat(vals, axis), np.concatenate(vals, axis))
    with pytest.raises(O.OracleError):
        O.concat([np.ones((2, 2), np.float32)], 0)


def test_gather_reference_cases():
    rng = np.random.default_rng(62)
    x = rng.random((10, 10)).astype(np.float32)
    want = np.stack([x[0:2], x[1:3]])
    assert np.array_equal(O.gather(x, np.array([[0, 1], [1, 2]])), want)
    assert np.array_equal(O.gather(x, np.array([[-10, -9], [1, -8]])), want)
    d = rng.standard_normal((5, 4, 3, 2)).astype(np.float32)
    assert np.array_equal(O.gather(d, np.array([0, 1, 3]), 0), np.take(d, [0, 1, 3], axis=0))
    assert np.array_equal(O.gather(d, np.array([0, 1, 3]), 1), np.take(d, [0, 1, 3], axis=1))
    d2 = rng.standard_normal((3, 3)).astype(np.float32)
    assert np.array_equal(O.gather(d2, np.array([[0, 2]]), 1), np.take(d2, [[0, 2]], axis=1))
    a = np.arange(10).astype(np.float32)
    assert np.array_equal(O.gather(a, np.array([0, -9, -10]), 0), np.take(a, [0, -9, -10], axis=0))
    assert np.array_equal(O.gather(a, np.array(1), 0), np.take(a, 1, axis=0))
    # SliceTests.cs CanGather: [[1.0,1.2],[2.3,3.4],[4.5,5.7]] with [[0,1],[1,2]]
    g = O.gather(np.array([[1.0, 1.2], [2.3, 3.4], [4.5, 5.7]]), np.array([[0, 1], [1, 2]], np.int32))
    assert g.shape == (2, 2, 2) and g[1, 1, 1] == 5.7
    with pytest.raises(O.OracleError):
        O.gather(a, np.array([10]), 0)


def test_slice_reference_cases():
    rng = np.random.default_rng(63)
    x = rng.random(1000).astype(np.float32).reshape(10, 10, 10)
    assert np.array_equal(O.slice_(x, [0, 0, 0], [2, 2, 2], [0, 1, 2], [1, 1, 1]), x[0:2, 0:2, 0:2])
    assert np.array_equal(O.slice_(x, [0, -7], [-8, 20], [0, 2]), x[0:-8, :, -7:20])
    y = rng.standard_normal((20, 10, 5)).astype(np.float32)
    assert np.array_equal(O.slice_(y, [0, 0], [3, 10], [0, 1], [1, 1]), y[0:3, 0:10])
    assert np.array_equal(O.slice_(y, [0], [-1], [1], [1]), y[:, 0:-1])
    assert np.array_equal(O.slice_(y, [1000], [1000], [1], [1]), y[:, 1000:1000])
    assert np.array_equal(O.slice_(y, [1], [1000], [1], [1]), y[:, 1:1000])
    assert np.array_equal(O.slice_(y, [0, 0, 3], [20, 10, 4]), y[:, :, 3:4])
    assert np.array_equal(O.slice_(y, [0, 0, 3], [20, 10, 4], [0, 1, 2]), y[:, :, 3:4])
    assert np.array_equal(O.slice_(y, [20, 10, 4], [0, 0, 1], [0, 1, 2], [-1, -3, -2]), y[20:0:-1, 10:0:-3, 4:1:-2])
    # SliceTests.cs CanSlice: Arange(12).Reshape(3,4)[.., 2..4] -> [[2,3],[6,7],[10,11]]
    t = np.arange(12, dtype=np.int32).reshape(3, 4)
    s1 = O.slice_(t, [2], [4], [1])
    assert s1.shape == (3, 2) and s1[2, 1] == 11 and s1[0, 0] == t[0, 2]


def test_movement_empty_outputs_fail_like_the_reference():
    """TensorDimensionsIterator yields its first index [0, ..., 0] even for an empty shape
    (TensorDimensionsIterator.cs:17-20, 36-40), so the reference's Transpose / Gather / pairwise Concat copy
    loops touch element 0 of an empty buffer and fail with IndexOutOfRangeException; Slice returns a lazy
    view and does not."""
    e = np.zeros((3, 0, 2), np.float32)
    with pytest.raises(O.OracleError, match="outside the bounds"):
        O.transpose(e, [2, 0, 1])
    assert O.transpose(np.zeros((0,), np.float32)).shape == (0,)  # rank <= 1: the input itself
    with pytest.raises(O.OracleError, match="outside the bounds"):
        O.gather(np.arange(10, dtype=np.float32), np.zeros((0,), np.int64), 0)
    with pytest.raises(O.OracleError, match="outside the bounds"):
        O.gather(np.zeros((3, 0), np.float32), np.array([1]), 0)
    with pytest.raises(O.OracleError, match="outside the bounds"):
        O.concat([np.zeros((2, 0), np.float32), np.zeros((2, 0), np.float32), np.ones((2, 3), np.float32)], 1)
    assert O.concat([np.zeros((2, 0), np.float32), np.ones((2, 3), np.float32)], 1).shape == (2, 3)
    with pytest.raises(O.OracleError, match="outside the bounds"):
        O.concat([np.zeros((0, 2), np.float32), np.ones((0, 3), np.float32)], 1)
    assert O.slice_(np.ones((4, 5), np.float32), [3], [1], [0]).shape == (0, 5)
