"""Parity at the full BASELINE.json config sizes, HIP path against the CPU
oracle on the same seeded inputs (the oracle finishes each in seconds).

Bars: bit-exact for the elementwise / integer / Cast work and for the GELU
chain; reductions |gpu - ref| <= 1e-5 * sum|x| of each slice; Softmax and
LayerNorm outputs |gpu - ref| <= 1e-5 * max(|ref|, 1) (LayerNorm) or
1e-5 * |ref| (Softmax), with NaN where the reference gives NaN.
Size-independent properties are checked where the oracle is not run.
"""
import gc

import numpy as np
import pytest

from onnx_amd import DeviceTensor, HipExecutionProvider as HIP, OpStatus
from oracle import oracle as O

pytestmark = pytest.mark.gpu


def dev(a):
    return DeviceTensor.from_numpy(a)


def ok(r):
    assert r.Status == OpStatus.Success, r.Message
    return r.Outputs[0]


def bits_equal(a, b):
    return np.array_equal(np.ascontiguousarray(a).reshape(-1).view(np.uint8),
                          np.ascontiguousarray(b).reshape(-1).view(np.uint8))


def test_c1_bias_add_then_scale(hip):
    rng = np.random.default_rng(101)
    a = rng.standard_normal((1, 128, 384)).astype(np.float32)
    b = rng.uniform(-0.1, 0.1, 384).astype(np.float32)
    s = np.array(0.125, np.float32)
    c = ok(HIP.Add(dev(a), dev(b)))
    y = ok(HIP.Mul(c, dev(s))).to_numpy()
    assert bits_equal(y, O.binary(O.MUL, O.binary(O.ADD, a, b), s))


def test_c2_layernorm_fused_and_by_node(hip):
    rng = np.random.default_rng(102)
    x = (rng.standard_normal((8, 512, 768)) * 2).astype(np.float32)
    g = (1 + 0.02 * rng.standard_normal(768)).astype(np.float32)
    be = (0.02 * rng.standard_normal(768)).astype(np.float32)
    eps = np.float32(1e-12)
    ref = O.layernorm_decomposed(x, g, be, eps)
    y = ok(HIP.LayerNormDecomposed(dev(x), dev(g), dev(be), 1e-12)).to_numpy()
    assert np.all(np.abs(y.astype(np.float64) - ref) <= 1e-5 * np.maximum(1.0, np.abs(ref)))
    # node by node: every elementwise node is bit-exact on the inputs it got,
    # the two ReduceMean nodes meet the reduction bar
    X = dev(x)
    mean = ok(HIP.ReduceMean(X, [-1], 1)).to_numpy()
    rm = O.reduce(O.RMEAN, x, [-1], True)
    assert np.all(np.abs(mean - rm) <= 1e-5 * np.abs(x).sum(-1, keepdims=True) / 768)
    d = ok(HIP.Sub(X, dev(mean))).to_numpy()
    assert bits_equal(d, O.binary(O.SUB, x, mean))
    two = np.array(2.0, np.float32)
    p = ok(HIP.Pow(dev(d), dev(two))).to_numpy()
    assert bits_equal(p, d * d)  # exponent 2 is the correctly rounded square
    var = ok(HIP.ReduceMean(dev(p), [-1], 1)).to_numpy()
    assert np.all(np.abs(var - O.reduce(O.RMEAN, p, [-1], True)) <= 1e-5 * p.sum(-1, keepdims=True) / 768)
    ve = ok(HIP.Add(dev(var), dev(np.array(eps)))).to_numpy()
    assert bits_equal(ve, O.binary(O.ADD, var, np.array(eps)))
    sd = ok(HIP.Sqrt(dev(ve))).to_numpy()
    assert bits_equal(sd, O.unary(O.SQRT, ve))
    n = ok(HIP.Div(dev(d), dev(sd))).to_numpy()
    assert bits_equal(n, O.binary(O.DIV, d, sd))
    m = ok(HIP.Mul(dev(n), dev(g))).to_numpy()
    assert bits_equal(m, O.binary(O.MUL, n, g))
    yy = ok(HIP.Add(dev(m), dev(be))).to_numpy()
    assert bits_equal(yy, O.binary(O.ADD, m, be))


def _c3_inputs():
    rng = np.random.default_rng(103)
    s = (rng.standard_normal((16, 12, 512, 512), dtype=np.float32) * np.float32(3))
    m = np.zeros((16, 1, 1, 512), np.float32)
    for bi in range(16):
        m[bi, 0, 0, rng.permutation(512)[:64]] = -10000.0
    return s, m


def test_c3_mask_add_and_softmax(hip):
    s, m = _c3_inputs()
    S, M = dev(s), dev(m)
    t = ok(HIP.Add(S, M))
    tn = t.to_numpy()
    ref_t = O.binary(O.ADD, s, m)
    assert bits_equal(tn, ref_t)
    y = ok(HIP.Softmax(t, -1)).to_numpy()
    ref = O.softmax(ref_t, -1)
    assert np.all(np.abs(y.astype(np.float64) - ref) <= 1e-5 * np.abs(ref) + 1e-30)
    del y
    yf = ok(HIP.AddSoftmax(S, M, -1)).to_numpy()
    assert np.all(np.abs(yf.astype(np.float64) - ref) <= 1e-5 * np.abs(ref) + 1e-30)
    # rows sum to 1; masked columns are exactly 0
    assert np.allclose(yf[:2].sum(-1), 1.0, atol=1e-5)
    assert np.all(yf[np.broadcast_to(m == -10000.0, yf.shape)] == 0.0)


@pytest.mark.parametrize("dt", [np.int64, np.int32])
def test_c4_integer_broadcast_ops(hip, dt):
    rng = np.random.default_rng(104)
    a = rng.integers(-(2**20), 2**20, (64, 1, 4096), endpoint=True).astype(dt)
    b = rng.integers(1, 1024, (1, 256, 4096), endpoint=True).astype(dt)
    A, B = dev(a), dev(b)
    for op, code in (("Add", O.ADD), ("Mul", O.MUL), ("Div", O.DIV)):
        y = ok(getattr(HIP, op)(A, B)).to_numpy()
        assert bits_equal(y, O.binary(code, a, b)), op
        del y
        gc.collect()


def test_c4_cast_and_reducesum_int64(hip):
    rng = np.random.default_rng(105)
    a = rng.integers(-(2**20), 2**20, (64, 1, 4096), endpoint=True)
    b = rng.integers(1, 1024, (1, 256, 4096), endpoint=True)
    x = O.binary(O.ADD, a, b)
    X = dev(x)
    f = ok(HIP.Cast(X, O.FLOAT)).to_numpy()
    assert bits_equal(f, O.cast(x, O.FLOAT))
    r = ok(HIP.ReduceSum(X, [1], 1)).to_numpy()
    assert bits_equal(r, O.reduce(O.RSUM, x, [1], True))
    # wrap-around: sums far outside int64 range stay two's-complement exact
    big = np.full((2, 300, 3), 2**62, np.int64)
    rb = ok(HIP.ReduceSum(dev(big), [1], 1)).to_numpy()
    assert bits_equal(rb, O.reduce(O.RSUM, big, [1], True))


def test_c5_gelu_chain(hip):
    rng = np.random.default_rng(106)
    x = rng.standard_normal((32, 2048, 3072), dtype=np.float32)
    y = ok(HIP.GeluErf(dev(x))).to_numpy()
    assert bits_equal(y, O.gelu_chain_fast(x))


def test_c5_strided_reducesum_and_full_mean(hip):
    rng = np.random.default_rng(107)
    yv = rng.uniform(-1, 1, (256, 4096, 256)).astype(np.float32)
    Y = dev(yv)
    r1 = ok(HIP.ReduceSum(Y, [1], 1)).to_numpy()
    ref1 = O.reduce(O.RSUM, yv, [1], True)
    absum = np.abs(yv).sum(axis=1, keepdims=True, dtype=np.float64)
    assert np.all(np.abs(r1.astype(np.float64) - ref1) <= 1e-5 * absum)
    r2 = ok(HIP.ReduceMean(Y, None, 1)).to_numpy()
    ref2 = O.reduce(O.RMEAN, yv, None, True)
    tot = float(np.abs(yv).sum(dtype=np.float64))
    truth = float(yv.sum(dtype=np.float64)) / yv.size
    assert abs(float(r2.reshape(-1)[0]) - float(ref2.reshape(-1)[0])) <= 1e-5 * tot / yv.size
    # against float64 truth the device sum is closer than the serial fold
    assert abs(float(r2.reshape(-1)[0]) - truth) <= abs(float(ref2.reshape(-1)[0]) - truth) + 1e-9
