"""GPU parity tests: every operator of the HIP path against the CPU oracle on
the same seeded inputs, through the C ABI (HipExecutionProvider over ctypes).

Bars (written per test):
  bit-exact : integer ops, Cast, float Add/Sub/Mul/Div, Sqrt, Erf (expf is
              bit-identical to the host expf), the fused GELU chain
  <= 2 ulp  : Pow with a non-2 exponent (device pow vs host powf)
  reductions: |gpu - ref| <= 1e-5 * sum|x| over the reduced slice (the
              reference folds serially; any parallel order differs)
  softmax   : |gpu - ref| <= 1e-5 * |ref| (+1e-30 for underflowed entries); rows of any
              length: + |ref - truth|, the reference's own rounding against float64 (its
              serial sum of a long row is up to ~1e-4 relative away from the exact one)
"""
import ctypes
import json
import os

import numpy as np
import pytest

from onnx_amd import DeviceTensor, HipExecutionProvider as HIP, OpStatus
from onnx_amd import _lib as L
from oracle import oracle as O

pytestmark = pytest.mark.gpu

HERE = os.path.dirname(os.path.abspath(__file__))
KATS = json.load(open(os.path.join(HERE, "golden", "reference_kats.json")))


def dev(a):
    return DeviceTensor.from_numpy(np.asarray(a))


def ok(r):
    assert r.Status == OpStatus.Success, r.Message
    return r.Outputs[0].to_numpy()


def ulps(a, b):
    a = np.asarray(a, np.float32).view(np.int32).astype(np.int64)
    b = np.asarray(b, np.float32).view(np.int32).astype(np.int64)
    a = np.where(a < 0, -(a & 0x7fffffff), a)
    b = np.where(b < 0, -(b & 0x7fffffff), b)
    return np.abs(a - b)


def assert_bits(gpu, ref):
    assert gpu.shape == ref.shape and gpu.dtype == ref.dtype
    g = np.ascontiguousarray(gpu).reshape(-1).view(np.uint8)
    r = np.ascontiguousarray(ref).reshape(-1).view(np.uint8)
    if not np.array_equal(g, r):
        bad = np.flatnonzero(gpu.reshape(-1) != ref.reshape(-1))
        raise AssertionError(f"{bad.size} mismatches, first at {bad[:5]}: gpu {gpu.reshape(-1)[bad[:5]]} "
                             f"ref {ref.reshape(-1)[bad[:5]]}")


def assert_reduction(gpu, ref, x_abs_sum):
    assert gpu.shape == ref.shape
    err = np.abs(gpu.astype(np.float64) - ref.astype(np.float64))
    tol = 1e-5 * x_abs_sum + 1e-30
    assert np.all(err <= tol), f"max err {err.max()} tol {tol.reshape(-1)[np.argmax(err)]}"


SHAPES = [
    ((1, 128, 384), (384,)),          # C1 bias
    ((1, 128, 384), ()),              # scalar
    ((8, 512, 768), (8, 512, 1)),     # per-row
    ((8, 512, 768), (768,)),          # gamma
    ((4, 3, 64, 64), (4, 1, 1, 64)),  # C3 mask pattern
    ((8, 1, 256), (1, 16, 256)),      # C4 pattern
    ((7, 5, 33), (5, 1)),             # ragged, outer broadcast
    ((5, 1), (7, 5, 33)),             # broadcast on A
    ((1001,), (1001,)),               # odd length
    ((3, 1, 5), (1, 4, 1)),           # two-sided, odd inner
    ((2, 3), (0, 1, 3)),              # empty output
    ((), ()),                          # scalars
    ((13,), ()),
    ((), (6, 7)),
]


@pytest.mark.parametrize("sa,sb", SHAPES)
@pytest.mark.parametrize("op", ["Add", "Sub", "Mul", "Div"])
def test_float_binary_bit_exact(hip, op, sa, sb):
    rng = np.random.default_rng(hash((op, sa, sb)) & 0xffff)
    a = rng.standard_normal(sa).astype(np.float32)
    b = rng.standard_normal(sb).astype(np.float32)
    code = {"Add": O.ADD, "Sub": O.SUB, "Mul": O.MUL, "Div": O.DIV}[op]
    ref = O.binary(code, np.asarray(a), np.asarray(b))
    got = ok(getattr(HIP, op)(dev(a), dev(b)))
    assert_bits(got, ref)


@pytest.mark.parametrize("op", ["Add", "Sub", "Mul", "Div"])
def test_double_binary_bit_exact(hip, op):
    rng = np.random.default_rng(11)
    a = rng.standard_normal((6, 7, 9))
    b = rng.standard_normal((7, 1))
    code = {"Add": O.ADD, "Sub": O.SUB, "Mul": O.MUL, "Div": O.DIV}[op]
    assert_bits(ok(getattr(HIP, op)(dev(a), dev(b))), O.binary(code, a, b))


def test_float_special_values(hip):
    a = np.array([0.0, -0.0, np.inf, -np.inf, np.nan, 1e-40, -1e-45, 3.4e38, 1.0, -2.5, 1e-30, 7.0], np.float32)
    b = np.array([-0.0, 0.0, np.inf, 1.0, 2.0, 1e-40, 3.0, 10.0, 0.0, -0.0, 1e30, 3.0], np.float32)
    for op, code in [("Add", O.ADD), ("Sub", O.SUB), ("Mul", O.MUL), ("Div", O.DIV)]:
        assert_bits(ok(getattr(HIP, op)(dev(a), dev(b))), O.binary(code, a, b))


@pytest.mark.parametrize("dt", [np.int32, np.int64, np.uint8])
@pytest.mark.parametrize("op", ["Add", "Sub", "Mul", "Div"])
def test_int_binary_bit_exact(hip, op, dt):
    rng = np.random.default_rng(12)
    info = np.iinfo(dt)
    a = rng.integers(info.min, info.max, (9, 1, 130), dtype=dt, endpoint=True)
    b = rng.integers(info.min, info.max, (1, 5, 130), dtype=dt, endpoint=True)
    if op == "Div":
        b[b == 0] = 3
        if dt != np.uint8:
            a[0, 0, :4] = info.min  # MIN / -1 itself is covered by test_int_div_errors
    code = {"Add": O.ADD, "Sub": O.SUB, "Mul": O.MUL, "Div": O.DIV}[op]
    if op == "Div" and dt != np.uint8:
        b[b == -1] = 5
    assert_bits(ok(getattr(HIP, op)(dev(a), dev(b))), O.binary(code, a, b))


# Large outputs with one operand read once take the one-wave tile kernel (2 x 64 vectors per block): shapes
# past 2^16 vectors whose vector counts leave a partial last tile, operand A or B streamed, the other
# broadcast along rows, columns or both.
TILE_SHAPES = [
    ((67, 1531, 16), (1531, 16)),      # B broadcast along the outer axis
    ((3, 1, 262160), (3, 7, 262160)),  # A broadcast along the middle axis
    ((8191, 144), (8191, 1)),          # per-row statistic
    ((1, 96), (12007, 96)),            # A broadcast, B streamed
]


@pytest.mark.parametrize("sa,sb", TILE_SHAPES)
@pytest.mark.parametrize("dt", [np.float32, np.float64, np.int32, np.int64, np.uint8])
def test_binary_streamed_operand_tiles(hip, sa, sb, dt):
    rng = np.random.default_rng(hash((sa, sb, np.dtype(dt).str)) & 0xffff)
    if np.issubdtype(dt, np.floating):
        a, b = rng.standard_normal(sa).astype(dt), rng.standard_normal(sb).astype(dt)
    else:
        info = np.iinfo(dt)
        a = rng.integers(info.min, info.max, sa, dtype=dt, endpoint=True)
        b = rng.integers(info.min, info.max, sb, dtype=dt, endpoint=True)
        b[b == 0] = 3
        if dt != np.uint8:
            b[b == -1] = 5
    for op, code in (("Add", O.ADD), ("Sub", O.SUB), ("Mul", O.MUL), ("Div", O.DIV)):
        assert_bits(ok(getattr(HIP, op)(dev(a), dev(b))), O.binary(code, a, b))


# Arrays of 2^19 to 2^21 vectors run as one-wave tiles of 4 x 64 vectors (broadcast, same-shape and scalar
# layouts, casts): sizes at both ends of that window, with tails and partial tiles.
MID_VEC = {np.float32: 4, np.float64: 2, np.int32: 4, np.int64: 2, np.uint8: 16}


@pytest.mark.parametrize("dt", [np.float32, np.float64, np.int32, np.int64, np.uint8])
@pytest.mark.parametrize("edge", ["low", "high"])
def test_binary_mid_size_tiles(hip, dt, edge):
    vw = MID_VEC[dt]
    nvec = (1 << 19) + 77 if edge == "low" else (1 << 21) - 131
    n = nvec * vw + 3
    rows = 1031
    per_row = -(-(nvec * vw) // rows) if edge == "low" else (nvec * vw) // rows
    inner = (-(-per_row // vw) if edge == "low" else per_row // vw) * vw
    assert (1 << 19) <= rows * inner // vw < (1 << 21)
    rng = np.random.default_rng(nvec % 1000 + vw)
    def draw(shape):
        if np.issubdtype(dt, np.floating):
            return rng.standard_normal(shape).astype(dt)
        info = np.iinfo(dt)
        v = rng.integers(max(info.min, -1000), min(info.max, 1000), shape, dtype=dt, endpoint=True)
        v[v == 0] = 3
        if dt != np.uint8:
            v[v == -1] = 5
        return v
    a, b, c = draw(n), draw(n), draw(())
    m, r = draw((rows, inner)), draw((rows, 1))
    for op, code in (("Add", O.ADD), ("Sub", O.SUB), ("Mul", O.MUL), ("Div", O.DIV)):
        assert_bits(ok(getattr(HIP, op)(dev(a), dev(b))), O.binary(code, a, b))           # same shape
        assert_bits(ok(getattr(HIP, op)(dev(a), dev(c))), O.binary(code, a, c))           # scalar B
        assert_bits(ok(getattr(HIP, op)(dev(c), dev(b))), O.binary(code, c, b))           # scalar A
        if not (op == "Div" and dt in (np.int32, np.int64)):
            assert_bits(ok(getattr(HIP, op)(dev(m), dev(r))), O.binary(code, m, r))       # per-row operand


# Outputs built only from re-read broadcast operands, 8-byte elements, at least 2^20 vectors: 128-lane
# tiles of one vector per lane.  Even inner axes run two elements per vector, odd ones one; the vector
# counts are not multiples of 128.
@pytest.mark.parametrize("dt", [np.float64, np.int64])
@pytest.mark.parametrize("shape_a,shape_b", [((33, 1, 4002), (1, 17, 4002)), ((37, 1, 6001), (1, 29, 6001)),
                                              ((2, 1, 30, 1, 962), (1, 5, 1, 37, 962))])
def test_binary_wide_broadcast_8byte(hip, dt, shape_a, shape_b):
    rng = np.random.default_rng(sum(shape_a) + sum(shape_b))
    if dt == np.float64:
        a, b = rng.standard_normal(shape_a), rng.standard_normal(shape_b)
    else:
        a = rng.integers(-(1 << 40), 1 << 40, shape_a, dtype=np.int64)
        b = rng.integers(-(1 << 20), 1 << 20, shape_b, dtype=np.int64)
        a[a == 0], b[b == 0] = 3, 7
    a, b = a.astype(dt), b.astype(dt)
    assert np.broadcast_shapes(shape_a, shape_b) and np.prod(np.broadcast_shapes(shape_a, shape_b)) >= 1 << 21
    for op, code in (("Add", O.ADD), ("Sub", O.SUB), ("Mul", O.MUL), ("Div", O.DIV)):
        assert_bits(ok(getattr(HIP, op)(dev(a), dev(b))), O.binary(code, a, b))
        assert_bits(ok(getattr(HIP, op)(dev(b), dev(a))), O.binary(code, b, a))


def test_uint8_div_by_zero_in_mid_size_tiles(hip):
    n = ((1 << 19) + 5) * 16 + 7
    a = np.full(n, 200, np.uint8)
    for pos in [0, n // 2, n - 8, n - 1]:
        b = np.full(n, 7, np.uint8)
        b[pos] = 0
        r = HIP.Div(dev(a), dev(b))
        assert r.Status == OpStatus.Failure and r.Code == L.ERR_DIVIDE_BY_ZERO, pos


@pytest.mark.parametrize("src,to", [(np.float32, O.FLOAT), (np.int64, O.FLOAT), (np.float32, O.INT32),
                                    (np.int32, O.INT64), (np.float64, O.UINT8), (np.int64, O.INT32)])
def test_cast_mid_size_tiles(hip, src, to):
    narrow = min(np.dtype(src).itemsize, np.dtype(O.NP_OF[to]).itemsize)
    e = 16 // narrow
    rng = np.random.default_rng(int(e) + to)
    for nvec in [(1 << 19) + 9, (1 << 21) - 3]:
        n = nvec * e + 5
        if np.issubdtype(src, np.floating):
            x = (rng.standard_normal(n) * 50).astype(src)
        else:
            x = rng.integers(-100, 100, n, dtype=src)
        if to == O.UINT8:
            x = (np.abs(x) % 250).astype(src)
        assert_bits(ok(HIP.Cast(dev(x), to)), O.cast(x, to))
        if to in (O.INT32, O.UINT8) and src != np.int32:
            for pos in [0, n // 3, n - 1]:
                y = x.copy()
                y[pos] = 1e10 if np.issubdtype(src, np.floating) else 2 ** 40
                r = HIP.Cast(dev(y), to)
                assert r.Status == OpStatus.Failure and r.Code == L.ERR_OVERFLOW, pos


def test_uint8_div_by_zero_in_tiles(hip):
    """A zero divisor in a streamed uint8 operand fails the call with the reference's status, whichever tile
    holds it, and the next call succeeds."""
    a = np.full((8191, 1, 144), 200, np.uint8)
    for pos in [(0, 0, 0), (4096, 1, 64), (8190, 2, 143)]:
        b = np.full((8191, 3, 144), 7, np.uint8)
        b[pos] = 0
        r = HIP.Div(dev(a), dev(b))
        assert r.Status == OpStatus.Failure and r.Code == L.ERR_DIVIDE_BY_ZERO, pos
        assert "divide by zero" in r.Message
    b = np.full((8191, 3, 144), 7, np.uint8)
    assert_bits(ok(HIP.Div(dev(a), dev(b))), O.binary(O.DIV, a, b))


def test_int64_div_large_operands(hip):
    rng = np.random.default_rng(13)
    a = rng.integers(-(2**62), 2**62, 4099, dtype=np.int64)
    b = rng.integers(-(2**40), 2**40, 4099, dtype=np.int64)
    b[b == 0] = 1
    a[:100] = rng.integers(-(2**20), 2**20, 100)  # 32-bit fast path mixed in
    b[:50] = rng.integers(1, 1024, 50)
    assert_bits(ok(HIP.Div(dev(a), dev(b))), O.binary(O.DIV, a, b))


RAGGED_BINARY_SHAPES = [((262, 1023), (1023,)), ((262, 1023), (262, 1)), ((5, 1, 1023), (1, 7, 1023)),
                        ((9, 3), (4, 9, 3)), ((2, 3, 5, 1), (1, 1, 5, 7)), ((4001,), (1,)), ((33, 17), (17,)),
                        ((64, 1, 4095), (1, 256, 4095))]


@pytest.mark.parametrize("sa,sb", RAGGED_BINARY_SHAPES)
@pytest.mark.parametrize("dt", [np.float32, np.float64, np.uint8, np.int32, np.int64])
def test_binary_ragged_inner_axis(hip, sa, sb, dt):
    """Broadcast outputs whose inner axis is not a multiple of the vector width: whole 16-byte output
    vectors over the flat index, an operand of the output's shape read by vectors, a broadcast operand
    element by element across row boundaries (inner axes of 3 and 7 cross several per vector).  Bit-exact
    for all four ops; integer Div with a zero divisor reports DivideByZero as the reference does."""
    rng = np.random.default_rng(len(sa) * 100 + sa[-1])
    if np.dtype(dt).kind == "f":
        a, b = rng.standard_normal(sa).astype(dt), rng.standard_normal(sb).astype(dt)
    else:
        info = np.iinfo(dt)
        a = rng.integers(info.min, info.max, sa, dtype=dt, endpoint=True)
        b = rng.integers(1 if dt == np.uint8 else -1000, 1000, sb).astype(dt)
        b[b == 0] = 3
        if dt != np.uint8:
            b[b == -1] = 5
    for op, code in [("Add", O.ADD), ("Sub", O.SUB), ("Mul", O.MUL), ("Div", O.DIV)]:
        assert_bits(ok(getattr(HIP, op)(dev(a), dev(b))), O.binary(code, a, b))
    if np.dtype(dt).kind != "f" and b.size > 1:
        b0 = b.copy()
        b0.reshape(-1)[b0.size // 2] = 0
        r = HIP.Div(dev(a), dev(b0))
        assert r.Status == OpStatus.Failure and r.Code == L.ERR_DIVIDE_BY_ZERO


@pytest.mark.parametrize("dt", [np.int32, np.int64])
def test_int_div_reused_divisor(hip, dt):
    """Broadcast and scalar divisors, all magnitudes: bit-exact quotients,
    wide int64 operands, errors keep the first-element rule."""
    rng = np.random.default_rng(26)
    info = np.iinfo(dt)
    a = rng.integers(info.min, info.max, (40, 1, 96), dtype=dt, endpoint=True)
    b = rng.integers(-3000, 3000, (1, 24, 96), dtype=dt)
    b[b == 0] = 7
    b[0, 0, :8] = [1, -1, 2, -2, info.max, info.min, 3, -3]
    if dt == np.int64:
        b[0, 1, :4] = [2**40, -(2**40), 2**33 + 1, -(2**35)]
        a[1, 0, :4] = [2**20, -(2**31), 2**31 - 1, -(2**20)]
    a[0, 0, :6] = [info.min + 1, info.max, 0, -1, 1, info.min + 2]
    a[a == info.min] = info.min + 1  # MIN / -1 is the error case below
    assert_bits(ok(HIP.Div(dev(a), dev(b))), O.binary(O.DIV, a, b))
    for d in [1, -1, 7, -13, 1 << 20, info.max, info.min]:
        s = np.array(d, dt)
        assert_bits(ok(HIP.Div(dev(a), dev(s))), O.binary(O.DIV, a, s))
    b0 = b.copy()
    b0[0, 5, 3] = 0
    r = HIP.Div(dev(a), dev(b0))
    assert r.Code == L.ERR_DIVIDE_BY_ZERO
    a1 = a.copy()
    a1[2, 0, 1] = info.min  # meets divisor -1 at b[0, 0, 1]
    r = HIP.Div(dev(a1), dev(b))
    assert r.Code == L.ERR_OVERFLOW
    r = HIP.Div(dev(a1), dev(np.array(0, dt)))
    assert r.Code == L.ERR_DIVIDE_BY_ZERO


@pytest.mark.parametrize("dt", [np.int32, np.int64])
def test_int_div_quotients_next_to_multiples(hip, dt):
    """Dividends k*b - 1, k*b and k*b + b - 1 (and their negations) for divisors across the 32-bit range
    -- where a quotient computed through a reciprocal would first go wrong -- bit-exact."""
    rng = np.random.default_rng(27)
    b = np.concatenate([np.arange(1, 2049), rng.integers(2049, 2**31 - 1, 6000),
                        [2**31 - 1, 2**31 - 2, 2**30, 2**30 + 1, 65535, 65536, 65537]]).astype(np.int64)
    kmax = (2**31 - 1) // b
    k = np.minimum(rng.integers(0, 2**31, b.size) % (kmax + 1), kmax)
    cols = [k * b - 1, k * b, k * b + b - 1, kmax * b, kmax * b + (2**31 - 1 - kmax * b)]
    a = np.clip(np.stack(cols, 1), -(2**31) + 1, 2**31 - 1)
    bb = np.broadcast_to(b[:, None], a.shape)
    a = np.concatenate([a, -a, a, -a]).astype(dt)
    bb = np.concatenate([bb, bb, -bb, -bb]).astype(dt)
    a[:3, 0] = np.iinfo(np.int32).min   # |INT_MIN| = 2^31 over 1, 2, 3
    assert_bits(ok(HIP.Div(dev(a), dev(bb))), O.binary(O.DIV, a, bb))


@pytest.mark.parametrize("dt", [np.int32, np.int64])
@pytest.mark.parametrize("inner", [700003, 700004])
def test_int_div_large_broadcast(hip, dt, inner):
    """Over 2^20 vectors (several vectors per lane, loaded before they are divided), a ragged total and an
    inner axis that does / does not take 16-byte vectors: bit-exact, and the first failing element decides the
    error when the failures lie in a lane's later vectors (output rows 1 and 2 of 3)."""
    rng = np.random.default_rng(28)
    a = rng.integers(-(2**31), 2**31, (1, 2, inner), dtype=np.int64).astype(dt)
    b = rng.integers(-(2**31), 2**31, (3, 1, inner), dtype=np.int64).astype(dt)
    b[b == 0] = 9
    b[b == -1] = -9
    a[a == np.iinfo(dt).min] = 5
    assert_bits(ok(HIP.Div(dev(a), dev(b))), O.binary(O.DIV, a, b))
    for ovf_row, dbz_row, code in ((1, 2, L.ERR_OVERFLOW), (2, 1, L.ERR_DIVIDE_BY_ZERO)):
        a1, b1 = a.copy(), b.copy()
        k = inner // 3
        a1[0, 1, k], b1[ovf_row, 0, k] = np.iinfo(dt).min, -1   # fails at (ovf_row, 1, k) only
        b1[dbz_row, 0, 2 * k] = 0                                # fails at (dbz_row, 0 and 1, 2k)
        flat_a = np.broadcast_to(a1, (3, 2, inner)).reshape(-1)
        flat_b = np.broadcast_to(b1, (3, 2, inner)).reshape(-1)
        first_dbz = np.flatnonzero(flat_b == 0)[0]
        first_ovf = np.flatnonzero((flat_a == np.iinfo(dt).min) & (flat_b == -1))[0]
        assert (first_ovf < first_dbz) == (code == L.ERR_OVERFLOW)
        assert HIP.Div(dev(a1), dev(b1)).Code == code


@pytest.mark.parametrize("dt", [np.int32, np.int64])
@pytest.mark.parametrize("a_shape,b_shape", [((7, 3, 200004), (1, 3, 200004)),   # 16-byte vectors
                                             ((7, 3, 200003), (1, 3, 200003)),   # one element per vector
                                             ((5, 1, 4096), (1, 256, 4096)),     # C4's layout, 5 rows
                                             ((6, 4, 262148), (1, 4, 1))])       # divisor broadcast on the inner axis
def test_int_div_divisor_shared_along_the_outer_axis(hip, dt, a_shape, b_shape):
    """A divisor that is constant along the outermost output axis has its reciprocal computed once for several
    quotients (row counts 5-7: not a multiple of the rows per lane).  Bit-exact against the oracle, int64
    operands outside int32 take the 64-bit path, and the first failing element in output order decides the
    error."""
    rng = np.random.default_rng(29)
    a = rng.integers(-(2**31), 2**31, a_shape, dtype=np.int64)
    big = rng.integers(-(2**31), 2**31, b_shape, dtype=np.int64)
    b = np.where(rng.random(b_shape) < 0.5, rng.integers(-1000, 1001, b_shape), big)
    b[b == 0] = 9
    b[b == -1] = -9
    if dt == np.int64:
        a.flat[::101] *= 3**20
        b.flat[::103] = b.flat[::103] * 1000 + 1
    a, b = a.astype(dt), b.astype(dt)
    a[a == np.iinfo(dt).min] = 5
    assert_bits(ok(HIP.Div(dev(a), dev(b))), O.binary(O.DIV, a, b))
    out = np.broadcast_shapes(a_shape, b_shape)

    def at(shape, o):
        return tuple(o[d] if shape[d] > 1 else 0 for d in range(3))
    for o_ovf in ((0, 0, 1), tuple(n - 1 for n in out)):
        a1, b1 = a.copy(), b.copy()
        b1[at(b_shape, tuple(n // 2 for n in out))] = 0
        a1[at(a_shape, o_ovf)], b1[at(b_shape, o_ovf)] = np.iinfo(dt).min, -1
        flat_a = np.broadcast_to(a1, out).reshape(-1)
        flat_b = np.broadcast_to(b1, out).reshape(-1)
        first_dbz = np.flatnonzero(flat_b == 0)[0]
        first_ovf = np.flatnonzero((flat_a == np.iinfo(dt).min) & (flat_b == -1))[0]
        code = L.ERR_OVERFLOW if first_ovf < first_dbz else L.ERR_DIVIDE_BY_ZERO
        assert HIP.Div(dev(a1), dev(b1)).Code == code


@pytest.mark.parametrize("dt", [np.int32, np.int64, np.uint8])
@pytest.mark.parametrize("a_shape,b_shape", [((33, 1, 4096), (1, 16, 4096)),   # B 1/33 of the output
                                             ((17, 1, 4093), (1, 16, 4093)),   # ragged: B's tail outside the vectors
                                             ((16, 1, 4096), (1, 256, 4096))])  # 256 scan blocks (C4's B)
def test_int_div_divisor_scanned_before_the_quotients(hip, dt, a_shape, b_shape):
    """An eager integer Div whose divisor is at most 1/16 of its output scans the divisor first and returns
    once the scan finds neither 0 nor (signed) -1; otherwise it waits for the quotient kernel's record.  A
    0, and separately a -1 against MIN in A, at B's last element (the last output element) give the
    synchronous status and the oracle's error; a -1 with no MIN opposite it divides normally; clean calls
    before and after failing ones return their own status and the oracle's bits."""
    rng = np.random.default_rng(31)
    info = np.iinfo(dt)
    if dt == np.uint8:
        a = rng.integers(0, 256, a_shape).astype(dt)
        b = rng.integers(1, 256, b_shape).astype(dt)
    else:
        a = rng.integers(-(2**20), 2**20 + 1, a_shape).astype(dt)
        b = rng.integers(1, 1025, b_shape).astype(dt) * np.where(rng.random(b_shape) < 0.5, -1, 1).astype(dt)
    assert np.prod(b_shape) * 16 <= np.prod(np.broadcast_shapes(a_shape, b_shape))
    clean = O.binary(O.DIV, a, b)
    assert_bits(ok(HIP.Div(dev(a), dev(b))), clean)
    b0 = b.copy()
    b0.flat[-1] = 0
    r = HIP.Div(dev(a), dev(b0))
    assert r.Status == OpStatus.Failure and r.Code == L.ERR_DIVIDE_BY_ZERO, r.Message
    with pytest.raises(O.OracleError) as e:
        O.binary(O.DIV, a, b0)
    assert e.value.status == L.ERR_DIVIDE_BY_ZERO
    assert_bits(ok(HIP.Div(dev(a), dev(b))), clean)
    if dt != np.uint8:
        bm = b.copy()
        bm.flat[-1] = -1
        # -1 with no MIN in A: every quotient is defined
        assert_bits(ok(HIP.Div(dev(a), dev(bm))), O.binary(O.DIV, a, bm))
        am = a.copy()
        am.flat[-1] = info.min
        r = HIP.Div(dev(am), dev(bm))
        assert r.Status == OpStatus.Failure and r.Code == L.ERR_OVERFLOW, r.Message
        with pytest.raises(O.OracleError) as e:
            O.binary(O.DIV, am, bm)
        assert e.value.status == L.ERR_OVERFLOW
        # both: the zero comes first in output order
        bz = bm.copy()
        bz.flat[0] = 0
        assert HIP.Div(dev(am), dev(bz)).Code == L.ERR_DIVIDE_BY_ZERO
    assert_bits(ok(HIP.Div(dev(a), dev(b))), clean)


@pytest.mark.parametrize("dt", [np.int32, np.int64])
def test_int_div_errors(hip, dt):
    info = np.iinfo(dt)
    r = HIP.Div(dev(np.array([4, 5, 6, 7], dt)), dev(np.array([1, 2, 0, 1], dt)))
    assert r.Status == OpStatus.Failure and r.Code == L.ERR_DIVIDE_BY_ZERO
    assert "divide by zero" in r.Message
    r = HIP.Div(dev(np.array([info.min, 5], dt)), dev(np.array([-1, 2], dt)))
    assert r.Status == OpStatus.Failure and r.Code == L.ERR_OVERFLOW
    # the first failing element decides, as in the C# loop
    r = HIP.Div(dev(np.array([info.min, 5], dt)), dev(np.array([-1, 0], dt)))
    assert r.Code == L.ERR_OVERFLOW
    r = HIP.Div(dev(np.array([1, info.min], dt)), dev(np.array([0, -1], dt)))
    assert r.Code == L.ERR_DIVIDE_BY_ZERO
    # the device flags are reset: the next division succeeds
    ok(HIP.Div(dev(np.array([4], dt)), dev(np.array([2], dt))))


def test_operator_failures_mirror_reference(hip):
    a = dev(np.ones((1, 3), np.float32))
    r = HIP.Add(a, dev(np.ones((2,), np.float32)))
    assert r.Status == OpStatus.Failure and r.Code == L.ERR_CANNOT_BROADCAST
    assert "not compatible for broadcasting" in r.Message
    r = HIP.Add(a, dev(np.ones((1, 3), np.float64)))
    assert r.Code == L.ERR_WRONG_INPUT_TYPE
    r = HIP.Add(None, a)
    assert r.Code == L.ERR_MISSING_INPUT and "parameter A" in r.Message
    r = HIP.Pow(dev(np.ones(3, np.int32)), dev(np.ones(3, np.int32)))
    assert r.Code == L.ERR_INPUT_TYPE_NOT_SUPPORTED and "Int32" in r.Message
    r = HIP.Sqrt(dev(np.ones(3, np.int64)))
    assert r.Code == L.ERR_INPUT_TYPE_NOT_SUPPORTED
    r = HIP.Cast(a, 10)  # Float16
    assert r.Code == L.ERR_ATTRIBUTE_NOT_SUPPORTED
    r = HIP.ReduceMax(dev(np.ones(3, np.int32)), [0])
    assert r.Code == L.ERR_NOT_SUPPORTED
    r = HIP.ReduceSum(dev(np.ones((2, 3), np.float32)), [2])
    assert r.Code == L.ERR_INVALID_ARGUMENT
    r = HIP.Softmax(dev(np.ones((2, 3), np.float32)), 2)
    assert r.Code == L.ERR_INVALID_ARGUMENT


def test_reference_kats(hip):
    for k in KATS["broadcast_shape"]:
        r = HIP.Add(dev(np.ones(k["a"], np.float32)), dev(np.ones(k["b"], np.float32)))
        if k["out"] is None:
            assert r.Code == L.ERR_CANNOT_BROADCAST, k["src"]
        else:
            y = ok(r)
            assert y.shape == tuple(k["out"]) and np.all(y == 2.0), k["src"]
    k = KATS["add_int"]
    a = np.zeros(k["shape"], np.int32)
    a[tuple(k["set_index"])] = k["set_value"]
    c = ok(HIP.Add(dev(a), dev(a)))
    for e in k["expect"]:
        assert c[tuple(e["index"])] == e["value"]
    for name, op in [("sub_f32", "Sub"), ("mul_f32", "Mul"), ("div_f32", "Div")]:
        k = KATS[name]
        z = ok(getattr(HIP, op)(dev(np.array(k["x"], np.float32)), dev(np.array(k["y"], np.float32))))
        np.testing.assert_array_equal(z, np.array(k["z"], np.float32))
    for k in KATS["pow"]:
        z = ok(HIP.Pow(dev(np.array(k["x"], np.float32)), dev(np.array(k["y"], np.float32))))
        np.testing.assert_array_equal(z, np.array(k["z"], np.float32))
    for k in KATS["softmax"]:
        y = ok(HIP.Softmax(dev(np.array(k["x"], np.float32)), k["axis"]))
        np.testing.assert_almost_equal(y, np.array(k["y"], np.float32), decimal=k["decimal"])
    for k in KATS["reduce_sum_int"]:
        y = ok(HIP.ReduceSum(dev(np.array(k["data"], np.int32)), k["axes"], k["keepdims"]))
        np.testing.assert_array_equal(y, np.array(k["out"], np.int32))
    for k in KATS["reduce_mean_f32"]:
        y = ok(HIP.ReduceMean(dev(np.array(k["data"], np.float32)), k["axes"], k["keepdims"]))
        np.testing.assert_almost_equal(y, np.array(k["out"], np.float32), decimal=6)
    k = KATS["reduce_mean_double"]
    for c in k["cases"]:
        y = ok(HIP.ReduceMean(dev(np.array(k["data"], np.float64)), c["axes"]))
        np.testing.assert_almost_equal(y, np.array(c["out"]))
    k = KATS["cast_dtypes"]
    for to in k["to"]:
        y = ok(HIP.Cast(dev(np.array(k["input"], np.int64)), to))
        assert y.dtype == np.dtype(O.NP_OF[to])


def test_pow(hip):
    rng = np.random.default_rng(14)
    x = (rng.uniform(0, 1, 5000) / 2 + 0.5).astype(np.float32)
    y = (rng.uniform(-1, 1, 5000) / 2 + 0.5).astype(np.float32)
    got = ok(HIP.Pow(dev(x), dev(y)))
    assert ulps(got, O.binary(O.POW, x, y)).max() <= 2
    x2 = rng.standard_normal((64, 768)).astype(np.float32) * 3
    two = np.array(2.0, np.float32)
    got2 = ok(HIP.Pow(dev(x2), dev(two)))
    # exponent 2 evaluates x*x; host powf(x, 2) differs by at most 1 ulp
    assert ulps(got2, O.binary(O.POW, x2, two)).max() <= 1
    np.testing.assert_array_equal(got2, x2 * x2)
    xn = np.array([-2.0, -2.0, 0.0, 0.0, 1.0, np.nan, -1.0, 4.0], np.float32)
    yn = np.array([3.0, 0.5, -1.0, 0.0, np.nan, 0.0, np.inf, -0.5], np.float32)
    g, r = ok(HIP.Pow(dev(xn), dev(yn))), O.binary(O.POW, xn, yn)
    same = (g == r) | (np.isnan(g) & np.isnan(r))
    assert same.all(), (g, r)


def _pow_cases(rng, n):
    """Pairs over the regimes of powf: positive bases with exponents up to |y| = 100, negative bases with
    integer exponents (sign from the exponent's parity), results that overflow to inf or underflow through
    the denormals to 0, and bases near 1."""
    q = n // 5
    x = [np.exp(rng.uniform(-2.3, 2.3, q)), -np.exp(rng.uniform(-2.3, 2.3, q)), rng.uniform(0.5, 2.0, q),
         np.exp(rng.uniform(2.3, 7, q)), np.exp(rng.uniform(-12, -7, n - 4 * q))]
    y = [rng.uniform(-30, 30, q), rng.integers(-40, 41, q).astype(np.float64), rng.uniform(-100, 100, q),
         rng.uniform(10, 20, q), rng.uniform(8, 16, n - 4 * q)]
    return np.concatenate(x).astype(np.float32), np.concatenate(y).astype(np.float32)


def test_pow_wide(hip):
    """10^6 pairs against the host powf within 2 ulp: the device evaluates (float)pow((double)x, (double)y),
    the double result within about one double ulp, so one float rounding from the correctly rounded float;
    overflow, underflow (denormals included), signs of negative bases and NaN for negative bases with
    non-integer exponents agree exactly."""
    rng = np.random.default_rng(16)
    x, y = _pow_cases(rng, 10**6)
    got = ok(HIP.Pow(dev(x), dev(y)))
    ref = O.binary(O.POW, x, y)
    nan = np.isnan(ref)
    np.testing.assert_array_equal(np.isnan(got), nan)
    np.testing.assert_array_equal(np.isinf(got), np.isinf(ref))
    fin = ~nan & np.isfinite(ref)
    assert np.array_equal(np.signbit(got[fin]), np.signbit(ref[fin]))
    u = ulps(got[fin], ref[fin])
    assert u.max() <= 2, (u.max(), x[fin][np.argmax(u)], y[fin][np.argmax(u)])
    # the regimes are all present: overflow, exact zeros from underflow, denormals, negative results
    assert np.isinf(ref).sum() > 1000 and (ref == 0).sum() > 1000
    assert ((ref != 0) & (np.abs(ref) < np.finfo(np.float32).tiny)).sum() > 100 and (ref < 0).sum() > 10000
    # negative bases with non-integer exponents: NaN
    xn = -np.exp(rng.uniform(-2, 2, 10000)).astype(np.float32)
    yn = (rng.integers(-20, 20, 10000) + 0.5).astype(np.float32)
    assert np.isnan(ok(HIP.Pow(dev(xn), dev(yn)))).all() and np.isnan(O.binary(O.POW, xn, yn)).all()


def test_sqrt_bit_exact(hip):
    rng = np.random.default_rng(15)
    x = np.concatenate([rng.uniform(0, 1e6, 100000), [0.0, -0.0, 1e-45, 1e-40, np.inf, -1.0, np.nan]]).astype(np.float32)
    assert_bits(ok(HIP.Sqrt(dev(x))), O.unary(O.SQRT, x))
    bits = np.arange(0, 1 << 31, 4093, dtype=np.uint32).view(np.float32)  # positive floats, all exponents
    assert_bits(ok(HIP.Sqrt(dev(bits))), O.unary(O.SQRT, bits))


def test_erf_bit_exact(hip):
    rng = np.random.default_rng(16)
    x = np.concatenate([rng.standard_normal(200000) / np.sqrt(2), np.linspace(-6, 6, 50001),
                        [0.0, -0.0, 1e-6, -1e-6, 1e-40, np.inf, -np.inf, np.nan, 9.5, -9.5, 1e-3]]).astype(np.float32)
    got = ok(HIP.Erf(dev(x)))
    ref = O.unary(O.ERF, x)
    same = (got.view(np.uint32) == ref.view(np.uint32)) | (np.isnan(got) & np.isnan(ref))
    assert same.all(), f"{(~same).sum()} mismatches, max ulp {ulps(got[~same], ref[~same]).max()}"
    bits = np.arange(0, 1 << 32, 65521, dtype=np.uint64).astype(np.uint32).view(np.float32)
    g2, r2 = ok(HIP.Erf(dev(bits))), O.unary(O.ERF, bits)
    same = (g2.view(np.uint32) == r2.view(np.uint32)) | (np.isnan(g2) & np.isnan(r2))
    assert same.all()


def test_erf_double(hip):
    """MathOps.Erf(double) with the device's double exp against the formula with the host's exp.  The result
    is 1 - P with P = poly * t * exp(-x^2) <= 1, and a one-ulp difference of the exponential moves P by at most
    one ulp of 1 (2^-53), so the bar is 2 ulp at the scale max(|erf|, 0.5), the granularity of 1 - P: within
    2 ulp of erf itself wherever |erf| >= 0.5, within 2^-52 absolute below."""
    rng = np.random.default_rng(17)
    x = np.concatenate([np.linspace(-6, 6, 20001), rng.standard_normal(200000), rng.uniform(-1e-3, 1e-3, 20000),
                        [0.0, -0.0, 1e-300, -1e-300, 30.0, -30.0]])
    got = ok(HIP.Erf(dev(x)))
    ref = O.unary(O.ERF, x)
    scale = np.spacing(np.maximum(np.abs(ref), 0.5))
    err = np.abs(got - ref) / scale
    assert err.max() <= 2, (err.max(), x[np.argmax(err)])
    # the formula's values at the ends: at 0 the coefficients sum to 0.999999999, so erf(+-0) = 1e-9 (sign +1
    # for -0 too, as x < 0 is false); erf(+-30) = +-1
    assert got[-6] == ref[-6] == got[-5] and abs(got[-6] - 1e-9) < 1e-16 and got[-2] == 1.0 and got[-1] == -1.0
    xn = np.array([np.nan, np.inf, -np.inf])
    gn = ok(HIP.Erf(dev(xn)))
    assert np.isnan(gn[0]) and gn[1] == 1.0 and gn[2] == -1.0


CAST_TYPES = [O.FLOAT, O.DOUBLE, O.UINT8, O.INT8, O.UINT16, O.INT16, O.INT32, O.UINT32, O.INT64, O.UINT64, O.BOOL]


def _cast_inputs(src, rng):
    dt = np.dtype(O.NP_OF[src])
    if dt == np.bool_:
        return rng.integers(0, 2, 517).astype(np.bool_)
    if dt.kind == "f":
        return np.concatenate([rng.uniform(-3, 300, 500), [0.5, 1.5, 2.5, -0.5, -0.4, 254.5, 255.5]]).astype(dt)
    info = np.iinfo(dt)
    lo, hi = max(info.min, -200), min(info.max, 300)
    return rng.integers(lo, hi, 517, dtype=dt, endpoint=True)


@pytest.mark.parametrize("src", CAST_TYPES)
def test_cast_matrix(hip, src):
    rng = np.random.default_rng(17 + src)
    x = _cast_inputs(src, rng)
    for dst in CAST_TYPES:
        r = HIP.Cast(dev(x), dst)
        try:
            ref = O.cast(x, dst)
        except O.OracleError as e:
            assert r.Status == OpStatus.Failure and r.Code == e.status, (src, dst)
            continue
        assert_bits(ok(r), ref)


def test_cast_int64_to_float_rounding(hip):
    rng = np.random.default_rng(18)
    x = rng.integers(-(2**62), 2**62, 100000, dtype=np.int64)
    x[:1000] = rng.integers(-(2**25), 2**25, 1000)
    x[1000:1010] = [2**24 + 1, 2**24 + 3, 2**53 + 1, -(2**53) - 3, 2**63 - 1, -(2**63), 0, -1, 1, 2**25 + 2]
    assert_bits(ok(HIP.Cast(dev(x), O.FLOAT)), O.cast(x, O.FLOAT))


def test_checked_calls_in_a_row_report_their_own_status(hip):
    """Integer Div, Gather and narrowing Cast share one device error record; after each eager check the
    read-back leaves it cleared, and the next check starts from that.  A failure is never reported again by
    a later call, and a success never hides a later failure."""
    a = np.arange(1, 9, dtype=np.int32)
    table = np.arange(12, dtype=np.float32).reshape(4, 3)
    steps = [
        ("div", lambda: HIP.Div(dev(a), dev(np.full(8, 2, np.int32))), None),
        ("div by zero", lambda: HIP.Div(dev(a), dev(np.array([1, 2, 3, 0, 5, 6, 7, 8], np.int32))),
         L.ERR_DIVIDE_BY_ZERO),
        ("gather", lambda: HIP.Gather(dev(table), dev(np.array([3, -4, 0], np.int64)), 0), None),
        ("gather out of range", lambda: HIP.Gather(dev(table), dev(np.array([1, 4], np.int64)), 0),
         L.ERR_INVALID_ARGUMENT),
        ("gather out of range again", lambda: HIP.Gather(dev(table), dev(np.array([-5], np.int64)), 0),
         L.ERR_INVALID_ARGUMENT),
        ("cast", lambda: HIP.Cast(dev(np.array([1.5, -2.5], np.float64)), O.INT32), None),
        ("cast overflow", lambda: HIP.Cast(dev(np.array([300], np.int32)), O.UINT8), L.ERR_OVERFLOW),
        ("div overflow", lambda: HIP.Div(dev(np.array([-(2**31)], np.int32)), dev(np.array([-1], np.int32))),
         L.ERR_OVERFLOW),
        ("div after failures", lambda: HIP.Div(dev(a), dev(np.full(8, 3, np.int32))), None),
        ("cast after", lambda: HIP.Cast(dev(np.array([255], np.int32)), O.UINT8), None),
    ]
    for _ in range(2):
        for name, call, code in steps:
            r = call()
            if code is None:
                assert r.Status == OpStatus.Success, (name, r.Message)
            else:
                assert r.Status == OpStatus.Failure and r.Code == code, (name, r.Code, r.Message)
    assert_bits(ok(HIP.Div(dev(a), dev(np.full(8, -3, np.int32)))), O.binary(O.DIV, a, np.full(8, -3, np.int32)))


def test_cast_overflow_errors(hip):
    for vals, dt, to in [([1.0, 2147483647.5], np.float64, O.INT32), ([np.nan], np.float32, O.INT64),
                         ([300], np.int32, O.UINT8), ([-1], np.int64, O.UINT64), ([2**40], np.int64, O.INT32)]:
        r = HIP.Cast(dev(np.array(vals, dt)), to)
        assert r.Status == OpStatus.Failure and r.Code == L.ERR_OVERFLOW, (vals, to)
        assert "too large or too small" in r.Message


REDUCE_CASES = [
    ((64, 768), [-1]),
    ((8, 512, 768), [-1]),
    ((3, 50000), [1]),            # long rows, split path
    ((2, 700001), [1]),           # long ragged rows
    ((16, 300, 64), [1]),         # strided middle axis
    ((4, 4096, 33), [1]),         # ragged inner
    ((256, 64, 256), [1]),
    ((300, 777, 256), [1]),       # whole 1 KB rows per tile, unsplit
    ((5, 4096, 192), [1]),        # whole rows per tile, split over row slices
    ((3, 300, 1040), [1]),        # wide rows over 256+ reduced rows: 512-lane blocks
    ((5, 6, 7, 8), [0, 2]),       # two passes
    ((5, 6, 7, 8), [3, 1]),
    ((4, 5, 6), None),            # all axes
    ((3000000,), None),           # full reduction, split
    ((7, 1, 9), [1]),             # size-1 reduced axis
    ((6, 0, 4), [1]),             # empty reduced axis
]


@pytest.mark.parametrize("shape,axes", REDUCE_CASES)
@pytest.mark.parametrize("kd", [1, 0])
def test_reduce_float(hip, shape, axes, kd):
    rng = np.random.default_rng(19)
    x = rng.uniform(-1, 1, shape).astype(np.float32)
    ax = tuple(range(len(shape))) if axes is None else tuple(a % len(shape) for a in axes)
    absum = np.abs(x.astype(np.float64)).sum(axis=ax, keepdims=bool(kd))
    for name, code in [("ReduceSum", O.RSUM), ("ReduceMean", O.RMEAN), ("ReduceMax", O.RMAX)]:
        got = ok(getattr(HIP, name)(dev(x), axes, kd))
        ref = O.reduce(code, x, axes, bool(kd))
        if name == "ReduceMax":
            assert_bits(got, ref)
        elif name == "ReduceMean":
            r = max(1, int(np.prod([shape[a] for a in ax])))
            if 0 in shape:
                assert got.shape == ref.shape
                np.testing.assert_array_equal(np.isnan(got), np.isnan(ref))
            else:
                assert_reduction(got, ref, absum / r)
        else:
            assert_reduction(got, ref, absum)


@pytest.mark.parametrize("dt", [np.int32, np.int64])
@pytest.mark.parametrize("shape,axes", [((64, 256, 40), [1]), ((8, 300, 1032), [1]), ((9, 777), [-1]), ((3, 4, 5, 6), [0, 2]), ((2, 300000), None),
                                        ((2, 5, 3), [1])])
def test_reduce_int_exact(hip, dt, shape, axes):
    rng = np.random.default_rng(20)
    info = np.iinfo(dt)
    x = rng.integers(info.min // 2, info.max // 2, shape, dtype=dt)
    for name, code in [("ReduceSum", O.RSUM), ("ReduceMean", O.RMEAN)]:
        assert_bits(ok(getattr(HIP, name)(dev(x), axes)), O.reduce(code, x, axes, True))


def test_reduce_double(hip):
    rng = np.random.default_rng(21)
    x = rng.standard_normal((33, 1000, 17))
    for name, code in [("ReduceSum", O.RSUM), ("ReduceMean", O.RMEAN), ("ReduceMax", O.RMAX)]:
        got = ok(getattr(HIP, name)(dev(x), [1]))
        ref = O.reduce(code, x, [1], True)
        np.testing.assert_allclose(got, ref, rtol=0, atol=1e-12)


RAGGED_REDUCE_CASES = [
    ((7, 1), [-1]), ((7, 3), [-1]), ((7, 5), [-1]), ((9, 63), [-1]), ((9, 65), [-1]), ((9, 1023), [-1]),
    ((1031, 1), [-1]), ((1031, 4), [-1]), ((1031, 7), [-1]), ((1031, 16), [-1]), ((777, 49), [-1]),   # L lanes
    ((1031, 64), [-1]), ((515, 128), [-1]), ((515, 100), [-1]), ((4097, 2), [-1]), ((3, 5, 33), [-1]),  # per row
    ((5, 8191), [-1]), ((3, 8193), [-1]), ((3, 100003), [-1]),   # row per wave, split rows (r > 8192)
    ((1000001,), None), ((3000003,), None), ((2, 3, 1000001), None),  # whole tensors not a multiple of 4
    ((5, 1000, 255), [1]), ((3, 77, 49), [1]), ((2, 3001, 7), [1]), ((64, 3, 1022), [1]),  # inner not % 4
]


@pytest.mark.parametrize("shape,axes", RAGGED_REDUCE_CASES)
@pytest.mark.parametrize("dt", [np.float32, np.float64, np.int32, np.int64])
def test_reduce_ragged_rows_and_columns(hip, shape, axes, dt):
    """Rows whose length is not a multiple of the vector width (an unaligned head and a tail read element
    by element around whole 16-byte vectors; several rows, so every head length occurs), whole tensors of
    such sizes (the split row kernel), and column reductions over an inner axis of such a width."""
    rng = np.random.default_rng(sum(shape))
    if np.dtype(dt).kind == "f":
        x = rng.uniform(-1, 1, shape).astype(dt)
    else:
        x = rng.integers(-(2**20), 2**20, shape).astype(dt)
    ax = tuple(range(len(shape))) if axes is None else tuple(a % len(shape) for a in axes)
    absum = np.abs(x.astype(np.float64)).sum(axis=ax, keepdims=True)
    names = [("ReduceSum", O.RSUM), ("ReduceMean", O.RMEAN)] + ([("ReduceMax", O.RMAX)] if np.dtype(dt).kind == "f" else [])
    for name, code in names:
        got = ok(getattr(HIP, name)(dev(x), axes, 1))
        ref = O.reduce(code, x, axes, True)
        if name == "ReduceMax" or np.dtype(dt).kind != "f":
            assert_bits(got, ref)
        else:
            r = int(np.prod([shape[a] for a in ax]))
            assert_reduction(got, ref, absum / (r if name == "ReduceMean" else 1))


def test_reduce_max_seed_zero_and_nan(hip):
    x = np.array([[-3, -1, -2], [1, np.nan, 5], [np.nan, np.nan, -1]], np.float32)
    assert_bits(ok(HIP.ReduceMax(dev(x), [1])), O.reduce(O.RMAX, x, [1], True))


@pytest.mark.parametrize("shape,axis", [((64, 512), -1), ((5, 12, 77, 128), -1), ((10, 2048), -1), ((4, 3001), 1),
                                        ((3, 4, 5), 0), ((6, 100, 7), 1), ((2, 3, 1000), 1), ((9, 3), -1)])
@pytest.mark.parametrize("dt", [np.float32, np.float64])
def test_softmax(hip, shape, axis, dt):
    rng = np.random.default_rng(22)
    x = (rng.standard_normal(shape) * 3).astype(dt)
    got = ok(HIP.Softmax(dev(x), axis))
    ref = O.softmax(x, axis)
    err = np.abs(got.astype(np.float64) - ref)
    assert np.all(err <= 1e-5 * np.abs(ref) + 1e-30), err.max()


def test_softmax_default_axis_and_masked_rows(hip):
    x = np.full((4, 64), -20000.0, np.float32)  # every row below the seed 0 of ReduceMax
    x[1, 3] = 5.0
    got = ok(HIP.Softmax(dev(x)))
    ref = O.softmax(x, -1)
    # rows below the ReduceMax seed 0 underflow to a zero sum: 0/0 = NaN as in
    # the reference; the one-hot row is exact
    np.testing.assert_array_equal(np.isnan(got), np.isnan(ref))
    assert np.isnan(ref[0]).all() and not np.isnan(ref[1]).any()
    assert_bits(got[1], ref[1])


@pytest.mark.parametrize("r", [256, 512, 768, 500, 96])
def test_softmax_special_values_in_rows(hip, r):
    """Rows holding a quiet NaN, a signalling NaN, +-0, +-inf and all-negative values, on the straight-line
    path (rows that fill the wave's vectors: 256, 512, 768) and the bounded one: the NaN rows, the infinite
    rows and the finite ones come out as the reference's five-step composite gives them."""
    rng = np.random.default_rng(28)
    x = (rng.standard_normal((12, r)) * 3).astype(np.float32)
    x[0, 5] = np.nan                                             # quiet NaN: the whole row NaN
    x[1, 7] = np.uint32(0x7f800001).view(np.float32)             # signalling NaN: the whole row NaN
    x[2, :] = -np.abs(x[2, :]) - 1.0                             # max below the seed 0
    x[2, 3] = -0.0
    x[3, :] = 0.0                                                # all zeros, one -0
    x[3, 9] = -0.0
    x[4, 11] = np.inf                                            # +inf: inf - inf = NaN
    x[5, 13] = -np.inf                                           # -inf: exp(-inf) = 0
    x[6, :] = -30000.0                                           # every entry below the seed: 0 / 0
    got = ok(HIP.Softmax(dev(x), -1))
    ref = O.softmax(x, -1)
    nan = np.isnan(ref)
    np.testing.assert_array_equal(np.isnan(got), nan)
    assert nan[0].all() and nan[1].all() and nan[4].all() and nan[6].all() and not nan[5].any()
    err = np.abs(got.astype(np.float64) - ref)[~nan]
    assert np.all(err <= 1e-5 * np.abs(ref[~nan]) + 1e-30), err.max()


@pytest.mark.parametrize("s_shape,m_shape", [((4, 3, 64, 512), (4, 1, 1, 512)), ((2, 3, 5, 96), (3, 1, 96)),
                                             ((2, 8, 128), (8, 1)), ((6, 77), (77,)), ((3, 4, 5, 6), (3, 4, 5, 6)),
                                             ((2, 2, 4000), (2, 1, 4000))])
def test_add_softmax(hip, s_shape, m_shape):
    rng = np.random.default_rng(23)
    s = (rng.standard_normal(s_shape) * 3).astype(np.float32)
    m = np.where(rng.uniform(size=m_shape) < 0.125, -10000.0, 0.0).astype(np.float32)
    got = ok(HIP.AddSoftmax(dev(s), dev(m), -1))
    ref = O.add_softmax(s, m, -1)
    # a row masked everywhere stays below the ReduceMax seed 0: exp underflows
    # to 0 for every entry and 0/0 gives NaN, in the reference as here
    nan = np.isnan(ref)
    np.testing.assert_array_equal(np.isnan(got), nan)
    err = np.abs(got.astype(np.float64) - ref)[~nan]
    assert np.all(err <= 1e-5 * np.abs(ref[~nan]) + 1e-30), err.max()


@pytest.mark.parametrize("s_shape,m_shape", [((3, 5, 1001, 64), (3, 1, 1, 64)), ((2, 7, 999, 128), (2, 1, 999, 1)),
                                             ((5, 2003, 96), (5, 1, 96)), ((2, 7, 4999, 64), (2, 1, 4999, 1))])
def test_add_softmax_mask_rows_change_along_the_rows(hip, s_shape, m_shape):
    """Mask rows that change part-way through a block's rows (odd rows per batch), a mask that changes on
    every row ([b, 1, q, 1], broadcast along the row), and more rows than the row kernel has waves (69,986
    rows: waves take a second row, whose mask row differs from their first)."""
    rng = np.random.default_rng(31)
    s = (rng.standard_normal(s_shape) * 3).astype(np.float32)
    m = np.where(rng.uniform(size=m_shape) < 0.125, -10000.0, rng.uniform(-1, 1, size=m_shape)).astype(np.float32)
    got = ok(HIP.AddSoftmax(dev(s), dev(m), -1))
    ref = O.add_softmax(s, m, -1)
    nan = np.isnan(ref)
    np.testing.assert_array_equal(np.isnan(got), nan)
    err = np.abs(got.astype(np.float64) - ref)[~nan]
    assert np.all(err <= 1e-5 * np.abs(ref[~nan]) + 1e-30), err.max()


def softmax_close(got, ref, pre):
    """got within 1e-5 * |ref| of the reference's Softmax of `pre` (the scores after any Div / Add node),
    beyond the reference's own rounding: its serial float sum of a long row is up to ~1e-4 relative away
    from the exact sum (8e-5 at 65535 N(0, 3) entries), which no other order of the sum can reproduce.  So
    |got - ref| <= 1e-5 |ref| + |ref - truth|, truth being the same Softmax in float64 (seed-0 max, NaN rows
    NaN): whatever the device gets within 1e-5 of the truth passes, and the bar is 1e-5 where the
    reference's sum is exact enough."""
    nan = np.isnan(ref)
    np.testing.assert_array_equal(np.isnan(got), nan)
    p = pre.astype(np.float64)
    with np.errstate(all="ignore"):
        m = np.fmax(np.max(np.where(np.isnan(p), -np.inf, p), -1, keepdims=True), 0.0)
        e = np.exp(p - m)
        truth = e / e.sum(-1, keepdims=True)
    slack = np.abs(ref.astype(np.float64) - truth)
    err = np.abs(got.astype(np.float64) - ref)
    bad = ~nan & ~(err <= 1e-5 * np.abs(ref) + slack + 1e-30)
    assert not bad.any(), (np.flatnonzero(bad)[:5], err[bad][:5], ref[bad][:5])


SOFTMAX_ROW_LENGTHS = [1, 2, 3, 4, 5, 7, 8, 16, 31, 49, 63, 64, 65, 100, 127, 128, 129, 255, 256, 257, 513, 1023,
                       2047, 2049, 2051, 2052, 4093, 4097, 8191, 8195, 16389, 32767, 32771, 65535, 65539, 70001]


@pytest.mark.parametrize("r", SOFTMAX_ROW_LENGTHS)
@pytest.mark.parametrize("dt", [np.float32, np.float64])
def test_softmax_any_row_length(hip, r, dt):
    """Rows of every length class: short rows with L lanes per row (several rows per wave), row per wave
    (whole vectors, or an unaligned head and a tail held one element per lane), row per block in registers
    (256 or 1024 lanes, 4 to 16 vectors each), and the three-pass kernel beyond.  1031 short rows or seven
    long ones, so every head length 0..3 occurs; special values in the head, the tail and the body."""
    rng = np.random.default_rng(r)
    x = (rng.standard_normal((1031 if r <= 256 else 7, r)) * 3).astype(dt)
    if r >= 16:
        x[1, 0] = np.nan                   # in the first row's head or first vector
        x[2, r - 1] = np.inf               # in a tail: inf - inf = NaN
        x[3, r - 2] = -np.inf              # exp(-inf) = 0
        x[4, :] = -30000.0                 # below the seed 0: 0 / 0
        x[5, r // 2] = 80.0                # one dominant entry
    got = ok(HIP.Softmax(dev(x), -1))
    softmax_close(got, O.softmax(x, -1), x)


@pytest.mark.parametrize("r", [3, 7, 49, 64, 70, 128, 513, 1023, 2049, 4093, 9001, 32771])
@pytest.mark.parametrize("dt", [np.float32, np.float64])
def test_add_softmax_any_row_length(hip, r, dt):
    """A mask row contiguous along the row whose rows start off 16-byte boundaries ([b, 1, 1, r] with r not
    a multiple of 4: read by elements), a mask broadcast along the row ([b, h, q, 1]) and a scale, on every
    row kernel: bit-identical to the Div / Add / Softmax nodes and within the bar of the oracle."""
    rng = np.random.default_rng(r + 7)
    q = 37 if r <= 128 else 3
    s = (rng.standard_normal((2, 3, q, r)) * 3).astype(dt)
    for mshape in [(2, 1, 1, r), (2, 3, q, 1), (r,)]:
        m = np.where(rng.uniform(size=mshape) < 0.125, -10000.0, rng.uniform(-1, 1, mshape)).astype(dt)
        got = ok(HIP.AddSoftmax(dev(s), dev(m), -1))
        softmax_close(got, O.add_softmax(s, m, -1), O.binary(O.ADD, s, m))
        c = np.array(8.0, dt)
        r2 = HIP.ScaleAddSoftmax(dev(s), dev(c), True, dev(m))
        assert r2.Status == OpStatus.Success, r2.Message
        t = HIP.Add(HIP.Div(dev(s), dev(c)).Outputs[0], dev(m)).Outputs[0]
        assert_bits(r2.Outputs[0].to_numpy(), ok(HIP.Softmax(t, -1)))


def test_device_reciprocal_is_correctly_rounded(hip):
    """The Erf / GELU reciprocal (v_rcp_f32 seed, one float Newton step) equals
    IEEE 1.0f / d on the device for every float d in [1, 2^126): the step
    repairs every seed v_rcp_f32 gives one ulp off (about a tenth of them), and
    v_rcp_f32 is exact at the 33 significands per binade where a one-ulp seed
    would not be repaired (the host enumeration finds exactly those)."""
    lib = ctypes.CDLL(os.path.join(HERE, "native", "librcp_check.so"))
    out = (ctypes.c_longlong * 3)()
    assert lib.lx_test_device_recip(out) == 0
    assert out[0] == 0, f"{out[0]} reciprocals differ from 1/d ({out[1]} seeds off by one ulp)"
    assert out[1] > 0   # the check sees off-by-one seeds: the Newton step is doing work


def test_device_rcp_f32_error_bound(hip):
    """v_rcp_f32 is within 2^-22 relative of 1/d for every float d in [1, 2^31]: with the 2^-24 of rounding an
    int32 divisor to float, the integer-division seed stays inside the 2^-21 that the host check of
    sdiv32_core proves sufficient (tests/test_host_abi.py)."""
    lib = ctypes.CDLL(os.path.join(HERE, "native", "librcp_check.so"))
    out = ctypes.c_double()
    assert lib.lx_test_device_rcp_error(ctypes.byref(out)) == 0
    print(f"v_rcp_f32 largest relative error on [1, 2^31]: {out.value:.3g} (2^{np.log2(out.value):.2f})")
    assert 0 < out.value <= 2.0 ** -22


@pytest.mark.parametrize("offset", [0, 1])
def test_table_maps_at_tile_edges(hip, offset):
    """GELU and Erf run in one-wave blocks over tiles of 2 x 64 vectors: sizes on both sides of every
    tile, vector and wave edge, the scalar tail, and (offset 1) pointers 4 bytes past 16-byte alignment,
    which take the one-float-per-vector form.  Bits equal the oracle's; the float before and after the
    output stay untouched."""
    rng = np.random.default_rng(31 + offset)
    for n in [1, 3, 4, 5, 63, 64, 65, 127, 128, 129, 255, 256, 257, 511, 512, 513, 4099, 65536 + 7]:
        x = (rng.standard_normal(n) * 3).astype(np.float32)
        x[rng.integers(0, n, max(1, n // 50))] = np.float32(np.inf)
        # x at the start of a (256-byte aligned) allocation, or one float into it
        pad = np.full(offset, 7.0, np.float32)
        buf = dev(np.concatenate([pad, x, [7.0, 7.0]]).astype(np.float32))
        base = buf.h.data + 4 * offset
        for op, ref in (("GeluErf", O.gelu_erf(x)), ("Erf", O.unary(O.ERF, x))):
            out = dev(np.full(n + 2, 9.0, np.float32))
            xo = DeviceTensor.wrap(base, (n,), np.float32, 4 * n, keepalive=buf)
            yo = DeviceTensor.wrap(out.h.data + 4 * offset, (n,), np.float32, 4 * n, keepalive=out)
            r = getattr(HIP, op)(xo, out=yo)
            assert r.Status == OpStatus.Success, r.Message
            full = out.to_numpy()
            got = full[offset:offset + n]
            same = (got.view(np.uint32) == ref.view(np.uint32)) | (np.isnan(got) & np.isnan(ref))
            assert same.all(), f"{op} n={n} offset={offset}: {(~same).sum()} mismatches"
            guard = np.delete(full, np.arange(offset, offset + n))
            assert (guard == 9.0).all(), f"{op} n={n} offset={offset} wrote outside its output"


def test_gelu_chain_bit_exact(hip):
    rng = np.random.default_rng(24)
    x = np.concatenate([rng.standard_normal(300001), [0.0, -0.0, 1e-7, -8.0, 8.0, np.inf, -np.inf]]).astype(np.float32)
    assert_bits(ok(HIP.GeluErf(dev(x))), O.gelu_erf(x))
    # the same chain op by op through the C ABI
    sq2 = np.array(np.float32(np.sqrt(2.0)), np.float32)
    a = ok(HIP.Div(dev(x), dev(sq2)))
    e = ok(HIP.Erf(dev(a)))
    b = ok(HIP.Add(dev(e), dev(np.array(1.0, np.float32))))
    c = ok(HIP.Mul(dev(x), dev(b)))
    y = ok(HIP.Mul(dev(c), dev(np.array(0.5, np.float32))))
    assert_bits(y, O.gelu_erf(x))


@pytest.mark.parametrize("shape", [(8, 512, 768), (3, 5, 1024), (7, 4096), (4, 12), (2, 3, 770)])
def test_layernorm(hip, shape):
    rng = np.random.default_rng(25)
    r = shape[-1]
    x = (rng.standard_normal(shape) * 2).astype(np.float32)
    g = (1 + 0.02 * rng.standard_normal(r)).astype(np.float32)
    b = (0.02 * rng.standard_normal(r)).astype(np.float32)
    got = ok(HIP.LayerNormDecomposed(dev(x), dev(g), dev(b), 1e-12))
    ref = O.layernorm_decomposed(x, g, b, np.float32(1e-12))
    # mean / variance are sums in a different order: 1e-5 relative to max(1, |y|)
    err = np.abs(got.astype(np.float64) - ref)
    assert np.all(err <= 1e-5 * np.maximum(1.0, np.abs(ref))), err.max()


@pytest.mark.parametrize("r", [1, 2, 3, 4, 5, 7, 8, 16, 31, 49, 64, 100, 127, 128, 255, 257, 1023, 2049, 4093, 4099,
                               4100])
def test_layernorm_any_row_length(hip, r):
    """Every row-length class of the fused LayerNorm: short rows with L lanes per row (several rows per
    wave, 1031 rows so every head length and partial waves occur), rows of any length with an unaligned
    head and a tail (gamma / beta read element by element where a row's vectors are off their 16-byte
    boundaries), the wave-per-row kernel, and beyond 4099 the nine nodes."""
    rng = np.random.default_rng(r + 3)
    rows = 1031 if r <= 256 else 9
    x = (rng.standard_normal((rows, r)) * 2).astype(np.float32)
    g = (1 + 0.02 * rng.standard_normal(r)).astype(np.float32)
    b = (0.02 * rng.standard_normal(r)).astype(np.float32)
    got = ok(HIP.LayerNormDecomposed(dev(x), dev(g), dev(b), 1e-12))
    ref = O.layernorm_decomposed(x, g, b, np.float32(1e-12))
    err = np.abs(got.astype(np.float64) - ref)
    assert np.all(err <= 1e-5 * np.maximum(1.0, np.abs(ref))), err.max()


def _layernorm_nodes(x, g, b):
    """The nine operators one by one through the C ABI (what the reference's graph runs)."""
    two, eps, ax = dev(np.array(2.0, np.float32)), dev(np.array(1e-12, np.float32)), [-1]
    X = dev(x)
    mean = HIP.ReduceMean(X, ax, 1).Outputs[0]
    d = HIP.Sub(X, mean).Outputs[0]
    p = HIP.Pow(d, two).Outputs[0]
    var = HIP.ReduceMean(p, ax, 1).Outputs[0]
    sd = HIP.Sqrt(HIP.Add(var, eps).Outputs[0]).Outputs[0]
    m = HIP.Mul(HIP.Div(d, sd).Outputs[0], dev(g))
    if m.Status != OpStatus.Success:
        return m
    return HIP.Add(m.Outputs[0], dev(b))


@pytest.mark.parametrize("xs,gs,bs,expect", [
    ((8, 512, 768), (768, 1), (768,), "cannot"),     # Mul [8,512,768] x [768,1]: 512 vs 768
    ((4, 16, 768), (2, 384), (768,), "cannot"),      # same element count, other shape
    ((4, 16, 768), (768,), (1, 2, 384), "cannot"),   # beta of the wrong shape
    ((768, 768), (768, 1), (768,), "columns"),       # gamma broadcast down the columns
    ((64, 64), (64,), (64, 1), "columns"),           # beta down the columns
    ((8, 512, 768), (1, 1, 768), (1, 768), "fused"),  # leading ones: the fused kernel's shape
])
def test_layernorm_affine_shapes_follow_the_nodes(hip, xs, gs, bs, expect):
    """The fused LayerNorm applies gamma / beta along the last axis; any other affine shape must give what
    the reference's Mul / Add nodes give: CannotBroadcast (ITensor.cs:113-117) or their broadcast."""
    rng = np.random.default_rng(26)
    x = (rng.standard_normal(xs) * 2).astype(np.float32)
    g = (1 + 0.02 * rng.standard_normal(gs)).astype(np.float32)
    b = (0.02 * rng.standard_normal(bs)).astype(np.float32)
    r = HIP.LayerNormDecomposed(dev(x), dev(g), dev(b), 1e-12)
    if expect == "cannot":
        assert r.Code == L.ERR_CANNOT_BROADCAST, (r.Code, r.Message)
        with pytest.raises(O.OracleError):
            O.layernorm_decomposed(x, g, b, np.float32(1e-12))
        return
    assert r.Status == OpStatus.Success, r.Message
    got = r.Outputs[0].to_numpy()
    ref = O.layernorm_decomposed(x, g, b, np.float32(1e-12))
    assert got.shape == ref.shape == x.shape
    err = np.abs(got.astype(np.float64) - ref)
    assert np.all(err <= 1e-5 * np.maximum(1.0, np.abs(ref))), err.max()
    if expect == "columns":
        # not the last-axis application: the node-by-node path, bit for bit
        assert_bits(got, ok(_layernorm_nodes(x, g, b)))
        wrong = O.layernorm_decomposed(x, g.reshape(-1), b.reshape(-1), np.float32(1e-12))
        assert np.abs(wrong - ref).max() > 1e-3


def test_output_reuse_and_capacity(hip):
    a = dev(np.arange(12, dtype=np.float32).reshape(3, 4))
    out = DeviceTensor.empty((3, 4), np.float32)
    r = HIP.Add(a, a, out=out)
    assert r.Status == OpStatus.Success and r.Outputs[0].h.data == out.h.data
    np.testing.assert_array_equal(out.to_numpy(), 2 * np.arange(12, dtype=np.float32).reshape(3, 4))
    small = DeviceTensor.empty((2,), np.float32)
    r = HIP.Add(a, a, out=small)
    assert r.Code == L.ERR_BUFFER_TOO_SMALL


def test_reshape_alias(hip):
    a = dev(np.arange(24, dtype=np.float32))
    v = a.reshape((2, 3, 4))
    assert v.shape == (2, 3, 4) and v.h.data == a.h.data
    y = ok(HIP.ReduceSum(v, [2], 0))
    np.testing.assert_array_equal(y, np.arange(24, dtype=np.float32).reshape(2, 3, 4).sum(2))


def test_read_probe_folds_what_it_reads(hip):
    """lx_read_probe, the read-ceiling diagnostic: with g blocks (one per 1024 16-byte vectors, at most
    out_bytes / 4), block b writes the XOR of every vector v with (v mod 1024 g) // 1024 == b.  Checked against
    a numpy fold of the same words with a partial last block, with grids clipped by out_bytes, and an out
    pointer that is not 4-byte aligned is refused."""
    rng = np.random.default_rng(41)
    nv = 10 * 1024 + 37
    words = rng.integers(0, 2**32, nv * 4, dtype=np.uint64).astype(np.uint32)
    src = dev(words)
    vx = np.bitwise_xor.reduce(words.reshape(nv, 4), axis=1)
    lib = L.lib()
    for g in (11, 3, 1):
        out = DeviceTensor.from_numpy(np.full(g + 2, 0xDEADBEEF, np.uint32))
        assert lib.lx_read_probe(ctypes.c_void_p(src.h.data), nv * 16, ctypes.c_void_p(out.h.data), 4 * g) == L.OK
        got = out.to_numpy()
        want = np.zeros(g, np.uint32)
        blk = (np.arange(nv) % (1024 * g)) // 1024
        for b in range(g):
            want[b] = np.bitwise_xor.reduce(vx[blk == b])
        assert np.array_equal(got[:g], want), g
        assert np.all(got[g:] == 0xDEADBEEF), g
    out = DeviceTensor.from_numpy(np.zeros(4, np.uint32))
    assert lib.lx_read_probe(ctypes.c_void_p(src.h.data), nv * 16, ctypes.c_void_p(out.h.data + 2), 8) == \
        L.ERR_INVALID_ARGUMENT
    assert "4-byte aligned" in L.last_error()
