"""Randomised differential tests: many small random cases per operator family, the HIP path against the CPU
oracle on the same inputs.  Results are compared bit for bit (integer ops, Cast, float elementwise ops, data
movement; a NaN matches any NaN) or within the reduction / Softmax bars, and where the reference fails
(shapes that do not broadcast, integer division by zero or MIN / -1, casts out of range, gather indices out
of range) the device must fail with the same status.  Shapes are drawn with ranks 0-5 and dimensions 1-7,
broadcast operands with dropped leading axes and size-1 axes, values with special values mixed in.  Seeded:
every run draws the same cases."""
import numpy as np
import pytest

from onnx_amd import DeviceTensor, HipExecutionProvider as HIP, OpStatus
from oracle import oracle as O

pytestmark = pytest.mark.gpu

FLOATS = (np.float32, np.float64)
CAST_TYPES = [O.FLOAT, O.DOUBLE, O.UINT8, O.INT8, O.UINT16, O.INT16, O.INT32, O.UINT32, O.INT64, O.UINT64, O.BOOL]


def dev(a):
    return DeviceTensor.from_numpy(np.asarray(a))


def same_bits(got, ref):
    """Bit-equal arrays of one shape and dtype, any NaN matching any NaN."""
    if got.shape != ref.shape or got.dtype != ref.dtype:
        return False
    if got.dtype.kind == "f":
        nan = np.isnan(ref)
        if not np.array_equal(np.isnan(got), nan):
            return False
        g, r = got[~nan], ref[~nan]
        return np.array_equal(g.view(np.uint8) if g.size else g, r.view(np.uint8) if r.size else r)
    return np.array_equal(got, ref)


def check(r, oracle_fn, compare, case):
    """The device result r against the oracle: equal statuses when the oracle fails, else compare()."""
    try:
        ref = oracle_fn()
    except O.OracleError as e:
        assert r.Status != OpStatus.Success and r.Code == e.status, (case, r.Code, e.status, r.Message)
        return
    assert r.Status == OpStatus.Success, (case, r.Message)
    got = r.Outputs[0].to_numpy()
    assert compare(got, ref), (case, got, ref)


def rand_shape(rng, rmin=0, rmax=5, dmax=7):
    return tuple(int(d) for d in rng.integers(1, dmax + 1, int(rng.integers(rmin, rmax + 1))))


def broadcast_pair(rng):
    out = rand_shape(rng)

    def operand():
        r = int(rng.integers(0, len(out) + 1))
        return tuple(1 if rng.random() < 0.3 else d for d in out[len(out) - r:])
    a, b = operand(), operand()
    if rng.random() < 0.1 and len(b) > 0:  # a pair that does not broadcast (when a dimension can clash)
        k = int(rng.integers(0, len(b)))
        b = b[:k] + (b[k] + 1 if b[k] > 1 else 2,) + b[k + 1:]
    return a, b


def values(rng, shape, dt, special=0.05):
    if np.dtype(dt).kind == "f":
        x = np.array(rng.standard_normal(shape) * 10.0 ** rng.uniform(-3, 3, shape), dt)
        if x.size:
            m = np.asarray(rng.random(x.shape) < special)
            pool = np.array([0.0, -0.0, np.inf, -np.inf, np.nan, 1e-40, -3e-39, 1.0, -1.0], dt)
            x[m] = pool[rng.integers(0, pool.size, int(m.sum()))]
        return np.asarray(x, dt)
    if dt == np.bool_:
        return rng.random(shape) < 0.5
    info = np.iinfo(dt)
    return np.asarray(rng.integers(info.min, info.max, shape, dtype=dt, endpoint=True))


def divisors(rng, shape, dt):
    """Divisors for integer Div: mostly small magnitudes, with zeros and -1 now and then."""
    if np.dtype(dt).kind == "f":
        return values(rng, shape, dt)
    info = np.iinfo(dt)
    lo = -1000 if info.min < 0 else 0
    b = np.asarray(rng.integers(lo, 1000, shape, dtype=np.int64), np.int64)
    if b.size:
        b = np.where(b == 0, 7, b)
        m = rng.random(b.shape)
        b = np.where(m < 0.03, 0, b)
        if info.min < 0:
            b = np.where((m >= 0.03) & (m < 0.06), -1, b)
        big = rng.integers(info.min // 2 + 1, info.max // 2, b.shape, dtype=np.int64) if info.max > 2**31 else b
        b = np.where((m >= 0.06) & (m < 0.12), big, b)
    return np.asarray(b, dt)


def dividends(rng, shape, dt):
    a = values(rng, shape, dt)
    if np.dtype(dt).kind == "i" and a.size:  # MIN now and then, to meet a divisor of -1
        a = np.where(rng.random(a.shape) < 0.05, np.iinfo(dt).min, a).astype(dt)
    return np.asarray(a, dt)


@pytest.mark.parametrize("dt", [np.float32, np.float64, np.uint8, np.int32, np.int64])
@pytest.mark.parametrize("op", ["Add", "Sub", "Mul", "Div"])
def test_binary_random(hip, op, dt):
    rng = np.random.default_rng([11, ["Add", "Sub", "Mul", "Div"].index(op), np.dtype(dt).num])
    code = {"Add": O.ADD, "Sub": O.SUB, "Mul": O.MUL, "Div": O.DIV}[op]
    for case in range(150):
        sa, sb = broadcast_pair(rng)
        if op == "Div":
            a, b = dividends(rng, sa, dt), divisors(rng, sb, dt)
        else:
            a, b = values(rng, sa, dt), values(rng, sb, dt)
        r = getattr(HIP, op)(dev(a), dev(b))
        check(r, lambda: O.binary(code, a, b), same_bits, (op, dt, sa, sb, case))


def large_broadcast_pair(rng, vw):
    """An output of 2^18 to 2^23 elements (about 2^16 to 2^21 vectors: the one-wave tile paths), ranks 2-4,
    the inner axis a whole number of 16-byte vectors or not, each axis held by one operand or both."""
    r = int(rng.integers(2, 5))
    total = int(2 ** rng.uniform(18, 23))
    lead = [int(d) for d in rng.integers(2, 12, r - 1)]
    inner = max(1, total // int(np.prod(lead)))
    if rng.random() < 0.7:
        inner = max(vw, inner // vw * vw)
    out = tuple(lead + [inner])

    # per axis: which operand holds it (the other broadcasts it), so the output is `out` itself; half the time
    # one operand holds every axis (it is read once); leading axes broadcast may also be dropped
    owner = rng.integers(0, 3, r)   # 0: both, 1: a only, 2: b only
    if rng.random() < 0.5:
        owner = np.where(owner == 2, 0, owner)
    a = [d if o != 2 else 1 for d, o in zip(out, owner)]
    b = [d if o != 1 else 1 for d, o in zip(out, owner)]
    while len(a) > 0 and a[0] == 1 and rng.random() < 0.5:
        a = a[1:]
    while len(b) > 0 and b[0] == 1 and rng.random() < 0.5:
        b = b[1:]
    if rng.random() < 0.5:
        a, b = b, a
    return tuple(a), tuple(b)


@pytest.mark.parametrize("dt", [np.float32, np.float64, np.uint8, np.int32, np.int64])
def test_binary_random_large(hip, dt):
    """Random broadcast pairs at the sizes of the tile kernels, every op, bit for bit against the oracle."""
    rng = np.random.default_rng([14, np.dtype(dt).num])
    vw = 16 // np.dtype(dt).itemsize
    for case in range(24):
        op = ["Add", "Sub", "Mul", "Div"][case % 4]
        code = {"Add": O.ADD, "Sub": O.SUB, "Mul": O.MUL, "Div": O.DIV}[op]
        sa, sb = large_broadcast_pair(rng, vw)
        if op == "Div":
            a, b = dividends(rng, sa, dt), divisors(rng, sb, dt)
        else:
            a, b = values(rng, sa, dt), values(rng, sb, dt)
        r = getattr(HIP, op)(dev(a), dev(b))
        check(r, lambda: O.binary(code, a, b), same_bits, (op, dt, sa, sb, case))


@pytest.mark.parametrize("dt", [np.uint8, np.int32, np.int64])
def test_int_div_small_divisor_random(hip, dt):
    """Integer Div whose divisor is at most 1/16 of the output, the shapes on which an eager call scans the
    divisor and returns once it holds no 0 (and, signed, no -1): half the divisors are clean, the others hold
    one 0, or one -1 with or without MIN at a random position of A; the status and the bits are the oracle's
    (the first failing element in output order decides the error)."""
    rng = np.random.default_rng([17, np.dtype(dt).num])
    info = np.iinfo(dt)
    signed = info.min < 0
    for case in range(60):
        r = int(rng.integers(2, 5))
        out = [int(d) for d in rng.integers(2, 9, r)]
        out[-1] = int(rng.integers(1, 300))
        if rng.random() < 0.5:
            out[-1] = out[-1] // 16 * 16 + 16
        # the divisor keeps the inner axis and some of the others, the dividend the rest (or all)
        keep = rng.random(r) < 0.4
        keep[-1] = True
        keep[0] = False
        sb = tuple(d if k else 1 for d, k in zip(out, keep))
        sa = tuple(out) if rng.random() < 0.5 else tuple(1 if k and i < r - 1 else d for i, (d, k) in enumerate(zip(out, keep)))
        n_out = int(np.prod(np.broadcast_shapes(sa, sb)))
        if np.prod(sb) * 16 > n_out:
            sa = (16,) + sa
            n_out *= 16
        a = dividends(rng, sa, dt) if signed else values(rng, sa, dt)
        lo = 1 if not signed else -1000
        b = rng.integers(lo, 1001, sb).astype(np.int64)
        b = np.where((b == 0) | (b == -1), 3, b).astype(dt)
        if signed:
            a = np.where(a == info.min, 5, a).astype(dt)
        kind = rng.random()
        if kind < 0.5:
            pass
        elif kind < 0.7 or not signed:
            b.flat[int(rng.integers(0, b.size))] = 0
        else:
            b.flat[int(rng.integers(0, b.size))] = -1
            if rng.random() < 0.6:
                a.flat[int(rng.integers(0, a.size))] = info.min
        r_ = HIP.Div(dev(a), dev(b))
        check(r_, lambda: O.binary(O.DIV, a, b), same_bits, ("Div", dt, sa, sb, case))


def reduction_bar(dt):
    def compare(got, ref, x_abs):
        if got.shape != ref.shape:
            return False
        nan = np.isnan(ref)
        if not np.array_equal(np.isnan(got), nan):
            return False
        err = np.abs(got.astype(np.float64) - ref.astype(np.float64))[~nan]
        return bool(np.all(err <= (1e-5 if dt == np.float32 else 1e-12) * x_abs[~nan] + 1e-30))
    return compare


@pytest.mark.parametrize("dt", [np.float32, np.float64, np.int32, np.int64])
@pytest.mark.parametrize("op", ["ReduceSum", "ReduceMean", "ReduceMax"])
def test_reduce_random(hip, op, dt):
    rng = np.random.default_rng([12, ["ReduceSum", "ReduceMean", "ReduceMax"].index(op), np.dtype(dt).num])
    code = {"ReduceSum": O.RSUM, "ReduceMean": O.RMEAN, "ReduceMax": O.RMAX}[op]
    for case in range(150):
        shape = rand_shape(rng, 1, 4, 9)
        x = values(rng, shape, dt, special=0.0) if np.dtype(dt).kind == "f" else \
            np.asarray(rng.integers(-(2**20), 2**20, shape), dt)
        r_ = len(shape)
        k = int(rng.integers(0, r_ + 1))
        axes = None if k == 0 else [int(a) - (r_ if rng.random() < 0.3 else 0)
                                    for a in rng.choice(r_, size=k, replace=False)]
        kd = int(rng.integers(0, 2))
        r = getattr(HIP, op)(dev(x), axes, kd)
        ax = tuple(range(r_)) if axes is None else tuple(a % r_ for a in axes)
        if np.dtype(dt).kind != "f" or op == "ReduceMax":
            compare = same_bits
        else:
            x_abs = np.abs(x.astype(np.float64)).sum(axis=ax, keepdims=bool(kd))
            if op == "ReduceMean":
                x_abs = x_abs / max(1, int(np.prod([shape[a] for a in ax])))
            bar = reduction_bar(dt)
            compare = lambda got, ref, bar=bar, x_abs=x_abs: bar(got, ref, np.asarray(x_abs))  # noqa: E731
        check(r, lambda: O.reduce(code, x, axes, bool(kd)), compare, (op, dt, shape, axes, kd, case))


def large_reduce_case(rng, vw):
    """A shape of 2^14 to 2^22 elements and the axes to reduce, drawn to reach each reduction plan: long rows
    split over blocks (a few rows of more than 8192 elements), many short rows, column reductions with narrow
    (at most 64 vectors) and wide inner axes, few output columns (rows split into slices), and two reduced
    axis groups (two passes).  Dimensions are multiples of the vector width or ragged."""
    def dim(lo, hi):
        d = int(rng.integers(lo, hi + 1))
        return d - d % vw + (0 if rng.random() < 0.5 else int(rng.integers(1, vw))) if d > vw else d
    kind = int(rng.integers(0, 6))
    if kind == 0:    # long rows, few of them
        shape, axes = (int(rng.integers(1, 33)), dim(8193, 120000)), [-1]
    elif kind == 1:  # many short rows
        shape, axes = (int(rng.integers(2000, 30000)), dim(1, 150)), [1]
    elif kind == 2:  # columns, narrow inner axis
        shape, axes = (int(rng.integers(1, 40)), int(rng.integers(200, 3000)), dim(1, 64 * vw)), [1]
    elif kind == 3:  # columns, wide inner axis
        shape, axes = (int(rng.integers(1, 6)), int(rng.integers(256, 1200)), dim(64 * vw + 1, 3000)), [1]
    elif kind == 4:  # few output columns: rows cut into slices
        shape, axes = (int(rng.integers(1, 3)), int(rng.integers(5000, 60000)), dim(1, 24)), [-2]
    else:            # two reduced groups
        shape, axes = (int(rng.integers(2, 9)), int(rng.integers(2, 50)), int(rng.integers(2, 9)), dim(100, 2000)), [0, 2]
    n = int(np.prod(shape))
    if n > (1 << 22):
        shape = (max(1, shape[0] * (1 << 22) // n),) + shape[1:]
    return shape, axes


@pytest.mark.parametrize("dt", [np.float32, np.float64, np.int32, np.int64])
@pytest.mark.parametrize("op", ["ReduceSum", "ReduceMean", "ReduceMax"])
def test_reduce_random_large(hip, op, dt):
    """Random shapes at the sizes where the reduction planner picks its split-row, row-group, whole-row-tile,
    wide-column and row-slice kernels: bit for bit for integers and ReduceMax, within the reduction bar for
    float sums and means."""
    rng = np.random.default_rng([16, ["ReduceSum", "ReduceMean", "ReduceMax"].index(op), np.dtype(dt).num])
    code = {"ReduceSum": O.RSUM, "ReduceMean": O.RMEAN, "ReduceMax": O.RMAX}[op]
    vw = 16 // np.dtype(dt).itemsize
    for case in range(18):
        shape, axes = large_reduce_case(rng, vw)
        x = values(rng, shape, dt, special=0.0) if np.dtype(dt).kind == "f" else \
            np.asarray(rng.integers(-(2**20), 2**20, shape), dt)
        kd = case % 2
        r = getattr(HIP, op)(dev(x), axes, kd)
        ax = tuple(a % len(shape) for a in axes)
        if np.dtype(dt).kind != "f" or op == "ReduceMax":
            compare = same_bits
        else:
            x_abs = np.abs(x.astype(np.float64)).sum(axis=ax, keepdims=bool(kd))
            if op == "ReduceMean":
                x_abs = x_abs / int(np.prod([shape[a] for a in ax]))
            bar = reduction_bar(dt)
            compare = lambda got, ref, bar=bar, x_abs=x_abs: bar(got, ref, np.asarray(x_abs))  # noqa: E731
        check(r, lambda: O.reduce(code, x, axes, bool(kd)), compare, (op, dt, shape, axes, kd, case))


@pytest.mark.parametrize("dt", FLOATS)
def test_softmax_random(hip, dt):
    rng = np.random.default_rng([13, np.dtype(dt).num])
    for case in range(200):
        shape = rand_shape(rng, 1, 4, 9)
        x = (rng.standard_normal(shape) * 4).astype(dt)
        axis = int(rng.integers(-len(shape), len(shape)))
        r = HIP.Softmax(dev(x), axis)

        def compare(got, ref):
            nan = np.isnan(ref)
            if got.shape != ref.shape or not np.array_equal(np.isnan(got), nan):
                return False
            err = np.abs(got.astype(np.float64) - ref)[~nan]
            return bool(np.all(err <= 1e-5 * np.abs(ref[~nan]) + 1e-30))
        check(r, lambda: O.softmax(x, axis), compare, (dt, shape, axis, case))


@pytest.mark.parametrize("dt", FLOATS)
def test_softmax_random_large(hip, dt):
    """Rows of 1 to 6000 elements, up to 2^21 elements in all, along the last axis or an inner one (ragged
    and vector-aligned rows alike): within 1e-5 |ref| of the oracle beyond the reference's own rounding.
    The reference sums a row serially in float32, which drifts up to ~1e-5 relative from the exact sum over
    a few thousand N(0, 4) entries (1.08e-5 on a row of 2703), an error no other summation order can
    reproduce; so |got - ref| <= 1e-5 |ref| + |ref - truth|, truth being the same Softmax in float64 (seed-0
    max), the rule of the fixed-shape Softmax tests."""
    rng = np.random.default_rng([17, np.dtype(dt).num])
    for case in range(30):
        n = int(rng.integers(1, 6001))
        if case % 3 == 2:
            shape, axis = (int(rng.integers(1, 9)), n, int(rng.integers(1, 40))), 1
        else:
            shape, axis = (int(rng.integers(1, 6)), int(rng.integers(1, max(2, (1 << 21) // n // 5))), n), -1
        x = (rng.standard_normal(shape) * 4).astype(dt)
        r = HIP.Softmax(dev(x), axis)

        def compare(got, ref, x=x, axis=axis):
            nan = np.isnan(ref)
            if got.shape != ref.shape or not np.array_equal(np.isnan(got), nan):
                return False
            p = x.astype(np.float64)
            m = np.fmax(p.max(axis=axis, keepdims=True), 0.0)
            e = np.exp(p - m)
            truth = e / e.sum(axis=axis, keepdims=True)
            slack = np.abs(ref.astype(np.float64) - truth)
            err = np.abs(got.astype(np.float64) - ref)
            return bool(np.all((err <= 1e-5 * np.abs(ref) + slack + 1e-30)[~nan]))
        check(r, lambda: O.softmax(x, axis), compare, (dt, shape, axis, case))


def test_cast_random(hip):
    rng = np.random.default_rng(14)
    for case in range(400):
        src, dst = (int(v) for v in rng.choice(CAST_TYPES, 2))
        shape = rand_shape(rng, 0, 3, 9)
        dt = O.NP_OF[src]
        if np.dtype(dt).kind == "f":
            x = values(rng, shape, dt)
            x = np.asarray(x * np.asarray(10.0 ** rng.integers(0, 12, shape), dt), dt) if x.size else x
        else:
            x = values(rng, shape, dt)
        r = HIP.Cast(dev(x), dst)
        check(r, lambda: O.cast(x, dst), same_bits, (src, dst, shape, case))


MOVE_TYPES = [np.float32, np.float64, np.uint8, np.int16, np.int32, np.int64, np.bool_]


def test_transpose_random(hip):
    rng = np.random.default_rng(15)
    for case in range(200):
        dt = MOVE_TYPES[case % len(MOVE_TYPES)]
        shape = rand_shape(rng, 0, 5, 7)
        x = values(rng, shape, dt, special=0.0)
        perm = None if rng.random() < 0.2 else [int(p) - (len(shape) if rng.random() < 0.3 else 0)
                                                for p in rng.permutation(len(shape))]
        r = HIP.Transpose(dev(x), perm)
        check(r, lambda: O.transpose(x, perm), same_bits, (dt, shape, perm, case))


def test_slice_random(hip):
    rng = np.random.default_rng(16)
    for case in range(250):
        dt = MOVE_TYPES[case % len(MOVE_TYPES)]
        shape = rand_shape(rng, 1, 4, 9)
        x = values(rng, shape, dt, special=0.0)
        r_ = len(shape)
        n = int(rng.integers(1, r_ + 1))
        axes = [int(a) for a in rng.choice(r_, size=n, replace=False)]
        starts = [int(rng.integers(-12, 12)) for _ in range(n)]
        ends = [int(rng.integers(-12, 12)) for _ in range(n)]
        steps = [int(rng.choice([-3, -2, -1, 1, 2, 3])) for _ in range(n)]
        ax = [a - r_ if rng.random() < 0.3 else a for a in axes]
        r = HIP.Slice(dev(x), starts, ends, ax, steps)
        check(r, lambda: O.slice_(x, starts, ends, ax, steps), same_bits, (dt, shape, starts, ends, ax, steps, case))


def test_gather_random(hip):
    rng = np.random.default_rng(17)
    for case in range(250):
        dt = MOVE_TYPES[case % len(MOVE_TYPES)]
        shape = rand_shape(rng, 1, 4, 7)
        x = values(rng, shape, dt, special=0.0)
        axis = int(rng.integers(-len(shape), len(shape)))
        dim = shape[axis]
        ishape = rand_shape(rng, 0, min(2, len(shape)), 5)
        lo, hi = (-dim - 1, dim + 1) if rng.random() < 0.2 else (-dim, dim)
        idx = np.asarray(rng.integers(lo, hi, ishape), np.int64 if rng.random() < 0.5 else np.int32)
        r = HIP.Gather(dev(x), dev(idx), axis)
        check(r, lambda: O.gather(x, idx, axis), same_bits, (dt, shape, axis, ishape, case))


def test_concat_random(hip):
    rng = np.random.default_rng(18)
    for case in range(200):
        dt = MOVE_TYPES[case % len(MOVE_TYPES)]
        shape = rand_shape(rng, 1, 4, 6)
        axis = int(rng.integers(-len(shape), len(shape)))
        xs = []
        for _ in range(int(rng.integers(2, 5))):
            s = list(shape)
            s[axis] = int(rng.integers(1, 6))
            xs.append(values(rng, tuple(s), dt, special=0.0))
        r = HIP.Concat([dev(v) for v in xs], axis)
        check(r, lambda: O.concat(xs, axis), same_bits, (dt, shape, axis, case))


def matmul_case(rng):
    """Operands of a random MatMul: ranks 1-4, batch axes that broadcast (size 1 or missing), rows and columns
    across the tile edges, K across the direct-load kernel's, the split's and the batch fold's conditions; one
    case in twenty with mismatched inner dimensions."""
    m = int(rng.choice([1, 2, 5, 8, 31, 32, 33, 63, 64, 65, 100, 130, 200]))
    n = int(rng.choice([1, 3, 4, 8, 20, 32, 36, 64, 68, 100, 128, 196]))
    k = int(rng.choice([1, 3, 8, 16, 32, 64, 100, 128, 192, 256, 384, 512, 1024]))
    nb = int(rng.integers(0, 3))
    batch = tuple(int(d) for d in rng.integers(1, 4, nb))
    sa = tuple(1 if rng.random() < 0.3 else d for d in batch[int(rng.integers(0, nb + 1)):]) + (m, k)
    sb = tuple(1 if rng.random() < 0.3 else d for d in batch[int(rng.integers(0, nb + 1)):]) + (k, n)
    if rng.random() < 0.05:
        sb = sb[:-2] + (k + 1, n)
    if rng.random() < 0.08:  # a rank-1 operand (the reference's element-wise broadcast rule)
        if rng.random() < 0.5:
            sa = (k,)
        else:
            sb = (k,)
    return sa, sb


@pytest.mark.parametrize("dt", [np.float32, np.float64, np.int32])
def test_matmul_random(hip, dt):
    """Random MatMuls against the oracle: Int32 bit-exact (wrapping), Float / Double within 1e-5 (1e-13) of
    sum |a b| per output, the oracle's status where the shapes fail; for Float, MatMulAdd (a bias row, and a
    residual of the product's shape) bit for bit the MatMul and the Add nodes."""
    rng = np.random.default_rng({np.float32: 70, np.float64: 71, np.int32: 72}[dt])
    tol = 1e-5 if dt == np.float32 else 1e-13
    for case in range(160):
        sa, sb = matmul_case(rng)
        if dt == np.int32:
            a = rng.integers(-1000, 1000, sa).astype(dt)
            b = rng.integers(-1000, 1000, sb).astype(dt)
        else:
            a = rng.standard_normal(sa).astype(dt)
            b = rng.standard_normal(sb).astype(dt)
        r = HIP.MatMul(dev(a), dev(b))
        try:
            ref = O.matmul(a, b)
        except O.OracleError as e:
            assert r.Status != OpStatus.Success and r.Code == e.status, (case, sa, sb, r.Code, e.status)
            continue
        assert r.Status == OpStatus.Success, (case, sa, sb, r.Message)
        got = r.Outputs[0].to_numpy()
        assert got.shape == ref.shape and got.dtype == ref.dtype, (case, sa, sb)
        if dt == np.int32:
            assert np.array_equal(got, ref), (case, sa, sb)
            continue
        mag = O.matmul(np.abs(a).astype(np.float64), np.abs(b).astype(np.float64))
        err = np.abs(got.astype(np.float64) - ref.astype(np.float64))
        assert np.all(err <= tol * mag + 1e-30), (case, sa, sb, float((err / (mag + 1e-30)).max()))
        if dt == np.float32 and len(sa) >= 2 and len(sb) >= 2:
            bias = rng.standard_normal(ref.shape[-1]).astype(dt)
            res = rng.standard_normal(ref.shape).astype(dt)
            fused = HIP.MatMulAdd(dev(a), dev(b), dev(bias), dev(res))
            assert fused.Status == OpStatus.Success, (case, sa, sb, fused.Message)
            nodes = HIP.Add(HIP.Add(r.Outputs[0], dev(bias)).Outputs[0], dev(res)).Outputs[0].to_numpy()
            assert same_bits(fused.Outputs[0].to_numpy(), nodes), (case, sa, sb)
