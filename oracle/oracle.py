"""TEST INFRASTRUCTURE ONLY -- ctypes front of the CPU oracle (lonnx_oracle.c).

The oracle is a C restatement of the Lokad.Onnx C# CPU operators (see the file
header of lonnx_oracle.c for the reference lines each function follows).  Only
tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg import this
module; the product package never does.
"""
import ctypes
import os

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(_HERE, "_build", "liblonnx_oracle.so")

# TensorElementType codes (Tensor.cs:31-50)
FLOAT, UINT8, INT8, UINT16, INT16, INT32, INT64, BOOL, DOUBLE, UINT32, UINT64 = 1, 2, 3, 4, 5, 6, 7, 9, 11, 12, 13
NP_OF = {FLOAT: np.float32, UINT8: np.uint8, INT8: np.int8, UINT16: np.uint16, INT16: np.int16,
         INT32: np.int32, INT64: np.int64, BOOL: np.bool_, DOUBLE: np.float64, UINT32: np.uint32,
         UINT64: np.uint64}
CODE_OF = {np.dtype(v): k for k, v in NP_OF.items()}

ADD, SUB, MUL, DIV, POW = 0, 1, 2, 3, 4
SQRT, ERF, NEG, EXP = 0, 1, 2, 3
RSUM, RMEAN, RMAX = 0, 1, 2

OK, ERR_CANNOT_BROADCAST, ERR_NOT_SUPPORTED, ERR_ATTRIBUTE_NOT_SUPPORTED = 0, 3, 5, 6
ERR_INVALID_ARGUMENT, ERR_DIVIDE_BY_ZERO, ERR_OVERFLOW, ERR_OUT_OF_MEMORY = 8, 9, 10, 11

MAX_RANK = 8


class OracleError(Exception):
    def __init__(self, status, msg=""):
        super().__init__(f"oracle status {status} {msg}")
        self.status = status


_lib = None


def lib():
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise RuntimeError(f"oracle library not built: {LIB_PATH} (run make -C oracle)")
        L = ctypes.CDLL(LIB_PATH)
        i64p = ctypes.POINTER(ctypes.c_int64)
        ip = ctypes.POINTER(ctypes.c_int)
        vp = ctypes.c_void_p
        L.lxo_broadcast_shape.argtypes = [ctypes.c_int, i64p, ctypes.c_int, i64p, ip, i64p]
        L.lxo_op_binary.argtypes = [ctypes.c_int, ctypes.c_int, ctypes.c_int, i64p, vp, ctypes.c_int, i64p, vp,
                                    vp, ip, i64p, i64p]
        L.lxo_binary.argtypes = [ctypes.c_int, ctypes.c_int, ctypes.c_int64, vp, vp, vp, i64p]
        L.lxo_unary.argtypes = [ctypes.c_int, ctypes.c_int, ctypes.c_int64, vp, vp]
        L.lxo_cast.argtypes = [ctypes.c_int, ctypes.c_int, ctypes.c_int64, vp, vp]
        L.lxo_reduce.argtypes = [ctypes.c_int, ctypes.c_int, ctypes.c_int, i64p, vp, ctypes.c_int, i64p,
                                 ctypes.c_int, vp, ip, i64p]
        L.lxo_softmax.argtypes = [ctypes.c_int, ctypes.c_int, i64p, vp, ctypes.c_int, vp]
        L.lxo_gelu_chain.argtypes = [ctypes.c_int64, vp, vp]
        L.lxo_matmul2d.argtypes = [ctypes.c_int, ctypes.c_int64, ctypes.c_int64, ctypes.c_int64, vp, vp, vp]
        L.lxo_erf_f32.argtypes = [ctypes.c_float]
        L.lxo_erf_f32.restype = ctypes.c_float
        L.lxo_erf_f64.argtypes = [ctypes.c_double]
        L.lxo_erf_f64.restype = ctypes.c_double
        L.lxo_expf.argtypes = [ctypes.c_float]
        L.lxo_expf.restype = ctypes.c_float
        L.lxo_powf.argtypes = [ctypes.c_float, ctypes.c_float]
        L.lxo_powf.restype = ctypes.c_float
        _lib = L
    return _lib


def _contig(a):
    """C-contiguous copy that keeps rank 0 (np.ascontiguousarray returns at least 1-D)."""
    a = np.asarray(a)
    return np.ascontiguousarray(a).reshape(a.shape)


def _dims(shape):
    arr = (ctypes.c_int64 * MAX_RANK)(*([int(d) for d in shape] + [0] * (MAX_RANK - len(shape))))
    return arr


def _ptr(a):
    return ctypes.c_void_p(a.ctypes.data) if a.size else ctypes.c_void_p(0)


def broadcast_shape(sa, sb):
    """ITensor.Broadcast shape rule; returns a tuple or None."""
    ro = ctypes.c_int(0)
    do = _dims([])
    st = lib().lxo_broadcast_shape(len(sa), _dims(sa), len(sb), _dims(sb), ctypes.byref(ro), do)
    if st != 0:
        return None
    return tuple(do[i] for i in range(ro.value))


def binary(op, a, b):
    """CPUExecutionProvider.Add/Sub/Mul/Div/Pow on numpy arrays (same dtype)."""
    a = _contig(a)
    b = _contig(b)
    assert a.dtype == b.dtype
    code = CODE_OF[a.dtype]
    shape = broadcast_shape(a.shape, b.shape)
    if shape is None:
        raise OracleError(ERR_CANNOT_BROADCAST)
    out = np.empty(shape, dtype=a.dtype)
    ro = ctypes.c_int(0)
    do = _dims([])
    err = ctypes.c_int64(-1)
    st = lib().lxo_op_binary(op, code, a.ndim, _dims(a.shape), _ptr(a), b.ndim, _dims(b.shape), _ptr(b),
                             _ptr(out), ctypes.byref(ro), do, ctypes.byref(err))
    if st != 0:
        raise OracleError(st, f"at element {err.value}")
    return out


def unary(op, x):
    x = _contig(x)
    out = np.empty_like(x)
    st = lib().lxo_unary(op, CODE_OF[x.dtype], x.size, _ptr(x), _ptr(out))
    if st != 0:
        raise OracleError(st)
    return out


def cast(x, to_code):
    x = _contig(x)
    out = np.empty(x.shape, dtype=NP_OF[to_code])
    st = lib().lxo_cast(CODE_OF[x.dtype], to_code, x.size, _ptr(x), _ptr(out))
    if st != 0:
        raise OracleError(st)
    return out


def reduce(op, x, axes=None, keepdims=True):
    """ReduceSum/ReduceMean/ReduceMax; axes None or [] = all axes."""
    x = _contig(x)
    ax = list(axes) if axes is not None else []
    axarr = (ctypes.c_int64 * max(1, len(ax)))(*ax) if ax else (ctypes.c_int64 * 1)(0)
    # output buffer large enough for any result shape
    nred = 1
    norm = [a + x.ndim if a < 0 else a for a in ax] if ax else list(range(x.ndim))
    for a in norm:
        if 0 <= a < x.ndim:
            nred *= x.shape[a]
    nout = max(1, x.size // nred if nred else int(np.prod([d for i, d in enumerate(x.shape) if i not in norm])))
    out = np.empty(nout, dtype=x.dtype)
    ro = ctypes.c_int(0)
    do = _dims([])
    st = lib().lxo_reduce(op, CODE_OF[x.dtype], x.ndim, _dims(x.shape), _ptr(x), len(ax), axarr,
                          1 if keepdims else 0, _ptr(out), ctypes.byref(ro), do)
    if st != 0:
        raise OracleError(st)
    shape = tuple(do[i] for i in range(ro.value))
    return out[: int(np.prod(shape)) if shape else 1].reshape(shape)


def softmax(x, axis=-1):
    x = _contig(x)
    out = np.empty_like(x)
    st = lib().lxo_softmax(CODE_OF[x.dtype], x.ndim, _dims(x.shape), _ptr(x), axis, _ptr(out))
    if st != 0:
        raise OracleError(st)
    return out


def _mm2d(x, y):
    """MatMul2D (TensorOps.cs:356-407): the serial loop of MathOps.mm_unsafe_vectorized."""
    if x.shape[1] != y.shape[0]:
        raise OracleError(ERR_INVALID_ARGUMENT, "columns != rows")
    x = _contig(x)
    y = _contig(y)
    out = np.empty((x.shape[0], y.shape[1]), dtype=x.dtype)
    st = lib().lxo_matmul2d(CODE_OF[x.dtype], x.shape[0], x.shape[1], y.shape[1], _ptr(x), _ptr(y), _ptr(out))
    if st != 0:
        raise OracleError(st)
    return out


def matmul(x, y):
    """Tensor<T>.MatMul (TensorOps.cs:600-705): 2-D, batch-broadcast, rank-1 cases."""
    x, y = np.asarray(x), np.asarray(y)
    if x.dtype != y.dtype or x.dtype not in (np.float32, np.float64, np.int32):
        raise OracleError(ERR_NOT_SUPPORTED)
    if x.ndim == 0 or y.ndim == 0:
        raise OracleError(ERR_INVALID_ARGUMENT, "rank 0")
    if x.ndim == 2 and y.ndim == 2:
        return _mm2d(x, y)
    if x.ndim >= 2 and y.ndim >= 2:
        if x.shape[-1] != y.shape[-2]:
            raise OracleError(ERR_INVALID_ARGUMENT, "columns != rows")
        bd = broadcast_shape(x.shape[:-2], y.shape[:-2])
        if bd is None:
            raise OracleError(ERR_INVALID_ARGUMENT, "batch shapes")
        bx = np.broadcast_to(x, bd + x.shape[-2:])
        by = np.broadcast_to(y, bd + y.shape[-2:])
        out = np.empty(bd + (x.shape[-2], y.shape[-1]), dtype=x.dtype)
        for idx in np.ndindex(*bd):
            out[idx] = _mm2d(bx[idx], by[idx])
        return out
    if x.ndim >= 2 or y.ndim >= 2:
        s = broadcast_shape(x.shape, y.shape)
        if s is None:
            raise OracleError(ERR_INVALID_ARGUMENT, "shapes")
        return matmul(np.broadcast_to(x, s), np.broadcast_to(y, s))
    return _mm2d(x.reshape(1, -1), y.reshape(-1, 1)).reshape(1)


def erf_f32(v):
    return lib().lxo_erf_f32(float(v))


def expf(v):
    return lib().lxo_expf(float(v))


# ---------------------------------------------------------------------------
# Composite graphs of the BASELINE configs, run op by op exactly as the
# reference's graph executor would run the ONNX nodes.
# ---------------------------------------------------------------------------
def layernorm_decomposed(x, gamma, beta, eps=np.float32(1e-12)):
    """ReduceMean, Sub, Pow(2), ReduceMean, Add eps, Sqrt, Div, Mul gamma, Add beta."""
    mean = reduce(RMEAN, x, [-1], True)
    d = binary(SUB, x, mean)
    p = binary(POW, d, np.array(2.0, dtype=np.float32))
    var = reduce(RMEAN, p, [-1], True)
    ve = binary(ADD, var, np.array(eps, dtype=np.float32))
    sd = unary(SQRT, ve)
    nrm = binary(DIV, d, sd)
    m = binary(MUL, nrm, gamma)
    return binary(ADD, m, beta)


def gelu_erf(x):
    """Div(x, sqrt2) -> Erf -> Add 1 -> Mul x -> Mul 0.5 (BERT-style GELU subgraph)."""
    a = binary(DIV, x, np.array(np.float32(np.sqrt(2.0)), dtype=np.float32))
    e = unary(ERF, a)
    b = binary(ADD, e, np.array(1.0, dtype=np.float32))
    c = binary(MUL, x, b)
    return binary(MUL, c, np.array(0.5, dtype=np.float32))


def gelu_chain_fast(x):
    """gelu_erf without materialising the scalar operands (same values)."""
    x = np.ascontiguousarray(x, dtype=np.float32)
    out = np.empty_like(x)
    lib().lxo_gelu_chain(x.size, _ptr(x), _ptr(out))
    return out


def add_softmax(s, mask, axis=-1):
    """Add(S, mask) then Softmax(axis)."""
    return softmax(binary(ADD, s, mask), axis)


# ---------------------------------------------------------------------------
# Data movement (TensorOps.cs:1358-1531, SliceIndex.cs:271-324): numpy moves
# the elements; the shape rules, index handling and failures are the
# reference's.
# ---------------------------------------------------------------------------
def transpose(x, perm=None):
    """Tensor<T>.Transpose (TensorOps.cs:1358-1405)."""
    x = np.asarray(x)
    r = x.ndim
    if perm is not None:
        perm = [int(p) for p in perm]
        if len(perm) != r or any(p >= r for p in perm) or len(set(perm)) != len(perm):
            raise OracleError(ERR_INVALID_ARGUMENT, "perm")
        perm = [p if p >= 0 else r + p for p in perm]
    else:
        perm = list(range(r))[::-1]
    if r <= 1:
        return x
    if x.size == 0:  # the copy loop still visits index [0, ..., 0] (TensorDimensionsIterator.cs:36-40)
        raise OracleError(ERR_INVALID_ARGUMENT, "Index was outside the bounds of the array.")
    return np.ascontiguousarray(np.transpose(x, perm))


def concat(xs, axis=0):
    """Tensor<T>.Concat(Tensor<T>[], axis) (TensorOps.cs:1446-1498): the dims check uses the raw axis."""
    xs = [np.asarray(x) for x in xs]
    if len(xs) < 2 or any(x.ndim != xs[0].ndim for x in xs):
        raise OracleError(ERR_INVALID_ARGUMENT, "inputs")
    r = xs[0].ndim
    if any(x.shape[d] != xs[0].shape[d] for x in xs for d in range(r) if d != axis):
        raise OracleError(ERR_INVALID_ARGUMENT, "dims")
    ax = axis if axis >= 0 else r + axis
    if ax < 0 or ax >= r:
        raise OracleError(ERR_INVALID_ARGUMENT, "Index was outside the bounds of the array.")
    first = (xs[0].shape[ax] + xs[1].shape[ax]) * int(np.prod([d for k, d in enumerate(xs[0].shape) if k != ax]))
    if first == 0:  # the first pairwise concat writes index [0, ..., 0] of its empty output
        raise OracleError(ERR_INVALID_ARGUMENT, "Index was outside the bounds of the array.")
    return np.concatenate(xs, ax)


def gather(data, indices, axis=None):
    """Tensor<T>.Gather (TensorOps.cs:1407-1444): a negative index counts from the end once."""
    data, indices = np.asarray(data), np.asarray(indices)
    if indices.ndim > data.ndim or data.ndim == 0:
        raise OracleError(ERR_INVALID_ARGUMENT, "rank")
    ax = 0 if axis is None else (axis if axis >= 0 else data.ndim + axis)
    if ax > data.ndim - 1 or ax < 0:
        raise OracleError(ERR_INVALID_ARGUMENT, "axis")
    dim = data.shape[ax]
    if data.size == 0 or indices.size == 0:  # an empty output: the loop still visits its index [0, ..., 0]
        raise OracleError(ERR_INVALID_ARGUMENT, "Index was outside the bounds of the array.")
    k = indices.astype(np.int64)
    k = np.where(k < 0, k + dim, k)
    if np.any((k < 0) | (k >= dim)):
        raise OracleError(ERR_INVALID_ARGUMENT, "index")
    return np.take(data, k, axis=ax)


def slice_(data, starts, ends, axes=None, steps=None):
    """Tensor<T>.Slice (TensorOps.cs:1500-1531) + SliceIndex.ToSliceDef (SliceIndex.cs:271-324): starts and
    ends wrap once when negative and clamp to [0, dim]; a negative step starts at dim-1 at most."""
    data = np.asarray(data)
    r = data.ndim
    n = len(starts)
    if r == 0 or n > r or len(ends) != n:
        raise OracleError(ERR_INVALID_ARGUMENT, "shape")
    ax = [int(a) if a >= 0 else r + int(a) for a in axes] if axes is not None else list(range(n))
    st = [int(s) for s in steps] if steps is not None else [1] * n
    out = data
    for d in range(r):
        if d not in ax:
            continue
        i = ax.index(d)
        dim = data.shape[d]

        def clamp(v):
            v = v if v >= 0 else dim + v
            return min(max(v, 0), dim)
        start, stop, step = clamp(int(starts[i])), clamp(int(ends[i])), st[i]
        idx = []
        if step > 0 and start < dim and start < stop:
            idx = list(range(start, stop, step))
        elif step < 0:
            start = min(start, dim - 1)
            if start > stop:
                idx = list(range(start, stop, step))
        out = np.take(out, np.array(idx, dtype=np.int64), axis=d)
    return np.ascontiguousarray(out)
