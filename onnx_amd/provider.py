"""HipExecutionProvider -- the device twin of the reference's
CPUExecutionProvider (src/Lokad.Onnx.Backend/CPUExecutionProvider.cs), over the
C ABI of include/lonnx.h.

Same operator names, argument meaning and failure behaviour: every operator
returns an OpResult (OpResult.cs:15-64) and never raises for operator errors.
Tensors are DeviceTensor handles (device twin of DenseTensor<T>) with explicit
residency: from_numpy uploads, to_numpy downloads.
"""
import ctypes
import enum
from dataclasses import dataclass, field
from typing import List, Optional

import numpy as np

from . import _lib as L

NP_OF = {L.FLOAT: np.float32, L.UINT8: np.uint8, L.INT8: np.int8, L.UINT16: np.uint16, L.INT16: np.int16,
         L.INT32: np.int32, L.INT64: np.int64, L.BOOL: np.bool_, L.DOUBLE: np.float64, L.UINT32: np.uint32,
         L.UINT64: np.uint64}
CODE_OF = {np.dtype(v): k for k, v in NP_OF.items()}

_initialised = False


def init(device: int = 0):
    """Select the device and create the library stream (idempotent)."""
    global _initialised
    if not _initialised:
        st = L.lib().lx_init(device)
        if st != L.OK:
            raise RuntimeError(f"lx_init failed ({st}): {L.last_error()}")
        _initialised = True


def synchronize():
    _check(L.lib().lx_synchronize(), "lx_synchronize")


def set_stream(hip_stream_handle: Optional[int]):
    init()
    _check(L.lib().lx_set_stream(ctypes.c_void_p(hip_stream_handle or 0)), "lx_set_stream")


def _check(st, what):
    if st != L.OK:
        raise RuntimeError(f"{what} failed ({st}): {L.last_error()}")


class DeviceTensor:
    """Device-resident tensor: row-major storage in HBM, int64 dims."""

    def __init__(self, handle: L.LxTensor, keepalive=None):
        self.h = handle
        self._keepalive = keepalive

    # ---- construction -------------------------------------------------
    @classmethod
    def empty(cls, shape, dtype):
        init()
        h = L.LxTensor()
        code = CODE_OF[np.dtype(dtype)]
        _check(L.lib().lx_tensor_alloc(code, len(shape), L.dims_array(shape), ctypes.byref(h)), "lx_tensor_alloc")
        return cls(h)

    @classmethod
    def from_numpy(cls, arr):
        arr = np.asarray(arr)
        arr = np.ascontiguousarray(arr).reshape(arr.shape)  # keeps rank 0
        t = cls.empty(arr.shape, arr.dtype)
        _check(L.lib().lx_tensor_upload(ctypes.byref(t.h), ctypes.c_void_p(arr.ctypes.data), arr.nbytes),
               "lx_tensor_upload")
        return t

    def upload(self, arr):
        """Writes host values into this tensor's device storage in place (same shape and dtype): what a
        captured graph execution's inputs need between replays."""
        arr = np.ascontiguousarray(np.asarray(arr, dtype=self.dtype)).reshape(self.shape)
        _check(L.lib().lx_tensor_upload(ctypes.byref(self.h), ctypes.c_void_p(arr.ctypes.data), arr.nbytes),
               "lx_tensor_upload")

    @classmethod
    def wrap(cls, ptr: int, shape, dtype, capacity: int, keepalive=None):
        """Non-owning view of existing device memory (e.g. a torch tensor)."""
        init()
        h = L.LxTensor()
        _check(L.lib().lx_tensor_wrap(CODE_OF[np.dtype(dtype)], len(shape), L.dims_array(shape),
                                      ctypes.c_void_p(ptr), capacity, ctypes.byref(h)), "lx_tensor_wrap")
        return cls(h, keepalive)

    @classmethod
    def wrap_torch(cls, t):
        import torch  # plumbing only: device memory comes from torch's allocator
        np_dtype = {torch.float32: np.float32, torch.float64: np.float64, torch.int32: np.int32,
                    torch.int64: np.int64, torch.uint8: np.uint8, torch.int8: np.int8, torch.int16: np.int16,
                    torch.bool: np.bool_}[t.dtype]
        assert t.is_contiguous()
        return cls.wrap(t.data_ptr(), tuple(t.shape), np_dtype, t.numel() * t.element_size(), keepalive=t)

    # ---- properties ---------------------------------------------------
    @property
    def shape(self):
        return tuple(self.h.dims[i] for i in range(self.h.rank))

    @property
    def dtype(self):
        return np.dtype(NP_OF[self.h.dtype])

    @property
    def ElementType(self):
        return self.h.dtype

    @property
    def Rank(self):
        return self.h.rank

    def numel(self):
        n = 1
        for d in self.shape:
            n *= d
        return n

    def to_numpy(self):
        out = np.empty(self.shape, dtype=self.dtype)
        _check(L.lib().lx_tensor_download(ctypes.byref(self.h), ctypes.c_void_p(out.ctypes.data), out.nbytes),
               "lx_tensor_download")
        return out

    def reshape(self, shape):
        h = L.LxTensor()
        _check(L.lib().lx_tensor_reshape(ctypes.byref(self.h), len(shape), L.dims_array(shape), ctypes.byref(h)),
               "lx_tensor_reshape")
        return DeviceTensor(h, keepalive=self)

    def free(self):
        if self.h.owns and self.h.data:
            L.lib().lx_tensor_free(ctypes.byref(self.h))

    def __del__(self):
        try:
            self.free()
        except Exception:
            pass


class OpStatus(enum.Enum):
    Success = 0
    Failure = 1


@dataclass
class OpResult:
    """OpResult (OpResult.cs:15-64) plus the C ABI status code."""
    Op: str
    Status: OpStatus
    Message: Optional[str] = None
    Outputs: List[DeviceTensor] = field(default_factory=list)
    Code: int = 0


def _ptr(t: Optional[DeviceTensor]):
    return ctypes.byref(t.h) if t is not None else None


def _as_tensor(x):
    if x is None or isinstance(x, DeviceTensor):
        return x
    return DeviceTensor.from_numpy(np.asarray(x))


def _result(op, st, out_h, out=None):
    """OpResult from a status; `out` is the caller's output tensor when one was given."""
    if st == L.OK:
        return OpResult(op, OpStatus.Success, None, [out if out is not None else DeviceTensor(out_h)], 0)
    if out is None and out_h.owns and out_h.data:
        L.lib().lx_tensor_free(ctypes.byref(out_h))
    return OpResult(op, OpStatus.Failure, L.last_error(), [], st)


def _axes_args(axes):
    """axes: None (absent input) or a sequence / array of ints (Int64 tensor in the reference)."""
    if axes is None:
        return None, -1
    a = np.asarray(axes, dtype=np.int64).reshape(-1)
    arr = (ctypes.c_int64 * max(1, a.size))(*a.tolist())
    return arr, int(a.size)


class HipExecutionProvider:
    """Static operators with CPUExecutionProvider's signatures."""

    # ---- profiling: the OpStage.Math stage of each call (Profiler.StartOpStage, Profiler.cs:71-80) ----
    @staticmethod
    def EnableProfiling(enabled: bool = True):
        """Device timing of later operator calls (lx_set_op_profiling): each call made while enabled appends
        one record whose math_ms is the device time between HIP events around its launches."""
        init()
        _check(L.lib().lx_set_op_profiling(1 if enabled else 0), "lx_set_op_profiling")

    @staticmethod
    def Profile() -> List[dict]:
        """The records since the last reset: op, math_ms (OpStage.Math on the device), host_ms (the call on
        the host) and start_ms (device time from the first record's start); waits for the calls' events."""
        init()
        lib = L.lib()
        out = []
        for i in range(lib.lx_op_profile_count()):
            p = L.LxOpProfile()
            _check(lib.lx_op_profile(i, ctypes.byref(p)), "lx_op_profile")
            out.append({"op": p.op.decode(), "math_ms": p.math_ms, "host_ms": p.host_ms, "start_ms": p.start_ms})
        return out

    @staticmethod
    def ResetProfile():
        init()
        _check(L.lib().lx_op_profile_reset(), "lx_op_profile_reset")

    @staticmethod
    def _binary(name, A, B, out=None):
        init()
        A, B = _as_tensor(A), _as_tensor(B)
        y = out.h if out is not None else L.LxTensor()
        st = getattr(L.lib(), "lx_" + name)(_ptr(A), _ptr(B), ctypes.byref(y))
        return _result(name, st, y, out)

    @staticmethod
    def Add(A, B, out=None):
        return HipExecutionProvider._binary("Add", A, B, out)

    @staticmethod
    def Sub(A, B, out=None):
        return HipExecutionProvider._binary("Sub", A, B, out)

    @staticmethod
    def Mul(A, B, out=None):
        return HipExecutionProvider._binary("Mul", A, B, out)

    @staticmethod
    def Div(A, B, out=None):
        return HipExecutionProvider._binary("Div", A, B, out)

    @staticmethod
    def Pow(A, B, out=None):
        return HipExecutionProvider._binary("Pow", A, B, out)

    @staticmethod
    def Sqrt(A, out=None):
        init()
        A = _as_tensor(A)
        y = out.h if out is not None else L.LxTensor()
        return _result("Sqrt", L.lib().lx_Sqrt(_ptr(A), ctypes.byref(y)), y, out)

    @staticmethod
    def Erf(X, out=None):
        init()
        X = _as_tensor(X)
        y = out.h if out is not None else L.LxTensor()
        return _result("Erf", L.lib().lx_Erf(_ptr(X), ctypes.byref(y)), y, out)

    @staticmethod
    def Cast(input, to, out=None):
        init()
        input = _as_tensor(input)
        y = out.h if out is not None else L.LxTensor()
        return _result("Cast", L.lib().lx_Cast(_ptr(input), int(to), ctypes.byref(y)), y, out)

    @staticmethod
    def _reduce(name, data, axes, keep_dims, noop, out=None):
        init()
        data = _as_tensor(data)
        arr, n = _axes_args(axes)
        kd = -1 if keep_dims is None else int(keep_dims)
        y = out.h if out is not None else L.LxTensor()
        if name == "ReduceMax":
            st = L.lib().lx_ReduceMax(_ptr(data), arr, n, kd, ctypes.byref(y))
        else:
            nw = -1 if noop is None else int(noop)
            st = getattr(L.lib(), "lx_" + name)(_ptr(data), arr, n, kd, nw, ctypes.byref(y))
        return _result(name, st, y, out)

    @staticmethod
    def ReduceSum(data, axes=None, keep_dims=None, noop_with_empty_axes=None, out=None):
        return HipExecutionProvider._reduce("ReduceSum", data, axes, keep_dims, noop_with_empty_axes, out)

    @staticmethod
    def ReduceMean(data, axes=None, keep_dims=None, noop_with_empty_axes=None, out=None):
        return HipExecutionProvider._reduce("ReduceMean", data, axes, keep_dims, noop_with_empty_axes, out)

    @staticmethod
    def ReduceMax(data, axes=None, keep_dims=None, out=None):
        return HipExecutionProvider._reduce("ReduceMax", data, axes, keep_dims, None, out)

    @staticmethod
    def Softmax(input, axis=None, out=None):
        init()
        input = _as_tensor(input)
        y = out.h if out is not None else L.LxTensor()
        st = L.lib().lx_Softmax(_ptr(input), 0 if axis is None else int(axis), 0 if axis is None else 1,
                                ctypes.byref(y))
        return _result("Softmax", st, y, out)

    @staticmethod
    def MatMul(A, B, out=None):
        """CPUExecutionProvider.MatMul (CPUExecutionProvider.cs:359-378)."""
        init()
        A, B = _as_tensor(A), _as_tensor(B)
        y = out.h if out is not None else L.LxTensor()
        st = L.lib().lx_MatMul(_ptr(A), _ptr(B), ctypes.byref(y))
        return _result("MatMul", st, y, out)

    @staticmethod
    def Transpose(data, perm=None, out=None):
        """CPUExecutionProvider.Transpose (CPUExecutionProvider.cs:411-433)."""
        init()
        data = _as_tensor(data)
        parr, n = _axes_args(perm)
        y = out.h if out is not None else L.LxTensor()
        st = L.lib().lx_Transpose(_ptr(data), parr, n, ctypes.byref(y))
        if st == L.OK and out is None and not y.owns:  # rank <= 1: the input itself
            return OpResult("Transpose", OpStatus.Success, None, [DeviceTensor(y, keepalive=data)], 0)
        return _result("Transpose", st, y, out)

    @staticmethod
    def Concat(inputs, axis=None, out=None):
        """CPUExecutionProvider.Concat (CPUExecutionProvider.cs:477-501)."""
        init()
        ts = [_as_tensor(t) for t in (inputs or [])]
        arr = (ctypes.POINTER(L.LxTensor) * max(1, len(ts)))(*[ctypes.pointer(t.h) for t in ts])
        y = out.h if out is not None else L.LxTensor()
        st = L.lib().lx_Concat(arr if inputs is not None else None, len(ts), 0 if axis is None else int(axis),
                               0 if axis is None else 1, ctypes.byref(y))
        return _result("Concat", st, y, out)

    @staticmethod
    def Gather(data, indices, axis=None, out=None):
        """CPUExecutionProvider.Gather (CPUExecutionProvider.cs:516-546)."""
        init()
        data, indices = _as_tensor(data), _as_tensor(indices)
        y = out.h if out is not None else L.LxTensor()
        st = L.lib().lx_Gather(_ptr(data), _ptr(indices), 0 if axis is None else int(axis), 0 if axis is None else 1,
                               ctypes.byref(y))
        return _result("Gather", st, y, out)

    @staticmethod
    def Slice(data, starts, ends, axes=None, steps=None, out=None):
        """CPUExecutionProvider.Slice (CPUExecutionProvider.cs:548-600); starts / ends / axes / steps as
        integer sequences."""
        init()
        data = _as_tensor(data)
        s_, ns = _axes_args(starts)
        e_, ne = _axes_args(ends)
        a_, na = _axes_args(axes)
        p_, np_ = _axes_args(steps)
        y = out.h if out is not None else L.LxTensor()
        st = L.lib().lx_Slice(_ptr(data), s_, ns, e_, ne, a_, na, p_, np_, ctypes.byref(y))
        return _result("Slice", st, y, out)

    # ---- fused subgraphs ---------------------------------------------------
    CHAIN_OPS = {"Add": 0, "Sub": 1, "Mul": 2, "Div": 3, "Pow": 4, "Sqrt": 16, "Erf": 17}

    @staticmethod
    def ElementwiseChain(inputs, program, out=None):
        """A linear chain of Float elementwise nodes in one kernel.  acc = inputs[0]; program is a list of
        (op, j) for binary ops (acc = acc op inputs[j]), (op, j, True) for acc = inputs[j] op acc, or (op,)
        for Sqrt / Erf.  Bit-identical to running the nodes one by one."""
        init()
        ts = [_as_tensor(t) for t in inputs]
        arr = (ctypes.POINTER(L.LxTensor) * max(1, len(ts)))(*[ctypes.pointer(t.h) for t in ts])
        ops, operands = [], []
        for ins in program:
            ops.append(HipExecutionProvider.CHAIN_OPS[ins[0]])
            j = ins[1] if len(ins) > 1 else 0
            operands.append(-(j + 1) if len(ins) > 2 and ins[2] else j)
        n = max(1, len(ops))
        o = (ctypes.c_int32 * n)(*ops)
        p = (ctypes.c_int32 * n)(*operands)
        y = out.h if out is not None else L.LxTensor()
        st = L.lib().lx_ElementwiseChain(arr, len(ts), o, p, len(ops), ctypes.byref(y))
        return _result("ElementwiseChain", st, y, out)

    @staticmethod
    def MatMulAdd(A, B, bias, residual=None, out=None):
        """MatMul(A, B) -> Add bias [-> Add residual] with the Adds in the MatMul's epilogue (lx_MatMulAdd)."""
        init()
        A, B, bias = _as_tensor(A), _as_tensor(B), _as_tensor(bias)
        r = _as_tensor(residual) if residual is not None else None
        y = out.h if out is not None else L.LxTensor()
        st = L.lib().lx_MatMulAdd(_ptr(A), _ptr(B), _ptr(bias), _ptr(r), ctypes.byref(y))
        return _result("MatMulAdd", st, y, out)

    @staticmethod
    def MatMulAddGelu(A, B, bias, out=None):
        """MatMul(A, B) -> Add bias -> the ONNX GELU subgraph, the Add and GELU in the MatMul's epilogue
        (lx_MatMulAddGelu)."""
        init()
        A, B, bias = _as_tensor(A), _as_tensor(B), _as_tensor(bias)
        y = out.h if out is not None else L.LxTensor()
        st = L.lib().lx_MatMulAddGelu(_ptr(A), _ptr(B), _ptr(bias), ctypes.byref(y))
        return _result("MatMulAddGelu", st, y, out)

    @staticmethod
    def ScaleAddSoftmax(S, scale, divide=True, mask=None, axis=-1, out=None):
        """Div(S, scale) (or Mul) -> Add(., mask) -> Softmax(axis) in one kernel (lx_ScaleAddSoftmax)."""
        init()
        S, scale = _as_tensor(S), _as_tensor(scale)
        m = _as_tensor(mask) if mask is not None else None
        y = out.h if out is not None else L.LxTensor()
        st = L.lib().lx_ScaleAddSoftmax(_ptr(S), _ptr(scale), int(bool(divide)), _ptr(m) if m is not None else None,
                                        int(axis), ctypes.byref(y))
        return _result("ScaleAddSoftmax", st, y, out)

    @staticmethod
    def GeluErf(X, out=None):
        init()
        X = _as_tensor(X)
        y = out.h if out is not None else L.LxTensor()
        return _result("GeluErf", L.lib().lx_GeluErf(_ptr(X), ctypes.byref(y)), y, out)

    @staticmethod
    def LayerNormDecomposed(X, gamma, beta, eps=1e-12, out=None):
        init()
        X, gamma, beta = _as_tensor(X), _as_tensor(gamma), _as_tensor(beta)
        y = out.h if out is not None else L.LxTensor()
        st = L.lib().lx_LayerNormDecomposed(_ptr(X), _ptr(gamma), _ptr(beta), ctypes.c_float(eps), ctypes.byref(y))
        return _result("LayerNormDecomposed", st, y, out)

    @staticmethod
    def AddSoftmax(S, mask, axis=-1, out=None):
        init()
        S, mask = _as_tensor(S), _as_tensor(mask)
        y = out.h if out is not None else L.LxTensor()
        return _result("AddSoftmax", L.lib().lx_AddSoftmax(_ptr(S), _ptr(mask), int(axis), ctypes.byref(y)), y, out)
