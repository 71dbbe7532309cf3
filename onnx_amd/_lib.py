"""ctypes binding of the C ABI in include/lonnx.h (the same cdecl symbols a C#
[DllImport] table binds).  Loading fails loudly when the HIP library is not
built: there is no CPU fallback."""
import ctypes
import os

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "liblonnx_hip.so")
MAX_RANK = 8

# TensorElementType codes (Tensor.cs:31-50)
FLOAT, UINT8, INT8, UINT16, INT16, INT32, INT64, BOOL, DOUBLE, UINT32, UINT64 = 1, 2, 3, 4, 5, 6, 7, 9, 11, 12, 13

# lx_status
OK = 0
ERR_MISSING_INPUT = 1
ERR_WRONG_INPUT_TYPE = 2
ERR_CANNOT_BROADCAST = 3
ERR_INPUT_TYPE_NOT_SUPPORTED = 4
ERR_NOT_SUPPORTED = 5
ERR_ATTRIBUTE_NOT_SUPPORTED = 6
ERR_WRONG_INPUT_SHAPE = 7
ERR_INVALID_ARGUMENT = 8
ERR_DIVIDE_BY_ZERO = 9
ERR_OVERFLOW = 10
ERR_OUT_OF_MEMORY = 11
ERR_HIP = 12
ERR_NOT_INITIALIZED = 13
ERR_BUFFER_TOO_SMALL = 14

PLAN_EMPTY, PLAN_SAME, PLAN_SCALAR_A, PLAN_SCALAR_B, PLAN_ND = 0, 1, 2, 3, 4


class LxTensor(ctypes.Structure):
    _fields_ = [
        ("dtype", ctypes.c_int32),
        ("rank", ctypes.c_int32),
        ("dims", ctypes.c_int64 * MAX_RANK),
        ("data", ctypes.c_void_p),
        ("capacity", ctypes.c_int64),
        ("owns", ctypes.c_int32),
        ("reserved", ctypes.c_int32),
    ]


class LxNodeProfile(ctypes.Structure):
    _fields_ = [
        ("node_id", ctypes.c_int64),
        ("node_index", ctypes.c_int32),
        ("op", ctypes.c_char * 36),
        ("math_ms", ctypes.c_double),
        ("host_ms", ctypes.c_double),
        ("start_ms", ctypes.c_double),
    ]


class LxOpProfile(ctypes.Structure):
    _fields_ = [
        ("op", ctypes.c_char * 36),
        ("math_ms", ctypes.c_double),
        ("host_ms", ctypes.c_double),
        ("start_ms", ctypes.c_double),
    ]


class LxPlan(ctypes.Structure):
    _fields_ = [
        ("status", ctypes.c_int32),
        ("out_rank", ctypes.c_int32),
        ("out_dims", ctypes.c_int64 * MAX_RANK),
        ("kind", ctypes.c_int32),
        ("rank", ctypes.c_int32),
        ("dims", ctypes.c_int64 * MAX_RANK),
        ("a_strides", ctypes.c_int64 * MAX_RANK),
        ("b_strides", ctypes.c_int64 * MAX_RANK),
        ("numel", ctypes.c_int64),
    ]


# name -> (restype, argtypes); every symbol declared in include/lonnx.h
_T = ctypes.POINTER(LxTensor)
_i64p = ctypes.POINTER(ctypes.c_int64)
_i32p = ctypes.POINTER(ctypes.c_int32)
_c = ctypes
SIGNATURES = {
    "lx_init": (_c.c_int, [_c.c_int32]),
    "lx_shutdown": (_c.c_int, []),
    "lx_last_error": (_c.c_char_p, []),
    "lx_version": (_c.c_char_p, []),
    "lx_set_stream": (_c.c_int, [_c.c_void_p]),
    "lx_set_op_profiling": (_c.c_int, [_c.c_int32]),
    "lx_op_profile_count": (_c.c_int32, []),
    "lx_op_profile": (_c.c_int, [_c.c_int32, _c.c_void_p]),
    "lx_op_profile_reset": (_c.c_int, []),
    "lx_get_stream": (_c.c_void_p, []),
    "lx_synchronize": (_c.c_int, []),
    "lx_dtype_size": (_c.c_int64, [_c.c_int32]),
    "lx_tensor_alloc": (_c.c_int, [_c.c_int32, _c.c_int32, _i64p, _T]),
    "lx_tensor_wrap": (_c.c_int, [_c.c_int32, _c.c_int32, _i64p, _c.c_void_p, _c.c_int64, _T]),
    "lx_tensor_free": (_c.c_int, [_T]),
    "lx_tensor_upload": (_c.c_int, [_T, _c.c_void_p, _c.c_int64]),
    "lx_tensor_download": (_c.c_int, [_T, _c.c_void_p, _c.c_int64]),
    "lx_tensor_reshape": (_c.c_int, [_T, _c.c_int32, _i64p, _T]),
    "lx_plan_broadcast": (_c.c_int, [_c.c_int32, _i64p, _c.c_int32, _i64p, _c.POINTER(LxPlan)]),
    "lx_Add": (_c.c_int, [_T, _T, _T]),
    "lx_Sub": (_c.c_int, [_T, _T, _T]),
    "lx_Mul": (_c.c_int, [_T, _T, _T]),
    "lx_Div": (_c.c_int, [_T, _T, _T]),
    "lx_Pow": (_c.c_int, [_T, _T, _T]),
    "lx_Sqrt": (_c.c_int, [_T, _T]),
    "lx_Erf": (_c.c_int, [_T, _T]),
    "lx_Cast": (_c.c_int, [_T, _c.c_int64, _T]),
    "lx_ReduceSum": (_c.c_int, [_T, _i64p, _c.c_int32, _c.c_int32, _c.c_int32, _T]),
    "lx_ReduceSum_noalloc": (_c.c_int, [_T, _i64p, _c.c_int32, _c.c_int32, _c.c_int32, _T]),
    "lx_ReduceMean": (_c.c_int, [_T, _i64p, _c.c_int32, _c.c_int32, _c.c_int32, _T]),
    "lx_ReduceMax": (_c.c_int, [_T, _i64p, _c.c_int32, _c.c_int32, _T]),
    "lx_Softmax": (_c.c_int, [_T, _c.c_int32, _c.c_int32, _T]),
    "lx_GeluErf": (_c.c_int, [_T, _T]),
    "lx_LayerNormDecomposed": (_c.c_int, [_T, _T, _T, _c.c_float, _T]),
    "lx_AddSoftmax": (_c.c_int, [_T, _T, _c.c_int32, _T]),
    "lx_MatMul": (_c.c_int, [_T, _T, _T]),
    "lx_Transpose": (_c.c_int, [_T, _i64p, _c.c_int32, _T]),
    "lx_Concat": (_c.c_int, [_c.POINTER(_T), _c.c_int32, _c.c_int32, _c.c_int32, _T]),
    "lx_Gather": (_c.c_int, [_T, _T, _c.c_int32, _c.c_int32, _T]),
    "lx_Slice": (_c.c_int, [_T, _i64p, _c.c_int32, _i64p, _c.c_int32, _i64p, _c.c_int32, _i64p, _c.c_int32, _T]),
    "lx_MatMulAdd": (_c.c_int, [_T, _T, _T, _T, _T]),
    "lx_MatMulAddGelu": (_c.c_int, [_T, _T, _T, _T]),
    "lx_ScaleAddSoftmax": (_c.c_int, [_T, _T, _c.c_int32, _T, _c.c_int32, _T]),
    "lx_ElementwiseChain": (_c.c_int, [_c.POINTER(_T), _c.c_int32, _i32p, _i32p, _c.c_int32, _T]),
    "lx_read_probe": (_c.c_int, [_c.c_void_p, _c.c_int64, _c.c_void_p, _c.c_int64]),
    "lx_pool_trim": (_c.c_int, []),
    "lx_pool_stats": (_c.c_int, [_i64p, _i64p]),
    # graph runtime
    "lx_graph_create": (_c.c_int, [_c.c_int64, _c.POINTER(_c.c_void_p)]),
    "lx_graph_free": (_c.c_int, [_c.c_void_p]),
    "lx_graph_add_input": (_c.c_int, [_c.c_void_p, _c.c_char_p, _c.c_int32, _c.c_int32, _i64p]),
    "lx_graph_add_output": (_c.c_int, [_c.c_void_p, _c.c_char_p]),
    "lx_graph_add_initializer": (_c.c_int, [_c.c_void_p, _c.c_char_p, _c.c_int32, _c.c_int32, _i64p, _c.c_void_p,
                                            _c.c_int64]),
    "lx_graph_add_node": (_c.c_int, [_c.c_void_p, _c.c_char_p, _c.c_char_p, _c.c_int32, _c.POINTER(_c.c_char_p),
                                     _c.c_int32, _c.POINTER(_c.c_char_p), _c.POINTER(_c.c_int32)]),
    "lx_graph_set_attr_int": (_c.c_int, [_c.c_void_p, _c.c_int32, _c.c_char_p, _c.c_int64]),
    "lx_graph_set_attr_ints": (_c.c_int, [_c.c_void_p, _c.c_int32, _c.c_char_p, _i64p, _c.c_int32]),
    "lx_graph_set_attr_float": (_c.c_int, [_c.c_void_p, _c.c_int32, _c.c_char_p, _c.c_float]),
    "lx_graph_set_attr_floats": (_c.c_int, [_c.c_void_p, _c.c_int32, _c.c_char_p, _c.POINTER(_c.c_float),
                                            _c.c_int32]),
    "lx_graph_set_attr_string": (_c.c_int, [_c.c_void_p, _c.c_int32, _c.c_char_p, _c.c_char_p]),
    "lx_graph_set_attr_tensor": (_c.c_int, [_c.c_void_p, _c.c_int32, _c.c_char_p, _c.c_int32, _c.c_int32, _i64p,
                                            _c.c_void_p, _c.c_int64]),
    "lx_graph_load_onnx": (_c.c_int, [_c.c_void_p, _c.c_int64, _c.POINTER(_c.c_void_p)]),
    "lx_graph_fuse": (_c.c_int, [_c.c_void_p, _c.POINTER(_c.c_int32)]),
    "lx_graph_execute": (_c.c_int, [_c.c_void_p, _c.c_int32, _c.POINTER(_c.c_char_p), _T, _c.c_int32]),
    "lx_graph_capture": (_c.c_int, [_c.c_void_p, _c.c_int32, _c.POINTER(_c.c_char_p), _T, _c.c_int32]),
    "lx_graph_replay": (_c.c_int, [_c.c_void_p]),
    "lx_graph_release_capture": (_c.c_int, [_c.c_void_p]),
    "lx_graph_execute_node": (_c.c_int, [_c.c_void_p, _c.c_char_p, _c.c_int32, _c.POINTER(_c.c_char_p), _T,
                                         _c.c_int32]),
    "lx_graph_output": (_c.c_int, [_c.c_void_p, _c.c_char_p, _T]),
    "lx_graph_reset": (_c.c_int, [_c.c_void_p]),
    "lx_graph_set_profiling": (_c.c_int, [_c.c_void_p, _c.c_int32]),
    "lx_graph_profile_count": (_c.c_int32, [_c.c_void_p]),
    "lx_graph_profile": (_c.c_int, [_c.c_void_p, _c.c_int32, _c.POINTER(LxNodeProfile)]),
    "lx_graph_profile_reset": (_c.c_int, [_c.c_void_p]),
    "lx_graph_node_count": (_c.c_int32, [_c.c_void_p]),
    "lx_graph_node_info": (_c.c_int, [_c.c_void_p, _c.c_int32, _c.c_char_p, _c.c_int32, _c.c_char_p, _c.c_int32]),
    "lx_graph_input_count": (_c.c_int32, [_c.c_void_p]),
    "lx_graph_input_info": (_c.c_int, [_c.c_void_p, _c.c_int32, _c.c_char_p, _c.c_int32, _c.POINTER(_c.c_int32),
                                       _c.POINTER(_c.c_int32), _i64p]),
    "lx_graph_initializer_count": (_c.c_int32, [_c.c_void_p]),
    "lx_graph_initializer_info": (_c.c_int, [_c.c_void_p, _c.c_int32, _c.c_char_p, _c.c_int32,
                                             _c.POINTER(_c.c_int32), _c.POINTER(_c.c_int32), _i64p]),
    "lx_graph_output_count": (_c.c_int32, [_c.c_void_p]),
    "lx_graph_output_name": (_c.c_int, [_c.c_void_p, _c.c_int32, _c.c_char_p, _c.c_int32]),
}

_lib = None


def pool_stats():
    """(live, cached) bytes of the library's device memory pool."""
    live, cached = ctypes.c_int64(), ctypes.c_int64()
    lib().lx_pool_stats(ctypes.byref(live), ctypes.byref(cached))
    return live.value, cached.value


def lib():
    """The loaded library (raises if it is not built)."""
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise RuntimeError(
                f"HIP library not built: {LIB_PATH}. Run `python -m onnx_amd.build` (hipcc, gfx950).")
        L = ctypes.CDLL(LIB_PATH)
        for name, (res, args) in SIGNATURES.items():
            f = getattr(L, name)
            f.restype = res
            f.argtypes = args
        _lib = L
    return _lib


def last_error():
    m = lib().lx_last_error()
    # messages are cut at 1023 bytes, which can split a multi-byte character of a name
    return m.decode(errors="replace") if m else ""


def dims_array(shape):
    shape = [int(d) for d in shape]
    if len(shape) > MAX_RANK:
        raise ValueError(f"rank {len(shape)} > {MAX_RANK}")
    return (ctypes.c_int64 * MAX_RANK)(*(shape + [0] * (MAX_RANK - len(shape))))


def plan_broadcast(shape_a, shape_b):
    """Host-only planner call (no device needed)."""
    p = LxPlan()
    st = lib().lx_plan_broadcast(len(shape_a), dims_array(shape_a), len(shape_b), dims_array(shape_b),
                                 ctypes.byref(p))
    return st, p
