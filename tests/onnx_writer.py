"""TEST HELPER: a minimal ONNX ModelProto encoder (protobuf wire format, field
numbers of the public onnx.proto), so tests can build model files for the
device graph runtime without the onnx package.  Also a generic wire decoder
used to read model files independently of the library's loader."""
import struct

import numpy as np

ELEM = {np.dtype(np.float32): 1, np.dtype(np.uint8): 2, np.dtype(np.int8): 3, np.dtype(np.int32): 6,
        np.dtype(np.int64): 7, np.dtype(np.bool_): 9, np.dtype(np.float64): 11}


def _varint(v):
    v &= (1 << 64) - 1
    out = bytearray()
    while True:
        b = v & 0x7F
        v >>= 7
        if v:
            out.append(b | 0x80)
        else:
            out.append(b)
            return bytes(out)


def _key(field, wt):
    return _varint((field << 3) | wt)


def f_varint(field, v):
    return _key(field, 0) + _varint(int(v))


def f_bytes(field, b):
    if isinstance(b, str):
        b = b.encode()
    return _key(field, 2) + _varint(len(b)) + b


def f_fixed32(field, v):
    return _key(field, 5) + struct.pack("<f", float(v))


def f_packed_varints(field, vals):
    body = b"".join(_varint(int(v)) for v in vals)
    return f_bytes(field, body)


def tensor(name, arr, raw=True):
    """TensorProto: dims (1), data_type (2), name (8), raw_data (9) or typed fields."""
    arr = np.ascontiguousarray(arr)
    out = b"".join(f_varint(1, d) for d in arr.shape)
    out += f_varint(2, ELEM[arr.dtype]) + f_bytes(8, name)
    if raw:
        out += f_bytes(9, arr.tobytes())
    elif arr.dtype == np.float32:
        out += f_bytes(4, arr.astype("<f4").tobytes())  # packed float_data
    elif arr.dtype == np.int64:
        out += f_packed_varints(7, arr.reshape(-1))
    elif arr.dtype == np.int32:
        out += f_packed_varints(5, arr.reshape(-1))
    elif arr.dtype == np.float64:
        out += f_bytes(10, arr.astype("<f8").tobytes())
    return out


def attribute(name, v):
    """AttributeProto with its type (field 20)."""
    out = f_bytes(1, name)
    if isinstance(v, np.ndarray):
        return out + f_bytes(5, tensor("", v)) + f_varint(20, 4)
    if isinstance(v, float):
        return out + f_fixed32(2, v) + f_varint(20, 1)
    if isinstance(v, (bool, int, np.integer)):
        return out + f_varint(3, int(v)) + f_varint(20, 2)
    if isinstance(v, str):
        return out + f_bytes(4, v) + f_varint(20, 3)
    if isinstance(v, (list, tuple)) and all(isinstance(x, (int, np.integer)) for x in v):
        return out + b"".join(f_varint(8, x) for x in v) + f_varint(20, 7)
    if isinstance(v, (list, tuple)):
        return out + f_bytes(7, struct.pack(f"<{len(v)}f", *v)) + f_varint(20, 6)
    raise TypeError(v)


def node(op, inputs, outputs, name="", **attrs):
    out = b"".join(f_bytes(1, i) for i in inputs) + b"".join(f_bytes(2, o) for o in outputs)
    out += f_bytes(3, name) + f_bytes(4, op)
    out += b"".join(f_bytes(5, attribute(k, v)) for k, v in attrs.items())
    return out


def value_info(name, dtype, shape):
    dims = b"".join(f_bytes(1, f_varint(1, d) if isinstance(d, int) else f_bytes(2, d)) for d in shape)
    tt = f_varint(1, ELEM[np.dtype(dtype)]) + f_bytes(2, dims)
    return f_bytes(1, name) + f_bytes(2, f_bytes(1, tt))


def model(nodes, inputs, outputs, initializers=(), opset=13, name="test"):
    """nodes: encoded NodeProtos; inputs/outputs: (name, dtype, shape); initializers: (name, array)."""
    g = b"".join(f_bytes(1, n) for n in nodes) + f_bytes(2, name)
    g += b"".join(f_bytes(5, tensor(n, a)) for n, a in initializers)
    g += b"".join(f_bytes(11, value_info(*i)) for i in inputs)
    g += b"".join(f_bytes(12, value_info(*o)) for o in outputs)
    return f_varint(1, 7) + f_bytes(2, "onnx_amd-tests") + f_bytes(7, g) + f_bytes(8, f_bytes(1, "") + f_varint(2, opset))


# ---- generic decoder ---------------------------------------------------------
def decode(buf):
    """{field: [values]}: varints as int, LEN as bytes, fixed32/64 as raw bytes."""
    out, i = {}, 0
    while i < len(buf):
        k, i = _read_varint(buf, i)
        field, wt = k >> 3, k & 7
        if wt == 0:
            v, i = _read_varint(buf, i)
        elif wt == 2:
            n, i = _read_varint(buf, i)
            v, i = buf[i:i + n], i + n
        elif wt == 5:
            v, i = buf[i:i + 4], i + 4
        elif wt == 1:
            v, i = buf[i:i + 8], i + 8
        else:
            raise ValueError(wt)
        out.setdefault(field, []).append(v)
    return out


def _read_varint(buf, i):
    v, s = 0, 0
    while True:
        b = buf[i]
        i += 1
        v |= (b & 0x7F) << s
        s += 7
        if not b & 0x80:
            return v, i
