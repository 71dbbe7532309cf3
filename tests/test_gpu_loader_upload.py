"""Damaged models loaded with the library initialised, so that every initializer of a model that parses is
uploaded to HBM at load time: each seeded mutation (truncation, bit flips, 0xFF runs, inserted bytes) of
mnist-8.onnx and of a BERT encoder layer either loads, uploads and fuses, or is refused with the loader's own
statuses (invalid argument for a malformed protobuf, not supported for an unconvertible field)."""
import ctypes
import os

import numpy as np
import pytest

from onnx_amd import _lib as L
from onnx_amd.graph import ComputationalGraph

pytestmark = pytest.mark.gpu

HERE = os.path.dirname(os.path.abspath(__file__))


def test_damaged_models_with_initializer_upload(hip):
    from bert_layer import bert_layer
    seeds = [open(os.path.join(HERE, "golden", "mnist-8.onnx"), "rb").read(), bert_layer(1, 8, 3)[0]]
    lib = L.lib()
    rng = np.random.default_rng(11)
    loaded, refused = 0, {}
    for it in range(160):
        b = bytearray(seeds[it % 2])
        kind = (it // 2) % 4
        if kind == 0:
            b = b[:int(rng.integers(0, len(b)))]
        elif kind == 1:
            for _ in range(int(rng.integers(1, 9))):
                b[int(rng.integers(len(b)))] ^= 1 << int(rng.integers(8))
        elif kind == 2:
            p = int(rng.integers(len(b)))
            b[p:p + int(rng.integers(1, 10))] = b"\xff" * int(rng.integers(1, 10))
        else:
            p = int(rng.integers(len(b)))
            b[p:p] = bytes(rng.integers(0, 256, int(rng.integers(1, 16))).astype(np.uint8))
        h = ctypes.c_void_p()
        buf = ctypes.create_string_buffer(bytes(b), len(b))
        st = lib.lx_graph_load_onnx(buf, len(b), ctypes.byref(h))
        if st == L.OK:
            g = ComputationalGraph(_handle=h)
            _ = g.Nodes, g.InputInfo, g.InitializerInfo
            g.Fuse()
            loaded += 1
        else:
            assert st in (L.ERR_INVALID_ARGUMENT, L.ERR_NOT_SUPPORTED), (it, st, L.last_error())
            assert L.last_error()
            refused[st] = refused.get(st, 0) + 1
    assert loaded > 0 and sum(refused.values()) > 0, (loaded, refused)
