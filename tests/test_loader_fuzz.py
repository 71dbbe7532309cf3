"""Robustness of the ONNX loader against damaged models (CPU, no device).

Seeded mutations of two well-formed models (the reference's mnist-8.onnx fixture and a
BERT encoder layer written here): truncation, bit flips, runs of 0xFF bytes and inserted
random bytes. Every mutated model must either load, after which its node list, input
information and the fusion pass work, or be refused with the loader's own statuses
(malformed protobuf -> invalid argument, an unconvertible field -> not supported) and a
message. The loop runs in a child process so that a crash of the native decoder shows up
as a failing test and not as a dead test runner."""
import json
import os
import subprocess
import sys

import pytest

from onnx_amd import _lib as L

HERE = os.path.dirname(os.path.abspath(__file__))

CHILD = r"""
import ctypes, json, sys
import numpy as np
sys.path[:0] = [sys.argv[1], sys.argv[2]]
from onnx_amd import _lib as L
from onnx_amd.graph import ComputationalGraph
from bert_layer import bert_layer
seeds = [open(sys.argv[3], "rb").read(), bert_layer(1, 8, 3)[0]]
rng = np.random.default_rng(int(sys.argv[4]))
lib = L.lib()
loaded, refused, silent = 0, {}, 0
for it in range(int(sys.argv[5])):
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
        _ = g.Nodes
        loaded += 1
    else:
        refused[str(st)] = refused.get(str(st), 0) + 1
        silent += not L.last_error()
print(json.dumps({"loaded": loaded, "refused": refused, "silent": silent}), flush=True)
"""


@pytest.mark.parametrize("seed", [1, 2])
def test_damaged_models_load_or_are_refused_cleanly(seed):
    mnist = os.path.join(HERE, "golden", "mnist-8.onnx")
    r = subprocess.run([sys.executable, "-c", CHILD, os.path.dirname(HERE), HERE, mnist, str(seed), "240"],
                       capture_output=True, text=True, timeout=600)
    assert r.returncode == 0, (r.returncode, r.stderr[-2000:])
    res = json.loads(r.stdout.strip().splitlines()[-1])
    assert res["silent"] == 0
    assert set(res["refused"]) <= {str(L.ERR_INVALID_ARGUMENT), str(L.ERR_NOT_SUPPORTED)}, res
    # the mutations hit both sides: some damaged models still parse, most truncations do not
    assert res["loaded"] > 0 and sum(res["refused"].values()) > 0, res
