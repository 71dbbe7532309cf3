"""The Attention node -- an attention layer's scores MatMul, scaled masked Softmax and context MatMul in one
launch -- against the three fused nodes it replaces, bit for bit.  The same model with the scores made a graph
output keeps those three nodes (MatMulPermuted, ScaleAddSoftmax or AddSoftmax, MatMulPermuted), since a value
another reader sees is never fused away.  Heads of every size up to 64 rows, keys and columns, ragged ones
included; masks broadcast over heads and rows, per row, one per key or a single value; Div, Mul and no scale;
executed and captured.  Larger heads keep the node and run the three nodes inside it."""
import numpy as np
import pytest

import onnx_writer as W
from onnx_amd import DeviceTensor
from onnx_amd.graph import Model

pytestmark = pytest.mark.gpu


def attention_model(b, h, s, sk, d, dv, mask_kind, scale, extra_outputs=(), dtype=np.float32):
    rng = np.random.default_rng(s * 1000 + sk * 100 + d + 7 * dv)
    nodes = [W.node("Transpose", ["k"], ["kt"], "tk", perm=[0, 1, 3, 2]),
             W.node("MatMul", ["q", "kt"], ["sc"], "scores")]
    inits = []
    x = "sc"
    if scale is not None:
        inits.append(("c", np.array(np.sqrt(d) if scale == "div" else 1.0 / np.sqrt(d), dtype)))
        nodes.append(W.node("Div" if scale == "div" else "Mul", ["sc", "c"], ["scaled"], "scale"))
        x = "scaled"
    mshape = {"b11s": (b, 1, 1, sk), "bhss": (b, h, s, sk), "b1ss": (b, 1, s, sk), "s": (sk,), "one": (1,)}[mask_kind]
    mask = np.where(rng.random(mshape) < 0.2, -10000.0, rng.normal(0, 0.5, mshape)).astype(dtype)
    inits.append(("mask", mask))
    nodes += [W.node("Add", [x, "mask"], ["t"], "addmask"), W.node("Softmax", ["t"], ["p"], "softmax", axis=-1),
              W.node("MatMul", ["p", "v"], ["ctx"], "context"),
              W.node("Transpose", ["ctx"], ["y"], "heads", perm=[0, 2, 1, 3])]
    ins = {"q": rng.normal(0, 1, (b, h, s, d)).astype(dtype),
           "k": rng.normal(0, 1, (b, h, sk, d)).astype(dtype),
           "v": rng.normal(0, 1, (b, h, sk, dv)).astype(dtype)}
    outs = [("y", dtype, (b, s, h, dv))] + [(o, dtype, ()) for o in extra_outputs]
    model = W.model(nodes, [(n, dtype, a.shape) for n, a in ins.items()], outs, inits)
    return model, ins


CASES = [  # b, h, s, sk, d, dv, mask, scale
    (1, 1, 1, 1, 1, 1, "b11s", "div"),
    (2, 3, 8, 8, 32, 32, "b11s", "div"),       # the me5s heads at 8 tokens
    (1, 12, 8, 8, 64, 64, "b11s", "mul"),      # BERT-base heads at 8 tokens
    (2, 2, 5, 7, 13, 9, "bhss", "div"),
    (1, 2, 13, 13, 64, 64, "b11s", None),
    (2, 1, 31, 33, 17, 40, "one", "mul"),
    (1, 2, 32, 32, 32, 32, "bhss", None),
    (2, 3, 10, 10, 32, 32, "b11s", "div"),     # rows of 10 keys: head and tail elements per row
    (1, 2, 33, 6, 3, 64, "b11s", "div"),
    (1, 1, 64, 64, 64, 64, "bhss", "div"),
    (2, 2, 64, 64, 32, 32, "b11s", "mul"),     # the me5s heads at 64 tokens
    (2, 2, 33, 64, 64, 33, "s", "div"),
    (2, 3, 5, 6, 8, 8, "b1ss", "div"),         # a mask over batch and rows, not heads: three row axes
    (1, 1, 65, 65, 32, 32, "b11s", "div"),     # larger than one launch's heads: the three nodes
    (1, 2, 8, 8, 80, 32, "b11s", "div"),
]


@pytest.mark.parametrize("case", CASES, ids=lambda c: "x".join(map(str, c[:6])) + f"-{c[6]}-{c[7]}")
def test_attention_node_equals_the_three_nodes(hip, case):
    b, h, s, sk, d, dv, mask_kind, scale = case
    model, ins = attention_model(b, h, s, sk, d, dv, mask_kind, scale)
    kept, _ = attention_model(b, h, s, sk, d, dv, mask_kind, scale, extra_outputs=("sc",))
    dev = {k: DeviceTensor.from_numpy(v) for k, v in ins.items()}
    g = Model.Load(model)
    g.Fuse()
    assert [n.Op for n in g.Nodes] == ["Attention"]
    g3 = Model.Load(kept)
    g3.Fuse()
    soft = "ScaleAddSoftmax" if scale else "AddSoftmax"
    assert [n.Op for n in g3.Nodes] == ["MatMulPermuted", soft, "MatMulPermuted"]
    assert g3.Execute(dev), g3.LastError
    want = g3.Output("y").to_numpy()
    assert g.Execute(dev), g.LastError
    got = g.Output("y").to_numpy()
    assert got.shape == (b, s, h, dv) and np.isfinite(got).all()
    assert np.array_equal(got.view(np.uint32), want.view(np.uint32))
    # captured: replays on new inputs written into the captured buffers, checked against the three nodes
    assert g.Capture(dev), g.LastError
    assert np.array_equal(g.Output("y").to_numpy().view(np.uint32), want.view(np.uint32))
    for rep in range(2):
        q2 = (ins["q"] * (0.5 + rep)).astype(np.float32)
        dev["q"].upload(q2)
        assert g.Replay(), g.LastError
        got2 = g.Output("y").to_numpy().copy()
        assert g3.Execute(dev), g3.LastError
        assert np.array_equal(got2.view(np.uint32), g3.Output("y").to_numpy().view(np.uint32))
    g.ReleaseCapture()


@pytest.mark.parametrize("seed", range(3))
def test_attention_node_random_heads(hip, seed):
    """Seeded random heads (rows, keys, head and value widths from 1 to 64, masks and scales of every kind): the
    Attention node equals the three nodes it replaces bit for bit."""
    rng = np.random.default_rng(100 + seed)
    for _ in range(8):
        b, h = int(rng.integers(1, 4)), int(rng.integers(1, 5))
        s, sk, d, dv = (int(rng.integers(1, 65)) for _ in range(4))
        mask_kind = ["b11s", "bhss", "b1ss", "one"][int(rng.integers(4))]
        scale = [None, "div", "mul"][int(rng.integers(3))]
        if scale is None and mask_kind == "one":  # MatMul -> Add of a [1] constant fuses as a bias row instead
            mask_kind = "b11s"
        model, ins = attention_model(b, h, s, sk, d, dv, mask_kind, scale)
        kept, _ = attention_model(b, h, s, sk, d, dv, mask_kind, scale, extra_outputs=("sc",))
        dev = {k: DeviceTensor.from_numpy(v) for k, v in ins.items()}
        g, g3 = Model.Load(model), Model.Load(kept)
        g.Fuse()
        g3.Fuse()
        assert [n.Op for n in g.Nodes] == ["Attention"], (b, h, s, sk, d, dv, mask_kind, scale)
        assert g3.Execute(dev) and g.Execute(dev), (g.LastError, g3.LastError)
        got, want = g.Output("y").to_numpy(), g3.Output("y").to_numpy()
        assert np.array_equal(got.view(np.uint32), want.view(np.uint32)), (b, h, s, sk, d, dv, mask_kind, scale)


def test_attention_node_of_doubles_runs_the_nodes(hip):
    """Float64 heads: the Attention node runs its three nodes, and they their original nodes (the fused kernels are
    Float); the result equals the unfused graph's bit for bit."""
    # unscaled (a Div by a Float64 constant does not join the Softmax: the scaled pattern takes Float scalars)
    model, ins = attention_model(2, 3, 8, 8, 32, 32, "bhss", None, dtype=np.float64)
    dev = {k: DeviceTensor.from_numpy(v) for k, v in ins.items()}
    g, plain = Model.Load(model), Model.Load(model)
    g.Fuse()
    assert [n.Op for n in g.Nodes] == ["Attention"]
    assert plain.Execute(dev), plain.LastError
    want = plain.Output("y").to_numpy().copy()
    assert g.Execute(dev), g.LastError
    got = g.Output("y").to_numpy()
    assert got.dtype == np.float64 and np.array_equal(got.view(np.uint64), want.view(np.uint64))


def test_attention_node_launch_count(hip):
    """The Attention node is one kernel where the three nodes are three (profiled per node)."""
    model, ins = attention_model(2, 12, 8, 8, 32, 32, "b11s", "div")
    dev = {k: DeviceTensor.from_numpy(v) for k, v in ins.items()}
    g = Model.Load(model)
    g.Fuse()
    assert g.Execute(dev), g.LastError
    g.EnableProfiling(True)
    assert g.Execute(dev), g.LastError
    prof = g.Profile
    g.EnableProfiling(False)
    assert [p["op"] for p in prof] == ["Attention"]
