"""CPU checks of the graph runtime's host side: the ONNX loader against an
independent decode of the reference's mnist-8.onnx fixture and of models built
here, its error statuses, and the pattern fusion pass (lx_graph_fuse needs no
device)."""
import struct

import numpy as np
import pytest

import onnx_amd  # noqa: F401
from onnx_amd import _lib as L
from onnx_amd.graph import ComputationalGraph, Model

import onnx_writer as W

MNIST = __import__("os").path.join(__import__("os").path.dirname(__file__), "golden", "mnist-8.onnx")
SQRT2 = np.float32(np.sqrt(2.0))


def _independent(path):
    """Node ops/names, inputs, initializer shapes of a ModelProto via the generic decoder."""
    m = W.decode(open(path, "rb").read())
    g = W.decode(m[7][0])
    nodes = []
    for nb in g.get(1, []):
        n = W.decode(nb)
        nodes.append((n.get(3, [b""])[0].decode(), n[4][0].decode()))
    inits = []
    for tb in g.get(5, []):
        t = W.decode(tb)
        dims = []
        for d in t.get(1, []):
            dims += [W._read_varint(d, i)[0] for i in [0]] if isinstance(d, bytes) else [d]
        inits.append((t[8][0].decode(), t[2][0], tuple(dims)))
    ins = []
    for vb in g.get(11, []):
        v = W.decode(vb)
        tt = W.decode(W.decode(v[2][0])[1][0])
        shape = W.decode(tt[2][0]) if 2 in tt else {}
        dims = tuple(W.decode(d).get(1, [0])[0] for d in shape.get(1, []))
        ins.append((v[1][0].decode(), tt[1][0], dims))
    outs = [W.decode(vb)[1][0].decode() for vb in g.get(12, [])]
    opset = [W.decode(o) for o in m.get(8, [])]
    return nodes, ins, inits, outs, opset


def test_loader_reads_reference_mnist_fixture():
    nodes, ins, inits, outs, _ = _independent(MNIST)
    g = Model.Load(MNIST)
    assert [(n.Name, n.Op) for n in g.Nodes] == nodes
    assert g.InputInfo == ins
    assert sorted(g.InitializerInfo) == sorted(inits)
    assert g.OutputNames == outs
    # the bias-broadcast Adds the reference's tests name (test_backend.py:85, 96)
    assert ("Plus30", "Add") in nodes and ("Plus214", "Add") in nodes


def _all_kinds_model():
    nodes = [W.node("Add", ["x", "w"], ["y"], "add1"),
             W.node("Constant", [], ["c"], "const1", value=np.arange(6, dtype=np.float32).reshape(2, 3)),
             W.node("Cast", ["y"], ["z"], "cast1", to=7, note="text", ratio=0.5, axes=[0, -1], scales=[1.5, 2.5])]
    inits = [("w", np.arange(12, dtype=np.float32).reshape(3, 4)), ("i64", np.array([-3, 2**40], np.int64)),
             ("d", np.array([1.25], np.float64)), ("i32", np.array([[7, -8]], np.int32))]
    return W.model(nodes, [("x", np.float32, (3, 4)), ("n", np.float32, ("batch", 4))],
                   [("z", np.int64, (3, 4))], inits)


def test_loader_roundtrip_of_written_model():
    g = Model.Load(W.model([W.node("Add", ["x", "w"], ["y"], "add1")], [("x", np.float32, (3, 4))],
                           [("y", np.float32, (3, 4))], [("w", np.ones((3, 4), np.float32))]))
    assert [(n.Name, n.Op) for n in g.Nodes] == [("add1", "Add")]
    g = Model.Load(_all_kinds_model())
    assert [(n.Name, n.Op) for n in g.Nodes] == [("add1", "Add"), ("const1", "Constant"), ("cast1", "Cast")]
    # a symbolic dim reads as DimValue 0 (TensorUtil.cs:62-84)
    assert g.InputInfo == [("x", L.FLOAT, (3, 4)), ("n", L.FLOAT, (0, 4))]
    assert g.InitializerInfo == [("w", L.FLOAT, (3, 4)), ("i64", L.INT64, (2,)), ("d", L.DOUBLE, (1,)),
                                 ("i32", L.INT32, (1, 2))]
    assert g.OutputNames == ["z"]


@pytest.mark.parametrize("typed", [False, True])
def test_loader_typed_and_raw_initializer_fields(typed):
    """GetTensorData (TensorUtil.cs:14-31): typed fields when present, else raw_data."""
    for arr in [np.array([1.5, -2.25], np.float32), np.array([[-3, 2**40]], np.int64),
                np.array([7, -8, 9], np.int32), np.array([0.1], np.float64)]:
        t = W.tensor("p", arr, raw=not typed)
        buf = W.f_varint(1, 7) + W.f_bytes(7, W.f_bytes(5, t)) + W.f_bytes(8, W.f_varint(2, 13))
        g = Model.Load(buf)
        assert g.InitializerInfo == [("p", W.ELEM[arr.dtype], arr.shape)]


def test_loader_error_statuses():
    lib = L.lib()
    import ctypes
    h = ctypes.c_void_p()
    junk = b"\x0a\xff\xff\xff\xff\x0f"
    assert lib.lx_graph_load_onnx(junk, len(junk), ctypes.byref(h)) == L.ERR_INVALID_ARGUMENT
    assert "Malformed ONNX model" in L.last_error()
    # uint8 initializers are refused by GetTensorData (TensorUtil.cs:29)
    bad = W.model([], [], [], [("u", np.array([1, 2], np.uint8))])
    assert lib.lx_graph_load_onnx(bad, len(bad), ctypes.byref(h)) == L.ERR_NOT_SUPPORTED
    assert L.last_error() == "Cannot get embedded tensor data of tensor element type 2."
    # a graph-valued attribute has no conversion in AttributeProto.Value (NodeUtil.cs:20)
    att = W.f_bytes(1, "body") + W.f_bytes(6, b"") + W.f_varint(20, 5)
    nd = W.f_bytes(1, "x") + W.f_bytes(2, "y") + W.f_bytes(4, "If") + W.f_bytes(5, att)
    bad = W.model([nd], [], [])
    assert lib.lx_graph_load_onnx(bad, len(bad), ctypes.byref(h)) == L.ERR_NOT_SUPPORTED
    assert L.last_error() == "Cannot convert attribute proto value of type Graph."


@pytest.mark.parametrize("name,ok", [(b"caf\xc3\xa9", True), ("节\U0001f600".encode(), True),
                                     (b"\xc3", False),              # cut short
                                     (b"\xc0\x80", False),          # overlong NUL
                                     (b"\xed\xa0\x80", False),      # a UTF-16 surrogate
                                     (b"\xf4\x90\x80\x80", False),  # above U+10FFFF
                                     (b"a\xffb", False)])
def test_loader_names_must_be_utf8(name, ok):
    """Names are protobuf string fields, which hold UTF-8 text; other bytes make the model malformed."""
    lib = L.lib()
    import ctypes
    h = ctypes.c_void_p()
    nd = W.f_bytes(1, "x") + W.f_bytes(2, "y") + W.f_bytes(3, name) + W.f_bytes(4, "Sqrt")
    buf = W.model([nd], [("x", np.float32, (2,))], [("y", np.float32, (2,))])
    st = lib.lx_graph_load_onnx(buf, len(buf), ctypes.byref(h))
    if ok:
        assert st == L.OK
        g = ComputationalGraph(_handle=h)
        assert [n.Name for n in g.Nodes] == [name.decode()]
    else:
        assert st == L.ERR_INVALID_ARGUMENT
        assert L.last_error() == "Malformed ONNX model: node."


# ---- fusion ---------------------------------------------------------------------
def gelu_nodes(x="x", y="y", half="half", extra=()):
    return [W.node("Div", [x, "sqrt2"], ["a"], "div"), W.node("Erf", ["a"], ["e"], "erf"),
            W.node("Add", ["e", "one"], ["b"], "add"), W.node("Mul", [x, "b"], ["c"], "mul"),
            W.node("Mul", ["c", half], [y], "mul2")] + list(extra)


GELU_INITS = [("sqrt2", np.array(SQRT2, np.float32)), ("one", np.array(1.0, np.float32)),
              ("half", np.array(0.5, np.float32))]


def ln_nodes(x="x", y="y"):
    return [W.node("ReduceMean", [x, "axes"], ["mean"], "rm1"), W.node("Sub", [x, "mean"], ["d"], "sub"),
            W.node("Pow", ["d", "two"], ["p"], "pow"), W.node("ReduceMean", ["p", "axes"], ["var"], "rm2"),
            W.node("Add", ["var", "eps"], ["ve"], "addeps"), W.node("Sqrt", ["ve"], ["sd"], "sqrt"),
            W.node("Div", ["d", "sd"], ["n"], "div"), W.node("Mul", ["n", "gamma"], ["m"], "mulg"),
            W.node("Add", ["m", "beta"], [y], "addb")]


def LN_INITS(r=8):
    return [("axes", np.array([-1], np.int64)), ("two", np.array(2.0, np.float32)),
            ("eps", np.array(1e-12, np.float32)), ("gamma", np.ones(r, np.float32)), ("beta", np.zeros(r, np.float32))]


def _fused(nodes, inits, outputs=("y",), inputs=(("x", np.float32, (2, 8)),)):
    g = Model.Load(W.model(nodes, list(inputs), [(o, np.float32, (2, 8)) for o in outputs], inits))
    n = g.Fuse()
    return n, [(nd.Name, nd.Op) for nd in g.Nodes]


def test_fusion_replaces_the_three_subgraphs():
    assert _fused(gelu_nodes(), GELU_INITS) == (1, [("mul2", "GeluErf")])
    assert _fused(ln_nodes(), LN_INITS()) == (1, [("addb", "LayerNormDecomposed")])
    sm = [W.node("Add", ["x", "mask"], ["t"], "add"), W.node("Softmax", ["t"], ["y"], "sm", axis=-1)]
    assert _fused(sm, [("mask", np.zeros((1, 8), np.float32))]) == (1, [("sm", "AddSoftmax")])
    # the three in one graph, chained
    nodes = ln_nodes(y="h") + gelu_nodes(x="h", y="g") + [W.node("Add", ["g", "mask"], ["t"], "add3"),
                                                          W.node("Softmax", ["t"], ["y"], "sm")]
    inits = LN_INITS() + GELU_INITS + [("mask", np.zeros((1, 8), np.float32))]
    assert _fused(nodes, inits) == (3, [("addb", "LayerNormDecomposed"), ("mul2", "GeluErf"), ("sm", "AddSoftmax")])


def test_fusion_keeps_subgraphs_whose_intermediates_escape():
    """A pattern whose intermediate escapes is not replaced by its fused kernel; the elementwise-chain pass
    then fuses only the runs of nodes whose intermediates have no other consumer."""
    # an intermediate is also a graph output: Div -> Erf stops at the escaping e
    n, ops = _fused(gelu_nodes(), GELU_INITS, outputs=("y", "e"))
    assert (n, ops) == (2, [("erf", "ElementwiseChain"), ("mul2", "ElementwiseChain")])
    # an intermediate has a consumer outside the pattern: b feeds Mul and Sqrt
    n, ops = _fused(gelu_nodes(extra=[W.node("Sqrt", ["b"], ["z"], "other")]), GELU_INITS, outputs=("y", "z"))
    assert (n, ops) == (2, [("add", "ElementwiseChain"), ("mul2", "ElementwiseChain"), ("other", "Sqrt")])
    # a constant with other bits than float32(sqrt 2): no GeluErf, one chain of the five nodes
    inits = [("sqrt2", np.array(1.4142, np.float32))] + GELU_INITS[1:]
    assert _fused(gelu_nodes(), inits) == (1, [("mul2", "ElementwiseChain")])
    # a "constant" the caller may replace (an initializer that is also a graph input)
    n, ops = _fused(gelu_nodes(), GELU_INITS, inputs=(("x", np.float32, (2, 8)), ("half", np.float32, ())))
    assert (n, ops) == (1, [("mul2", "ElementwiseChain")])
    # LayerNorm reducing another axis: only Add eps -> Sqrt -> Div -> Mul -> Add chains
    inits = LN_INITS()
    inits[0] = ("axes", np.array([0], np.int64))
    n, ops = _fused(ln_nodes(), inits)
    assert n == 1 and [o for _, o in ops] == ["ReduceMean", "Sub", "Pow", "ReduceMean", "ElementwiseChain"]


def test_chain_fusion_boundaries():
    # C1: Add bias -> Mul scalar
    c1 = [W.node("Add", ["x", "bias"], ["h"], "add"), W.node("Mul", ["h", "k"], ["y"], "mul")]
    inits = [("bias", np.zeros(8, np.float32)), ("k", np.array(0.125, np.float32))]
    assert _fused(c1, inits) == (1, [("mul", "ElementwiseChain")])
    # a node using the chain value twice ends the chain before it
    sq = [W.node("Sub", ["x", "bias"], ["h"], "sub"), W.node("Mul", ["h", "h"], ["y"], "sq")]
    assert _fused(sq, inits) == (0, [("sub", "Sub"), ("sq", "Mul")])
    # a non-elementwise consumer ends it; single nodes are left alone
    sm = [W.node("Add", ["x", "bias"], ["h"], "add"), W.node("Softmax", ["h"], ["y"], "sm")]
    assert _fused(sm, inits)[0] == 1   # Add -> Softmax is the AddSoftmax pattern
    rs = [W.node("Add", ["x", "bias"], ["h"], "add"), W.node("ReduceSum", ["h"], ["y"], "rs")]
    assert _fused(rs, inits) == (0, [("add", "Add"), ("rs", "ReduceSum")])
    # at most 8 distinct inputs per chain: a ninth starts a new chain
    nodes, prev = [], "x"
    for k in range(9):
        nodes.append(W.node("Add", [prev, f"c{k}"], [f"t{k}" if k < 8 else "y"], f"n{k}"))
        prev = f"t{k}"
    inits9 = [(f"c{k}", np.full(8, k, np.float32)) for k in range(9)]
    n, ops = _fused(nodes, inits9)
    assert (n, ops) == (2, [("n6", "ElementwiseChain"), ("n8", "ElementwiseChain")])


def test_graph_builder_api_and_fusion_without_onnx_bytes():
    g = ComputationalGraph(13)
    g.AddInput("x", np.float32, (4, 8))
    for name, v in GELU_INITS:
        g.AddInitializer(name, v)
    g.AddNode("Div", ["x", "sqrt2"], ["a"], "div")
    g.AddNode("Erf", ["a"], ["e"], "erf")
    g.AddNode("Add", ["one", "e"], ["b"], "add")   # operands in the other order
    g.AddNode("Mul", ["b", "x"], ["c"], "mul")
    g.AddNode("Mul", ["half", "c"], ["y"], "mul2")
    g.AddOutput("y")
    assert g.Fuse() == 1 and [n.Op for n in g.Nodes] == ["GeluErf"]


# ---- a whole BERT-base encoder layer ---------------------------------------------------------
def test_bert_layer_oracle_against_float64():
    """The oracle's node-by-node float32 evaluation of a BERT layer (the reference's arithmetic) stays within
    1e-5 of an independent float64 evaluation: pins the graph oracle on a composite of every op kind."""
    from bert_layer import bert_layer, bert_layer_f64
    from oracle import graph_oracle as GO
    from test_gpu_graph import _dict_nodes
    _, ins, inits, nodes = bert_layer(1, 16, 3)
    ref = GO.run(_dict_nodes(nodes), ins, inits)["y"]
    assert np.abs(ref - bert_layer_f64(ins, inits)).max() < 1e-5


def test_encoder_oracle_against_float64():
    """The oracle's node-by-node float32 evaluation of a two-layer me5s-shaped encoder (embedding Gathers, the
    attention-mask Unsqueeze / Cast / scale, two encoder layers) stays within 1e-5 of an independent float64
    evaluation."""
    from bert_layer import encoder_model, encoder_model_f64
    from oracle import graph_oracle as GO
    from test_gpu_graph import _dict_nodes
    _, ins, inits, nodes = encoder_model(1, 16, layers=2, vocab=500, seed=4)
    ref = GO.run(_dict_nodes(nodes), ins, inits)["last_hidden_state"]
    assert np.abs(ref - encoder_model_f64(ins, inits, layers=2)).max() < 1e-5


def test_encoder_fusion_plan():
    """Every layer of the encoder fuses as the single layer does (5 fused nodes), plus the embedding sum, the
    embedding LayerNorm and the mask's Sub -> Mul."""
    from bert_layer import encoder_model
    model, _, _, _ = encoder_model(1, 16, layers=3, vocab=500, seed=4)
    g = Model.Load(model)
    assert g.Fuse() == 3 * 5 + 3
    ops = [n.Op for n in g.Nodes]
    assert ops[:7] == ["Gather", "Gather", "ElementwiseChain", "LayerNormDecomposed", "Unsqueeze", "Cast",
                       "ElementwiseChain"]
    assert ops.count("MatMulAddGroup") == 3 and ops.count("MatMulAddGelu") == 3 and ops.count("Attention") == 3
    assert ops.count("LayerNormDecomposed") == 1 and ops.count("MatMulAddLayerNorm") == 2 * 3
    assert "Add" not in ops and "Div" not in ops
    assert "MatMulPermuted" not in ops and "ScaleAddSoftmax" not in ops and "Transpose" not in ops
    assert "MatMul" not in ops


def test_bert_layer_fusion_plan():
    from bert_layer import bert_layer
    model, _, _, _ = bert_layer(1, 16, 3)
    g = Model.Load(model)
    assert g.Fuse() == 5
    ops = [n.Op for n in g.Nodes]
    assert ops.count("MatMulAddLayerNorm") == 2 and ops.count("Attention") == 1
    assert "Div" not in ops   # the scores' Div by sqrt(64) went into ScaleAddSoftmax
    # the six projections carry their bias (and the two residual Adds) in the MatMul epilogue, the FFN's
    # first one its GELU too, the two before a LayerNorm that LayerNorm; the Q, K, V projections of the same
    # input run as one grouped launch
    assert "MatMulAdd" not in ops and "LayerNormDecomposed" not in ops and "Add" not in ops and "GeluErf" not in ops
    # the attention products read Q, K (by columns) and V and write the context through the heads'
    # transposed views: no Transpose node is left; scores, masked Softmax and context form one Attention node
    # (placed where the context's output Transpose was)
    assert "MatMulPermuted" not in ops and "ScaleAddSoftmax" not in ops and "Transpose" not in ops
    assert "MatMul" not in ops and [n.Name for n in g.Nodes if n.Op == "Attention"] == ["c_perm"]
    assert [n.Name for n in g.Nodes if n.Op == "MatMulAddLayerNorm"] == ["addb1", "addb2"]
    assert [n.Name for n in g.Nodes if n.Op == "MatMulAddGelu"] == ["gelu_half"]
    assert [n.Name for n in g.Nodes if n.Op == "MatMulAddGroup"] == ["q_bias"]
    assert ops.index("MatMulAddGroup") == 0   # placed before the first consumer of any of its outputs


def test_scaled_softmax_pattern():
    nodes = [W.node("Div", ["x", "c"], ["s"], "scale"), W.node("Add", ["mask", "s"], ["t"], "add"),
             W.node("Softmax", ["t"], ["y"], "sm", axis=-1)]
    inits = [("c", np.array(8.0, np.float32)), ("mask", np.zeros((1, 8), np.float32))]
    assert _fused(nodes, inits) == (1, [("sm", "ScaleAddSoftmax")])
    mul = [W.node("Mul", ["c", "x"], ["s"], "scale")] + nodes[1:]
    assert _fused(mul, inits) == (1, [("sm", "ScaleAddSoftmax")])
    # a divisor that is not a scalar constant: the plain Add -> Softmax pattern
    inits2 = [("c", np.full(8, 8.0, np.float32)), ("mask", np.zeros((1, 8), np.float32))]
    assert _fused(nodes, inits2) == (1, [("scale", "Div"), ("sm", "AddSoftmax")])


def test_grouped_projection_constants_are_not_initializers():
    """Grouping unnamed projections makes one stacked weight / bias pair per group under names no other
    tensor uses; the graph's initializer list (graph.Initializers) stays what the model holds."""
    from test_gpu_matmul import _two_unnamed_projection_layers
    rng = np.random.default_rng(94)
    nodes, inits = _two_unnamed_projection_layers(rng)
    outs = ["q0", "k0", "v0", "q1", "k1", "v1"]
    g = Model.Load(W.model(nodes, [("x", np.float32, (2, 40, 64))], [(o, np.float32, ()) for o in outs], inits))
    before = g.InitializerInfo
    assert g.Fuse() == 2
    assert [n.Op for n in g.Nodes] == ["MatMulAddGroup", "MatMulAddGroup"]
    assert g.InitializerInfo == before and len(before) == 12


def test_profiling_switch_and_empty_profile():
    """The profiling switch and the record list exist without a device: nothing is recorded until an
    execution runs, and a record index past the end fails with a status, not a crash."""
    import ctypes
    from onnx_amd import _lib as L
    g = Model.Load(W.model(ln_nodes(), [("x", np.float32, (2, 8))], [("y", np.float32, (2, 8))], LN_INITS()))
    assert g.Profile == []
    g.EnableProfiling(True)
    g.EnableProfiling(False)
    g.ResetProfile()
    rec = L.LxNodeProfile()
    assert L.lib().lx_graph_profile(g._h, 0, ctypes.byref(rec)) != L.OK
    assert ctypes.sizeof(L.LxNodeProfile) == 8 + 4 + 36 + 8 + 8 + 8
    # the eager calls' records (lx_set_op_profiling): the same behaviour without a device
    assert ctypes.sizeof(L.LxOpProfile) == 36 + 4 + 8 + 8 + 8   # op[36], padding to 8, three doubles
    assert L.lib().lx_op_profile_count() == 0
    assert L.lib().lx_op_profile(0, ctypes.byref(L.LxOpProfile())) == L.ERR_INVALID_ARGUMENT
    assert L.lib().lx_op_profile_reset() == L.OK
