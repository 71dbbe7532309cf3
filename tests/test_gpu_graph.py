"""GPU tests of the device graph runtime (lx_graph_*): whole graphs of the
BASELINE subgraphs executed with every tensor in HBM, with and without pattern
fusion, against the CPU restatement of the reference's graph executor
(oracle/graph_oracle.py) on the same inputs.

Bars as for the single operators: bit-exact for elementwise / integer / Cast /
the GELU chain; reductions, Softmax and LayerNorm within 1e-5 of the reference
relative to the magnitude of the reduced slice."""
import ctypes

import numpy as np
import pytest

from onnx_amd import DeviceTensor, HipExecutionProvider as HIP, OpStatus
from onnx_amd import _lib as L
from onnx_amd.graph import ComputationalGraph, Model
from oracle import graph_oracle as GO

import onnx_writer as W
from test_graph_host import GELU_INITS, LN_INITS, gelu_nodes, ln_nodes

pytestmark = pytest.mark.gpu


def _dict_nodes(encoded):
    """NodeProto bytes -> graph_oracle node dicts (through the generic decoder)."""
    out = []
    for nb in encoded:
        n = W.decode(nb)
        attrs = {}
        for ab in n.get(5, []):
            a = W.decode(ab)
            t = a[20][0]
            nm = a[1][0].decode()
            if t == 2:
                v = a[3][0]
                attrs[nm] = v - (1 << 64) if v >= 1 << 63 else v
            elif t == 1:
                attrs[nm] = np.frombuffer(a[2][0], np.float32)[0]
            elif t == 7:
                attrs[nm] = [v - (1 << 64) if v >= 1 << 63 else v for v in a[8]]
            elif t == 4:  # TensorProto written raw by onnx_writer.tensor
                tp = W.decode(a[5][0])
                np_dt = {v: k for k, v in W.ELEM.items()}[tp[2][0]]
                attrs[nm] = np.frombuffer(tp[9][0], np_dt).reshape(tp.get(1, []))
        out.append({"op": n[4][0].decode(), "inputs": [x.decode() for x in n.get(1, [])],
                    "outputs": [x.decode() for x in n.get(2, [])], "name": n.get(3, [b""])[0].decode(),
                    "attrs": attrs})
    return out


def run_both(nodes, inputs, inits, outputs, fuse, opset=13):
    """Device graph (optionally fused) and oracle graph on the same inputs."""
    model = W.model(nodes, [(k, v.dtype, v.shape) for k, v in inputs.items()],
                    [(o, np.float32, ()) for o in outputs], inits, opset=opset)
    g = Model.Load(model)
    nf = g.Fuse() if fuse else 0
    ok = g.Execute({k: DeviceTensor.from_numpy(v) for k, v in inputs.items()}, True)
    assert ok, g.LastError
    got = {o: g.Output(o).to_numpy() for o in outputs}
    ref = GO.run(_dict_nodes(nodes), inputs, dict(inits), opset)
    return got, {o: ref[o] for o in outputs}, nf, g


def bits(a, b):
    return np.array_equal(np.ascontiguousarray(a).view(np.uint8), np.ascontiguousarray(b).view(np.uint8))


def close(got, ref, x_abs_scale):
    err = np.abs(got.astype(np.float64) - ref.astype(np.float64))
    return np.all(err <= 1e-5 * np.maximum(1.0, x_abs_scale))


def test_c1_bias_add_scale_graph(hip):
    rng = np.random.default_rng(1)
    x = rng.standard_normal((1, 128, 384)).astype(np.float32)
    nodes = [W.node("Add", ["x", "bias"], ["h"], "add"), W.node("Mul", ["h", "k"], ["y"], "mul")]
    inits = [("bias", rng.uniform(-0.1, 0.1, 384).astype(np.float32)), ("k", np.array(0.125, np.float32))]
    got, ref, _, _ = run_both(nodes, {"x": x}, inits, ["y"], False)
    assert bits(got["y"], ref["y"])


@pytest.mark.parametrize("fuse", [False, True])
@pytest.mark.parametrize("shape", [(8, 512, 768), (3, 5, 64)])
def test_c2_layernorm_graph(hip, fuse, shape):
    rng = np.random.default_rng(2)
    r = shape[-1]
    x = (rng.standard_normal(shape) * 2).astype(np.float32)
    inits = LN_INITS(r)
    inits[3] = ("gamma", (1 + 0.02 * rng.standard_normal(r)).astype(np.float32))
    inits[4] = ("beta", (0.02 * rng.standard_normal(r)).astype(np.float32))
    got, ref, nf, g = run_both(ln_nodes(), {"x": x}, inits, ["y"], fuse)
    assert nf == (1 if fuse else 0)
    assert [n.Op for n in g.Nodes] == (["LayerNormDecomposed"] if fuse else
                                        ["ReduceMean", "Sub", "Pow", "ReduceMean", "Add", "Sqrt", "Div", "Mul", "Add"])
    assert close(got["y"], ref["y"], np.abs(ref["y"]))


@pytest.mark.parametrize("shape,gshape", [((8, 512, 768), (768, 1)), ((768, 768), (768, 1)), ((16, 64), (2, 32))])
def test_layernorm_graph_affine_shapes_follow_the_nodes(hip, shape, gshape):
    """A fused LayerNorm node whose gamma is not [1, ..., 1, r] runs its nine nodes: the same result bit for
    bit as the unfused graph when gamma broadcasts down the columns, the same failure (node, op, message)
    when it cannot broadcast."""
    rng = np.random.default_rng(27)
    r = shape[-1]
    x = (rng.standard_normal(shape) * 2).astype(np.float32)
    inits = LN_INITS(r)
    inits[3] = ("gamma", (1 + 0.02 * rng.standard_normal(gshape)).astype(np.float32))
    inits[4] = ("beta", (0.02 * rng.standard_normal(r)).astype(np.float32))
    res = {}
    for fuse in (False, True):
        g = Model.Load(W.model(ln_nodes(), [("x", np.float32, shape)], [("y", np.float32, shape)], inits))
        if fuse:
            assert g.Fuse() == 1 and [n.Op for n in g.Nodes] == ["LayerNormDecomposed"]
        ok_ = g.Execute({"x": DeviceTensor.from_numpy(x)})
        res[fuse] = (ok_, g.LastError if not ok_ else g.Output("y").to_numpy())
        g.close()
    try:
        ref = GO.run(_dict_nodes(ln_nodes()), {"x": x}, dict(inits), 13)["y"]
    except Exception:
        ref = None
    if gshape[0] == shape[-2]:
        assert res[False][0] and res[True][0], res
        assert bits(res[False][1], res[True][1])
        assert ref is not None and close(res[True][1], ref, np.abs(ref))
    else:
        assert not res[False][0] and not res[True][0] and ref is None
        assert res[False][1] == res[True][1] and "mulg" in res[True][1], res


@pytest.mark.parametrize("fuse", [False, True])
def test_c3_mask_softmax_graph(hip, fuse):
    rng = np.random.default_rng(3)
    s = (rng.standard_normal((2, 12, 64, 512)) * 3).astype(np.float32)
    m = np.where(rng.uniform(size=(2, 1, 1, 512)) < 0.125, -10000.0, 0.0).astype(np.float32)
    nodes = [W.node("Add", ["s", "mask"], ["t"], "add"), W.node("Softmax", ["t"], ["y"], "sm", axis=-1)]
    got, ref, nf, _ = run_both(nodes, {"s": s}, [("mask", m)], ["y"], fuse)
    assert nf == (1 if fuse else 0)
    assert close(got["y"], ref["y"], np.abs(ref["y"]))


@pytest.mark.parametrize("dt", [np.int64, np.int32])
def test_c4_integer_graph(hip, dt):
    rng = np.random.default_rng(4)
    a = rng.integers(-(2**20), 2**20, (16, 1, 256), dtype=dt)
    b = rng.integers(1, 1025, (1, 64, 256), dtype=dt)
    nodes = [W.node("Add", ["a", "b"], ["s"], "add"), W.node("Mul", ["a", "b"], ["p"], "mul"),
             W.node("Div", ["p", "b"], ["q"], "div"), W.node("Cast", ["s"], ["f"], "cast", to=1),
             W.node("ReduceSum", ["q", "ax1"], ["r"], "rsum", keepdims=1)]
    got, ref, _, _ = run_both(nodes, {"a": a, "b": b}, [("ax1", np.array([1], np.int64))], ["s", "p", "q", "f", "r"],
                              False)
    for k in ["s", "p", "q", "f", "r"]:
        assert bits(got[k], ref[k]), k


@pytest.mark.parametrize("fuse", [False, True])
def test_c5_gelu_and_reductions_graph(hip, fuse):
    rng = np.random.default_rng(5)
    x = rng.standard_normal((4, 64, 768)).astype(np.float32)
    extra = [W.node("ReduceSum", ["y", "ax1"], ["rs"], "rsum", keepdims=1),
             W.node("ReduceMean", ["y", "noaxes"], ["rm"], "rmean", keepdims=1)]
    nodes = gelu_nodes(extra=extra)
    inits = GELU_INITS + [("ax1", np.array([1], np.int64)), ("noaxes", np.zeros((0,), np.int64))]
    got, ref, nf, _ = run_both(nodes, {"x": x}, inits, ["y", "rs", "rm"], fuse)
    assert nf == (1 if fuse else 0)
    assert bits(got["y"], ref["y"])
    assert close(got["rs"], ref["rs"], np.abs(ref["y"]).sum(axis=1, keepdims=True))
    # a serial float32 fold of 196608 mostly positive terms is itself off by
    # ~1e-5 of the mean: judge both against the float64 sum, the device within the
    # bar or no farther from it than the reference's serial order
    truth = ref["y"].astype(np.float64).mean()
    e_dev = abs(float(got["rm"].reshape(-1)[0]) - truth)
    e_ref = abs(float(ref["rm"].reshape(-1)[0]) - truth)
    assert e_dev <= max(e_ref, 1e-5 * float(np.abs(ref["y"]).mean())), (e_dev, e_ref)


def test_shape_ops_graph(hip):
    """Reshape / Unsqueeze (views), Shape, Constant (host-known values) mixed with device ops."""
    rng = np.random.default_rng(6)
    x = rng.standard_normal((6, 8)).astype(np.float32)
    cval = rng.standard_normal((1, 2, 24)).astype(np.float32)
    nodes = [W.node("Shape", ["x"], ["xs"], "shape"),
             W.node("Reshape", ["x", "newshape"], ["r"], "reshape"),
             W.node("Unsqueeze", ["r", "uax"], ["u"], "unsq"),
             W.node("Constant", [], ["c"], "const", value=cval),
             W.node("Add", ["u", "c"], ["y"], "add"),
             W.node("Cast", ["xs"], ["xsf"], "cast", to=1)]
    inits = [("newshape", np.array([2, -1], np.int64)), ("uax", np.array([0], np.int64))]
    got, ref, _, _ = run_both(nodes, {"x": x}, inits, ["y", "xs", "xsf"], False)
    assert got["y"].shape == (1, 2, 24) and bits(got["y"], ref["y"])
    assert np.array_equal(got["xs"], [6, 8]) and bits(got["xsf"], ref["xsf"])


def test_opset11_attribute_axes(hip):
    x = np.random.default_rng(7).standard_normal((4, 6, 5)).astype(np.float32)
    nodes = [W.node("ReduceMean", ["x"], ["m"], "rm", axes=[1], keepdims=0),
             W.node("Unsqueeze", ["m"], ["u"], "unsq", axes=[1])]
    got, ref, _, _ = run_both(nodes, {"x": x}, [], ["u"], False, opset=11)
    assert got["u"].shape == (4, 1, 5) and close(got["u"], ref["u"], np.abs(x).mean(axis=1, keepdims=True))


def test_execution_stops_at_first_failing_node(hip):
    a = np.array([4, 6, 8], np.int32)
    b = np.array([2, 0, 2], np.int32)
    nodes = [W.node("Add", ["a", "a"], ["s"], "add"), W.node("Div", ["s", "b"], ["q"], "div"),
             W.node("Mul", ["q", "q"], ["y"], "mul")]
    g = Model.Load(W.model(nodes, [("a", np.int32, (3,)), ("b", np.int32, (3,))], [("y", np.int32, (3,))]))
    assert not g.Execute([a, b])
    assert g.LastStatus == L.ERR_DIVIDE_BY_ZERO
    assert g.LastError.startswith("Execution of node 2 div with op Div failed:")
    assert "y" not in g.Outputs
    # an unsupported op stops the run with NotSupported
    g = Model.Load(W.model([W.node("Relu", ["a"], ["y"], "relu")], [("a", np.float32, (3,))], [("y", np.float32, (3,))]))
    assert not g.Execute([np.ones(3, np.float32)])
    assert g.LastStatus == L.ERR_NOT_SUPPORTED
    assert g.LastError == "Execution of node 1 relu with op Relu failed: The operation Relu is not supported by the backend."
    # wrong number of user inputs (ComputationalGraph.cs:83-89)
    assert not g.Execute([])
    assert "user input(s) required" in g.LastError


def test_use_initializers_and_execute_node(hip):
    w = np.arange(4, dtype=np.float32)
    nodes = [W.node("Add", ["x", "w"], ["y"], "add")]
    g = Model.Load(W.model(nodes, [("x", np.float32, (4,)), ("w", np.float32, (4,))], [("y", np.float32, (4,))],
                           [("w", w)]))
    x = np.full(4, 2.0, np.float32)
    assert g.Execute([x], True) and np.array_equal(g.Output("y").to_numpy(), x + w)   # w served by its initializer
    assert not g.Execute([x], False)                                                    # now w is required
    assert g.Execute({"x": x, "w": -w}, False) and np.array_equal(g.Output("y").to_numpy(), x - w)
    assert g.ExecuteNode([x], "add", True) and np.array_equal(g.Output("y").to_numpy(), x + w)


def test_repeated_execution_reuses_device_memory(hip):
    """Steady state: executions after the first take every block from the pool."""
    rng = np.random.default_rng(8)
    x = DeviceTensor.from_numpy((rng.standard_normal((8, 512, 768)) * 2).astype(np.float32))
    g = Model.Load(W.model(ln_nodes(), [("x", np.float32, (8, 512, 768))], [("y", np.float32, (8, 512, 768))],
                           LN_INITS(768)))
    live, cached = ctypes.c_int64(), ctypes.c_int64()
    stats = []
    for _ in range(4):
        assert g.Execute([x]), g.LastError
        L.lib().lx_pool_stats(ctypes.byref(live), ctypes.byref(cached))
        stats.append((live.value, cached.value))
        g.Reset()
    assert len(set(stats[1:])) == 1, stats
    y1 = None
    for _ in range(2):
        assert g.Execute([x])
        y = g.Output("y").to_numpy()
        assert y1 is None or bits(y, y1)
        y1 = y


# ---- device-side checks deferred to one readback per execution ------------------------------
def _exec(nodes, inputs, inits, outputs, fuse=False):
    model = W.model(nodes, [(k, v.dtype, v.shape) for k, v in inputs.items()],
                    [(o, np.float32, ()) for o in outputs], inits)
    g = Model.Load(model)
    if fuse:
        g.Fuse()
    ok = g.Execute({k: DeviceTensor.from_numpy(v) for k, v in inputs.items()}, True)
    return g, ok


def test_deferred_gather_failure_is_reported_as_its_node(hip):
    """An out-of-range Gather index is found after the last node ran (one readback per execution); the
    failure names the Gather node with the operator's own message, and no later node's output is kept."""
    table = np.arange(12, dtype=np.float32).reshape(4, 3)
    nodes = [W.node("Gather", ["table", "ids"], ["e"], "gather"), W.node("Add", ["e", "one"], ["h"], "add"),
             W.node("Mul", ["h", "two"], ["y"], "mul")]
    inits = [("table", table), ("one", np.array(1.0, np.float32)), ("two", np.array(2.0, np.float32))]
    g, ok = _exec(nodes, {"ids": np.array([0, 7], np.int64)}, inits, ["y"])
    assert not ok
    assert g.LastError == "Execution of node 1 gather with op Gather failed: Index was outside the bounds of the array."
    assert "y" not in g.Outputs
    # the same graph with valid indices runs through, and again after the failure
    g2, ok = _exec(nodes, {"ids": np.array([3, -4], np.int64)}, inits, ["y"])
    assert ok, g2.LastError
    assert np.array_equal(g2.Output("y").to_numpy(), (table[[3, 0]] + 1) * 2)


def test_deferred_device_failure_precedes_a_later_host_failure(hip):
    """Node 1 fails on the device (Gather), node 3 on the host (shapes that do not broadcast): node by node
    the reference stops at node 1, so node 1 is reported."""
    nodes = [W.node("Gather", ["table", "ids"], ["e"], "gather"), W.node("Add", ["e", "one"], ["h"], "add"),
             W.node("Mul", ["h", "bad"], ["y"], "mul")]
    inits = [("table", np.ones((4, 3), np.float32)), ("one", np.array(1.0, np.float32)),
             ("bad", np.ones(5, np.float32))]
    g, ok = _exec(nodes, {"ids": np.array([9], np.int64)}, inits, ["y"])
    assert not ok and g.LastError.startswith("Execution of node 1 gather with op Gather failed")
    g, ok = _exec(nodes, {"ids": np.array([1], np.int64)}, inits, ["y"])
    assert not ok and g.LastError.startswith("Execution of node 3 mul with op Mul failed")


@pytest.mark.parametrize("dt", [np.int32, np.int64])
def test_deferred_integer_division_and_cast_checks(hip, dt):
    a = np.array([7, -9, 4], dt)
    nodes = [W.node("Div", ["a", "b"], ["q"], "div"), W.node("Cast", ["q"], ["y"], "cast", to=3)]  # to Int8
    g, ok = _exec(nodes, {"a": a, "b": np.array([2, 0, 1], dt)}, [], ["y"])
    assert not ok and g.LastError == "Execution of node 1 div with op Div failed: Attempted to divide by zero."
    g, ok = _exec(nodes, {"a": np.array([7, -900, 4], dt), "b": np.array([2, 1, 1], dt)}, [], ["y"])
    assert not ok
    assert g.LastError == ("Execution of node 2 cast with op Cast failed: Value was either too large or too small "
                           "for a signed byte.")
    # the messages equal the operators' own
    r = HIP.Div(DeviceTensor.from_numpy(a), DeviceTensor.from_numpy(np.array([2, 0, 1], dt)))
    assert r.Message == "Attempted to divide by zero."
    g, ok = _exec(nodes, {"a": a, "b": np.array([2, 3, 1], dt)}, [], ["y"])
    assert ok, g.LastError
    assert np.array_equal(g.Output("y").to_numpy(), np.array([3, -3, 4], np.int8))


# ---- captured executions (lx_graph_capture / lx_graph_replay) ---------------------------------
def _ln_graph(fuse):
    model = W.model(ln_nodes(), [("x", np.float32, (4, 64, 128))], [("y", np.float32, ())], LN_INITS(128))
    g = Model.Load(model)
    if fuse:
        g.Fuse()
    return g


@pytest.mark.parametrize("fuse", [False, True])
def test_capture_replays_match_eager_executions(hip, fuse):
    """Every replay, with new data written into the captured input buffer and eager executions and
    synchronisations between the replays, equals an eager execution on the same data bit for bit."""
    rng = np.random.default_rng(70)
    g, eager = _ln_graph(fuse), _ln_graph(fuse)
    xs = [(rng.standard_normal((4, 64, 128)) * 3).astype(np.float32) for _ in range(4)]
    xd = DeviceTensor.from_numpy(xs[0])
    assert g.Capture([xd]), g.LastError
    for i, x in enumerate(xs):
        xd.upload(x)
        assert g.Replay(), g.LastError
        got = g.Output("y").to_numpy()
        assert eager.Execute([DeviceTensor.from_numpy(x)]), eager.LastError
        assert bits(got, eager.Output("y").to_numpy()), i
        # eager work on the same graph object between replays does not disturb the record
        assert g.Execute([DeviceTensor.from_numpy(xs[(i + 1) % 4])]), g.LastError
    g.ReleaseCapture()
    assert not g.Replay() and "no captured execution" in g.LastError


def test_capture_with_gather_reports_failures_per_replay(hip):
    table = np.arange(12, dtype=np.float32).reshape(4, 3)
    nodes = [W.node("Gather", ["table", "ids"], ["e"], "gather"), W.node("Mul", ["e", "two"], ["y"], "mul")]
    model = W.model(nodes, [("ids", np.int64, (2,))], [("y", np.float32, ())],
                    [("table", table), ("two", np.array(2.0, np.float32))])
    g = Model.Load(model)
    ids = DeviceTensor.from_numpy(np.array([0, 1], np.int64))
    assert g.Capture([ids]), g.LastError
    for v, good in (([3, 2], True), ([1, 4], False), ([-1, -4], True)):
        ids.upload(np.array(v, np.int64))
        assert g.Replay() == good, g.LastError
        if good:
            assert np.array_equal(g.Output("y").to_numpy(), table[v] * 2)
        else:
            assert g.LastError == ("Execution of node 1 gather with op Gather failed: Index was outside the bounds "
                                   "of the array.")


def test_capture_refuses_device_computed_shapes(hip):
    """Reshape whose target shape is computed on the device needs that shape on the host mid-execution:
    such a graph executes but cannot be captured."""
    nodes = [W.node("Add", ["s", "zero"], ["shape"], "add"), W.node("Reshape", ["x", "shape"], ["y"], "reshape")]
    model = W.model(nodes, [("x", np.float32, (2, 6)), ("s", np.int64, (2,))], [("y", np.float32, ())],
                    [("zero", np.zeros(2, np.int64))])
    g = Model.Load(model)
    ins = {"x": DeviceTensor.from_numpy(np.arange(12, dtype=np.float32).reshape(2, 6)),
           "s": DeviceTensor.from_numpy(np.array([3, 4], np.int64))}
    assert g.Execute(ins), g.LastError
    assert g.Output("y").to_numpy().shape == (3, 4)
    assert not g.Capture(ins) and g.LastStatus == L.ERR_NOT_SUPPORTED
    assert g.Execute(ins), g.LastError   # the stream is usable afterwards


def test_capture_memory_is_released(hip):
    g = _ln_graph(False)
    x = DeviceTensor.from_numpy(np.ones((4, 64, 128), np.float32))
    live0 = L.pool_stats()[0]
    assert g.Capture([x]), g.LastError
    assert g.Replay(), g.LastError
    g.ReleaseCapture()
    g.Reset()
    assert L.pool_stats()[0] <= live0 + 4096   # the check records stay with the graph


def _dynamic_reshape_model(idx=0):
    """Shape -> Gather -> Concat -> Reshape: the shape arithmetic of an exported model (the batch size read
    at run time).  A rank-0 initializer loads as shape [1] here, as the reference's TensorUtil reads it, so
    the index is written as [idx] and no Unsqueeze is needed."""
    nodes = [W.node("Shape", ["x"], ["s"], "shape"),
             W.node("Gather", ["s", "i"], ["b"], "gather", axis=0),
             W.node("Concat", ["b", "rest"], ["tgt"], "concat", axis=0),
             W.node("Reshape", ["x", "tgt"], ["r"], "reshape"),
             W.node("Transpose", ["r"], ["y"], "perm", perm=[0, 2, 1, 3])]
    inits = [("i", np.array([idx], np.int64)), ("rest", np.array([40, 4, 24], np.int64))]
    return W.model(nodes, [("x", np.float32, (2, 40, 96))], [("y", np.float32, ())], inits)


def test_shape_arithmetic_runs_on_the_host_and_captures(hip):
    """Gather / Concat over small integer vectors the host knows are computed there: the Reshape reads its
    target without a download, and the graph can be captured and replayed (it could not while the shape
    vector came back from the device)."""
    x = np.random.default_rng(95).standard_normal((2, 40, 96)).astype(np.float32)
    ref = x.reshape(2, 40, 4, 24).transpose(0, 2, 1, 3)
    g = Model.Load(_dynamic_reshape_model())
    dx = DeviceTensor.from_numpy(x)
    assert g.Execute({"x": dx}), g.LastError
    assert np.array_equal(g.Output("y").to_numpy(), ref)
    assert g.Capture({"x": dx}), g.LastError
    for scale in (1.0, -2.0):
        dx.upload(x * scale)
        assert g.Replay(), g.LastError
        assert np.array_equal(g.Output("y").to_numpy(), (x * scale).reshape(2, 40, 4, 24).transpose(0, 2, 1, 3))


def test_shape_arithmetic_out_of_range_index_fails_as_the_device_operator(hip):
    g = Model.Load(_dynamic_reshape_model(idx=5))
    assert not g.Execute({"x": DeviceTensor.from_numpy(np.zeros((2, 40, 96), np.float32))})
    assert "gather" in g.LastError and "outside the bounds" in g.LastError


def _assert_telescoping(prof, wall_ms, tiled=0.99, min_share=0.3, boundary_ms=0.0):
    """Records of consecutive work on one stream never overlap (each starts at or after the previous one's
    end), and when the device is the bottleneck they tile it: the device times add up to at least `tiled` of
    the span from the first start to the last end, less `boundary_ms` per boundary between two records (the
    device time of the event packets there); the span lies within the host's wall time around the work (and
    is at least `min_share` of it)."""
    for a, b in zip(prof, prof[1:]):
        assert b["start_ms"] >= a["start_ms"] + a["math_ms"] - 2e-3, (a, b)
    span = prof[-1]["start_ms"] + prof[-1]["math_ms"] - prof[0]["start_ms"]
    total = sum(p["math_ms"] for p in prof)
    assert tiled * span - boundary_ms * (len(prof) - 1) <= total <= span * 1.0001 + 1e-3, (total, span)
    assert min_share * wall_ms <= span <= wall_ms, (span, wall_ms)
    return span


def test_profiling_c2_graph_node_times_add_up_to_the_execution():
    """Profiler.StartNodeProfile / StopNodeProfile on the device: one execution of the nine-node LayerNorm
    graph records nine nodes with the reference's op types in node order, every node with device time, and
    the node times add up to the device span between the execution's first and last boundary events (the
    events telescope: each node ends at the next node's start); a second execution appends nine more; reset
    clears them; a fused graph records its one fused node."""
    import time
    rng = np.random.default_rng(29)
    shape = (64, 512, 768)
    x = DeviceTensor.from_numpy((rng.standard_normal(shape) * 2).astype(np.float32))
    inits = LN_INITS(768)
    ops = ["ReduceMean", "Sub", "Pow", "ReduceMean", "Add", "Sqrt", "Div", "Mul", "Add"]
    g = Model.Load(W.model(ln_nodes(), [("x", np.float32, shape)], [("y", np.float32, shape)], inits))
    assert g.Execute({"x": x}), g.LastError      # warm: uploads, pool
    assert g.Profile == []                        # not enabled
    g.EnableProfiling(True)
    onnx_sync()
    t0 = time.perf_counter()
    assert g.Execute({"x": x}), g.LastError
    wall = (time.perf_counter() - t0) * 1e3
    prof = g.Profile
    assert [p["op"] for p in prof] == ops and [p["node_id"] for p in prof] == list(range(9))
    assert all(p["math_ms"] > 0 and p["host_ms"] > 0 for p in prof)
    assert prof[0]["start_ms"] == 0.0
    _assert_telescoping(prof, wall)
    assert g.Execute({"x": x}), g.LastError
    assert len(g.Profile) == 18 and g.Profile[9]["start_ms"] == 0.0
    g.ResetProfile()
    assert g.Profile == []
    g.EnableProfiling(False)
    assert g.Execute({"x": x}), g.LastError
    assert g.Profile == []
    g.close()
    gf = Model.Load(W.model(ln_nodes(), [("x", np.float32, shape)], [("y", np.float32, shape)], inits))
    assert gf.Fuse() == 1
    gf.EnableProfiling(True)
    assert gf.Execute({"x": x}), gf.LastError
    prof = gf.Profile
    assert [p["op"] for p in prof] == ["LayerNormDecomposed"] and prof[0]["node_id"] == 8 and prof[0]["math_ms"] > 0
    gf.close()


def test_profiling_eager_c2_calls_time_the_device_work():
    """OpStage.Math of eager calls (lx_set_op_profiling): the nine operator calls of the decomposed LayerNorm
    made through HipExecutionProvider with profiling on record nine calls in order, each with device time
    between the HIP events around its launches; the records telescope over the calls' device span, which
    lies within the host wall time; calls made by a graph execution are not recorded as eager calls; reset
    clears the records and a disabled profiler records nothing."""
    import time
    rng = np.random.default_rng(33)
    shape = (256, 512, 768)   # 400 MB per tensor: each call's kernel outlasts the next call's dispatch
    x = DeviceTensor.from_numpy((rng.standard_normal(shape) * 2).astype(np.float32))
    gamma = DeviceTensor.from_numpy((1 + 0.02 * rng.standard_normal(768)).astype(np.float32))
    beta = DeviceTensor.from_numpy((0.02 * rng.standard_normal(768)).astype(np.float32))
    two = DeviceTensor.from_numpy(np.array(2.0, np.float32))
    eps = DeviceTensor.from_numpy(np.array(1e-12, np.float32))
    axes = [-1]

    def calls():
        def out(r):
            assert r.Status == OpStatus.Success, r.Message
            return r.Outputs[0]
        mean = out(HIP.ReduceMean(x, axes, 1))
        d = out(HIP.Sub(x, mean))
        p = out(HIP.Pow(d, two))
        var = out(HIP.ReduceMean(p, axes, 1))
        ve = out(HIP.Add(var, eps))
        sd = out(HIP.Sqrt(ve))
        n = out(HIP.Div(d, sd))
        m = out(HIP.Mul(n, gamma))
        return out(HIP.Add(m, beta))
    y_ref = calls().to_numpy()                    # warm: pool
    # six 3 GiB Adds (about 3 ms of device work, not profiled) queued first: the nine calls are all queued
    # before the device reaches them, so no host gap between two calls can leave the device idle, and their
    # records tile the device span
    big = DeviceTensor.from_numpy(np.ones(1 << 28, np.float32))
    sink = DeviceTensor.from_numpy(np.zeros(1 << 28, np.float32))
    HIP.Add(big, big, out=sink)
    HIP.ResetProfile()
    onnx_sync()
    t0 = time.perf_counter()
    for _ in range(6):
        assert HIP.Add(big, big, out=sink).Status == OpStatus.Success
    HIP.EnableProfiling(True)
    y = calls()
    onnx_sync()
    wall = (time.perf_counter() - t0) * 1e3
    prof = HIP.Profile()
    assert [p["op"] for p in prof] == ["ReduceMean", "Sub", "Pow", "ReduceMean", "Add", "Sqrt", "Div", "Mul", "Add"]
    assert all(p["math_ms"] > 0 and p["host_ms"] > 0 for p in prof), prof
    assert prof[0]["start_ms"] == 0.0
    # each call records its own start and end events: two event packets (a few us of device time) lie
    # between one call's end and the next call's start
    _assert_telescoping(prof, wall, tiled=0.99, min_share=0.05, boundary_ms=0.008)
    # no call's device time beats its algorithmic bytes at the 8 TB/s HBM peak
    big, row = np.prod(shape) * 4, np.prod(shape[:-1]) * 4
    moved = [big + row, 2 * big + row, 2 * big + 4, big + row, 2 * row + 4, 2 * row, 2 * big + row,
             2 * big + 768 * 4, 2 * big + 768 * 4]
    for p, b in zip(prof, moved):
        assert p["math_ms"] >= b / 8e12 * 1e3, (p, b)
    assert np.array_equal(y.to_numpy(), y_ref)
    g = Model.Load(W.model(ln_nodes(), [("x", np.float32, shape)], [("y", np.float32, shape)], LN_INITS(768)))
    assert g.Execute({"x": x}), g.LastError
    assert len(HIP.Profile()) == 9
    g.close()
    HIP.ResetProfile()
    assert HIP.Profile() == []
    HIP.EnableProfiling(False)
    calls()
    assert HIP.Profile() == []


def test_profiling_records_the_failing_node():
    """As the reference stops its node profile after Execute returns, the failing node is recorded too,
    and nothing after it."""
    rng = np.random.default_rng(30)
    nodes = [W.node("Add", ["a", "b"], ["s"], "add"), W.node("Div", ["s", "z"], ["q"], "div"),
             W.node("Mul", ["q", "b"], ["p"], "mul")]
    a = rng.standard_normal((4, 64)).astype(np.float32)
    b = rng.standard_normal((4, 64)).astype(np.float32)
    z = rng.standard_normal((3, 64)).astype(np.float32)   # Div [4,64] / [3,64]: CannotBroadcast on the host
    g = Model.Load(W.model(nodes, [("a", np.float32, a.shape), ("b", np.float32, b.shape), ("z", np.float32, z.shape)],
                           [("p", np.float32, a.shape)], []))
    g.EnableProfiling(True)
    ok_ = g.Execute({"a": DeviceTensor.from_numpy(a), "b": DeviceTensor.from_numpy(b), "z": DeviceTensor.from_numpy(z)})
    assert not ok_ and "div" in g.LastError and "broadcast" in g.LastError
    assert [p["op"] for p in g.Profile] == ["Add", "Div"]
    g.close()


def onnx_sync():
    import onnx_amd
    onnx_amd.synchronize()
