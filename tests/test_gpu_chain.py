"""GPU tests of the elementwise-chain kernel (lx_ElementwiseChain) and of the
graph runtime's chain fusion: a linear run of Float Add/Sub/Mul/Div/Pow/Sqrt/Erf
nodes computed in one pass must equal, bit for bit, the reference's node-by-node
result (the oracle restates CPUExecutionProvider.Add/.../Erf,
CPUExecutionProvider.cs:82-236, 380-409)."""
import numpy as np
import pytest

from onnx_amd import DeviceTensor, HipExecutionProvider as HIP, OpStatus
from onnx_amd import _lib as L
from onnx_amd.graph import Model
from oracle import graph_oracle as GO
from oracle import oracle as O

import onnx_writer as W

pytestmark = pytest.mark.gpu

BIN = {"Add": O.ADD, "Sub": O.SUB, "Mul": O.MUL, "Div": O.DIV, "Pow": O.POW}


def dev(a):
    return DeviceTensor.from_numpy(np.asarray(a))


def bits(a, b):
    """Bit-identical, any NaN matching any NaN: when both operands of an op are NaNs the payload that
    survives depends on the operand order of the machine instruction, which the compiler may commute."""
    a, b = np.ascontiguousarray(a), np.ascontiguousarray(b)
    if a.shape != b.shape:
        return False
    same = (a.view(np.uint32) == b.view(np.uint32)) | (np.isnan(a) & np.isnan(b))
    return bool(same.all())


def oracle_chain(inputs, program):
    acc = inputs[0]
    for ins in program:
        if ins[0] in ("Sqrt", "Erf"):
            acc = O.unary(O.SQRT if ins[0] == "Sqrt" else O.ERF, acc)
        elif len(ins) > 2 and ins[2]:
            acc = O.binary(BIN[ins[0]], inputs[ins[1]], acc)
        else:
            acc = O.binary(BIN[ins[0]], acc, inputs[ins[1]])
    return acc


def device_chain(inputs, program):
    """The same program node by node through the separate device operators."""
    d = [dev(x) for x in inputs]
    acc = d[0]
    for ins in program:
        if ins[0] in ("Sqrt", "Erf"):
            r = getattr(HIP, ins[0])(acc)
        elif len(ins) > 2 and ins[2]:
            r = getattr(HIP, ins[0])(d[ins[1]], acc)
        else:
            r = getattr(HIP, ins[0])(acc, d[ins[1]])
        assert r.Status == OpStatus.Success, r.Message
        acc = r.Outputs[0]
    return acc.to_numpy()


def check(inputs, program):
    """Bit-identical to the separate device operators; and to the oracle's node-by-node result when the
    program has no Pow (Pow is within 2 ulp of the host powf, not bit-exact)."""
    got = run_chain(inputs, program)
    assert bits(got, device_chain(inputs, program))
    if not any(p[0] == "Pow" for p in program):
        assert bits(got, oracle_chain(inputs, program))


def run_chain(inputs, program):
    r = HIP.ElementwiseChain([dev(x) for x in inputs], program)
    assert r.Status == OpStatus.Success, r.Message
    return r.Outputs[0].to_numpy()


CASES = [
    # C1: bias Add, scalar Mul
    ([(1, 128, 384), (384,), ()], [("Add", 1), ("Mul", 2)]),
    # the GELU chain through the generic kernel: x / sqrt2 -> erf -> + 1 -> x * . -> * 0.5
    ([(4, 64, 768), (), (), ()], [("Div", 1), ("Erf",), ("Add", 2), ("Mul", 0, True), ("Mul", 3)]),
    # LayerNorm tail: (var + eps) -> sqrt -> d / . -> * gamma -> + beta
    ([(8, 33, 1), (), (8, 33, 64), (64,), (64,)], [("Add", 1), ("Sqrt",), ("Div", 2, True), ("Mul", 3), ("Add", 4)]),
    # every op, operands on both sides, several broadcast patterns, an inner axis that does not divide by 4
    ([(3, 5, 7), (7,), (3, 1, 7), (5, 1), (), (1, 1, 1)],
     [("Sub", 1), ("Mul", 2, True), ("Add", 3), ("Div", 4, True), ("Pow", 5), ("Sqrt",), ("Sub", 0, True)]),
    # the output shape grows along the chain (rank-0 and lower-rank starts)
    ([(), (6,), (2, 6), (3, 1, 1)], [("Add", 1), ("Mul", 2), ("Sub", 3, True), ("Erf",)]),
    ([(64,), (16, 64), (4, 16, 1)], [("Mul", 1), ("Add", 2), ("Pow", 0, True)]),
    # 2^16 vectors and more take the one-wave tile kernel: the C3 pattern, the GELU chain with Erf, eight
    # inputs with Pow, a partial last tile, and an inner axis that does not divide by 4 (one float per vector)
    ([(5, 300, 176), (5, 1, 176), ()], [("Add", 1), ("Mul", 2)]),
    ([(3, 301, 292), (), (), ()], [("Div", 1), ("Erf",), ("Add", 2), ("Mul", 0, True), ("Mul", 3)]),
    ([(2, 257, 516), (516,), (2, 1, 516), (257, 1), (), (1, 1, 1), (2, 257, 1), (1, 257, 516)],
     [("Sub", 1), ("Mul", 2, True), ("Add", 3), ("Div", 4, True), ("Pow", 5), ("Sqrt",), ("Sub", 6), ("Add", 7)]),
    ([(7, 9363), (9363,), ()], [("Mul", 1), ("Erf",), ("Sub", 2, True)]),
]


@pytest.mark.parametrize("case", range(len(CASES)))
def test_chain_matches_node_by_node(hip, case):
    shapes, program = CASES[case]
    rng = np.random.default_rng(100 + case)
    ins = [(rng.standard_normal(s) * 2).astype(np.float32) for s in shapes]
    if any(p[0] == "Pow" for p in program):
        ins = [np.abs(x) + np.float32(0.5) for x in ins]   # real powers of positive bases, plus NaN-free Sqrt
    check(ins, program)


def test_chain_special_values(hip):
    x = np.array([0.0, -0.0, 1e-45, -1e-45, np.inf, -np.inf, np.nan, 3.4e38, -3.4e38, 1.0, 2.0, 0.5] * 11,
                 np.float32)
    y = np.roll(x, 5)
    check([x, y], [("Div", 1), ("Erf",), ("Mul", 1, True), ("Sub", 0), ("Sqrt",), ("Add", 1)])
    check([x, y], [("Div", 1), ("Erf",), ("Mul", 1, True), ("Sub", 0), ("Pow", 1), ("Sqrt",), ("Add", 1)])


def test_chain_errors(hip):
    a, b = dev(np.ones((2, 3), np.float32)), dev(np.ones((4,), np.float32))
    r = HIP.ElementwiseChain([a, b], [("Add", 1)])
    assert r.Code == L.ERR_CANNOT_BROADCAST
    r = HIP.ElementwiseChain([a, dev(np.ones((2, 3), np.int32))], [("Add", 1)])
    assert r.Code == L.ERR_INPUT_TYPE_NOT_SUPPORTED
    r = HIP.ElementwiseChain([a], [("Add", 1)])
    assert r.Code == L.ERR_INVALID_ARGUMENT


def _graph_run(nodes, inputs, inits, outputs, fuse):
    model = W.model(nodes, [(k, v.dtype, v.shape) for k, v in inputs.items()],
                    [(o, np.float32, ()) for o in outputs], inits)
    g = Model.Load(model)
    n = g.Fuse() if fuse else 0
    ok = g.Execute({k: DeviceTensor.from_numpy(v) for k, v in inputs.items()}, True)
    return g, n, ok


def test_graph_c1_chain_fused_bit_exact(hip):
    from test_gpu_graph import _dict_nodes
    rng = np.random.default_rng(7)
    x = rng.standard_normal((1, 128, 384)).astype(np.float32)
    nodes = [W.node("Add", ["x", "bias"], ["h"], "add"), W.node("Mul", ["h", "k"], ["y"], "mul")]
    inits = [("bias", rng.uniform(-0.1, 0.1, 384).astype(np.float32)), ("k", np.array(0.125, np.float32))]
    g, n, ok = _graph_run(nodes, {"x": x}, inits, ["y"], True)
    assert ok, g.LastError
    assert n == 1 and [nd.Op for nd in g.Nodes] == ["ElementwiseChain"]
    ref = GO.run(_dict_nodes(nodes), {"x": x}, dict(inits))
    assert bits(g.Output("y").to_numpy(), ref["y"])


def test_graph_chain_with_escaping_intermediate(hip):
    """GELU-shaped graph whose Erf output is also a graph output: two chains around it."""
    from test_graph_host import GELU_INITS, gelu_nodes
    from test_gpu_graph import _dict_nodes
    x = np.random.default_rng(8).standard_normal((3, 50, 70)).astype(np.float32)
    g, n, ok = _graph_run(gelu_nodes(), {"x": x}, GELU_INITS, ["y", "e"], True)
    assert ok, g.LastError
    assert n == 2
    ref = GO.run(_dict_nodes(gelu_nodes()), {"x": x}, dict(GELU_INITS))
    assert bits(g.Output("y").to_numpy(), ref["y"]) and bits(g.Output("e").to_numpy(), ref["e"])


def test_graph_chain_broadcast_failure_reports_the_original_node(hip):
    """Shapes that fail at the second node: the fused node runs its original nodes, so the failure names the
    same node with the same message as the unfused graph."""
    x = np.ones((2, 3), np.float32)
    nodes = [W.node("Add", ["x", "b"], ["h"], "first"), W.node("Mul", ["h", "c"], ["y"], "second")]
    inits = [("b", np.ones(3, np.float32)), ("c", np.ones(4, np.float32))]
    g0, _, ok0 = _graph_run(nodes, {"x": x}, inits, ["y"], False)
    g1, n1, ok1 = _graph_run(nodes, {"x": x}, inits, ["y"], True)
    assert n1 == 1 and not ok0 and not ok1
    assert g1.LastError == g0.LastError and "second" in g0.LastError


# ---- Div / Mul by a scalar -> Add(mask) -> Softmax in one kernel (lx_ScaleAddSoftmax) ------------------
@pytest.mark.parametrize("dt", [np.float32, np.float64])
@pytest.mark.parametrize("shape,mshape", [((2, 12, 64, 512), (2, 1, 1, 512)), ((3, 5, 70), (3, 1, 70)),
                                          ((4, 8, 4096), None), ((2, 3, 9000), (2, 1, 9000))])
def test_scale_add_softmax_equals_the_nodes(hip, dt, shape, mshape):
    """Bit-identical to the node-by-node device path (Div, Add, Softmax), including the shapes the fused
    kernel does not take (rows longer than its registers hold: node by node inside the call)."""
    rng = np.random.default_rng(31)
    s = (rng.standard_normal(shape) * 20).astype(dt)
    c = np.array(8.0, dt)
    m = None if mshape is None else np.where(rng.uniform(size=mshape) < 0.2, -10000.0, 0.0).astype(dt)
    for divide in (True, False):
        r = HIP.ScaleAddSoftmax(dev(s), dev(c), divide, None if m is None else dev(m))
        assert r.Status == OpStatus.Success, r.Message
        got = r.Outputs[0].to_numpy()
        t = (HIP.Div if divide else HIP.Mul)(dev(s), dev(c)).Outputs[0]
        if m is not None:
            t = HIP.Add(t, dev(m)).Outputs[0]
        ref = HIP.Softmax(t, -1).Outputs[0].to_numpy()
        assert got.shape == ref.shape and np.array_equal(got.view(np.uint8), ref.view(np.uint8)), divide


@pytest.mark.parametrize("c", [8.0, -8.0, 0.125, 2.0 ** 126, 2.0 ** -126, 2.0 ** -140, 3.0, 1e-30])
def test_scale_add_softmax_scales_equal_the_div_node(hip, c):
    """A division by a power of two runs as the multiplication by its exact reciprocal (the same correctly
    rounded value); other divisors -- and powers of two whose reciprocal is not a normal float -- divide.
    Either way the node's bits, over magnitudes that overflow, underflow to denormals and cancel."""
    rng = np.random.default_rng(34)
    s = (rng.standard_normal((4, 8, 96)) * np.float32(10.0) ** rng.integers(-40, 39, (4, 8, 96))).astype(np.float32)
    s[0, 0, :8] = [3.4e38, -3.4e38, 1e-45, -1e-45, 1.17e-38, 0.0, -0.0, 6e-39]
    m = np.where(rng.uniform(size=(4, 1, 96)) < 0.2, -10000.0, 0.0).astype(np.float32)
    cc = np.array(c, np.float32)
    t = HIP.Add(HIP.Div(dev(s), dev(cc)).Outputs[0], dev(m)).Outputs[0]
    ref = HIP.Softmax(t, -1).Outputs[0].to_numpy()
    r = HIP.ScaleAddSoftmax(dev(s), dev(cc), True, dev(m))
    assert r.Status == OpStatus.Success, r.Message
    assert bits(r.Outputs[0].to_numpy(), ref)


@pytest.mark.parametrize("axis", [-1, 4])
def test_scale_add_softmax_with_a_mask_that_grows_the_scores(hip, axis):
    """A mask of higher rank than the scores makes the Add's output larger: Softmax's axis is the sum's,
    as for the Softmax node, and the result is the nodes' (fused and unfused paths)."""
    rng = np.random.default_rng(33)
    s = (rng.standard_normal((2, 4, 6, 32)) * 10).astype(np.float32)
    m = np.where(rng.uniform(size=(3, 2, 4, 1, 32)) < 0.3, -10000.0, 0.0).astype(np.float32)
    c = np.array(8.0, np.float32)
    t = HIP.Add(HIP.Div(dev(s), dev(c)).Outputs[0], dev(m)).Outputs[0]
    ref = HIP.Softmax(t, axis).Outputs[0].to_numpy()
    r = HIP.ScaleAddSoftmax(dev(s), dev(c), True, dev(m), axis)
    assert r.Status == OpStatus.Success, r.Message
    assert bits(r.Outputs[0].to_numpy(), ref) and np.isfinite(ref).all()
    ref2 = HIP.Softmax(HIP.Add(dev(s), dev(m)).Outputs[0], axis).Outputs[0].to_numpy()
    r2 = HIP.AddSoftmax(dev(s), dev(m), axis)
    assert r2.Status == OpStatus.Success, r2.Message
    assert bits(r2.Outputs[0].to_numpy(), ref2)


def test_scale_add_softmax_graph(hip):
    from test_gpu_graph import _dict_nodes
    rng = np.random.default_rng(32)
    s = (rng.standard_normal((2, 12, 64, 128)) * 30).astype(np.float32)
    mask = np.where(rng.uniform(size=(2, 1, 1, 128)) < 0.25, -10000.0, 0.0).astype(np.float32)
    nodes = [W.node("Div", ["s", "c"], ["t"], "scale"), W.node("Add", ["t", "mask"], ["u"], "add"),
             W.node("Softmax", ["u"], ["y"], "sm", axis=-1)]
    inits = [("c", np.array(8.0, np.float32))]
    outs = {}
    for fuse in (False, True):
        g, ok = None, None
        model = W.model(nodes, [("s", np.float32, s.shape), ("mask", np.float32, mask.shape)],
                        [("y", np.float32, ())], inits)
        g = Model.Load(model)
        n = g.Fuse() if fuse else 0
        assert g.Execute({"s": DeviceTensor.from_numpy(s), "mask": DeviceTensor.from_numpy(mask)}), g.LastError
        outs[fuse] = (n, g.Output("y").to_numpy())
    assert outs[True][0] == 1 and bits(outs[True][1], outs[False][1])
    ref = GO.run(_dict_nodes(nodes), {"s": s, "mask": mask}, dict(inits))["y"]
    err = np.abs(outs[True][1].astype(np.float64) - ref.astype(np.float64))
    assert np.all(err <= 1e-5 * np.maximum(1.0, np.abs(ref))), err.max()
