"""Random graphs built from the subgraphs the fusion pass recognises (elementwise chains, the Erf GELU, the
decomposed LayerNorm, projections with a bias, a residual and a GELU, attention with transposed heads and a
scaled masked Softmax), with intermediates randomly made graph outputs so that patterns are cut where a value
has another reader: each graph executed unfused, fused and fused-and-captured.  The fused graph equals the
unfused one bit for bit unless it holds a fused reduction (LayerNorm, Softmax), whose sums run in another order:
then within a loose bar (the numerical bars of those kernels are tested against the oracle elsewhere; this test
checks that fusion rewires nothing).  Seeded: every run draws the same graphs."""
import math

import numpy as np
import pytest

import onnx_writer as W
from onnx_amd import DeviceTensor
from onnx_amd.graph import Model

pytestmark = pytest.mark.gpu

REDUCING = {"LayerNormDecomposed", "MatMulAddLayerNorm", "AddSoftmax", "ScaleAddSoftmax", "Attention"}


class Builder:
    def __init__(self, rng, b, s, h):
        self.rng, self.b, self.s = rng, b, s
        self.nodes, self.inits, self.k, self.made = [], [], 0, []
        self.vals = {"x": (b, s, h)}  # value name -> shape
        self.order = ["x"]

    def name(self, p):
        self.k += 1
        return f"{p}{self.k}"

    def const(self, arr):
        n = self.name("c")
        self.inits.append((n, np.asarray(arr)))
        return n

    def node(self, op, ins, **attrs):
        out = self.name("v")
        self.nodes.append(W.node(op, ins, [out], self.name("n"), **attrs))
        self.made.append(out)
        return out

    def add_value(self, v, shape):
        self.vals[v] = shape
        self.order.append(v)

    def pick(self, shape=None):
        cands = [v for v in self.order if shape is None or self.vals[v] == shape]
        return cands[int(self.rng.integers(len(cands)))] if cands else None

    def row(self, h, lo=-1.0, hi=1.0):
        return self.const(self.rng.uniform(lo, hi, h).astype(np.float32))

    def chain(self):
        v = self.pick()
        shape = self.vals[v]
        h = shape[-1]
        for _ in range(int(self.rng.integers(1, 5))):
            c = int(self.rng.integers(6))
            if c == 0:
                v = self.node("Add", [v, self.row(h)])
            elif c == 1:
                v = self.node("Sub", [self.const(np.float32(self.rng.uniform(-1, 1))), v])
            elif c == 2:
                other = self.pick(shape)
                v = self.node("Mul", [v, other if other != v else self.row(h)])
            elif c == 3:
                v = self.node("Div", [v, self.row(h, 0.5, 2.0)])
            elif c == 4:
                v = self.node("Erf", [v])
            else:
                v = self.node("Sqrt", [self.node("Add", [self.node("Mul", [v, v]), self.const(np.float32(1.0))])])
        self.add_value(v, shape)

    def gelu(self, v=None):
        v = v or self.pick()
        d = self.node("Div", [v, self.const(np.float32(math.sqrt(2.0)))])
        e = self.node("Erf", [d])
        a = self.node("Add", [e, self.const(np.float32(1.0))])
        m = self.node("Mul", [v, a])
        y = self.node("Mul", [m, self.const(np.float32(0.5))])
        self.add_value(y, self.vals[v])
        return y

    def layernorm(self, v=None):
        v = v or self.pick()
        h = self.vals[v][-1]
        axes, two, eps = self.const(np.array([-1], np.int64)), self.const(np.float32(2.0)), self.const(np.float32(1e-12))
        mean = self.node("ReduceMean", [v, axes])
        dd = self.node("Sub", [v, mean])
        p = self.node("Pow", [dd, two])
        var = self.node("ReduceMean", [p, axes])
        ve = self.node("Add", [var, eps])
        sd = self.node("Sqrt", [ve])
        nrm = self.node("Div", [dd, sd])
        m = self.node("Mul", [nrm, self.const((1 + 0.1 * self.rng.standard_normal(h)).astype(np.float32))])
        y = self.node("Add", [m, self.row(h, -0.1, 0.1)])
        self.add_value(y, self.vals[v])
        return y

    def projection(self):
        v = self.pick()
        b, s, k = self.vals[v]
        n = int(self.rng.choice([64, 256, 384]))
        w = self.const((self.rng.standard_normal((k, n)) / math.sqrt(k)).astype(np.float32))
        y = self.node("Add", [self.node("MatMul", [v, w]), self.row(n, -0.1, 0.1)])
        res = self.pick((b, s, n))
        if res is not None and self.rng.random() < 0.5:
            y = self.node("Add", [y, res])
        self.add_value(y, (b, s, n))
        r = self.rng.random()
        if r < 0.3:
            self.gelu(y)
        elif r < 0.6:
            self.layernorm(y)

    def attention(self):
        v = self.pick()
        b, s, h = self.vals[v]
        heads, dh = h // 32, 32
        shp = self.const(np.array([b, s, heads, dh], np.int64))

        def heads_of(t, perm):
            return self.node("Transpose", [self.node("Reshape", [t, shp])], perm=perm)
        q = heads_of(v, [0, 2, 1, 3])
        k = heads_of(self.pick((b, s, h)), [0, 2, 3, 1])
        vv = heads_of(self.pick((b, s, h)), [0, 2, 1, 3])
        sc = self.node("Div", [self.node("MatMul", [q, k]), self.const(np.float32(math.sqrt(dh)))])
        mask = (self.rng.random((b, 1, 1, s)) < 0.2).astype(np.float32) * np.float32(-10000.0)
        p = self.node("Softmax", [self.node("Add", [sc, self.const(mask)])], axis=-1)
        ctx = self.node("Transpose", [self.node("MatMul", [p, vv])], perm=[0, 2, 1, 3])
        y = self.node("Reshape", [ctx, self.const(np.array([b, s, h], np.int64))])
        self.add_value(y, (b, s, h))


def build(rng):
    b, s = int(rng.choice([1, 2])), int(rng.choice([8, 16, 64]))
    h = int(rng.choice([64, 256, 384]))
    g = Builder(rng, b, s, h)
    for _ in range(int(rng.integers(3, 8))):
        [g.chain, g.gelu, g.layernorm, g.projection, g.attention][int(rng.integers(5))]()
    outs = [g.order[-1]]
    # intermediates of the patterns as extra graph outputs: a pattern must then stop at them
    for o in g.made:
        if o not in outs and rng.random() < 0.12:
            outs.append(o)
    x = rng.standard_normal((b, s, h)).astype(np.float32)
    model = W.model(g.nodes, [("x", np.float32, x.shape)], [(o, np.float32, ()) for o in outs], g.inits)
    return model, x, outs


@pytest.mark.parametrize("seed", range(12))
def test_random_graphs_fuse_without_changing_results(hip, seed):
    rng = np.random.default_rng(1000 + seed)
    fused_any = 0
    for case in range(5):
        model, x, outs = build(rng)
        dev = {"x": DeviceTensor.from_numpy(x)}
        res, ops = {}, []
        for mode in ("nodes", "fused", "captured"):
            g = Model.Load(model)
            if mode != "nodes":
                fused_any += g.Fuse()
                ops = [n.Op for n in g.Nodes]
            ok = (g.Capture(dev) and g.Replay()) if mode == "captured" else g.Execute(dev)
            assert ok, (seed, case, mode, g.LastError)
            res[mode] = [g.Output(o).to_numpy() for o in outs]
        exact = not (REDUCING & set(ops))
        for mode in ("fused", "captured"):
            for o, u, f in zip(outs, res["nodes"], res[mode]):
                assert u.shape == f.shape and u.dtype == f.dtype, (seed, case, mode, o)
                assert np.array_equal(np.isnan(u), np.isnan(f)), (seed, case, mode, o)
                if exact:
                    assert np.array_equal(u.view(np.uint32), f.view(np.uint32)), (seed, case, mode, o, ops)
                else:
                    fin = ~np.isnan(u)
                    assert np.allclose(f[fin], u[fin], rtol=1e-3, atol=1e-4), (seed, case, mode, o, ops)
        assert np.array_equal(res["fused"][0].view(np.uint32), res["captured"][0].view(np.uint32))
    assert fused_any > 0
