"""TEST / BENCH HELPER: one BERT-base encoder layer as an ONNX model (the node
sequence a PyTorch export of a BERT layer produces, with static shapes), plus a
float64 numpy evaluation of the same layer for accuracy checks.

    model_bytes, inputs, weights = bert_layer(batch, seq, seed)

Nodes: Q/K/V projections (MatMul + Add bias, Reshape to heads, Transpose),
scores (MatMul, Div by sqrt(64), Add mask, Softmax), context (MatMul, Transpose,
Reshape), output projection + residual, LayerNorm (9 nodes), FFN (MatMul + bias,
GELU as Div/Erf/Add/Mul/Mul, MatMul + bias) + residual, LayerNorm.  Every node is
one the reference's Node.ExecuteCPU switch handles (Node.cs:121-181)."""
import math

import numpy as np

import onnx_writer as W

H, HEADS, DH, FF = 768, 12, 64, 3072
SQRT2 = np.float32(math.sqrt(2.0))


def _ln(x, y, sfx):
    return [W.node("ReduceMean", [x, "axes"], [f"mean{sfx}"], f"rm1{sfx}"),
            W.node("Sub", [x, f"mean{sfx}"], [f"d{sfx}"], f"sub{sfx}"),
            W.node("Pow", [f"d{sfx}", "two"], [f"p{sfx}"], f"pow{sfx}"),
            W.node("ReduceMean", [f"p{sfx}", "axes"], [f"var{sfx}"], f"rm2{sfx}"),
            W.node("Add", [f"var{sfx}", "eps"], [f"ve{sfx}"], f"addeps{sfx}"),
            W.node("Sqrt", [f"ve{sfx}"], [f"sd{sfx}"], f"sqrt{sfx}"),
            W.node("Div", [f"d{sfx}", f"sd{sfx}"], [f"n{sfx}"], f"div{sfx}"),
            W.node("Mul", [f"n{sfx}", f"gamma{sfx}"], [f"m{sfx}"], f"mulg{sfx}"),
            W.node("Add", [f"m{sfx}", f"beta{sfx}"], [y], f"addb{sfx}")]


def bert_layer(batch, seq, seed=0):
    rng = np.random.default_rng(seed)
    f32 = np.float32

    def w(*shape, scale=0.02):
        return (rng.standard_normal(shape) * scale).astype(f32)

    weights = {
        "wq": w(H, H), "bq": w(H), "wk": w(H, H), "bk": w(H), "wv": w(H, H), "bv": w(H),
        "wo": w(H, H), "bo": w(H), "w1": w(H, FF), "b1": w(FF), "w2": w(FF, H), "b2": w(H),
        "gamma1": (1 + w(H)).astype(f32), "beta1": w(H), "gamma2": (1 + w(H)).astype(f32), "beta2": w(H),
    }
    consts = {
        "heads_shape": np.array([batch, seq, HEADS, DH], np.int64), "hidden_shape": np.array([batch, seq, H], np.int64),
        "scale": np.array(8.0, f32), "axes": np.array([-1], np.int64), "two": np.array(2.0, f32),
        "eps": np.array(1e-12, f32), "sqrt2": np.array(SQRT2, f32), "one": np.array(1.0, f32),
        "half": np.array(0.5, f32),
    }
    nodes = []
    for t, perm in (("q", [0, 2, 1, 3]), ("k", [0, 2, 3, 1]), ("v", [0, 2, 1, 3])):
        nodes += [W.node("MatMul", ["x", f"w{t}"], [f"{t}0"], f"{t}_proj"),
                  W.node("Add", [f"{t}0", f"b{t}"], [f"{t}1"], f"{t}_bias"),
                  W.node("Reshape", [f"{t}1", "heads_shape"], [f"{t}2"], f"{t}_heads"),
                  W.node("Transpose", [f"{t}2"], [f"{t}h"], f"{t}_perm", perm=perm)]
    nodes += [W.node("MatMul", ["qh", "kh"], ["s0"], "scores"),
              W.node("Div", ["s0", "scale"], ["s1"], "scale"),
              W.node("Add", ["s1", "mask"], ["s2"], "mask_add"),
              W.node("Softmax", ["s2"], ["probs"], "softmax", axis=-1),
              W.node("MatMul", ["probs", "vh"], ["c0"], "context"),
              W.node("Transpose", ["c0"], ["c1"], "c_perm", perm=[0, 2, 1, 3]),
              W.node("Reshape", ["c1", "hidden_shape"], ["c2"], "c_merge"),
              W.node("MatMul", ["c2", "wo"], ["o0"], "o_proj"),
              W.node("Add", ["o0", "bo"], ["o1"], "o_bias"),
              W.node("Add", ["o1", "x"], ["r1"], "residual1")]
    nodes += _ln("r1", "h1", "1")
    nodes += [W.node("MatMul", ["h1", "w1"], ["f0"], "ffn_in"),
              W.node("Add", ["f0", "b1"], ["f1"], "ffn_bias"),
              W.node("Div", ["f1", "sqrt2"], ["g0"], "gelu_div"), W.node("Erf", ["g0"], ["g1"], "gelu_erf"),
              W.node("Add", ["g1", "one"], ["g2"], "gelu_add"), W.node("Mul", ["f1", "g2"], ["g3"], "gelu_mul"),
              W.node("Mul", ["g3", "half"], ["g4"], "gelu_half"),
              W.node("MatMul", ["g4", "w2"], ["f2"], "ffn_out"),
              W.node("Add", ["f2", "b2"], ["f3"], "ffn_out_bias"),
              W.node("Add", ["f3", "h1"], ["r2"], "residual2")]
    nodes += _ln("r2", "y", "2")
    x = rng.standard_normal((batch, seq, H)).astype(f32)
    mask = np.zeros((batch, 1, 1, seq), f32)
    for b in range(batch):  # the padding of each sequence: its last positions masked
        mask[b, 0, 0, seq - (b * 7) % (seq // 4):] = -10000.0
    inits = list(weights.items()) + list(consts.items())
    model = W.model(nodes, [("x", f32, x.shape), ("mask", f32, mask.shape)], [("y", f32, x.shape)], inits)
    return model, {"x": x, "mask": mask}, dict(inits), nodes


def bert_layer_f64(inputs, inits):
    """The same layer in float64 numpy (an independent evaluation, for accuracy bounds)."""
    d = {k: np.asarray(v, np.float64) for k, v in inits.items()}
    x, mask = inputs["x"].astype(np.float64), inputs["mask"].astype(np.float64)
    b, s, _ = x.shape

    def heads(t):
        return t.reshape(b, s, HEADS, DH).transpose(0, 2, 1, 3)

    def ln(t, g, be):
        m = t.mean(-1, keepdims=True)
        v = ((t - m) ** 2).mean(-1, keepdims=True)
        return (t - m) / np.sqrt(v + 1e-12) * g + be

    q, k, v = (heads(x @ d[f"w{t}"] + d[f"b{t}"]) for t in "qkv")
    sc = q @ k.transpose(0, 1, 3, 2) / 8.0 + mask
    sc = np.exp(sc - sc.max(-1, keepdims=True))
    p = sc / sc.sum(-1, keepdims=True)
    c = (p @ v).transpose(0, 2, 1, 3).reshape(b, s, H)
    h1 = ln(c @ d["wo"] + d["bo"] + x, d["gamma1"], d["beta1"])
    f = h1 @ d["w1"] + d["b1"]
    from scipy.special import erf
    g = f * 0.5 * (1.0 + erf(f / math.sqrt(2.0)))
    return ln(g @ d["w2"] + d["b2"] + h1, d["gamma2"], d["beta2"])
