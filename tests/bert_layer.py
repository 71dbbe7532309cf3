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


def encoder_model(batch, seq, layers=12, hidden=384, heads=12, ff=1536, vocab=30522, max_pos=512, seed=0):
    """A whole BERT-class encoder as ONNX (the node sequence a PyTorch export of a BERT model produces, static
    shapes), by default shaped like me5s, the model the reference's benchmarks and model test run
    (multilingual-e5-small: 12 layers, hidden 384, 12 heads of 32, FFN 1536; random weights, a BERT-size
    vocabulary to keep the embedding table small):

      embeddings  Gather word rows by input_ids + Gather position rows + the token-type-0 row, LayerNorm
      mask        Unsqueeze attention_mask [B,S] to [B,1,1,S], Cast to float, (1 - m) * -10000
      layers      each as bert_layer's: Q/K/V projections + heads, scaled masked Softmax attention, output
                  projection + residual, LayerNorm, Erf-GELU FFN + residual, LayerNorm

    Returns (model bytes, inputs, initializers, node list)."""
    rng = np.random.default_rng(seed)
    f32 = np.float32
    dh = hidden // heads

    def w(*shape, scale=0.02):
        return (rng.standard_normal(shape) * scale).astype(f32)

    inits = {
        "word_emb": w(vocab, hidden, scale=0.5), "pos_emb": w(max_pos, hidden, scale=0.5),
        "tt_row": w(hidden, scale=0.5), "position_ids": np.arange(seq, dtype=np.int64).reshape(1, seq),
        "gamma_emb": (1 + w(hidden)).astype(f32), "beta_emb": w(hidden),
        "unsq_axes": np.array([1, 2], np.int64), "neg": np.array(-10000.0, f32),
        "heads_shape": np.array([batch, seq, heads, dh], np.int64),
        "hidden_shape": np.array([batch, seq, hidden], np.int64),
        "scale": np.array(math.sqrt(dh), f32), "axes": np.array([-1], np.int64), "two": np.array(2.0, f32),
        "eps": np.array(1e-12, f32), "sqrt2": np.array(SQRT2, f32), "one": np.array(1.0, f32),
        "half": np.array(0.5, f32),
    }
    nodes = [W.node("Gather", ["word_emb", "input_ids"], ["we"], "emb_word", axis=0),
             W.node("Gather", ["pos_emb", "position_ids"], ["pe"], "emb_pos", axis=0),
             W.node("Add", ["we", "pe"], ["e0"], "emb_add_pos"),
             W.node("Add", ["e0", "tt_row"], ["e1"], "emb_add_tt")]
    nodes += _ln("e1", "h_0", "_emb")
    nodes += [W.node("Unsqueeze", ["attention_mask", "unsq_axes"], ["m0"], "mask_unsqueeze"),
              W.node("Cast", ["m0"], ["m1"], "mask_cast", to=1),
              W.node("Sub", ["one", "m1"], ["m2"], "mask_invert"),
              W.node("Mul", ["m2", "neg"], ["mask"], "mask_scale")]
    for i in range(layers):
        sx = f"_L{i}"
        for k, shape in (("wq", (hidden, hidden)), ("wk", (hidden, hidden)), ("wv", (hidden, hidden)),
                         ("wo", (hidden, hidden)), ("w1", (hidden, ff)), ("w2", (ff, hidden))):
            inits[k + sx] = w(*shape)
        for k, n in (("bq", hidden), ("bk", hidden), ("bv", hidden), ("bo", hidden), ("b1", ff), ("b2", hidden)):
            inits[k + sx] = w(n)
        for k in ("1", "2"):
            inits[f"gamma{k}{sx}"] = (1 + w(hidden)).astype(f32)
            inits[f"beta{k}{sx}"] = w(hidden)
        x, y = f"h_{i}", f"h_{i + 1}"
        for t, perm in (("q", [0, 2, 1, 3]), ("k", [0, 2, 3, 1]), ("v", [0, 2, 1, 3])):
            nodes += [W.node("MatMul", [x, f"w{t}{sx}"], [f"{t}0{sx}"], f"{t}_proj{sx}"),
                      W.node("Add", [f"{t}0{sx}", f"b{t}{sx}"], [f"{t}1{sx}"], f"{t}_bias{sx}"),
                      W.node("Reshape", [f"{t}1{sx}", "heads_shape"], [f"{t}2{sx}"], f"{t}_heads{sx}"),
                      W.node("Transpose", [f"{t}2{sx}"], [f"{t}h{sx}"], f"{t}_perm{sx}", perm=perm)]
        nodes += [W.node("MatMul", [f"qh{sx}", f"kh{sx}"], [f"s0{sx}"], f"scores{sx}"),
                  W.node("Div", [f"s0{sx}", "scale"], [f"s1{sx}"], f"scale{sx}"),
                  W.node("Add", [f"s1{sx}", "mask"], [f"s2{sx}"], f"mask_add{sx}"),
                  W.node("Softmax", [f"s2{sx}"], [f"probs{sx}"], f"softmax{sx}", axis=-1),
                  W.node("MatMul", [f"probs{sx}", f"vh{sx}"], [f"c0{sx}"], f"context{sx}"),
                  W.node("Transpose", [f"c0{sx}"], [f"c1{sx}"], f"c_perm{sx}", perm=[0, 2, 1, 3]),
                  W.node("Reshape", [f"c1{sx}", "hidden_shape"], [f"c2{sx}"], f"c_merge{sx}"),
                  W.node("MatMul", [f"c2{sx}", f"wo{sx}"], [f"o0{sx}"], f"o_proj{sx}"),
                  W.node("Add", [f"o0{sx}", f"bo{sx}"], [f"o1{sx}"], f"o_bias{sx}"),
                  W.node("Add", [f"o1{sx}", x], [f"r1{sx}"], f"residual1{sx}")]
        nodes += _ln(f"r1{sx}", f"a{sx}", f"1{sx}")
        nodes += [W.node("MatMul", [f"a{sx}", f"w1{sx}"], [f"f0{sx}"], f"ffn_in{sx}"),
                  W.node("Add", [f"f0{sx}", f"b1{sx}"], [f"f1{sx}"], f"ffn_bias{sx}"),
                  W.node("Div", [f"f1{sx}", "sqrt2"], [f"g0{sx}"], f"gelu_div{sx}"),
                  W.node("Erf", [f"g0{sx}"], [f"g1{sx}"], f"gelu_erf{sx}"),
                  W.node("Add", [f"g1{sx}", "one"], [f"g2{sx}"], f"gelu_add{sx}"),
                  W.node("Mul", [f"f1{sx}", f"g2{sx}"], [f"g3{sx}"], f"gelu_mul{sx}"),
                  W.node("Mul", [f"g3{sx}", "half"], [f"g4{sx}"], f"gelu_half{sx}"),
                  W.node("MatMul", [f"g4{sx}", f"w2{sx}"], [f"f2{sx}"], f"ffn_out{sx}"),
                  W.node("Add", [f"f2{sx}", f"b2{sx}"], [f"f3{sx}"], f"ffn_out_bias{sx}"),
                  W.node("Add", [f"f3{sx}", f"a{sx}"], [f"r2{sx}"], f"residual2{sx}")]
        nodes += _ln(f"r2{sx}", y, f"2{sx}")
    ids = rng.integers(0, vocab, (batch, seq)).astype(np.int64)
    am = np.ones((batch, seq), np.int64)
    for b in range(batch):  # the padding of each sequence: its last positions
        am[b, seq - (b * 7) % (seq // 4):] = 0
    # the model's output is the last layer's hidden state (last_hidden_state)
    nodes[-1] = W.node("Add", [f"m2_L{layers - 1}", f"beta2_L{layers - 1}"], ["last_hidden_state"], f"addb2_L{layers - 1}")
    model = W.model(nodes, [("input_ids", np.int64, ids.shape), ("attention_mask", np.int64, am.shape)],
                    [("last_hidden_state", f32, (batch, seq, hidden))], list(inits.items()))
    return model, {"input_ids": ids, "attention_mask": am}, inits, nodes


def encoder_model_f64(inputs, inits, layers=12, heads=12):
    """The same encoder in float64 numpy (an independent evaluation, for accuracy bounds)."""
    from scipy.special import erf
    d = {k: np.asarray(v, np.float64) if np.asarray(v).dtype.kind == "f" else np.asarray(v) for k, v in inits.items()}
    ids, am = inputs["input_ids"], inputs["attention_mask"]
    b, s = ids.shape
    hidden = d["word_emb"].shape[1]
    dh = hidden // heads

    def ln(t, g, be):
        m = t.mean(-1, keepdims=True)
        v = ((t - m) ** 2).mean(-1, keepdims=True)
        return (t - m) / np.sqrt(v + 1e-12) * g + be

    def split(t):
        return t.reshape(b, s, heads, dh).transpose(0, 2, 1, 3)

    x = ln(d["word_emb"][ids] + d["pos_emb"][d["position_ids"]] + d["tt_row"], d["gamma_emb"], d["beta_emb"])
    mask = (1.0 - am.astype(np.float64)).reshape(b, 1, 1, s) * -10000.0
    for i in range(layers):
        sx = f"_L{i}"
        q, k, v = (split(x @ d[f"w{t}{sx}"] + d[f"b{t}{sx}"]) for t in "qkv")
        sc = q @ k.transpose(0, 1, 3, 2) / math.sqrt(dh) + mask
        sc = np.exp(sc - sc.max(-1, keepdims=True))
        c = (sc / sc.sum(-1, keepdims=True) @ v).transpose(0, 2, 1, 3).reshape(b, s, hidden)
        a = ln(c @ d[f"wo{sx}"] + d[f"bo{sx}"] + x, d[f"gamma1{sx}"], d[f"beta1{sx}"])
        f = a @ d[f"w1{sx}"] + d[f"b1{sx}"]
        g = f * 0.5 * (1.0 + erf(f / math.sqrt(2.0)))
        x = ln(g @ d[f"w2{sx}"] + d[f"b2{sx}"] + a, d[f"gamma2{sx}"], d[f"beta2{sx}"])
    return x
