"""A whole BERT-base encoder layer through the device graph runtime: every
operator family of the device path at once (elementwise / broadcast /
reductions / Softmax, MatMul, data movement, the graph executor with and
without fusion, capture).

Bar: the layer composes ~60 float32 operators whose summation orders differ from
the reference's serial loops, so it is judged against an independent float64
evaluation: the device's largest error is at most 4x the largest error of the
reference's own float32 node-by-node evaluation (the oracle) plus 1e-6."""
import numpy as np
import pytest

from onnx_amd import DeviceTensor
from onnx_amd.graph import Model
from oracle import graph_oracle as GO

from bert_layer import bert_layer, bert_layer_f64, encoder_model, encoder_model_f64
from test_gpu_graph import _dict_nodes

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def layer():
    model, ins, inits, nodes = bert_layer(2, 64, 11)
    ref = GO.run(_dict_nodes(nodes), ins, inits)["y"]
    t64 = bert_layer_f64(ins, inits)
    return model, ins, ref, t64


@pytest.mark.parametrize("mode", ["nodes", "fused", "captured"])
def test_bert_layer_accuracy(hip, layer, mode):
    model, ins, ref, t64 = layer
    g = Model.Load(model)
    if mode != "nodes":
        assert g.Fuse() == 5
    dev = {k: DeviceTensor.from_numpy(v) for k, v in ins.items()}
    ok = g.Capture(dev) if mode == "captured" else g.Execute(dev)
    assert ok, g.LastError
    y = g.Output("y").to_numpy()
    assert y.shape == ref.shape and np.isfinite(y).all()
    err_ref = np.abs(ref.astype(np.float64) - t64).max()
    err_dev = np.abs(y.astype(np.float64) - t64).max()
    print(f"BERT layer {mode}: device max error {err_dev:.3g}, reference float32 max error {err_ref:.3g}")
    assert err_dev <= 4 * err_ref + 1e-6, (err_dev, err_ref)
    if mode == "captured":   # a replay on new inputs written into the captured buffers
        x2 = (ins["x"] * 0.5).astype(np.float32)
        dev["x"].upload(x2)
        assert g.Replay(), g.LastError
        t64b = bert_layer_f64({"x": x2, "mask": ins["mask"]}, _inits(layer))
        assert np.abs(g.Output("y").to_numpy().astype(np.float64) - t64b).max() <= 4 * err_ref + 1e-6


def _inits(layer):
    # the initializers of the fixture's model (same seed)
    _, _, inits, _ = bert_layer(2, 64, 11)
    return inits


@pytest.fixture(scope="module")
def encoder():
    model, ins, inits, nodes = encoder_model(2, 64, layers=3, vocab=2000, seed=12)
    ref = GO.run(_dict_nodes(nodes), ins, inits)["last_hidden_state"]
    t64 = encoder_model_f64(ins, inits, layers=3)
    return model, ins, ref, t64


@pytest.mark.parametrize("mode", ["nodes", "fused", "captured"])
def test_me5s_shaped_encoder_accuracy(hip, encoder, mode):
    """A whole me5s-shaped encoder (embeddings by Gather, the attention mask's Unsqueeze / Cast / scale, three
    encoder layers of hidden 384, 12 heads of 32, FFN 1536) from int64 token ids and attention mask to the last
    hidden state, node by node, fused and captured: within 4x the reference's own float32 error against float64."""
    model, ins, ref, t64 = encoder
    g = Model.Load(model)
    if mode != "nodes":
        assert g.Fuse() == 3 * 5 + 3
    dev = {k: DeviceTensor.from_numpy(v) for k, v in ins.items()}
    ok = g.Capture(dev) if mode == "captured" else g.Execute(dev)
    assert ok, g.LastError
    y = g.Output("last_hidden_state").to_numpy()
    assert y.shape == ref.shape and np.isfinite(y).all()
    err_ref = np.abs(ref.astype(np.float64) - t64).max()
    err_dev = np.abs(y.astype(np.float64) - t64).max()
    print(f"encoder {mode}: device max error {err_dev:.3g}, reference float32 max error {err_ref:.3g}")
    assert err_dev <= 4 * err_ref + 1e-6, (err_dev, err_ref)
    if mode == "captured":   # a replay on other token ids written into the captured input buffer
        ids2 = (ins["input_ids"] * 7 + 3) % 2000
        dev["input_ids"].upload(ids2)
        assert g.Replay(), g.LastError
        _, _, inits, _ = encoder_model(2, 64, layers=3, vocab=2000, seed=12)
        t64b = encoder_model_f64({"input_ids": ids2, "attention_mask": ins["attention_mask"]}, inits, layers=3)
        assert np.abs(g.Output("last_hidden_state").to_numpy().astype(np.float64) - t64b).max() <= 4 * err_ref + 1e-6
