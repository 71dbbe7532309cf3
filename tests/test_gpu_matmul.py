"""GPU parity of MatMul (lx_MatMul: fp32 / fp64 MFMA, exact int32) against the
oracle's restatement of Tensor<T>.MatMul (TensorOps.cs:356-705, serial inner
loop of MathOps.mm_unsafe_vectorized).

Bars: Int32 bit-exact (wrapping).  Float / Double: the sums run in another
order than the reference's serial loop, so |gpu - ref| <= 1e-5 * sum_j |a_ij b_jk|
(float) and 1e-13 * sum_j |a_ij b_jk| (double), the reduction bar applied to
each dot product."""
import numpy as np
import pytest

from onnx_amd import DeviceTensor, HipExecutionProvider as HIP, OpStatus
from onnx_amd import _lib as L
from oracle import oracle as O

pytestmark = pytest.mark.gpu


def dev(a):
    return DeviceTensor.from_numpy(np.asarray(a))


def mm(a, b):
    r = HIP.MatMul(dev(a), dev(b))
    assert r.Status == OpStatus.Success, r.Message
    return r.Outputs[0].to_numpy()


def check_float(a, b, tol):
    got = mm(a, b)
    ref = O.matmul(a, b)
    assert got.shape == ref.shape and got.dtype == ref.dtype
    # sum_j |a_ij b_jk| under the reference's shape rules (the oracle's float64 MatMul of |a|, |b|)
    mag = O.matmul(np.abs(a).astype(np.float64), np.abs(b).astype(np.float64))
    err = np.abs(got.astype(np.float64) - ref.astype(np.float64))
    assert np.all(err <= tol * mag + 1e-30), float((err / (mag + 1e-30)).max())


def test_reference_kats(hip):
    """MathTests.cs:82-97 and test_backend.py:949-988 shapes."""
    ones = lambda *s: np.ones(s, np.int32)  # noqa: E731
    for a, b, shape in [((1, 1, 5, 6), (3, 6, 7), (1, 3, 5, 7)), ((2, 3, 5, 6), (3, 6, 7), (2, 3, 5, 7)),
                        ((4, 1, 5, 6), (4, 2, 6, 7), (4, 2, 5, 7))]:
        c = mm(ones(*a), ones(*b))
        assert c.shape == shape and np.all(c == 6)
    a = np.arange(16, dtype=np.int32).reshape(2, 2, 4)
    b = np.arange(16, dtype=np.int32).reshape(2, 4, 2)
    assert mm(a, b)[0, 1, 1] == 98
    f = mm(np.ones((1, 1, 5, 6), np.float32), np.ones((3, 6, 7), np.float32))
    assert f.shape == (1, 3, 5, 7) and np.all(f == 6)


@pytest.mark.parametrize("sa,sb", [((5, 6), (6, 5)), ((3, 4), (4, 3)), ((2, 3, 4), (2, 4, 3)),
                                   ((1, 2, 3, 4), (1, 2, 4, 3)), ((127, 65), (65, 129)), ((129, 33), (33, 130)),
                                   ((64, 7), (7, 9)), ((2, 1, 33, 40), (3, 40, 17)), ((1, 1000), (1000, 1)),
                                   ((300, 300), (300, 300))])
def test_float_shapes(hip, sa, sb):
    rng = np.random.default_rng(50)
    check_float(rng.standard_normal(sa).astype(np.float32), rng.standard_normal(sb).astype(np.float32), 1e-5)


def test_float_bert_sizes(hip):
    rng = np.random.default_rng(51)
    x = rng.standard_normal((8, 512, 768)).astype(np.float32)
    w = (rng.standard_normal((768, 768)) * 0.03).astype(np.float32)
    check_float(x, w, 1e-5)
    q = rng.standard_normal((2, 12, 512, 64)).astype(np.float32)
    k = rng.standard_normal((2, 12, 64, 512)).astype(np.float32)
    check_float(q, k, 1e-5)


@pytest.mark.parametrize("sa,sb", [((4000, 100), (100, 2300)), ((4000, 99), (99, 2300)), ((1536, 72), (72, 4096)),
                                   ((2100, 40), (40, 2300)), ((2, 1100, 40), (40, 1200)), ((4096, 24), (24, 3072))])
def test_float_every_block_tile(hip, sa, sb):
    """Shapes whose tile choice lands on each block tile (128x96, 96x128, 128x64, 64x64, 128x128), with ragged
    edges and, for K = 99, the unvectorised loads."""
    rng = np.random.default_rng(55)
    check_float(rng.standard_normal(sa).astype(np.float32), rng.standard_normal(sb).astype(np.float32), 1e-5)


@pytest.mark.parametrize("sa,sb", [((4096, 768), (768, 768)), ((2000, 192), (192, 2020)), ((4000, 192), (192, 740)),
                                   ((4096, 256), (256, 512)), ((200, 128), (128, 196)), ((3, 1, 130, 128), (1, 2, 128, 132)),
                                   ((64, 128), (128, 68)), ((2, 12, 512, 512), (2, 12, 512, 64)),
                                   ((2, 12, 512, 512), (2, 12, 512, 32)), ((300, 128), (128, 20))])
def test_float_direct_load_tiles(hip, sa, sb):
    """K a multiple of 64 above 64 with aligned operands: the direct-to-LDS kernel, on shapes whose tile choice
    lands on each of its tiles (128x96 one per CU, 128x128 and 128x96 with partial edge tiles, 128x64, 64x64 with
    partial tiles, broadcast batches, the smallest shape it takes, attention context with N = 64 and N = 32 (128x32
    tiles), a ragged N = 20)."""
    rng = np.random.default_rng(56)
    check_float(rng.standard_normal(sa).astype(np.float32), rng.standard_normal(sb).astype(np.float32), 1e-5)


def split_of(m, k, n, batch=1):
    """K ranges of a float product with 16-byte operands (lx_matmul.hip, f32_split): with T 64x64 tiles over
    the batch, the most equal ranges of whole 64-steps dividing K / 64 with T times them within 256; 1 from
    T = 128."""
    if k % 64 or n % 4:
        return 1
    tiles = -(-m // 64) * -(-n // 64) * batch
    if tiles >= 128:
        return 1
    steps, best = k // 64, 1
    for r in range(2, steps + 1):
        if steps % r == 0 and tiles * r <= 256:
            best = r
    return best


@pytest.mark.parametrize("m,k,n", [(256, 128, 8192), (8192, 192, 512), (320, 192, 260), (512, 512, 32),
                                   (2000, 200, 2020)])
def test_float_kernels_sum_in_one_order(hip, m, k, n):
    """The direct-load kernel and the register-staged one add the products of a dot product in the same order,
    so a product is the same bits whichever kernel and tile runs it, given the same K ranges: the whole product
    against its 32-row blocks (fewer than 64 rows: the register-staged kernel) and its 64-column blocks (N = 64:
    another tile), bit for bit, wherever the blocks split K as the whole does -- unsplit at [256,128] x
    [128,8192] (rows) and [8192,192] x [192,512] (columns), three ranges each at [320,192] x [192,260], eight
    at [512,512] x [512,32] (128x32 tiles whole); K = 200, the register-staged kernel's tiles only."""
    rng = np.random.default_rng(58)
    a = rng.standard_normal((m, k)).astype(np.float32)
    b = rng.standard_normal((k, n)).astype(np.float32)
    whole = mm(a, b)
    checked = 0
    if all(split_of(r, k, n) == split_of(m, k, n) for r in (32, m % 32 or 32)):
        rows = np.concatenate([mm(a[i:i + 32], b) for i in range(0, m, 32)])
        assert np.array_equal(whole.view(np.uint32), rows.view(np.uint32))
        checked += 1
    if n >= 128 and split_of(m, k, 64) == split_of(m, k, n):
        cols = np.concatenate([mm(a, np.ascontiguousarray(b[:, j:j + 64])) for j in range(0, n - n % 64, 64)], axis=1)
        assert np.array_equal(whole[:, :cols.shape[1]].view(np.uint32), cols.view(np.uint32))
        checked += 1
    assert checked >= 1


@pytest.mark.parametrize("sa,sb", [((8, 384), (384, 384)), ((8, 1536), (1536, 384)), ((8, 384), (384, 1536)),
                                   ((1, 1536), (1536, 384)), ((63, 512), (512, 100)), ((512, 768), (768, 768)),
                                   ((4, 8, 384), (4, 384, 384)), ((3, 1, 80, 1024), (1, 2, 1024, 36)),
                                   ((200, 4096), (4096, 4))])
def test_float_split_k_sums_its_ranges_in_order(hip, sa, sb):
    """Products with few output tiles split K into equal ranges, one partial product each, then add the partials
    in range order: the split product is, bit for bit, the float32 sum in that order of the unsplit products of
    its ranges (run whole by either kernel: fewer than 64 rows take the register-staged one; a range product
    that would split as a product of its own runs with its rows repeated until it has 128 tiles, which leaves
    each row's bits as they are), and within the MatMul bar of the oracle.  Rows of 8 tokens (the reference's
    short-text embeddings), M = 1, ragged M and N, a batch per operand, broadcast batches, N = 4, ranges that
    would split again."""
    rng = np.random.default_rng(59)
    a = rng.standard_normal(sa).astype(np.float32)
    b = rng.standard_normal(sb).astype(np.float32)
    m, k, n = sa[-2], sa[-1], sb[-1]
    batch = int(np.prod(np.broadcast_shapes(sa[:-2], sb[:-2])))
    r = split_of(m, k, n, batch)
    assert r > 1

    def unsplit(a, b):
        rep = 1
        while split_of(m * rep, a.shape[-1], n, batch) > 1:
            rep *= 2
        return mm(np.ascontiguousarray(np.concatenate([a] * rep, axis=-2)), b)[..., :m, :]

    kr, ref = k // r, None
    for i in range(r):
        part = unsplit(a[..., i * kr:(i + 1) * kr], np.ascontiguousarray(b[..., i * kr:(i + 1) * kr, :]))
        ref = part if ref is None else (ref + part).astype(np.float32)
    whole = mm(a, b)
    assert whole.shape == ref.shape and np.array_equal(whole.view(np.uint32), ref.view(np.uint32))
    check_float(a, b, 1e-5)


@pytest.mark.parametrize("batch", [524280, 524288])
def test_batch_fold_at_the_grid_limit(hip, batch):
    """A batch of left matrices over one right matrix runs as one product of batch * m rows while its 64-row
    tiles fit the grid (524280 x 8 rows: exactly 65535 tiles); one more row tile's worth keeps the batch
    (524288 matrices, in launches of 65535).  Integer values: every sum exact."""
    rng = np.random.default_rng(92)
    a = rng.integers(-8, 8, (batch, 8, 4)).astype(np.float32)
    b = rng.integers(-8, 8, (4, 4)).astype(np.float32)
    got = mm(a, b)
    assert got.shape == (batch, 8, 4) and np.array_equal(got, a @ b)


@pytest.mark.parametrize("sa,sb", [((5, 6), (6, 5)), ((3, 70, 33), (33, 65)), ((2, 1, 40, 17), (3, 17, 66)),
                                   ((300, 130), (130, 260)), ((1000, 512), (512, 700)), ((4096, 256), (256, 1030)),
                                   ((2, 1, 700, 96), (3, 96, 900)), ((257, 33), (33, 129)), ((2048, 33), (33, 2049)),
                                   ((1024, 64), (64, 1030))])
def test_double(hip, sa, sb):
    """Double: 128x128, 64x64 and 32x32 tiles (the largest that gives 256 of them), 16-byte and scalar loads (odd K
    or N), ragged edges, broadcast batches."""
    rng = np.random.default_rng(52)
    check_float(rng.standard_normal(sa), rng.standard_normal(sb), 1e-13)


@pytest.mark.parametrize("sa,sb", [((5, 9), (9, 4)), ((3, 70, 33), (33, 65)), ((2, 1, 17, 40), (3, 40, 17))])
def test_int32_wraps(hip, sa, sb):
    rng = np.random.default_rng(53)
    a = rng.integers(-2**31, 2**31, sa, dtype=np.int64).astype(np.int32)
    b = rng.integers(-2**31, 2**31, sb, dtype=np.int64).astype(np.int32)
    got = mm(a, b)
    assert np.array_equal(got, O.matmul(a, b))


def test_rank1_and_broadcast_rules(hip):
    v = np.arange(5, dtype=np.float32)
    c = mm(v, v)
    assert c.shape == (1,) and c[0] == 30.0
    rng = np.random.default_rng(54)
    m = rng.standard_normal((4, 4)).astype(np.float32)
    w = rng.standard_normal(4).astype(np.float32)
    check_float(m, w, 1e-5)   # w broadcast element-wise to [4,4] first, as the reference does
    check_float(w, m, 1e-5)


def test_errors(hip):
    r = HIP.MatMul(dev(np.ones((2, 3), np.float32)), dev(np.ones((4, 2), np.float32)))
    assert r.Code == L.ERR_INVALID_ARGUMENT
    assert r.Message == ("The number of columns in the first matrix (3) is not equal to the number of rows in the "
                         "second matrix (4).")
    r = HIP.MatMul(dev(np.ones((3, 4), np.float32)), dev(np.ones(4, np.float32)))
    assert r.Code == L.ERR_INVALID_ARGUMENT   # [3,4] x [3,4] after the element-wise broadcast
    r = HIP.MatMul(dev(np.ones((2, 2), np.float32)), dev(np.ones((2, 2), np.int32)))
    assert r.Code == L.ERR_WRONG_INPUT_TYPE
    assert r.Message == ("Unable to cast object of type 'Lokad.Onnx.DenseTensor`1[System.Int32]' to type "
                         "'Lokad.Onnx.Tensor`1[System.Single]'.")
    r = HIP.MatMul(dev(np.ones((2, 2), np.int64)), dev(np.ones((2, 2), np.int64)))
    assert r.Code == L.ERR_INPUT_TYPE_NOT_SUPPORTED
    r = HIP.MatMul(dev(np.array(1.0, np.float32)), dev(np.ones((2, 2), np.float32)))
    assert r.Message == "The rank of each tensor in matrix multiplication must be greater than 1."
    r = HIP.MatMul(dev(np.ones((2, 3, 4), np.float32)), dev(np.ones((5, 4, 2), np.float32)))
    assert r.Message == "The tensor shapes are not compatible for broadcasting."


# ---- MatMul -> Add bias [-> Add residual] with the Adds in the epilogue (lx_MatMulAdd) -------------------
def _nodes(a, b, bias, res):
    t = HIP.MatMul(dev(a), dev(b)).Outputs[0]
    t = HIP.Add(t, dev(bias)).Outputs[0]
    if res is not None:
        t = HIP.Add(t, dev(res)).Outputs[0]
    return t.to_numpy()


@pytest.mark.parametrize("sa,sb,sbias,sres", [
    ((256, 768), (768, 768), (768,), None), ((4, 64, 768), (768, 256), (256,), (4, 64, 256)),
    ((4000, 192), (192, 740), (740,), (4000, 740)), ((2000, 192), (192, 2020), (2020,), None),
    ((2, 3, 33, 40), (40, 70), (1, 70), (2, 3, 33, 70)), ((128, 64), (64, 96), (96,), (128, 96)),
    # split K (few output tiles): the epilogue after the ordered sum of the partials
    ((8, 384), (384, 384), (384,), (8, 384)), ((1, 8, 1536), (1536, 384), (384,), (1, 8, 384)),
    ((1, 96, 512), (3, 512, 80), (3, 1, 80), None),
    # shapes the epilogue does not take: the MatMul and the Adds one after the other
    ((64, 32), (32, 48), (64, 48), None), ((64, 32), (32, 48), (48,), (48,)), ((5, 32), (32, 48), (3, 1, 48), None)])
@pytest.mark.parametrize("dt", [np.float32, np.float64])
def test_matmul_add_equals_the_nodes(hip, sa, sb, sbias, sres, dt):
    rng = np.random.default_rng(57)
    a, b = rng.standard_normal(sa).astype(dt), rng.standard_normal(sb).astype(dt)
    bias = rng.standard_normal(sbias).astype(dt)
    res = None if sres is None else rng.standard_normal(sres).astype(dt)
    r = HIP.MatMulAdd(dev(a), dev(b), dev(bias), None if res is None else dev(res))
    assert r.Status == OpStatus.Success, r.Message
    got, ref = r.Outputs[0].to_numpy(), _nodes(a, b, bias, res)
    assert got.shape == ref.shape and np.array_equal(got.view(np.uint8), ref.view(np.uint8))


def test_matmul_add_into_caller_storage(hip):
    rng = np.random.default_rng(58)
    a, b = rng.standard_normal((96, 64)).astype(np.float32), rng.standard_normal((64, 80)).astype(np.float32)
    bias, res = rng.standard_normal(80).astype(np.float32), rng.standard_normal((96, 80)).astype(np.float32)
    out = DeviceTensor.empty((96, 80), np.float32)
    r = HIP.MatMulAdd(dev(a), dev(b), dev(bias), dev(res), out=out)
    assert r.Status == OpStatus.Success, r.Message
    assert np.array_equal(out.to_numpy().view(np.uint32), _nodes(a, b, bias, res).view(np.uint32))
    r = HIP.MatMulAdd(dev(a), dev(b), dev(np.ones(81, np.float32)))
    assert r.Code == L.ERR_CANNOT_BROADCAST


def test_matmul_add_bias_row_per_batch_equals_the_nodes(hip):
    """A bias of one row per batch ([G, 1, N] against a product [G, M, N]) in the epilogue: the MatMul, then
    the broadcast Add, bit for bit; a bias that matches neither form runs the Add node."""
    rng = np.random.default_rng(90)
    a = rng.standard_normal((1, 96, 64)).astype(np.float32)
    w = rng.standard_normal((3, 64, 80)).astype(np.float32)
    for bshape in [(3, 1, 80), (1, 80), (80,), (3, 96, 80)]:
        b = rng.standard_normal(bshape).astype(np.float32)
        r = HIP.MatMulAdd(dev(a), dev(w), dev(b))
        assert r.Status == OpStatus.Success, r.Message
        got = r.Outputs[0].to_numpy()
        ref = HIP.Add(HIP.MatMul(dev(a), dev(w)).Outputs[0], dev(b)).Outputs[0].to_numpy()
        assert got.shape == ref.shape and np.array_equal(got.view(np.uint32), ref.view(np.uint32)), bshape


@pytest.mark.parametrize("xs,n,g", [((2, 40, 96), 64, 3), ((1, 8, 384), 384, 3), ((1, 8, 1536), 1536, 3),
                                    ((1, 8, 384), 64, 17)])
def test_grouped_projections_equal_the_separate_ones(hip, xs, n, g):
    """g MatMul -> Add bias projections of one input become one MatMulAddGroup node (one batched launch,
    outputs as slices of one product); every output equals the unfused graph's bit for bit, including
    through a consumer that reads a slice (Reshape / Transpose of the second one).  Eight tokens split K in
    the grouped launch as in each separate product: six ranges at hidden 384, eight at 1536 (where the
    group's three matrices together would take three); a group of 17 runs its products one by one."""
    import onnx_writer as W
    from onnx_amd.graph import Model
    rng = np.random.default_rng(91)
    x = rng.standard_normal(xs).astype(np.float32)
    inits = []
    nodes = []
    names = [f"p{i}" for i in range(g)]
    for t in names:
        inits += [(f"w{t}", (rng.standard_normal((xs[-1], n)) * 0.1).astype(np.float32)),
                  (f"b{t}", rng.standard_normal(n).astype(np.float32))]
        nodes += [W.node("MatMul", ["x", f"w{t}"], [f"{t}_mm"], f"{t}_proj"),
                  W.node("Add", [f"{t}_mm", f"b{t}"], [f"{t}"], f"{t}_bias")]
    inits.append(("shape", np.array([xs[0], xs[1], 4, n // 4], np.int64)))
    nodes += [W.node("Reshape", ["p1", "shape"], ["kr"], "k_heads"),
              W.node("Transpose", ["kr"], ["kt"], "k_perm", perm=[0, 2, 3, 1])]
    outs = [names[0], "kt"] + names[2:]
    res = {}
    for fuse in (False, True):
        g = Model.Load(W.model(nodes, [("x", np.float32, x.shape)], [(o, np.float32, ()) for o in outs], inits))
        if fuse:
            assert g.Fuse() == 1 and [n.Op for n in g.Nodes][0] == "MatMulAddGroup"
        assert g.Execute({"x": dev(x)}), g.LastError
        res[fuse] = [g.Output(o).to_numpy() for o in outs]
    for u, f in zip(res[False], res[True]):
        assert u.shape == f.shape and np.array_equal(u.view(np.uint32), f.view(np.uint32))


@pytest.mark.parametrize("b,s,h,d", [(1, 8, 12, 32), (2, 64, 12, 32), (1, 512, 12, 32), (2, 10, 3, 6),
                                     (1, 8, 12, 128)])
@pytest.mark.parametrize("q_read_twice", [False, True])
def test_attention_transposes_fold_into_the_products(hip, b, s, h, d, q_read_twice):
    """Transpose (perm [0,2,1,3]) -> MatMul and MatMul -> Transpose (the attention heads' Q, V and context)
    fold into MatMulPermuted nodes that read and write the transposed views through their strides, and so
    does K's Transpose ([0,2,3,1]), read by columns; Q's stays a node when its output is also a graph output.
    Every output bit for bit the unfused graph's, executed and captured: 8 tokens, 64, 512 (the context
    product splits K), heads of 6 (no 16-byte accesses), heads of 128 at 8 tokens (the scores would split K,
    which a B read by columns does not: that node runs its Transpose and MatMul)."""
    import onnx_writer as W
    from onnx_amd.graph import Model
    rng = np.random.default_rng(93)
    ins = {t: rng.standard_normal((b, s, h, d)).astype(np.float32) for t in "qkv"}
    nodes = [W.node("Transpose", ["q"], ["qt"], "q_perm", perm=[0, 2, 1, 3]),
             W.node("Transpose", ["k"], ["kt"], "k_perm", perm=[0, 2, 3, 1]),
             W.node("Transpose", ["v"], ["vt"], "v_perm", perm=[0, 2, 1, 3]),
             W.node("MatMul", ["qt", "kt"], ["sc"], "scores"),
             W.node("Softmax", ["sc"], ["p"], "softmax", axis=-1),
             W.node("MatMul", ["p", "vt"], ["ctx"], "context"),
             W.node("Transpose", ["ctx"], ["y"], "ctx_perm", perm=[0, 2, 1, 3])]
    outs = ["y", "sc"] + (["qt"] if q_read_twice else [])
    dev = {t: DeviceTensor.from_numpy(v) for t, v in ins.items()}
    res = {}
    for mode in ("nodes", "fused", "captured"):
        g = Model.Load(W.model(nodes, [(t, np.float32, ins[t].shape) for t in "qkv"],
                               [(o, np.float32, ()) for o in outs], []))
        if mode != "nodes":
            assert g.Fuse() == 2
            assert [n.Op for n in g.Nodes] == (["Transpose"] if q_read_twice else []) + [
                "MatMulPermuted", "Softmax", "MatMulPermuted"]
        if mode == "captured":
            assert g.Capture(dev), g.LastError
            assert g.Replay(), g.LastError
        else:
            assert g.Execute(dev), g.LastError
        res[mode] = [g.Output(o).to_numpy() for o in outs]
    for mode in ("fused", "captured"):
        for u, f in zip(res["nodes"], res[mode]):
            assert u.shape == f.shape and np.array_equal(u.view(np.uint32), f.view(np.uint32)), mode
    ref = np.swapaxes(np.swapaxes(ins["q"], 1, 2) @ np.swapaxes(ins["k"], 1, 2).swapaxes(2, 3), 1, 1)
    assert np.allclose(res["fused"][1], ref, rtol=1e-4, atol=1e-4)


def _two_unnamed_projection_layers(rng):
    """Two layers of three MatMul -> Add bias projections each, every node unnamed (ONNX allows it); the
    second layer reads the first one's V and has weights of its own."""
    import onnx_writer as W
    inits, nodes = [], []
    for layer, src in ((0, "x"), (1, "v0")):
        for t in "qkv":
            inits += [(f"w{t}{layer}", (rng.standard_normal((64, 64)) * 0.1).astype(np.float32)),
                      (f"b{t}{layer}", rng.standard_normal(64).astype(np.float32))]
            nodes += [W.node("MatMul", [src, f"w{t}{layer}"], [f"{t}{layer}p"]),
                      W.node("Add", [f"{t}{layer}p", f"b{t}{layer}"], [f"{t}{layer}"])]
    return nodes, inits


def test_grouped_projections_of_unnamed_layers_keep_their_own_weights(hip):
    """Each group of unnamed projections stacks its own weights: the fused graph equals the unfused one bit
    for bit in both layers (a name derived from the node's name would let the second group read the
    first group's stacked weights)."""
    import onnx_writer as W
    from onnx_amd.graph import Model
    rng = np.random.default_rng(92)
    x = rng.standard_normal((2, 40, 64)).astype(np.float32)
    nodes, inits = _two_unnamed_projection_layers(rng)
    outs = ["q0", "k0", "v0", "q1", "k1", "v1"]
    res = {}
    for fuse in (False, True):
        g = Model.Load(W.model(nodes, [("x", np.float32, x.shape)], [(o, np.float32, ()) for o in outs], inits))
        if fuse:
            assert g.Fuse() == 2 and [n.Op for n in g.Nodes] == ["MatMulAddGroup", "MatMulAddGroup"]
        assert g.Execute({"x": dev(x)}), g.LastError
        res[fuse] = [g.Output(o).to_numpy() for o in outs]
        g.close()
    for o, u, f in zip(outs, res[False], res[True]):
        assert u.shape == f.shape and np.array_equal(u.view(np.uint32), f.view(np.uint32)), o


def test_grouped_projection_slice_capacity_is_its_own(hip):
    """An output slice of a grouped projection reports its own bytes as capacity, so reusing it as output
    storage cannot write past the slice."""
    import onnx_writer as W
    from onnx_amd.graph import Model
    rng = np.random.default_rng(93)
    x = rng.standard_normal((2, 40, 64)).astype(np.float32)
    nodes, inits = _two_unnamed_projection_layers(rng)
    g = Model.Load(W.model(nodes[:6], [("x", np.float32, x.shape)], [(o, np.float32, ()) for o in ("q0", "k0", "v0")],
                           inits[:6]))
    assert g.Fuse() == 1
    assert g.Execute({"x": dev(x)}), g.LastError
    for o in ("q0", "k0", "v0"):
        assert g.Output(o).h.capacity == 2 * 40 * 64 * 4, o
    g.close()


def _gelu_nodes(t):
    """The ONNX GELU subgraph's five separate device operators on t (the reference's node-by-node path)."""
    c = lambda v: dev(np.array(v, t.dtype))  # noqa: E731
    d = HIP.Div(dev(t), c(1.4142135623730951 if t.dtype == np.float64 else np.float32(1.4142135))).Outputs[0]
    e = HIP.Erf(d).Outputs[0]
    a = HIP.Add(e, c(1.0)).Outputs[0]
    m = HIP.Mul(dev(t), a).Outputs[0]
    return HIP.Mul(m, c(0.5)).Outputs[0].to_numpy()


@pytest.mark.parametrize("sa,sb,sbias", [((256, 768), (768, 3072), (3072,)), ((2, 64, 768), (768, 256), (256,)),
                                         ((2000, 192), (192, 2020), (2020,)), ((4096, 768), (768, 768), (768,)),
                                         ((4096, 768), (768, 2304), (2304,)), ((2048, 256), (256, 4096), (4096,)),
                                         ((98304, 128), (128, 64), (64,)),
                                         ((8, 384), (384, 1536), (1536,)), ((10, 8, 384), (384, 1536), (1536,)),
                                         ((127, 65), (65, 129), (129,)), ((3, 33, 40), (3, 40, 70), (3, 1, 70)),
                                         ((64, 32), (32, 48), (64, 48))])
@pytest.mark.parametrize("dt", [np.float32, np.float64])
def test_matmul_add_gelu_equals_the_nodes(hip, sa, sb, sbias, dt):
    """MatMul -> Add bias -> GELU (Div sqrt2, Erf, Add 1, Mul x, Mul 0.5) as one launch with the Add and the
    GELU in the MatMul's epilogue, bit for bit the seven separate operators: a BERT FFN shape, a batch, ragged
    tiles, a bias row per batch; shapes that put several blocks of each direct-load tile on a CU at once (64x64
    at [4096,768]x[768,2304], 128x128 two per CU, 128x64 three per CU); a bias that is no row vector, and
    Double, run the nodes."""
    rng = np.random.default_rng(61)
    a = rng.standard_normal(sa).astype(dt)
    b = (rng.standard_normal(sb) * 0.1).astype(dt)
    bias = rng.standard_normal(sbias).astype(dt)
    r = HIP.MatMulAddGelu(dev(a), dev(b), dev(bias))
    assert r.Status == OpStatus.Success, r.Message
    got = r.Outputs[0].to_numpy()
    pre = HIP.Add(HIP.MatMul(dev(a), dev(b)).Outputs[0], dev(bias)).Outputs[0].to_numpy()
    ref = _gelu_nodes(pre)
    assert got.shape == ref.shape and got.dtype == ref.dtype
    assert np.array_equal(got.view(np.uint8), ref.view(np.uint8))


def test_matmul_add_gelu_special_values_and_caller_storage(hip):
    """Pre-activations that saturate the GELU (|x| up to 1e5, where erf rounds to +-1), zeros, and NaN / inf
    products, into caller storage: bit for bit the separate operators."""
    rng = np.random.default_rng(62)
    a = (rng.standard_normal((96, 64)) * np.logspace(-3, 3, 64)).astype(np.float32)
    a[0, 0], a[1, :], a[2, 5] = np.nan, 0.0, np.inf
    b = rng.standard_normal((64, 80)).astype(np.float32)
    bias = rng.standard_normal(80).astype(np.float32)
    out = DeviceTensor.empty((96, 80), np.float32)
    r = HIP.MatMulAddGelu(dev(a), dev(b), dev(bias), out=out)
    assert r.Status == OpStatus.Success, r.Message
    pre = HIP.Add(HIP.MatMul(dev(a), dev(b)).Outputs[0], dev(bias)).Outputs[0].to_numpy()
    assert np.array_equal(out.to_numpy().view(np.uint32), _gelu_nodes(pre).view(np.uint32))


def test_ffn_gelu_graph_fuses_into_one_node(hip):
    """MatMul -> Add bias -> the GELU nodes in a graph become one MatMulAddGelu node whose output equals the
    unfused graph's bit for bit; with the biased product also a graph output the GELU stays a node of its own."""
    import onnx_writer as W
    from onnx_amd.graph import Model
    rng = np.random.default_rng(94)
    x = rng.standard_normal((2, 40, 96)).astype(np.float32)
    inits = [("w", (rng.standard_normal((96, 128)) * 0.1).astype(np.float32)),
             ("b", rng.standard_normal(128).astype(np.float32)), ("sqrt2", np.array(1.4142135, np.float32)),
             ("one", np.array(1.0, np.float32)), ("half", np.array(0.5, np.float32))]
    nodes = [W.node("MatMul", ["x", "w"], ["f0"], "ffn_in"), W.node("Add", ["f0", "b"], ["f1"], "ffn_bias"),
             W.node("Div", ["f1", "sqrt2"], ["g0"], "gelu_div"), W.node("Erf", ["g0"], ["g1"], "gelu_erf"),
             W.node("Add", ["g1", "one"], ["g2"], "gelu_add"), W.node("Mul", ["f1", "g2"], ["g3"], "gelu_mul"),
             W.node("Mul", ["g3", "half"], ["y"], "gelu_half")]
    res = {}
    for fuse, outs in ((False, ["y"]), (True, ["y"]), ("escape", ["y", "f1"])):
        g = Model.Load(W.model(nodes, [("x", np.float32, x.shape)], [(o, np.float32, ()) for o in outs], inits))
        if fuse is True:
            assert g.Fuse() == 1 and [n.Op for n in g.Nodes] == ["MatMulAddGelu"]
        elif fuse == "escape":
            assert g.Fuse() == 2 and [n.Op for n in g.Nodes] == ["MatMulAdd", "GeluErf"]
        assert g.Execute({"x": dev(x)}), g.LastError
        res[fuse] = g.Output("y").to_numpy()
        g.close()
    for k in (True, "escape"):
        assert np.array_equal(res[False].view(np.uint32), res[k].view(np.uint32)), k


def test_transposed_views_random(hip):
    """Random Transpose -> MatMul <- Transpose -> Transpose graphs of rank 3 and 4: each Transpose whose perm
    keeps the last axis last folds into the MatMul (read or written through strides), and so does the right
    operand's when it makes its last axis K (read by columns), the others stay nodes; the fused graph equals
    the unfused one bit for bit, executed and captured, and numpy's product within the MatMul bar."""
    import onnx_writer as W
    from onnx_amd.graph import Model
    rng = np.random.default_rng(94)

    def perm(r):
        if rng.random() < 0.6:  # keeps the last axis last
            return [int(v) for v in rng.permutation(r - 1)] + [r - 1]
        return [int(v) for v in rng.permutation(r)]

    folded = 0
    for case in range(24):
        r = int(rng.choice([3, 4]))
        batch = tuple(int(d) for d in rng.integers(1, 4, r - 2))
        m, k, n = (int(rng.choice(v)) for v in ([1, 8, 33, 64, 100], [16, 64, 128, 384], [4, 32, 36, 64, 128]))
        A = rng.standard_normal(batch + (m, k)).astype(np.float32)
        B = rng.standard_normal(batch + (k, n)).astype(np.float32)
        pa, pb, pc = perm(r), perm(r), perm(r)
        A0 = np.ascontiguousarray(np.transpose(A, np.argsort(pa)))
        B0 = np.ascontiguousarray(np.transpose(B, np.argsort(pb)))
        nodes = [W.node("Transpose", ["a0"], ["a"], "ta", perm=pa), W.node("Transpose", ["b0"], ["b"], "tb", perm=pb),
                 W.node("MatMul", ["a", "b"], ["c"], "mm"), W.node("Transpose", ["c"], ["y"], "tc", perm=pc)]
        dev_in = {"a0": DeviceTensor.from_numpy(A0), "b0": DeviceTensor.from_numpy(B0)}
        res = {}
        for mode in ("nodes", "fused", "captured"):
            g = Model.Load(W.model(nodes, [("a0", np.float32, A0.shape), ("b0", np.float32, B0.shape)],
                                   [("y", np.float32, ())], []))
            if mode != "nodes":
                nf = g.Fuse()
                folded += nf
                folds = pa[-1] == r - 1 or pb[-1] == r - 1 or pb[-2] == r - 1 or pc[-1] == r - 1
                assert nf == (1 if folds else 0), (case, pa, pb, pc)
            ok = g.Capture(dev_in) and g.Replay() if mode == "captured" else g.Execute(dev_in)
            assert ok, (case, g.LastError)
            res[mode] = g.Output("y").to_numpy()
        for mode in ("fused", "captured"):
            assert np.array_equal(res["nodes"].view(np.uint32), res[mode].view(np.uint32)), (case, mode, pa, pb, pc)
        ref = np.transpose(A.astype(np.float64) @ B.astype(np.float64), pc)
        mag = np.transpose(np.abs(A).astype(np.float64) @ np.abs(B).astype(np.float64), pc)
        assert np.all(np.abs(res["nodes"] - ref) <= 1e-5 * mag + 1e-30), case
    assert folded > 0


@pytest.mark.parametrize("xs,k,n,residual", [((1, 8, 384), 384, 384, True), ((1, 8, 1536), 1536, 384, True),
                                             ((2, 40, 384), 1536, 768, False), ((1, 8, 384), 384, 4096, True),
                                             ((8, 512, 384), 384, 384, True), ((1, 8, 384), 384, 200, True)])
def test_matmul_add_layernorm_equals_the_two_fused_nodes(hip, xs, k, n, residual):
    """MatMul -> Add bias [-> Add residual] -> the decomposed LayerNorm's nine nodes fuse to one
    MatMulAddLayerNorm node; it equals lx_MatMulAdd followed by lx_LayerNormDecomposed bit for bit, executed
    and captured.  Products that split K (8 tokens, hidden 384 and 1536, rows up to 4096) normalise in the
    ordered sum of the partials; [8,512] tokens (no split) and rows of 200 (another LayerNorm kernel) run the
    two kernels."""
    import onnx_writer as W
    from onnx_amd.graph import Model
    from bert_layer import _ln
    rng = np.random.default_rng(95)
    x = rng.standard_normal(xs[:-1] + (k,)).astype(np.float32)
    w = (rng.standard_normal((k, n)) * 0.05).astype(np.float32)
    b = rng.standard_normal(n).astype(np.float32)
    r = rng.standard_normal(xs[:-1] + (n,)).astype(np.float32)
    gamma = (1 + 0.1 * rng.standard_normal(n)).astype(np.float32)
    beta = (0.1 * rng.standard_normal(n)).astype(np.float32)
    inits = [("w", w), ("b", b), ("gamma1", gamma), ("beta1", beta), ("axes", np.array([-1], np.int64)),
             ("two", np.array(2.0, np.float32)), ("eps", np.array(1e-12, np.float32))]
    nodes = [W.node("MatMul", ["x", "w"], ["p"], "proj"), W.node("Add", ["p", "b"], ["h0"], "bias")]
    h = "h0"
    if residual:
        nodes.append(W.node("Add", ["h0", "r"], ["h1"], "residual"))
        h = "h1"
    nodes += _ln(h, "y", "1")
    ins = [("x", np.float32, x.shape)] + ([("r", np.float32, r.shape)] if residual else [])
    dev_in = {"x": dev(x), "r": dev(r)} if residual else {"x": dev(x)}
    pre = HIP.MatMulAdd(dev(x), dev(w), dev(b), dev(r) if residual else None)
    assert pre.Status == OpStatus.Success, pre.Message
    ln = HIP.LayerNormDecomposed(pre.Outputs[0], dev(gamma), dev(beta), 1e-12)
    assert ln.Status == OpStatus.Success, ln.Message
    ref = ln.Outputs[0].to_numpy()
    for mode in ("fused", "captured"):
        g = Model.Load(W.model(nodes, ins, [("y", np.float32, ())], inits))
        assert g.Fuse() == 1 and [nd.Op for nd in g.Nodes] == ["MatMulAddLayerNorm"]
        ok = (g.Capture(dev_in) and g.Replay()) if mode == "captured" else g.Execute(dev_in)
        assert ok, g.LastError
        got = g.Output("y").to_numpy()
        assert got.shape == ref.shape and np.array_equal(got.view(np.uint32), ref.view(np.uint32)), mode
