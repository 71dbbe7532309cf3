"""Parity at the reference's largest tensor.  A DenseTensor's storage is one .NET array, `new T[Length]`
(DenseTensor.cs:96-100), and a .NET array holds at most Array.MaxLength = 2,147,483,591 elements, so no
reference tensor is larger.  Every kernel family runs here on a tensor of about that many elements (8.6 GB in
float32, 17 GB in int64): every element index, byte offset and grid of the device path at that size.

Inputs are drawn on the device (torch as allocator and random source: plumbing).  Checks:
* bits fixed by IEEE or two's-complement arithmetic (Add, Sqrt, Cast, integer Div, data movement) against the
  same operation in torch, over every element;
* sums within the reduction bar (1e-5 * sum|x| of each slice) of float64 sums;
* the oracle on sampled elements and rows (the first and last 4096 elements always among them) for every op,
  including GELU, Softmax, AddSoftmax and LayerNorm, with the bars of the smaller-size tests."""
import gc

import numpy as np
import pytest

import onnx_amd
from onnx_amd import DeviceTensor, HipExecutionProvider as HIP, OpStatus
from oracle import oracle as O

pytestmark = pytest.mark.gpu

torch = pytest.importorskip("torch")

N_MAX = 2_147_483_591  # System.Array.MaxLength


@pytest.fixture(autouse=True)
def _release():
    yield
    gc.collect()
    torch.cuda.synchronize()
    torch.cuda.empty_cache()
    onnx_amd._lib.lib().lx_pool_trim()


def gen(seed):
    return torch.Generator(device="cuda").manual_seed(seed)


def w(t):
    return DeviceTensor.wrap_torch(t)


def run(r):
    """The operator's status, then its stream drained so torch may read the result."""
    assert r.Status == OpStatus.Success, r.Message
    onnx_amd.synchronize()


def same(a, b):
    """Equal bits over every element (no NaN in these inputs)."""
    torch.cuda.synchronize()
    return a.shape == b.shape and a.dtype == b.dtype and bool(torch.equal(a, b))


def sample(n, k, seed):
    rng = np.random.default_rng(seed)
    return np.unique(np.concatenate([np.arange(4096), np.arange(n - 4096, n), rng.integers(0, n, k)]))


def host(t, idx):
    """t.reshape(-1)[idx] or t[idx] (rows) on the host."""
    return t[torch.from_numpy(idx).cuda()].cpu().numpy()


def test_flat_binary_unary_and_gelu_at_max_length(hip):
    g = gen(1)
    x = torch.randn(N_MAX, device="cuda", generator=g)
    y = torch.randn(N_MAX, device="cuda", generator=g)
    out = torch.empty_like(x)
    torch.cuda.synchronize()
    run(HIP.Add(w(x), w(y), out=w(out)))
    assert same(out, x + y)
    idx = sample(N_MAX, 200_000, 1)
    xs, ys = host(x, idx), host(y, idx)
    assert np.array_equal(host(out, idx), O.binary(O.ADD, xs, ys))
    ax = x.abs()
    torch.cuda.synchronize()
    run(HIP.Sqrt(w(ax), out=w(out)))
    assert same(out, torch.sqrt(ax))
    del ax
    run(HIP.GeluErf(w(x), out=w(out)))
    assert np.array_equal(host(out, idx).view(np.uint32), O.gelu_erf(xs).view(np.uint32))
    run(HIP.Erf(w(x), out=w(out)))
    assert np.array_equal(host(out, idx).view(np.uint32), O.unary(O.ERF, xs).view(np.uint32))


def test_broadcast_binary_at_max_length(hip):
    g = gen(2)
    rows, inner = N_MAX // 4096, 4096
    x = torch.randn(rows, inner, device="cuda", generator=g)
    b = torch.randn(inner, device="cuda", generator=g)
    out = torch.empty_like(x)
    torch.cuda.synchronize()
    run(HIP.Mul(w(x), w(b), out=w(out)))
    assert same(out, x * b)
    ridx = sample(rows, 2000, 2)
    assert np.array_equal(host(out, ridx), O.binary(O.MUL, host(x, ridx), b.cpu().numpy()))
    # a column vector broadcast along the rows: [rows, 1] - [rows, inner]
    c = torch.randn(rows, 1, device="cuda", generator=g)
    torch.cuda.synchronize()
    run(HIP.Sub(w(c), w(x), out=w(out)))
    assert same(out, c - x)


def test_integer_ops_at_max_length(hip):
    g = gen(3)
    # C4's Div shape scaled to the largest output: [512,1,4096] / [1,1023,4096] -> 2,145,386,496 int32
    a = torch.randint(-(2**20), 2**20 + 1, (512, 1, 4096), dtype=torch.int32, device="cuda", generator=g)
    b = torch.randint(1, 1025, (1, 1023, 4096), dtype=torch.int32, device="cuda", generator=g)
    b = torch.where(torch.rand(b.shape, device="cuda", generator=g) < 0.5, b, -b)
    out = torch.empty(512, 1023, 4096, dtype=torch.int32, device="cuda")
    torch.cuda.synchronize()
    run(HIP.Div(w(a), w(b), out=w(out)))
    assert same(out, torch.div(a, b, rounding_mode="trunc"))
    ai, bi = a.cpu().numpy(), b.cpu().numpy()
    for k in (0, 511):
        assert np.array_equal(out[k].cpu().numpy()[None], O.binary(O.DIV, ai[k:k + 1], bi))
    del a, b, out
    # flat int32 Div over every element, then a zero divisor at the last element
    x = torch.randint(-(2**31), 2**31 - 1, (N_MAX,), dtype=torch.int32, device="cuda", generator=g)
    d = torch.randint(1, 2**16, (N_MAX,), dtype=torch.int32, device="cuda", generator=g)
    y = torch.empty_like(x)
    torch.cuda.synchronize()
    run(HIP.Div(w(x), w(d), out=w(y)))
    assert same(y, torch.div(x, d, rounding_mode="trunc"))
    d[-1] = 0
    torch.cuda.synchronize()
    r = HIP.Div(w(x), w(d), out=w(y))
    assert r.Status == OpStatus.Failure and r.Code == O.ERR_DIVIDE_BY_ZERO, (r.Code, r.Message)
    onnx_amd.synchronize()
    del x, d, y
    # int64 Add with wrap-around over every element
    p = torch.randint(-(2**62), 2**62, (N_MAX,), dtype=torch.int64, device="cuda", generator=g) * 2
    q = torch.randint(-(2**62), 2**62, (N_MAX,), dtype=torch.int64, device="cuda", generator=g) * 2
    s = torch.empty_like(p)
    torch.cuda.synchronize()
    run(HIP.Add(w(p), w(q), out=w(s)))
    assert same(s, p + q)
    idx = sample(N_MAX, 100_000, 3)
    assert np.array_equal(host(s, idx), O.binary(O.ADD, host(p, idx), host(q, idx)))


def test_cast_at_max_length(hip):
    g = gen(4)
    x = torch.randint(-(2**40), 2**40, (N_MAX,), dtype=torch.int64, device="cuda", generator=g)
    y = torch.empty(N_MAX, dtype=torch.float32, device="cuda")
    torch.cuda.synchronize()
    run(HIP.Cast(w(x), O.FLOAT, out=w(y)))
    assert same(y, x.float())  # round to nearest even, as (float)long
    idx = sample(N_MAX, 100_000, 4)
    assert np.array_equal(host(y, idx), O.cast(host(x, idx), O.FLOAT))
    del x
    z = torch.empty(N_MAX, dtype=torch.float64, device="cuda")
    torch.cuda.synchronize()
    run(HIP.Cast(w(y), O.DOUBLE, out=w(z)))
    assert same(z, y.double())


def within_bar(got, x64_sum, abs_sum):
    return bool(torch.all((got.double() - x64_sum).abs() <= 1e-5 * abs_sum + 1e-30))


def test_reductions_at_max_length(hip):
    g = gen(5)
    x = torch.randn(N_MAX, device="cuda", generator=g)
    o = torch.empty(1, dtype=torch.float32, device="cuda")
    tot, atot = x.sum(dtype=torch.float64), x.abs().sum(dtype=torch.float64)
    torch.cuda.synchronize()
    run(HIP.ReduceSum(w(x), None, 1, out=w(o)))
    assert within_bar(o, tot, atot)
    run(HIP.ReduceMean(w(x), None, 0, out=w(o)))
    assert within_bar(o, tot / N_MAX, atot / N_MAX)
    run(HIP.ReduceMax(w(x), None, 0, out=w(o)))
    assert same(o, torch.clamp(x.max(), min=0).reshape(1))  # the fold starts from 0
    # a middle axis (column reduction) and the last axis (row reduction) of shapes near the limit
    y = x[:512 * 1023 * 4096].view(512, 1023, 4096)
    oc = torch.empty(512, 1, 4096, dtype=torch.float32, device="cuda")
    torch.cuda.synchronize()
    run(HIP.ReduceSum(w(y), [1], 1, out=w(oc)))
    assert within_bar(oc, y.sum(1, keepdim=True, dtype=torch.float64), y.abs().sum(1, keepdim=True, dtype=torch.float64))
    yk = y[:2].cpu().numpy()
    ref = O.reduce(O.RSUM, yk, [1], True)
    assert np.all(np.abs(oc[:2].cpu().numpy().astype(np.float64) - ref) <= 1e-5 * np.abs(yk).sum(1, keepdims=True))
    z = x[:(N_MAX // 4096) * 4096].view(-1, 4096)
    orow = torch.empty(z.shape[0], 1, dtype=torch.float32, device="cuda")
    torch.cuda.synchronize()
    run(HIP.ReduceMean(w(z), [-1], 1, out=w(orow)))
    assert within_bar(orow, z.sum(-1, keepdim=True, dtype=torch.float64) / 4096,
                      z.abs().sum(-1, keepdim=True, dtype=torch.float64) / 4096)
    del x, y, z
    # int64 sum over every element: exact, wrapping
    xi = torch.randint(-(2**62), 2**62, (N_MAX,), dtype=torch.int64, device="cuda", generator=g)
    oi = torch.empty(1, dtype=torch.int64, device="cuda")
    torch.cuda.synchronize()
    run(HIP.ReduceSum(w(xi), None, 0, out=w(oi)))
    assert same(oi, xi.sum().reshape(1))


def softmax_rows_ok(got, ref):
    return np.array_equal(np.isnan(got), np.isnan(ref)) and bool(
        np.all(np.abs(got.astype(np.float64) - ref)[~np.isnan(ref)] <= 1e-5 * np.abs(ref[~np.isnan(ref)]) + 1e-30))


def test_row_kernels_at_max_length(hip):
    g = gen(6)
    rows, r = N_MAX // 512, 512
    s = torch.randn(rows, r, device="cuda", generator=g) * 3
    out = torch.empty_like(s)
    ridx = sample(rows, 2000, 6)
    torch.cuda.synchronize()
    run(HIP.Softmax(w(s), -1, out=w(out)))
    ss = host(s, ridx)
    assert softmax_rows_ok(host(out, ridx), O.softmax(ss, -1))
    mask = torch.where(torch.rand(r, device="cuda", generator=g) < 0.125, -10000.0, 0.0).float()
    torch.cuda.synchronize()
    run(HIP.AddSoftmax(w(s), w(mask), -1, out=w(out)))
    assert softmax_rows_ok(host(out, ridx), O.add_softmax(ss, mask.cpu().numpy(), -1))
    del s, out
    # LayerNorm rows of 768
    rows = N_MAX // 768
    x = torch.randn(rows, 768, device="cuda", generator=g) * 2
    gam = 1 + 0.02 * torch.randn(768, device="cuda", generator=g)
    bet = 0.02 * torch.randn(768, device="cuda", generator=g)
    y = torch.empty_like(x)
    torch.cuda.synchronize()
    run(HIP.LayerNormDecomposed(w(x), w(gam), w(bet), 1e-12, out=w(y)))
    ridx = sample(rows, 2000, 7)
    ref = O.layernorm_decomposed(host(x, ridx), gam.cpu().numpy(), bet.cpu().numpy(), np.float32(1e-12))
    assert np.all(np.abs(host(y, ridx).astype(np.float64) - ref) <= 1e-5 * np.maximum(1.0, np.abs(ref)))
    del x, y
    # Softmax over a middle axis: [2, 1023, 2^20], columns of 1023
    c = torch.randn(2, 1023, 1 << 20, device="cuda", generator=g)
    oc = torch.empty_like(c)
    torch.cuda.synchronize()
    run(HIP.Softmax(w(c), 1, out=w(oc)))
    cols = sample(1 << 20, 500, 8)
    ci = torch.from_numpy(cols).cuda()
    assert softmax_rows_ok(oc[:, :, ci].cpu().numpy(), O.softmax(np.ascontiguousarray(c[:, :, ci].cpu().numpy()), 1))


def test_movement_at_max_length(hip):
    g = gen(7)
    # Transpose of the largest square matrix, float32 (four elements per access: 46340 is a multiple of 4),
    # and of a uint8 matrix with an odd side (one element per access)
    a = torch.randn(46340, 46340, device="cuda", generator=g)
    t = torch.empty(46340, 46340, device="cuda")
    torch.cuda.synchronize()
    run(HIP.Transpose(w(a), None, out=w(t)))
    assert same(t, a.t().contiguous())
    del a, t
    a8 = torch.randint(0, 256, (46341, 46340), dtype=torch.uint8, device="cuda", generator=g)
    t8 = torch.empty(46340, 46341, dtype=torch.uint8, device="cuda")
    torch.cuda.synchronize()
    run(HIP.Transpose(w(a8), None, out=w(t8)))
    assert same(t8, a8.t().contiguous())
    del a8, t8
    # Slice with a positive and a negative step along the whole length
    x = torch.randn(N_MAX, device="cuda", generator=g)
    n3 = len(range(1, N_MAX - 1, 3))
    s3 = torch.empty(n3, device="cuda")
    run(HIP.Slice(w(x), [1], [N_MAX - 1], [0], [3], out=w(s3)))
    assert same(s3, x[1:N_MAX - 1:3])
    # ends = -(n + 5) wraps once to -5 and clamps to 0, an exclusive end: index 0 is not taken (the oracle's
    # rule on a short array fixes which indices a long one gives)
    assert np.array_equal(O.slice_(np.arange(11), [-1], [-16], [0], [-2]), np.arange(10, 0, -2))
    nb = len(range(N_MAX - 1, 0, -2))
    sb = torch.empty(nb, device="cuda")
    run(HIP.Slice(w(x), [-1], [-(N_MAX + 5)], [0], [-2], out=w(sb)))
    assert same(sb, x[torch.arange(N_MAX - 1, 0, -2, device="cuda")])
    xs = x.cpu().numpy()[: 1 << 20]
    assert np.array_equal(s3[: 1000].cpu().numpy(), O.slice_(xs, [1], [(1 << 20) - 1], [0], [3])[:1000])
    del s3, sb
    # Gather rows of [2097151, 1024] by random (also negative) indices
    d = x[: 2097151 * 1024].view(2097151, 1024)
    idx = torch.randint(-2097151, 2097151, (2097151,), dtype=torch.int64, device="cuda", generator=g)
    go = torch.empty_like(d)
    torch.cuda.synchronize()
    run(HIP.Gather(w(d), w(idx), 0, out=w(go)))
    assert same(go, d[torch.where(idx < 0, idx + 2097151, idx)])
    # which row each index names, by the oracle's rule (a negative index counts from the end once)
    ii = idx[:64].cpu().numpy()
    rows = O.gather(np.arange(2097151, dtype=np.int64), ii, 0)
    assert np.array_equal(go[:64].cpu().numpy(), host(d, rows))
    del go, idx
    # Concat of two halves along the last axis, output of 2,147,481,600 elements
    h = 2097151 // 2
    p, q = d[:h], d[h:2 * h]
    co = torch.empty(h, 2048, device="cuda")
    torch.cuda.synchronize()
    run(HIP.Concat([w(p), w(q)], 1, out=w(co)))
    assert same(co, torch.cat([p, q], 1))
    k = sample(h, 200, 9)
    assert np.array_equal(host(co, k), O.concat([host(p, k), host(q, k)], 1))
