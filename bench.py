"""Benchmark of the MI355X device path for the Lokad.Onnx elementwise /
broadcast / reduction operators.

Headline workload: the LayerNorm subgraph of ONNX
nodes ReduceMean(-1) -> Sub -> Pow 2 -> ReduceMean(-1) -> Add eps -> Sqrt ->
Div -> Mul gamma -> Add beta on X[8,512,768] float32 ~ N(0, 2),
gamma ~ N(1, 0.02), beta ~ N(0, 0.02), eps = 1e-12, run as one fused gfx950
kernel.  One step = one LayerNorm over one X.

Timing: inputs resident in HBM; 16 rotating buffer sets (403 MB touched per
16 steps, more than the 256 MB Infinity Cache) so that consecutive steps read
cold data; the K timed steps are captured in one HIP graph and replayed between
two HIP events on the launch stream (the stream the library launches on).
The CPU baseline is the oracle restatement of the reference's C# path, single
threaded, on the same workload shape.

`--all` also measures every BASELINE config op (written to stderr and to
gpurun_out/bench_configs.json); the single JSON line on stdout is the headline.

Usage: python bench.py [--gpus 1] [--steps K] [--warmup W] [--all] [--no-cpu]
"""
import argparse
import json
import os
import sys
import time

import numpy as np

ROOT = os.path.dirname(os.path.abspath(__file__))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)

PEAK_HBM_GBS = 8000.0
PEAK_FP32_MFMA_TFLOPS = 157.3  # MI355X dense fp32 matrix peak
LN_SHAPE = (8, 512, 768)
# algorithmic bytes of the fused LayerNorm: X read + Y written + gamma + beta
LN_BYTES = 2 * 8 * 512 * 768 * 4 + 2 * 768 * 4 + 4  # 25,171,972 (X + Y + gamma + beta + eps)
LN_SETS = 16


def log(*a):
    print(*a, file=sys.stderr, flush=True)


EAGER = False


def graph_time(torch, launch, steps, warmup, set_stream, reps=1):
    """Run `launch(i)` warmup times eagerly, capture `steps` launches in a HIP
    graph, replay it once untimed, then time `reps` replays with HIP events.
    Returns milliseconds per step (the median replay).  With EAGER (--eager,
    used under rocprofv3 counter collection) the steps run as ordinary launches
    instead."""
    for i in range(warmup):
        launch(i)
    torch.cuda.synchronize()
    if EAGER:
        e0 = torch.cuda.Event(enable_timing=True)
        e1 = torch.cuda.Event(enable_timing=True)
        e0.record()
        for i in range(steps):
            launch(i)
        e1.record()
        torch.cuda.synchronize()
        return e0.elapsed_time(e1) / steps
    g = torch.cuda.CUDAGraph()
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        set_stream(torch.cuda.current_stream().cuda_stream)
        with torch.cuda.graph(g, stream=s):
            for i in range(steps):
                launch(i)
    set_stream(torch.cuda.current_stream().cuda_stream)
    torch.cuda.synchronize()
    g.replay()
    torch.cuda.synchronize()
    times = []
    for _ in range(reps):
        e0 = torch.cuda.Event(enable_timing=True)
        e1 = torch.cuda.Event(enable_timing=True)
        torch.cuda.synchronize()
        e0.record()
        g.replay()
        e1.record()
        torch.cuda.synchronize()
        times.append(e0.elapsed_time(e1) / steps)
    return sorted(times)[len(times) // 2]


def wall_time(torch, fn, steps, warmup):
    """Host wall clock per call of `fn(i)` between two device synchronisations
    (for host-dispatched work that is not captured in a HIP graph)."""
    for i in range(warmup):
        fn(i)
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for i in range(steps):
        fn(i)
    torch.cuda.synchronize()
    return (time.perf_counter() - t0) / steps * 1e3


def measured_traffic():
    """HBM bytes per LayerNorm launch from the committed rocprofv3 counter
    summary (profiles/k_layernorm_c2_traffic.txt), or None when absent."""
    path = os.path.join(ROOT, "profiles", "k_layernorm_c2_traffic.txt")
    try:
        for line in open(path):
            if line.startswith("traffic_bytes_per_launch:"):
                return int(float(line.split(":", 1)[1]))
    except OSError:
        pass
    return None


def cpu_baseline_ln(target_s=10.0):
    """Oracle (C restatement of the reference path, 1 thread) on X[8,512,768]."""
    from oracle import oracle as O
    rng = np.random.default_rng(1)
    x = (rng.standard_normal(LN_SHAPE) * 2).astype(np.float32)
    g = (1 + 0.02 * rng.standard_normal(768)).astype(np.float32)
    b = (0.02 * rng.standard_normal(768)).astype(np.float32)
    O.layernorm_decomposed(x, g, b)
    n = 0
    t0 = time.perf_counter()
    while True:
        O.layernorm_decomposed(x, g, b)
        n += 1
        el = time.perf_counter() - t0
        if el >= target_s:
            break
    sec = el / n
    return {"value": round(LN_BYTES / sec / 1e9, 4), "unit": "GB/s", "cores": 1, "kind": "port",
            "sample": f"{n} full LayerNorm passes (9 ops) over X[8,512,768] f32 in {el:.1f} s, "
                      f"{sec * 1e3:.1f} ms each, single thread",
            "ms_per_step": round(sec * 1e3, 3)}


def cpu_ops(target_s=1.0):
    """CPU leg of --all: the oracle (C restatement of the reference's CPU algorithm, 1 thread) on a
    bounded sample of each config op, scaled to the full op by element count.  Returns
    {op name: (seconds for the full op, sample description)}."""
    from oracle import oracle as O
    rng = np.random.default_rng(3)

    def timed(fn, scale, sample):
        fn()
        n, t0 = 0, time.perf_counter()
        while True:
            fn()
            n += 1
            el = time.perf_counter() - t0
            if el >= target_s:
                break
        return el / n * scale, f"{sample}, {n} runs in {el:.1f} s, scaled x{scale:g}"

    out = {}
    f32 = np.float32
    A1 = rng.standard_normal((1, 128, 384)).astype(f32)
    B1 = rng.uniform(-0.1, 0.1, 384).astype(f32)
    out["C1 Add bias [1,128,384]+[384]"] = timed(lambda: O.binary(O.ADD, A1, B1), 1, "full op")
    out["C1 Mul scalar 0.125"] = timed(lambda: O.binary(O.MUL, A1, np.array(0.125, f32)), 1, "full op")
    X = (rng.standard_normal(LN_SHAPE) * 2).astype(f32)
    g = (1 + 0.02 * rng.standard_normal(768)).astype(f32)
    b = (0.02 * rng.standard_normal(768)).astype(f32)
    ln = timed(lambda: O.layernorm_decomposed(X, g, b), 1, "the 9 ops on X[8,512,768]")
    for k in ("C2 LayerNorm fused", "C2 LayerNorm 9 separate ops",
              "C2 LayerNorm graph executor, 9 nodes (host dispatch per execution)",
              "C2 LayerNorm graph executor, fused to 1 node (host dispatch per execution)"):
        out[k] = ln
    S = (rng.standard_normal((1, 12, 512, 512)) * 3).astype(f32)
    M = np.where(rng.uniform(size=(1, 1, 1, 512)) < 0.125, -10000.0, 0.0).astype(f32)
    T = O.binary(O.ADD, S, M)
    out["C3 Add mask"] = timed(lambda: O.binary(O.ADD, S, M), 16, "S[1,12,512,512] + mask[1,1,1,512]")
    out["C3 Softmax(-1)"] = timed(lambda: O.softmax(T, -1), 16, "[1,12,512,512]")
    out["C3 Add+Softmax fused"] = timed(lambda: O.add_softmax(S, M, -1), 16, "S[1,12,512,512] + mask, Softmax")
    for dt in (np.int64, np.int32):
        nm = np.dtype(dt).name
        A4 = rng.integers(-(2**20), 2**20 + 1, (4, 1, 4096)).astype(dt)
        B4 = rng.integers(1, 1025, (1, 256, 4096)).astype(dt)
        smp = "A[4,1,4096] op B[1,256,4096]"
        out[f"C4 Add {nm}"] = timed(lambda: O.binary(O.ADD, A4, B4), 16, smp)
        out[f"C4 Mul {nm}"] = timed(lambda: O.binary(O.MUL, A4, B4), 16, smp)
        out[f"C4 Div {nm} (eager, includes error-flag readback)"] = timed(lambda: O.binary(O.DIV, A4, B4), 16, smp)
        if dt == np.int64:
            Y4 = O.binary(O.ADD, A4, B4)
            out["C4 Cast i64->f32"] = timed(lambda: O.cast(Y4, 1), 16, "[4,256,4096] int64")
            out["C4 ReduceSum(axis=1) i64"] = timed(lambda: O.reduce(O.RSUM, Y4, [1], True), 16, "[4,256,4096] int64")
    X5 = rng.standard_normal((1, 2048, 3072)).astype(f32)
    out["C5 GELU chain fused"] = timed(lambda: O.gelu_erf(X5), 32, "the 5 ops on X[1,2048,3072]")
    Yb = rng.uniform(-1, 1, (16, 4096, 256)).astype(f32)
    out["C5 ReduceSum(axis=1)"] = timed(lambda: O.reduce(O.RSUM, Yb, [1], True), 16, "[16,4096,256]")
    out["C5 ReduceMean(all)"] = timed(lambda: O.reduce(O.RMEAN, Yb, None, True), 16, "[16,4096,256]")
    Am = rng.standard_normal((256, 768)).astype(f32)
    Bm = rng.standard_normal((768, 768)).astype(f32)
    out["MatMul fp32 [4096,768]x[768,768] (dense)"] = timed(lambda: O.matmul(Am, Bm), 16, "[256,768]x[768,768]")
    Bf = rng.standard_normal((768, 3072)).astype(f32)
    out["MatMul fp32 [4096,768]x[768,3072] (FFN in)"] = timed(lambda: O.matmul(Am, Bf), 16, "[256,768]x[768,3072]")
    return out


def attach_cpu(res, cpu):
    """Adds the CPU leg to each --all record it covers: CPU time of the full op, its GB/s (or TFLOP/s)
    and the GPU/CPU time ratio."""
    for d in res:
        c = cpu.get(d["op"])
        if c is None:
            continue
        sec, sample = c
        d["cpu_us"] = round(sec * 1e6, 1)
        if "algorithmic_bytes" in d:
            d["cpu_GB/s"] = round(d["algorithmic_bytes"] / sec / 1e9, 3)
        if "flops" in d:
            d["cpu_TFLOP/s"] = round(d["flops"] / sec / 1e12, 5)
        d["gpu_speedup"] = round(sec * 1e6 / d["us"], 1)
        d["cpu_sample"] = sample + " (oracle: C restatement of the reference's CPU algorithm, 1 thread)"


def bench_all(torch, HIP, DeviceTensor, set_stream, steps, warmup):
    """Every BASELINE config op, cold-cache, graph-timed; returns a list of dicts."""
    dev = torch.device("cuda:0")
    res = []
    gen = torch.Generator(device=dev)
    gen.manual_seed(0)

    def wrap(t):
        return DeviceTensor.wrap_torch(t)

    def record(name, nbytes, elems, ms, unit_elems="elements/s"):
        gbs = nbytes / (ms * 1e-3) / 1e9
        d = {"op": name, "algorithmic_bytes": nbytes, "us": round(ms * 1e3, 3), "GB/s": round(gbs, 1),
             "frac_of_peak": round(gbs / PEAK_HBM_GBS, 4), "elements_per_s": round(elems / (ms * 1e-3), 1)}
        log(json.dumps(d))
        res.append(d)

    def run(name, nbytes, elems, fn, nsets, k=None):
        ms = graph_time(torch, fn, k or steps, warmup, set_stream, reps=5)
        record(name, nbytes, elems, ms)

    # C1: A[1,128,384] + B[384], then * 0.125 (700 rotating sets: > 256 MB)
    n1 = 700
    A = [torch.randn(1, 128, 384, device=dev, generator=gen) for _ in range(n1)]
    B = torch.rand(384, device=dev, generator=gen) * 0.2 - 0.1
    C = [torch.empty(1, 128, 384, device=dev) for _ in range(n1)]
    D = [torch.empty(1, 128, 384, device=dev) for _ in range(n1)]
    s8 = torch.tensor(0.125, device=dev)
    wA, wB, wC, wD, ws8 = [wrap(t) for t in A], wrap(B), [wrap(t) for t in C], [wrap(t) for t in D], wrap(s8)
    run("C1 Add bias [1,128,384]+[384]", 394752, 49152, lambda i: HIP.Add(wA[i % n1], wB, out=wC[i % n1]), n1)
    run("C1 Mul scalar 0.125", 393220, 49152, lambda i: HIP.Mul(wC[i % n1], ws8, out=wD[i % n1]), n1)
    # the two nodes as one elementwise-chain kernel (what the graph runtime's fusion runs)
    run("C1 Add -> Mul as one ElementwiseChain kernel", 394756, 49152,
        lambda i: HIP.ElementwiseChain([wA[i % n1], wB, ws8], [("Add", 1), ("Mul", 2)], out=wD[i % n1]), n1)
    # and through the graph runtime, host dispatch per execution: 2 nodes, then fused
    from onnx_amd.graph import ComputationalGraph
    for fuse, label, nbytes in ((False, "2 nodes", 394752 + 393220), (True, "fused to 1 chain", 394756)):
        gr = ComputationalGraph(13)
        gr.AddInput("x", np.float32, (1, 128, 384))
        gr.AddInitializer("bias", B.cpu().numpy())
        gr.AddInitializer("k", np.array(0.125, np.float32))
        gr.AddNode("Add", ["x", "bias"], ["h"], name="add")
        gr.AddNode("Mul", ["h", "k"], ["y"], name="mul")
        gr.AddOutput("y")
        if fuse:
            assert gr.Fuse() == 1

        def step(i, gr=gr):
            if not gr.Execute([wA[i % n1]]):
                raise RuntimeError(gr.LastError)
        record(f"C1 graph executor, {label} (host dispatch per execution)", nbytes, 49152,
               wall_time(torch, step, max(64, steps), warmup))
        # the same execution recorded once into a HIP graph and replayed (one launch per execution)
        assert gr.Capture([wA[0]]), gr.LastError

        def replay(i, gr=gr):
            if not gr.Replay():
                raise RuntimeError(gr.LastError)
        record(f"C1 graph executor, {label}, captured (replay per execution, one input buffer)", nbytes, 49152,
               wall_time(torch, replay, max(64, steps), warmup))
        gr.close()
    # launch-bound graphs of many small nodes: 40 alternating Add / Mul nodes on C1's shape (no fusion),
    # host dispatch per execution against one captured replay
    gr = ComputationalGraph(13)
    gr.AddInput("x", np.float32, (1, 128, 384))
    gr.AddInitializer("bias", B.cpu().numpy())
    prev = "x"
    for k in range(40):
        gr.AddNode("Add" if k % 2 == 0 else "Mul", [prev, "bias"], [f"t{k}"], name=f"n{k}")
        prev = f"t{k}"
    gr.AddOutput(prev)

    def step40(i):
        if not gr.Execute([wA[0]]):
            raise RuntimeError(gr.LastError)

    def replay40(i):
        if not gr.Replay():
            raise RuntimeError(gr.LastError)
    nb40 = 40 * 394752
    record("40-node Add/Mul graph on [1,128,384] (host dispatch per execution)", nb40, 40 * 49152,
           wall_time(torch, step40, max(32, steps // 4), warmup))
    assert gr.Capture([wA[0]]), gr.LastError
    record("40-node Add/Mul graph on [1,128,384], captured (replay per execution)", nb40, 40 * 49152,
           wall_time(torch, replay40, max(32, steps // 4), warmup))
    gr.close()
    del A, C, D, wA, wC, wD
    torch.cuda.empty_cache()

    # C2: fused LayerNorm and the 9 separate ops
    X = [torch.randn(*LN_SHAPE, device=dev, generator=gen) * 2 for _ in range(LN_SETS)]
    Y = [torch.empty(*LN_SHAPE, device=dev) for _ in range(LN_SETS)]
    gam = 1 + 0.02 * torch.randn(768, device=dev, generator=gen)
    bet = 0.02 * torch.randn(768, device=dev, generator=gen)
    wX, wY, wg, wb = [wrap(t) for t in X], [wrap(t) for t in Y], wrap(gam), wrap(bet)
    run("C2 LayerNorm fused", LN_BYTES, 8 * 512 * 768,
        lambda i: HIP.LayerNormDecomposed(wX[i % LN_SETS], wg, wb, 1e-12, out=wY[i % LN_SETS]), LN_SETS)
    # the practical ceiling at this size: a plain device copy of the same bytes (Cast float -> float, 16-byte
    # nontemporal loads and stores) over the same 16 buffer sets; at 25 MB per launch the ramp and drain of
    # one launch cost about as much as the transfer itself
    run("C2 size-matched copy X -> Y (Cast float->float, same buffer sets)", 2 * 8 * 512 * 768 * 4, 8 * 512 * 768,
        lambda i: HIP.Cast(wX[i % LN_SETS], 1, out=wY[i % LN_SETS]), LN_SETS)
    # the same with the host round trip a caller holding host arrays pays (as the C# provider's managed
    # tensors are): X uploaded from pageable host memory, the kernel, Y read back; host clock per step
    Xh = [x.cpu().numpy() for x in X[:2]]

    def ln_host(i):
        wX[i % 2].upload(Xh[i % 2])
        HIP.LayerNormDecomposed(wX[i % 2], wg, wb, 1e-12, out=wY[i % 2])
        wY[i % 2].to_numpy()
    record("C2 LayerNorm fused, including upload of X and download of Y (pageable host memory)", LN_BYTES,
           8 * 512 * 768, wall_time(torch, ln_host, max(16, steps // 8), warmup))
    # unfused: 9 launches through the operator API, intermediates preallocated
    tm = {k: [torch.empty(8, 512, 1, device=dev) for _ in range(LN_SETS)] for k in ("mean", "var", "ve", "sd")}
    tf = {k: [torch.empty(*LN_SHAPE, device=dev) for _ in range(LN_SETS)] for k in ("d", "p", "n", "m")}
    wm = {k: [wrap(t) for t in v] for k, v in tm.items()}
    wf = {k: [wrap(t) for t in v] for k, v in tf.items()}
    two, eps = wrap(torch.tensor(2.0, device=dev)), wrap(torch.tensor(1e-12, device=dev))

    def ln_unfused(i):
        j = i % LN_SETS
        HIP.ReduceMean(wX[j], [-1], 1, out=wm["mean"][j])
        HIP.Sub(wX[j], wm["mean"][j], out=wf["d"][j])
        HIP.Pow(wf["d"][j], two, out=wf["p"][j])
        HIP.ReduceMean(wf["p"][j], [-1], 1, out=wm["var"][j])
        HIP.Add(wm["var"][j], eps, out=wm["ve"][j])
        HIP.Sqrt(wm["ve"][j], out=wm["sd"][j])
        HIP.Div(wf["d"][j], wm["sd"][j], out=wf["n"][j])
        HIP.Mul(wf["n"][j], wg, out=wf["m"][j])
        HIP.Add(wf["m"][j], wb, out=wY[j])
    run("C2 LayerNorm 9 separate ops", 151132168, 8 * 512 * 768, ln_unfused, LN_SETS, k=max(8, steps // 4))

    # the same ONNX subgraph through the device graph runtime (the ComputationalGraph twin), one
    # host-dispatched execution per step (wall clock, ctypes call included): 9 nodes, then fused

    def ln_graph(fuse):
        gr = ComputationalGraph(13)
        gr.AddInput("x", np.float32, LN_SHAPE)
        for name, v in (("axes", np.array([-1], np.int64)), ("two", np.array(2.0, np.float32)),
                        ("eps", np.array(1e-12, np.float32)), ("gamma", gam.cpu().numpy()),
                        ("beta", bet.cpu().numpy())):
            gr.AddInitializer(name, v)
        for op, ins, outs in (("ReduceMean", ["x", "axes"], ["mean"]), ("Sub", ["x", "mean"], ["d"]),
                              ("Pow", ["d", "two"], ["p"]), ("ReduceMean", ["p", "axes"], ["var"]),
                              ("Add", ["var", "eps"], ["ve"]), ("Sqrt", ["ve"], ["sd"]), ("Div", ["d", "sd"], ["n"]),
                              ("Mul", ["n", "gamma"], ["m"]), ("Add", ["m", "beta"], ["y"])):
            gr.AddNode(op, ins, outs, name=outs[0])
        gr.AddOutput("y")
        if fuse:
            assert gr.Fuse() == 1
        return gr

    for fuse, label, nbytes in ((False, "9 nodes", 151132168), (True, "fused to 1 node", LN_BYTES)):
        gr = ln_graph(fuse)

        def step(i, gr=gr):
            if not gr.Execute([wX[i % LN_SETS]]):
                raise RuntimeError(gr.LastError)
        ms = wall_time(torch, step, max(16, steps // 2), warmup)
        record(f"C2 LayerNorm graph executor, {label} (host dispatch per execution)", nbytes, 8 * 512 * 768, ms)
        if not fuse:
            assert gr.Capture([wX[0]]), gr.LastError

            def replay(i, gr=gr):
                if not gr.Replay():
                    raise RuntimeError(gr.LastError)
            record(f"C2 LayerNorm graph executor, {label}, captured (replay per execution, one input buffer)", nbytes, 8 * 512 * 768,
                   wall_time(torch, replay, max(16, steps // 2), warmup))
        gr.close()
    del X, Y, tm, tf, wX, wY, wm, wf
    torch.cuda.empty_cache()

    # C3: S[16,12,512,512] + mask[16,1,1,512], Softmax(-1); separately and fused
    S = torch.randn(16, 12, 512, 512, device=dev, generator=gen) * 3
    M = torch.zeros(16, 1, 1, 512, device=dev)
    for bi in range(16):
        idx = torch.randperm(512, device=dev, generator=gen)[:64]
        M[bi, 0, 0, idx] = -10000.0
    T = torch.empty_like(S)
    O2 = torch.empty_like(S)
    wS, wM, wT, wO = wrap(S), wrap(M), wrap(T), wrap(O2)
    k3 = max(4, steps // 8)
    run("C3 Add mask", 402685952, S.numel(), lambda i: HIP.Add(wS, wM, out=wT), 1, k=k3)
    run("C3 Softmax(-1)", 402653184, S.numel(), lambda i: HIP.Softmax(wT, -1, out=wO), 1, k=k3)
    run("C3 Add+Softmax fused", 402685952, S.numel(), lambda i: HIP.AddSoftmax(wS, wM, -1, out=wO), 1, k=k3)
    del S, M, T, O2, wS, wM, wT, wO
    torch.cuda.empty_cache()

    # C4: int64 / int32 A[64,1,4096] (U[-2^20,2^20]) op B[1,256,4096] (U[1,1024])
    for dt, es in ((torch.int64, 8), (torch.int32, 4)):
        A4 = torch.randint(-(2**20), 2**20 + 1, (64, 1, 4096), device=dev, dtype=dt, generator=gen)
        B4 = torch.randint(1, 1025, (1, 256, 4096), device=dev, dtype=dt, generator=gen)
        Y4 = torch.empty(64, 256, 4096, device=dev, dtype=dt)
        wA4, wB4, wY4 = wrap(A4), wrap(B4), wrap(Y4)
        nb = (64 * 4096 + 256 * 4096 + 64 * 256 * 4096) * es
        for op in ("Add", "Mul"):
            run(f"C4 {op} {str(dt)[6:]}", nb, Y4.numel(), lambda i, op=op: getattr(HIP, op)(wA4, wB4, out=wY4), 1, k=k3)
        # Div checks the device error flags (one readback per call): eager timing, host clock per call
        nd = max(8, k3)
        for _ in range(2):
            HIP.Div(wA4, wB4, out=wY4)
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        for _ in range(nd):
            HIP.Div(wA4, wB4, out=wY4)
        torch.cuda.synchronize()
        record(f"C4 Div {str(dt)[6:]} (eager, includes error-flag readback)", nb, Y4.numel(),
               (time.perf_counter() - t0) * 1e3 / nd)
        if dt == torch.int64:
            Yc = torch.empty(64, 256, 4096, device=dev, dtype=torch.float32)
            wYc = wrap(Yc)
            HIP.Add(wA4, wB4, out=wY4)
            run("C4 Cast i64->f32", 805306368, Y4.numel(), lambda i: HIP.Cast(wY4, 1, out=wYc), 1, k=k3)
            Yr = torch.empty(64, 1, 4096, device=dev, dtype=dt)
            wYr = wrap(Yr)
            run("C4 ReduceSum(axis=1) i64", 538968064, Y4.numel(), lambda i: HIP.ReduceSum(wY4, [1], 1, out=wYr), 1, k=k3)
            del Yc, wYc, Yr, wYr
        del A4, B4, Y4, wA4, wB4, wY4
        torch.cuda.empty_cache()

    # C5: GELU chain on X[32,2048,3072]; ReduceSum(axis=1) and ReduceMean(all) on Y[256,4096,256]
    X5 = torch.randn(32, 2048, 3072, device=dev, generator=gen)
    Y5 = torch.empty_like(X5)
    wX5, wY5 = wrap(X5), wrap(Y5)
    run("C5 GELU chain fused", 1610612736, X5.numel(), lambda i: HIP.GeluErf(wX5, out=wY5), 1, k=k3)
    # the same five nodes through the generic elementwise-chain kernel (the fusion used when the
    # constants do not match the GELU pattern)
    k5 = [wrap(torch.tensor(v, device=dev)) for v in (1.4142135381698608, 1.0, 0.5)]
    run("C5 GELU chain as a generic ElementwiseChain", 1610612736, X5.numel(),
        lambda i: HIP.ElementwiseChain([wX5] + k5, [("Div", 1), ("Erf",), ("Add", 2), ("Mul", 0, True), ("Mul", 3)],
                                       out=wY5), 1, k=k3)
    del X5, Y5, wX5, wY5
    torch.cuda.empty_cache()
    Yb = torch.rand(256, 4096, 256, device=dev, generator=gen) * 2 - 1
    R1 = torch.empty(256, 1, 256, device=dev)
    R2 = torch.empty(1, 1, 1, device=dev)
    wYb, wR1, wR2 = wrap(Yb), wrap(R1), wrap(R2)
    run("C5 ReduceSum(axis=1)", 1074003968, Yb.numel(), lambda i: HIP.ReduceSum(wYb, [1], 1, out=wR1), 1, k=k3)
    run("C5 ReduceMean(all)", 1073741828, Yb.numel(), lambda i: HIP.ReduceMean(wYb, None, 1, out=wR2), 1, k=k3)
    # copy-kernel ceiling on the same GPU (torch's device copy of 1 GiB)
    Zc = torch.empty_like(Yb)
    torch.cuda.synchronize()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    for _ in range(3):
        Zc.copy_(Yb)
    e0.record()
    for _ in range(10):
        Zc.copy_(Yb)
    e1.record()
    torch.cuda.synchronize()
    record("device copy 1 GiB (torch copy_, ceiling reference)", 2 * Yb.numel() * 4, Yb.numel(), e0.elapsed_time(e1) / 10)
    del Yb, Zc
    torch.cuda.empty_cache()

    # Data movement (row f3): HBM-bound; every element read once and written once (algorithmic bytes
    # = input bytes moved + output bytes + index bytes); rotating sets of > 256 MB keep the L2 and the
    # MALL cold
    def movement(name, in_shape, make_out, fn, sets=12):
        xs = [torch.randn(*in_shape, device=dev, generator=gen) for _ in range(sets)]
        ys = [make_out() for _ in range(sets)]
        wx, wy = [wrap(t) for t in xs], [wrap(t) for t in ys]
        out_bytes = ys[0].numel() * ys[0].element_size()  # the elements read equal the elements written
        run(name, 2 * out_bytes, ys[0].numel(), lambda i: fn(wx[i % sets], wy[i % sets]), sets)
        del xs, ys, wx, wy

    movement("Transpose [8,512,12,64] perm [0,2,1,3] (attention heads)", (8, 512, 12, 64),
             lambda: torch.empty(8, 12, 512, 64, device=dev), lambda x, y: HIP.Transpose(x, [0, 2, 1, 3], out=y))
    movement("Transpose [8,512,12,64] perm [0,2,3,1] (keys, innermost axis moves)", (8, 512, 12, 64),
             lambda: torch.empty(8, 12, 64, 512, device=dev), lambda x, y: HIP.Transpose(x, [0, 2, 3, 1], out=y))
    movement("Transpose [3072,768] (weight)", (3072, 768), lambda: torch.empty(768, 3072, device=dev),
             lambda x, y: HIP.Transpose(x, None, out=y), sets=40)
    movement("Slice [8,512,2304] -> [8,512,768] (QKV split)", (8, 512, 2304),
             lambda: torch.empty(8, 512, 768, device=dev),
             lambda x, y: HIP.Slice(x, [768], [1536], [-1], None, out=y), sets=8)
    cat_in = [[wrap(torch.randn(8, 512, 768, device=dev, generator=gen)) for _ in range(3)] for _ in range(8)]
    cat_out = [wrap(torch.empty(8, 512, 2304, device=dev)) for _ in range(8)]
    run("Concat 3 x [8,512,768] axis -1", 2 * 8 * 512 * 2304 * 4, 8 * 512 * 2304,
        lambda i: HIP.Concat(cat_in[i % 8], -1, out=cat_out[i % 8]), 8)
    del cat_in, cat_out
    table = wrap(torch.randn(30522, 768, device=dev, generator=gen))
    ids = [wrap(torch.randint(0, 30522, (8, 512), device=dev, generator=gen)) for _ in range(24)]
    emb = [wrap(torch.empty(8, 512, 768, device=dev)) for _ in range(24)]
    # Gather checks its indices on the device and reads the verdict back, so it is not captured:
    # host wall clock per call, the readback included
    record("Gather [30522,768] by ids [8,512] (word embedding; per call incl. index-check readback)",
           2 * 8 * 512 * 768 * 4 + 8 * 512 * 8, 8 * 512 * 768,
           wall_time(torch, lambda i: HIP.Gather(table, ids[i % 24], 0, out=emb[i % 24]), steps, warmup))
    del table, ids, emb
    torch.cuda.empty_cache()

    # a whole BERT-base encoder layer (batch 8 x 512 tokens) through the graph runtime: 74 ONNX nodes
    # node by node, fused (LayerNorm / GELU / mask+Softmax / residual chains), and the fused graph captured
    sys.path.insert(0, os.path.join(ROOT, "tests"))
    from bert_layer import bert_layer
    from onnx_amd.graph import Model
    model, bins, _, _ = bert_layer(8, 512, 5)
    bdev = {k: DeviceTensor.from_numpy(v) for k, v in bins.items()}
    layer_flops = 2.0 * 4096 * (4 * 768 * 768 + 2 * 768 * 3072) + 2 * 2.0 * 8 * 12 * 512 * 512 * 64
    for label, fuse, capture in (("74 nodes", False, False), ("fused", True, False), ("fused, captured", True, True)):
        gl = Model.Load(model)
        if fuse:
            gl.Fuse()
        if capture:
            assert gl.Capture(bdev), gl.LastError

        def layer_step(i, gl=gl, capture=capture):
            if not (gl.Replay() if capture else gl.Execute(bdev)):
                raise RuntimeError(gl.LastError)
        ms = wall_time(torch, layer_step, max(8, steps // 16), max(2, warmup // 4))
        d = {"op": f"BERT-base encoder layer [8,512,768], {label} (per execution)", "us": round(ms * 1e3, 1),
             "tokens_per_s": round(4096 / (ms * 1e-3), 1), "TFLOP/s": round(layer_flops / (ms * 1e-3) / 1e12, 2),
             "flops": layer_flops}
        log(json.dumps(d))
        res.append(d)
        gl.close()
    del bdev

    # MatMul (row f2): fp32 MFMA, compute-bound; BERT-base shapes at batch 8 x 512 tokens
    for name, sa, sb in (("MatMul fp32 [4096,768]x[768,768] (dense)", (4096, 768), (768, 768)),
                         ("MatMul fp32 [4096,768]x[768,2304] (fused QKV projection)", (4096, 768), (768, 2304)),
                         ("MatMul fp32 [4096,768]x[768,3072] (FFN in)", (4096, 768), (768, 3072)),
                         ("MatMul fp32 [4096,3072]x[3072,768] (FFN out)", (4096, 3072), (3072, 768)),
                         ("MatMul fp32 [16,12,512,64]x[16,12,64,512] (attention scores)", (16, 12, 512, 64),
                          (16, 12, 64, 512)),
                         ("MatMul fp32 [4096,4096]x[4096,4096]", (4096, 4096), (4096, 4096))):
        Am = torch.randn(*sa, device=dev, generator=gen)
        Bm = torch.randn(*sb, device=dev, generator=gen)
        Cm = torch.empty(*(sa[:-1] + sb[-1:]), device=dev)
        wAm, wBm, wCm = wrap(Am), wrap(Bm), wrap(Cm)
        flops = 2.0 * (Am.numel() // sa[-1]) * sa[-1] * sb[-1]
        ms = graph_time(torch, lambda i: HIP.MatMul(wAm, wBm, out=wCm), max(4, steps // 8), warmup, set_stream, reps=5)
        tf = flops / (ms * 1e-3) / 1e12
        d = {"op": name, "flops": flops, "us": round(ms * 1e3, 3), "TFLOP/s": round(tf, 2),
             "frac_of_peak": round(tf / PEAK_FP32_MFMA_TFLOPS, 4), "bound": "mfma"}
        log(json.dumps(d))
        res.append(d)
        del Am, Bm, Cm, wAm, wBm, wCm
    torch.cuda.empty_cache()
    return res


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=200)
    ap.add_argument("--warmup", type=int, default=20)
    ap.add_argument("--all", action="store_true", help="also measure every BASELINE config op")
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline leg")
    ap.add_argument("--eager", action="store_true", help="time ordinary launches instead of a HIP graph")
    ap.add_argument("--copy-calibration", action="store_true",
                    help="also run a plain 256 MiB device copy (Cast float->float) 4 times, the known-size "
                         "reference for scaling rocprofv3 FETCH_SIZE / WRITE_SIZE")
    args = ap.parse_args()
    global EAGER
    EAGER = args.eager
    if args.gpus != 1:
        print(f"bench.py measures one GPU only: this build has no multi-GPU path (asked for --gpus {args.gpus}).",
              file=sys.stderr)
        sys.exit(2)

    import torch

    import onnx_amd
    from onnx_amd import DeviceTensor, HipExecutionProvider as HIP

    onnx_amd.init(0)
    set_stream = onnx_amd.set_stream
    set_stream(torch.cuda.current_stream().cuda_stream)
    dev = torch.device("cuda:0")
    gen = torch.Generator(device=dev)
    gen.manual_seed(2)
    X = [torch.randn(*LN_SHAPE, device=dev, generator=gen) * 2 for _ in range(LN_SETS)]
    Y = [torch.empty(*LN_SHAPE, device=dev) for _ in range(LN_SETS)]
    gam = 1 + 0.02 * torch.randn(768, device=dev, generator=gen)
    bet = 0.02 * torch.randn(768, device=dev, generator=gen)
    wX = [DeviceTensor.wrap_torch(t) for t in X]
    wY = [DeviceTensor.wrap_torch(t) for t in Y]
    wg, wb = DeviceTensor.wrap_torch(gam), DeviceTensor.wrap_torch(bet)

    def step(i):
        r = HIP.LayerNormDecomposed(wX[i % LN_SETS], wg, wb, 1e-12, out=wY[i % LN_SETS])
        if r.Code:
            raise RuntimeError(r.Message)

    ms = graph_time(torch, step, args.steps, args.warmup, set_stream)
    gbs = LN_BYTES / (ms * 1e-3) / 1e9
    if args.copy_calibration:
        src = torch.randn(64 * 1024 * 1024, device=dev, generator=gen)
        dst = torch.empty_like(src)
        ws, wd = DeviceTensor.wrap_torch(src), DeviceTensor.wrap_torch(dst)
        for _ in range(4):
            HIP.Cast(ws, 1, out=wd)
        torch.cuda.synchronize()
    out = {
        "metric": "achieved HBM GB/s (% of MI355X peak) per op + elements/s vs C# CPU path",
        "value": round(gbs, 2),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms, 6),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f32",
        "data": "synthetic (torch.randn on device, seeded): X ~ N(0,2), gamma ~ N(1,0.02), beta ~ N(0,0.02)",
        "config": {"workload": "C2 LayerNorm decomposed into 9 ONNX ops, one fused kernel, X[8,512,768] f32",
                   "algorithmic_bytes_per_step": LN_BYTES, "buffer_sets": LN_SETS,
                   "elements_per_s": round(8 * 512 * 768 / (ms * 1e-3), 1)},
        "roofline": {"bound": "hbm", "achieved": round(gbs, 2), "peak": PEAK_HBM_GBS, "unit": "GB/s",
                     "frac": round(gbs / PEAK_HBM_GBS, 4), "traffic": measured_traffic()},
    }
    if args.all:
        res = bench_all(torch, HIP, DeviceTensor, set_stream, args.steps, args.warmup)
        if not args.no_cpu:
            attach_cpu(res, cpu_ops())
            for d in res:
                if "cpu_us" in d:
                    log(json.dumps({k: d[k] for k in ("op", "us", "cpu_us", "gpu_speedup")}))
        os.makedirs(os.path.join(ROOT, "gpurun_out"), exist_ok=True)
        with open(os.path.join(ROOT, "gpurun_out", "bench_configs.json"), "w") as f:
            json.dump(res, f, indent=1)
    if not args.no_cpu:
        cb = cpu_baseline_ln()
        out["cpu_baseline"] = {k: cb[k] for k in ("value", "unit", "cores", "kind", "sample")}
    print(json.dumps(out), flush=True)


if __name__ == "__main__":
    main()
