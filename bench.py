"""Benchmark of the MI355X device path for the Lokad.Onnx elementwise /
broadcast / reduction operators.

Headline workload: BASELINE.json configs[4] (C5, the largest), one step =
  the Erf-GELU subgraph Div(x, sqrt2) -> Erf -> Add 1 -> Mul x -> Mul 0.5 on
  X[32,2048,3072] f32 ~ N(0,1), run as one fused kernel, then
  ReduceSum(axis=1, keepdims) over Y[256,4096,256] f32 ~ U(-1,1), then
  ReduceMean over all of Y.
`value` = the step's algorithmic bytes (every input read once + every output
written once) / the step time, inputs resident in HBM (each step touches
3.5 GB, far above the 256 MB Infinity Cache).  The K timed steps run on the
library's launch stream with a HIP event between consecutive kernels; the
dominant kernel (the fused GELU) gives `roofline.achieved`.

`per_config` in the same JSON line holds every BASELINE config op (C1..C5),
each timed as a HIP-graph replay over rotating buffer sets (more than 256 MB
touched between two launches on the same data), with its HBM traffic from two
rocprofv3 counter passes (FETCH_SIZE, WRITE_SIZE) run as child processes over
`bench.py --probe`, scaled by a plain copy of known size, and its CPU leg: the
oracle (C restatement of the reference's C# CPU path, 1 thread) on a bounded
sample, scaled to the full op.

Usage: python bench.py [--gpus 1] [--steps K] [--warmup W] [--no-cpu]
                       [--traffic live|profile|none] [--all]
--all adds the graph executor, data movement, BERT layer and MatMul lines
(stderr and gpurun_out/bench_configs.json).
"""
import argparse
import csv
import glob
import json
import os
import platform
import shutil
import signal
import subprocess
import sys
import time

import numpy as np

ROOT = os.path.dirname(os.path.abspath(__file__))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)

PEAK_HBM_GBS = 8000.0
PEAK_FP32_MFMA_TFLOPS = 157.3  # MI355X dense fp32 matrix peak
LN_SHAPE = (8, 512, 768)
LN_BYTES = 2 * 8 * 512 * 768 * 4 + 2 * 768 * 4 + 4  # 25,171,972 (X + Y + gamma + beta + eps)
LN_SETS = 16
C5_X = (32, 2048, 3072)
C5_Y = (256, 4096, 256)
GELU_BYTES = 2 * 32 * 2048 * 3072 * 4                   # 1,610,612,736
RSUM_BYTES = 256 * 4096 * 256 * 4 + 256 * 256 * 4       # 1,074,003,968
RMEAN_BYTES = 256 * 4096 * 256 * 4 + 4                  # 1,073,741,828
C5_STEP_BYTES = GELU_BYTES + RSUM_BYTES + RMEAN_BYTES
CALIB_BYTES = 256 << 20   # counter calibration: a plain copy of 256 MiB
MARKER = "lx::k_cast<2, 5,"   # Cast uint8 -> int16 of a few elements: separates the probe's ops


def log(*a):
    print(*a, file=sys.stderr, flush=True)


EAGER = False


def graph_time(torch, launch, steps, warmup, set_stream, reps=1):
    """Run `launch(i)` warmup times eagerly, capture `steps` launches in a HIP
    graph, replay it once untimed, then time `reps` replays with HIP events.
    Returns milliseconds per step (the median replay).  With EAGER (--eager)
    the steps run as ordinary launches instead."""
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


def wall_time(torch, fn, steps, warmup, reps=5):
    """Host wall clock per call of `fn(i)` between two device synchronisations (for host-dispatched work
    that is not captured in a HIP graph): `warmup` calls, then `reps` blocks of `steps` calls, the median
    block.  The blocks make the figure robust to the first milliseconds of a workload, which on this part
    run slower than the rest (the clock settling after a change of load)."""
    for i in range(warmup):
        fn(i)
    torch.cuda.synchronize()
    times = []
    for _ in range(reps):
        t0 = time.perf_counter()
        for i in range(steps):
            fn(i)
        torch.cuda.synchronize()
        times.append((time.perf_counter() - t0) / steps * 1e3)
    return sorted(times)[len(times) // 2]


def host_info(torch):
    """The machine the numbers come from: host CPU, cores, glibc (whose expf / powf bits the oracle
    reproduces), ROCm, torch, GPU."""
    cpu = "unknown"
    try:
        for line in open("/proc/cpuinfo"):
            if line.startswith("model name"):
                cpu = line.split(":", 1)[1].strip()
                break
    except OSError:
        pass
    rocm = "unknown"
    for p in ("/opt/rocm/.info/version", "/opt/rocm/.info/version-dev"):
        if os.path.exists(p):
            rocm = open(p).read().strip()
            break
    try:
        glibc = os.confstr("CS_GNU_LIBC_VERSION")
    except (ValueError, OSError):
        glibc = " ".join(platform.libc_ver())
    p = torch.cuda.get_device_properties(0)
    return {"host_cpu": cpu, "host_cores_total": os.cpu_count(), "host_cores_usable": len(os.sched_getaffinity(0)),
            "glibc": glibc, "rocm": rocm, "hip_runtime": torch.version.hip, "torch": torch.__version__,
            "gpu": f"{p.name} ({getattr(p, 'gcnArchName', '?')}, {p.multi_processor_count} CUs, "
                   f"{p.total_memory / 2**30:.0f} GiB)", "kernel": platform.release()}


# ---------------------------------------------------------------------------
# workloads: every BASELINE config op on device buffers (shared by the timed run and the probe)
# ---------------------------------------------------------------------------
class Workloads:
    """Device buffers of every BASELINE config, generated on the device with a seeded torch generator,
    and one launch function per op.  `specs` lists the per-config ops in BASELINE order."""

    def __init__(self, torch, HIP, DeviceTensor, steps):
        self.torch, self.HIP = torch, HIP
        dev = torch.device("cuda:0")
        gen = torch.Generator(device=dev)
        gen.manual_seed(0)
        w = DeviceTensor.wrap_torch
        self.specs = []
        kbig = max(6, steps // 8)

        def spec(config, op, nbytes, elems, fn, sets, k, timing="graph", kernels=""):
            self.specs.append({"config": config, "op": op, "algorithmic_bytes": nbytes, "elements": elems,
                               "fn": fn, "sets": sets, "k": k, "timing": timing, "kernels": kernels})

        # C1: A[1,128,384] + B[384], then * 0.125 (700 rotating sets: 276 MB > 256 MB)
        n1 = 700
        self.A1 = [torch.randn(1, 128, 384, device=dev, generator=gen) for _ in range(n1)]
        self.B1 = torch.rand(384, device=dev, generator=gen) * 0.2 - 0.1
        self.C1 = [torch.empty(1, 128, 384, device=dev) for _ in range(n1)]
        self.D1 = [torch.empty(1, 128, 384, device=dev) for _ in range(n1)]
        self.s8 = torch.tensor(0.125, device=dev)
        wA, wB, wC, wD, ws8 = [w(t) for t in self.A1], w(self.B1), [w(t) for t in self.C1], [w(t) for t in self.D1], w(self.s8)
        self.wA1, self.wB1, self.ws8 = wA, wB, ws8
        k1 = max(64, 2 * steps)
        spec("C1", "Add bias [1,128,384]+[384]", 394752, 49152, lambda i: HIP.Add(wA[i % n1], wB, out=wC[i % n1]), n1,
             k1, kernels="k_binary_nd<0,float>")
        spec("C1", "Mul scalar 0.125", 393220, 49152, lambda i: HIP.Mul(wC[i % n1], ws8, out=wD[i % n1]), n1, k1,
             kernels="k_binary_flat<2,float,scalar B>")
        spec("C1", "Add -> Mul fused (one ElementwiseChain kernel, the graph runtime's fusion)", 394756, 49152,
             lambda i: HIP.ElementwiseChain([wA[i % n1], wB, ws8], [("Add", 1), ("Mul", 2)], out=wD[i % n1]), n1, k1,
             kernels="k_chain")

        # C2: LayerNorm over X[8,512,768] (16 sets: 403 MB)
        self.X2 = [torch.randn(*LN_SHAPE, device=dev, generator=gen) * 2 for _ in range(LN_SETS)]
        self.Y2 = [torch.empty(*LN_SHAPE, device=dev) for _ in range(LN_SETS)]
        self.gam = 1 + 0.02 * torch.randn(768, device=dev, generator=gen)
        self.bet = 0.02 * torch.randn(768, device=dev, generator=gen)
        wX, wY, wg, wb = [w(t) for t in self.X2], [w(t) for t in self.Y2], w(self.gam), w(self.bet)
        self.wX2, self.wY2, self.wg, self.wb = wX, wY, wg, wb
        k2 = max(32, steps)
        spec("C2", "LayerNorm, 9 ONNX ops as one fused kernel", LN_BYTES, 8 * 512 * 768,
             lambda i: HIP.LayerNormDecomposed(wX[i % LN_SETS], wg, wb, 1e-12, out=wY[i % LN_SETS]), LN_SETS, k2,
             kernels="k_layernorm<3>")
        tm = {k: [torch.empty(8, 512, 1, device=dev) for _ in range(LN_SETS)] for k in ("mean", "var", "ve", "sd")}
        tf = {k: [torch.empty(*LN_SHAPE, device=dev) for _ in range(LN_SETS)] for k in ("d", "p", "n", "m")}
        self.ln_tmp = (tm, tf)
        wm = {k: [w(t) for t in v] for k, v in tm.items()}
        wf = {k: [w(t) for t in v] for k, v in tf.items()}
        self.two, self.eps = torch.tensor(2.0, device=dev), torch.tensor(1e-12, device=dev)
        two, eps = w(self.two), w(self.eps)

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
        spec("C2", "LayerNorm as its 9 separate operator calls", 151132168, 8 * 512 * 768, ln_unfused, LN_SETS,
             max(16, steps // 4), kernels="9 kernels")

        # C3: S[16,12,512,512] + mask[16,1,1,512] (64 of 512 positions masked per batch row), Softmax(-1)
        self.S3 = torch.randn(16, 12, 512, 512, device=dev, generator=gen) * 3
        self.M3 = torch.zeros(16, 1, 1, 512, device=dev)
        for bi in range(16):
            idx = torch.randperm(512, device=dev, generator=gen)[:64]
            self.M3[bi, 0, 0, idx] = -10000.0
        self.T3 = torch.empty_like(self.S3)
        self.O3 = torch.empty_like(self.S3)
        wS, wM, wT, wO = w(self.S3), w(self.M3), w(self.T3), w(self.O3)
        ne3 = self.S3.numel()
        spec("C3", "Add mask [16,12,512,512]+[16,1,1,512]", 402685952, ne3, lambda i: HIP.Add(wS, wM, out=wT), 1, kbig,
             kernels="k_binary_tile<0,float,U=2>")
        spec("C3", "Softmax(-1) [16,12,512,512]", 402653184, ne3, lambda i: HIP.Softmax(wT, -1, out=wO), 1, kbig,
             kernels="k_softmax_row1")
        spec("C3", "Add mask + Softmax fused", 402685952, ne3, lambda i: HIP.AddSoftmax(wS, wM, -1, out=wO), 1, kbig,
             kernels="k_softmax_row1 (mask)")

        # C4: int64 / int32 A[64,1,4096] ~ U[-2^20,2^20] op B[1,256,4096] ~ U[1,1024]
        self.c4 = {}
        for dt, es, nm, kb in ((torch.int64, 8, "int64", "k_binary_tile<{},int64,128 lanes>"),
                               (torch.int32, 4, "int32", "k_binary_nd<{},int32>")):
            A4 = torch.randint(-(2**20), 2**20 + 1, (64, 1, 4096), device=dev, dtype=dt, generator=gen)
            B4 = torch.randint(1, 1025, (1, 256, 4096), device=dev, dtype=dt, generator=gen)
            Y4 = torch.empty(64, 256, 4096, device=dev, dtype=dt)
            self.c4[nm] = (A4, B4, Y4)
            wA4, wB4, wY4 = w(A4), w(B4), w(Y4)
            nb = (64 * 4096 + 256 * 4096 + 64 * 256 * 4096) * es
            ne = Y4.numel()
            spec("C4", f"Add {nm}", nb, ne, lambda i, a=wA4, b=wB4, y=wY4: HIP.Add(a, b, out=y), 1, kbig,
                 kernels=kb.format(0))
            spec("C4", f"Mul {nm}", nb, ne, lambda i, a=wA4, b=wB4, y=wY4: HIP.Mul(a, b, out=y), 1, kbig,
                 kernels=kb.format(2))
            # per eager call on the host clock: at least 24 calls between the two synchronisations, so the
            # first launch's latency and the final wait weigh little on the per-call figure
            spec("C4", f"Div {nm} (per eager call: divisor scan + kernel, verdict read back)", nb, ne,
                 lambda i, a=wA4, b=wB4, y=wY4: HIP.Div(a, b, out=y), 1, max(24, steps // 4), timing="eager",
                 kernels="k_div_scan + k_div_rows")
            if nm == "int64":
                self.Yc4 = torch.empty(64, 256, 4096, device=dev, dtype=torch.float32)
                self.Yr4 = torch.empty(64, 1, 4096, device=dev, dtype=dt)
                wYc, wYr = w(self.Yc4), w(self.Yr4)
                HIP.Add(wA4, wB4, out=wY4)
                spec("C4", "Cast int64 -> float32", 805306368, ne, lambda i, y=wY4: HIP.Cast(y, 1, out=wYc), 1, kbig,
                     kernels="k_cast<7,1>")
                spec("C4", "ReduceSum(axis=1) int64", 538968064, ne,
                     lambda i, y=wY4: HIP.ReduceSum(y, [1], 1, out=wYr), 1, kbig, kernels="k_reduce_cols<0,long>")

        # C5: GELU on X[32,2048,3072]; ReduceSum(axis=1) and ReduceMean(all) on Y[256,4096,256]
        self.X5 = torch.randn(*C5_X, device=dev, generator=gen)
        self.G5 = torch.empty_like(self.X5)
        self.Yb = torch.rand(*C5_Y, device=dev, generator=gen) * 2 - 1
        self.R1 = torch.empty(256, 1, 256, device=dev)
        self.R2 = torch.empty(1, 1, 1, device=dev)
        self.wX5, self.wG5, self.wYb, self.wR1, self.wR2 = w(self.X5), w(self.G5), w(self.Yb), w(self.R1), w(self.R2)
        spec("C5", "GELU chain (5 ONNX ops) as one fused kernel", GELU_BYTES, self.X5.numel(), self.gelu, 1, kbig,
             kernels="k_map_tab<GeluOp,4,2>")
        spec("C5", "ReduceSum(axis=1) [256,4096,256] -> [256,1,256]", RSUM_BYTES, self.Yb.numel(), self.rsum, 1, kbig,
             kernels="k_reduce_cols<0,float>")
        spec("C5", "ReduceMean(all) [256,4096,256] -> [1,1,1]", RMEAN_BYTES, self.Yb.numel(), self.rmean, 1, kbig,
             kernels="k_reduce_rows_split + finish")

        # ceilings on the same GPU: the library's copy (Cast float -> float, nontemporal 16-byte vectors) at
        # 1 GiB and at C2's 25 MB over the same 16 sets, and a pure 1 GiB read (lx_read_probe)
        self.Zc = torch.empty_like(self.Yb)
        wZc = w(self.Zc)
        self.probe_out = torch.empty(1 << 16, device=dev, dtype=torch.int32)
        lib = __import__("onnx_amd").lib()
        yb, po = self.Yb.data_ptr(), self.probe_out.data_ptr()
        self.ceilings = [
            ("copy 1 GiB (Cast float->float, nontemporal 16-byte vectors)", 2 * self.Yb.numel() * 4, self.Yb.numel(),
             lambda i: HIP.Cast(self.wYb, 1, out=wZc), 1, kbig),
            # 512 blocks (two per CU): the fastest read shape of a sweep over 256 .. 65536 blocks on MI355X
            ("read 1 GiB (lx_read_probe, nontemporal 16-byte vectors, 4 per lane, 512 blocks)", self.Yb.numel() * 4,
             self.Yb.numel(), lambda i: lib.lx_read_probe(yb, self.Yb.numel() * 4, po, 4 * 512), 1, kbig),
            ("copy 25 MB X -> Y over C2's 16 sets (Cast float->float)", 2 * 8 * 512 * 768 * 4, 8 * 512 * 768,
             lambda i: HIP.Cast(wX[i % LN_SETS], 1, out=wY[i % LN_SETS]), LN_SETS, k2),
        ]

    def gelu(self, i=0):
        return self.HIP.GeluErf(self.wX5, out=self.wG5)

    def rsum(self, i=0):
        return self.HIP.ReduceSum(self.wYb, [1], 1, out=self.wR1)

    def rmean(self, i=0):
        return self.HIP.ReduceMean(self.wYb, None, 1, out=self.wR2)


# ---------------------------------------------------------------------------
# CPU leg: the oracle on bounded samples
# ---------------------------------------------------------------------------
def cpu_ops(c5_target_s=4.0, target_s=1.0):
    """The oracle (C restatement of the reference's CPU algorithm, 1 thread) on a bounded sample of each
    config op, scaled to the full op by element count.  Returns {(config, op): (seconds for the full op,
    sample description)} keyed like Workloads.specs."""
    from oracle import oracle as O
    rng = np.random.default_rng(3)

    def timed(fn, scale, sample, tgt=target_s):
        fn()
        n, t0 = 0, time.perf_counter()
        while True:
            fn()
            n += 1
            el = time.perf_counter() - t0
            if el >= tgt:
                break
        return el / n * scale, f"{sample}, {n} runs in {el:.1f} s, scaled x{scale:g}"

    out = {}
    f32 = np.float32
    A1 = rng.standard_normal((1, 128, 384)).astype(f32)
    B1 = rng.uniform(-0.1, 0.1, 384).astype(f32)
    C1 = O.binary(O.ADD, A1, B1)
    out[("C1", "Add bias [1,128,384]+[384]")] = timed(lambda: O.binary(O.ADD, A1, B1), 1, "full op")
    out[("C1", "Mul scalar 0.125")] = timed(lambda: O.binary(O.MUL, C1, np.array(0.125, f32)), 1, "full op")
    out[("C1", "Add -> Mul fused (one ElementwiseChain kernel, the graph runtime's fusion)")] = timed(
        lambda: O.binary(O.MUL, O.binary(O.ADD, A1, B1), np.array(0.125, f32)), 1, "the 2 ops, full size")
    X = (rng.standard_normal(LN_SHAPE) * 2).astype(f32)
    g = (1 + 0.02 * rng.standard_normal(768)).astype(f32)
    b = (0.02 * rng.standard_normal(768)).astype(f32)
    ln = timed(lambda: O.layernorm_decomposed(X, g, b), 1, "the 9 ops on X[8,512,768]")
    out[("C2", "LayerNorm, 9 ONNX ops as one fused kernel")] = ln
    out[("C2", "LayerNorm as its 9 separate operator calls")] = ln
    S = (rng.standard_normal((1, 12, 512, 512)) * 3).astype(f32)
    M = np.where(rng.uniform(size=(1, 1, 1, 512)) < 0.125, -10000.0, 0.0).astype(f32)
    T = O.binary(O.ADD, S, M)
    out[("C3", "Add mask [16,12,512,512]+[16,1,1,512]")] = timed(lambda: O.binary(O.ADD, S, M), 16,
                                                                   "S[1,12,512,512] + mask[1,1,1,512]")
    out[("C3", "Softmax(-1) [16,12,512,512]")] = timed(lambda: O.softmax(T, -1), 16, "[1,12,512,512]")
    out[("C3", "Add mask + Softmax fused")] = timed(lambda: O.add_softmax(S, M, -1), 16,
                                                     "S[1,12,512,512] + mask, Softmax")
    for dt in (np.int64, np.int32):
        nm = np.dtype(dt).name
        A4 = rng.integers(-(2**20), 2**20 + 1, (4, 1, 4096)).astype(dt)
        B4 = rng.integers(1, 1025, (1, 256, 4096)).astype(dt)
        smp = "A[4,1,4096] op B[1,256,4096], C# semantics (the reference rejects this dtype)"
        if dt == np.int32:
            smp = "A[4,1,4096] op B[1,256,4096]"
        out[("C4", f"Add {nm}")] = timed(lambda: O.binary(O.ADD, A4, B4), 16, smp)
        out[("C4", f"Mul {nm}")] = timed(lambda: O.binary(O.MUL, A4, B4), 16, smp)
        out[("C4", f"Div {nm} (per eager call: divisor scan + kernel, verdict read back)")] = timed(
            lambda: O.binary(O.DIV, A4, B4), 16, smp + (", C# semantics (the reference rejects int32 Div)"
                                                       if dt == np.int32 else ""))
        if dt == np.int64:
            Y4 = O.binary(O.ADD, A4, B4)
            out[("C4", "Cast int64 -> float32")] = timed(lambda: O.cast(Y4, 1), 16, "[4,256,4096] int64")
            out[("C4", "ReduceSum(axis=1) int64")] = timed(lambda: O.reduce(O.RSUM, Y4, [1], True), 16,
                                                          "[4,256,4096] int64, C# semantics (the reference rejects "
                                                          "int64 ReduceSum)")
    X5 = rng.standard_normal((1, 2048, 3072)).astype(f32)
    out[("C5", "GELU chain (5 ONNX ops) as one fused kernel")] = timed(
        lambda: O.gelu_erf(X5), 32, "the 5 ops on X[1,2048,3072]", c5_target_s)
    Yb = rng.uniform(-1, 1, (16, 4096, 256)).astype(f32)
    out[("C5", "ReduceSum(axis=1) [256,4096,256] -> [256,1,256]")] = timed(
        lambda: O.reduce(O.RSUM, Yb, [1], True), 16, "Y[16,4096,256] (transpose, then serial folds)", c5_target_s)
    out[("C5", "ReduceMean(all) [256,4096,256] -> [1,1,1]")] = timed(
        lambda: O.reduce(O.RMEAN, Yb, None, True), 16, "Y[16,4096,256] (one serial float32 fold)", c5_target_s)
    return out


# ---------------------------------------------------------------------------
# HBM traffic: rocprofv3 counter passes over `bench.py --probe`
# ---------------------------------------------------------------------------
HEADLINE_PROBE_STEPS = 3


def run_probe(torch, HIP, DeviceTensor, steps):
    """Child of a rocprofv3 --pmc pass: a copy of known size (the calibration), then each per-config op
    launched twice, then three headline steps (GELU, ReduceSum, ReduceMean in the step's order), every
    segment opened by a marker kernel (Cast uint8 -> int16 of 16 elements)."""
    W = Workloads(torch, HIP, DeviceTensor, steps)
    mk_in = DeviceTensor.from_numpy(np.arange(16, dtype=np.uint8))
    mk_out = DeviceTensor.empty((16,), np.int16)
    src = torch.randn(CALIB_BYTES // 4, device="cuda:0")
    dst = torch.empty_like(src)
    ws, wd = DeviceTensor.wrap_torch(src), DeviceTensor.wrap_torch(dst)
    torch.cuda.synchronize()

    def marker():
        HIP.Cast(mk_in, 5, out=mk_out)
        torch.cuda.synchronize()
    marker()
    HIP.Cast(ws, 1, out=wd)
    torch.cuda.synchronize()
    for sp in W.specs:
        marker()
        for i in range(2):
            sp["fn"](i)
        torch.cuda.synchronize()
    marker()
    for _ in range(HEADLINE_PROBE_STEPS):
        W.gelu()
        W.rsum()
        W.rmean()
    torch.cuda.synchronize()
    marker()
    print("probe done", flush=True)


def parse_counters(path, counter):
    """Per-segment lists of (kernel name, counter value, duration in ns) from a counter_collection.csv,
    segments split at the marker kernel, and the markers' own (value, duration) pairs."""
    rows = []
    with open(path) as f:
        for r in csv.DictReader(f):
            if r["Counter_Name"] != counter:
                continue
            dur = int(r["End_Timestamp"]) - int(r["Start_Timestamp"]) if r.get("End_Timestamp") else 0
            rows.append((int(r["Dispatch_Id"]), r["Kernel_Name"], float(r["Counter_Value"]), dur))
    rows.sort()
    segs, cur, markers = [], None, []
    for _, name, v, dur in rows:
        if MARKER in name:
            markers.append((v, dur))
            if cur is not None:
                segs.append(cur)
            cur = []
            continue
        if cur is not None and "lx::" in name:
            cur.append((name, v, dur))
    # the probe ends with a marker: whatever follows it is not a segment
    return segs, markers


def short(name):
    return name.split("(")[0].replace("void ", "")


XCDS = 8            # MI355X: 256 CUs in 8 XCDs; rocprofv3 sums a GRBM counter over the XCDs
RATED_MHZ = 2400.0  # MI355X peak engine clock (the agent's Max_Engine_Clk_Fcompute)


def clock_of(seg, pred, c0):
    """Shader clock (MHz) of the dispatches in a GRBM_GUI_ACTIVE segment whose name satisfies `pred`: busy
    cycles per XCD, less the `c0` cycles the counter adds to every dispatch outside its timestamps, over
    the dispatches' durations."""
    sel = [(v / XCDS - c0, d) for n, v, d in seg if pred(n)]
    ns = sum(d for _, d in sel)
    return round(sum(c for c, _ in sel) / ns * 1e3, 1) if ns else None


def live_traffic(specs, steps, timeout_s=240):
    """Three rocprofv3 passes over `bench.py --probe`: FETCH_SIZE, WRITE_SIZE and GRBM_GUI_ACTIVE (busy
    cycles, for the shader clock).  Returns ({op index: (fetch bytes, write bytes, kernel names)},
    calibration dict, clock dict) or (None, reason, None)."""
    exe = shutil.which("rocprofv3")
    if not exe:
        return None, "rocprofv3 not found", None
    out = os.path.join(ROOT, "gpurun_out", "bench_counters")
    shutil.rmtree(out, ignore_errors=True)
    os.makedirs(out, exist_ok=True)
    env = dict(os.environ, TMPDIR="/tmp")
    res = {}
    for counter, tag in (("FETCH_SIZE", "f"), ("WRITE_SIZE", "w"), ("GRBM_GUI_ACTIVE", "c")):
        cmd = [exe, "--pmc", counter, "--output-format", "csv", "-d", os.path.join(out, tag), "-o", tag, "--",
               sys.executable, os.path.join(ROOT, "bench.py"), "--probe", "--steps", str(steps)]
        log(f"counter pass {counter}: " + " ".join(cmd))
        with open(os.path.join(out, f"{tag}.log"), "w") as lf:
            p = subprocess.Popen(cmd, cwd="/tmp", env=env, stdout=lf, stderr=subprocess.STDOUT,
                                 start_new_session=True)
            try:
                p.wait(timeout=timeout_s)
            except subprocess.TimeoutExpired:
                os.killpg(p.pid, signal.SIGKILL)
                p.wait()
                return None, f"{counter} pass timed out after {timeout_s} s", None
        done = "probe done" in open(os.path.join(out, f"{tag}.log")).read()
        files = glob.glob(os.path.join(out, tag, "**", "*counter_collection.csv"), recursive=True)
        if not done or not files:
            return None, f"{counter} pass failed (rc {p.returncode})", None
        res[counter], marks = parse_counters(files[0], counter)
        if counter == "GRBM_GUI_ACTIVE":
            # the counter's busy window is longer than the dispatch: a constant per dispatch, measured on the
            # 16-element marker kernels (about 2 us, taken to run at the rated clock, so that c0 errs by
            # at most a few hundred cycles: under 0.5% of a 150 us kernel's clock)
            mc = sorted(v / XCDS for v, _ in marks)
            md = sorted(d for _, d in marks)
            c0 = mc[len(mc) // 2] - RATED_MHZ * 1e-3 * md[len(md) // 2]
        log(f"counter pass {counter}: {len(res[counter])} segments (rc {p.returncode})")
    f, wr, ck = res["FETCH_SIZE"], res["WRITE_SIZE"], res["GRBM_GUI_ACTIVE"]
    nseg = len(specs) + 2
    if len(f) != nseg or len(wr) != nseg or len(ck) != nseg:
        return None, f"segment count {len(f)}/{len(wr)}/{len(ck)} != {nseg}", None
    cf = sum(v for _, v, _ in f[0])
    cw = sum(v for _, v, _ in wr[0])
    calib = {"kernel": short(f[0][0][0]) if f[0] else "?",
             "bytes_read": CALIB_BYTES, "bytes_written": CALIB_BYTES, "FETCH_SIZE_KiB": round(cf, 1),
             "WRITE_SIZE_KiB": round(cw, 1), "fetch_factor": round(CALIB_BYTES / (cf * 1024), 5),
             "write_factor": round(CALIB_BYTES / (cw * 1024), 5)}
    per = {}
    for i in range(len(specs)):
        fs, ws = f[i + 1], wr[i + 1]
        names = sorted({short(n) for n, _, _ in fs})
        per[i] = (sum(v for _, v, _ in fs) / 2 * 1024 * calib["fetch_factor"],
                  sum(v for _, v, _ in ws) / 2 * 1024 * calib["write_factor"], names)
    gi = next(i for i, sp in enumerate(specs) if sp["op"].startswith("GELU"))
    head = ck[-1]
    is_gelu = lambda n: "GeluOp" in n  # noqa: E731
    clock = {"source": "rocprofv3 --pmc GRBM_GUI_ACTIVE over bench.py --probe (the profiler serialises the "
                       f"dispatches): busy cycles / {XCDS} XCDs, less a per-dispatch constant of {round(c0)} "
                       "cycles measured on the marker kernels, / dispatch duration",
             "rated_mhz": RATED_MHZ,
             "calibration_copy_mhz": clock_of(ck[0], lambda n: True, c0),
             "gelu_back_to_back_mhz": clock_of(ck[gi + 1], is_gelu, c0),
             "gelu_in_headline_steps_mhz": clock_of(head, is_gelu, c0),
             "reduce_sum_in_headline_steps_mhz": clock_of(head, lambda n: "reduce_cols" in n, c0),
             "reduce_mean_in_headline_steps_mhz": clock_of(head, lambda n: "reduce_rows_split" in n, c0),
             "gelu_in_headline_steps_us": [round(d / 1e3, 1) for n, v, d in head if is_gelu(n)],
             "gelu_back_to_back_us": [round(d / 1e3, 1) for n, v, d in ck[gi + 1] if is_gelu(n)]}
    return per, calib, clock


def profile_traffic():
    """Fallback: the GELU kernel's traffic from the committed counter summary, or None."""
    path = os.path.join(ROOT, "profiles", "gelu_c5_traffic.txt")
    try:
        for line in open(path):
            if line.startswith("traffic_bytes_per_launch:"):
                return int(float(line.split(":", 1)[1]))
    except OSError:
        pass
    return None


# ---------------------------------------------------------------------------
# extras (--all): graph executor, data movement, a BERT layer, MatMul
# ---------------------------------------------------------------------------
def bench_extras(torch, HIP, DeviceTensor, set_stream, steps, warmup, W):
    dev = torch.device("cuda:0")
    res = []
    gen = torch.Generator(device=dev)
    gen.manual_seed(1)

    def wrap(t):
        return DeviceTensor.wrap_torch(t)

    def record(name, nbytes, elems, ms):
        gbs = nbytes / (ms * 1e-3) / 1e9
        d = {"op": name, "algorithmic_bytes": nbytes, "us": round(ms * 1e3, 3), "GB/s": round(gbs, 1),
             "frac_of_peak": round(gbs / PEAK_HBM_GBS, 4), "elements_per_s": round(elems / (ms * 1e-3), 1)}
        log(json.dumps(d))
        res.append(d)

    def run(name, nbytes, elems, fn, nsets, k=None):
        ms = graph_time(torch, fn, k or steps, warmup, set_stream, reps=5)
        record(name, nbytes, elems, ms)

    from onnx_amd.graph import ComputationalGraph
    n1 = len(W.A1)
    wA, B = W.wA1, W.B1
    # C1 through the graph runtime, host dispatch per execution: 2 nodes, then fused
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
    # C2: the host round trip a caller holding host arrays pays (X uploaded from pageable host memory, the
    # fused kernel, Y read back), then the ONNX subgraph through the device graph runtime
    wX, wY, wg, wb, gam, bet = W.wX2, W.wY2, W.wg, W.wb, W.gam, W.bet
    Xh = [x.cpu().numpy() for x in W.X2[:2]]

    def ln_host(i):
        wX[i % 2].upload(Xh[i % 2])
        HIP.LayerNormDecomposed(wX[i % 2], wg, wb, 1e-12, out=wY[i % 2])
        wY[i % 2].to_numpy()
    record("C2 LayerNorm fused, including upload of X and download of Y (pageable host memory)", LN_BYTES,
           8 * 512 * 768, wall_time(torch, ln_host, max(16, steps // 8), warmup))
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
    # the C5 GELU nodes through the generic elementwise-chain kernel (the fusion used when the constants
    # do not match the GELU pattern)
    k5 = [wrap(torch.tensor(v, device=dev)) for v in (1.4142135381698608, 1.0, 0.5)]
    run("C5 GELU chain as a generic ElementwiseChain", GELU_BYTES, W.X5.numel(),
        lambda i: HIP.ElementwiseChain([W.wX5] + k5, [("Div", 1), ("Erf",), ("Add", 2), ("Mul", 0, True), ("Mul", 3)],
                                       out=W.wG5), 1, k=max(4, steps // 8))

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

    # the whole encoder of the reference's benchmark and model-test model (me5s, multilingual-e5-small: 12
    # layers, hidden 384, 12 heads of 32, FFN 1536; random weights), token ids and attention mask to the last
    # hidden state, batch 8 x 512 tokens
    from bert_layer import encoder_model
    model, eins, _, _ = encoder_model(8, 512, seed=5)
    edev = {k: DeviceTensor.from_numpy(v) for k, v in eins.items()}
    h, ffw, heads, nl = 384, 1536, 12, 12
    enc_flops = nl * (2.0 * 4096 * (4 * h * h + 2 * h * ffw) + 2 * 2.0 * 8 * heads * 512 * 512 * (h // heads))
    for label, capture in (("fused", False), ("fused, captured", True)):
        ge = Model.Load(model)
        ge.Fuse()
        if capture:
            assert ge.Capture(edev), ge.LastError

        def enc_step(i, ge=ge, capture=capture):
            if not (ge.Replay() if capture else ge.Execute(edev)):
                raise RuntimeError(ge.LastError)
        ms = wall_time(torch, enc_step, max(8, steps // 16), max(2, warmup // 4))
        d = {"op": f"me5s-shaped encoder (12 layers, hidden 384) [8,512] tokens, {label} (per execution)",
             "us": round(ms * 1e3, 1), "tokens_per_s": round(4096 / (ms * 1e-3), 1),
             "TFLOP/s": round(enc_flops / (ms * 1e-3) / 1e12, 2), "flops": enc_flops}
        log(json.dumps(d))
        res.append(d)
        ge.close()
    del edev
    # the same encoder at the batch sizes of the reference's me5s run benchmarks (Benchmarks.cs:370-423: 1, 10
    # and 50 strings of 20 characters, 1 and 10 of 200), as b sequences of s tokens, s = 8 and 64 standing for
    # those strings (their exact token counts depend on the tokenizer), one captured execution each
    for b, sq in ((1, 8), (10, 8), (50, 8), (1, 64), (10, 64)):
        model, sins, _, _ = encoder_model(b, sq, seed=5)
        sdev = {k: DeviceTensor.from_numpy(v) for k, v in sins.items()}
        ge = Model.Load(model)
        ge.Fuse()
        assert ge.Capture(sdev), ge.LastError

        def small_step(i, ge=ge):
            if not ge.Replay():
                raise RuntimeError(ge.LastError)
        ms = wall_time(torch, small_step, max(16, steps // 4), max(2, warmup // 4))
        d = {"op": f"me5s-shaped encoder [{b},{sq}] tokens, fused, captured (per execution)",
             "us": round(ms * 1e3, 1), "tokens_per_s": round(b * sq / (ms * 1e-3), 1)}
        log(json.dumps(d))
        res.append(d)
        ge.close()
        del sdev

    # MatMul (row f2): fp32 MFMA, compute-bound; BERT-base shapes at batch 8 x 512 tokens
    for name, sa, sb in (("MatMul fp32 [4096,768]x[768,768] (dense)", (4096, 768), (768, 768)),
                         ("MatMul fp32 [4096,768]x[768,2304] (fused QKV projection)", (4096, 768), (768, 2304)),
                         ("MatMul fp32 [4096,768]x[768,3072] (FFN in)", (4096, 768), (768, 3072)),
                         ("MatMul fp32 [4096,3072]x[3072,768] (FFN out)", (4096, 3072), (3072, 768)),
                         ("MatMul fp32 [16,12,512,64]x[16,12,64,512] (attention scores)", (16, 12, 512, 64),
                          (16, 12, 64, 512)),
                         ("MatMul fp32 [4096,4096]x[4096,4096]", (4096, 4096), (4096, 4096)),
                         # the shapes of the reference's TensorMatMulBenchmarks (Benchmarks.cs:90-160)
                         ("MatMul fp32 [384,384]x[384,384]", (384, 384), (384, 384)),
                         ("MatMul fp32 [384,1536]x[1536,384]", (384, 1536), (1536, 384)),
                         ("MatMul fp32 [6,384,384]x[6,384,384]", (6, 384, 384), (6, 384, 384)),
                         ("MatMul fp32 [3,4,384,384]x[3,4,384,384]", (3, 4, 384, 384), (3, 4, 384, 384))):
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




# ---------------------------------------------------------------------------
def spread(v):
    """min / median / max / mean of a list of per-step times (us), and the means of its first and last
    fifth, which show a drift over the timed region (a clock still ramping, say)."""
    s = sorted(v)
    q = max(1, len(v) // 5)
    return {"min": round(s[0], 2), "median": round(s[len(s) // 2], 2), "max": round(s[-1], 2),
            "mean": round(sum(v) / len(v), 2), "first_fifth_mean": round(sum(v[:q]) / q, 2),
            "last_fifth_mean": round(sum(v[-q:]) / q, 2)}


def headline_c5(torch, W, steps, warmup):
    """K steps of C5 (GELU, ReduceSum(axis 1), ReduceMean(all)) on the launch stream.  A HIP event before
    and after every GELU launch (the roofline kernel) and one after the last step: each event is a queue
    packet that adds about 3.4 us of device time, so the two reductions are timed together, as the rest of
    the step.  Returns (ms per step, {"gelu": ms per launch, "reductions": ms per step}, host wall ms per
    step, {"gelu": [us per step], "reductions": [us per step]})."""
    fns = (W.gelu, W.rsum, W.rmean)
    for _ in range(warmup):
        for f in fns:
            r = f()
            if r.Code:
                raise RuntimeError(r.Message)
    torch.cuda.synchronize()
    ev = [[torch.cuda.Event(enable_timing=True) for _ in range(2)] for _ in range(steps)]
    end = torch.cuda.Event(enable_timing=True)
    t0 = time.perf_counter()
    for s in range(steps):
        ev[s][0].record()
        W.gelu()
        ev[s][1].record()
        W.rsum()
        W.rmean()
    end.record()
    torch.cuda.synchronize()
    wall_ms = (time.perf_counter() - t0) * 1e3
    total = ev[0][0].elapsed_time(end)
    gelu_us = [ev[s][0].elapsed_time(ev[s][1]) * 1e3 for s in range(steps)]
    nxt = [ev[s + 1][0] for s in range(steps - 1)] + [end]
    red_us = [ev[s][1].elapsed_time(nxt[s]) * 1e3 for s in range(steps)]
    return (total / steps, {"gelu": sum(gelu_us) / steps * 1e-3, "reductions": sum(red_us) / steps * 1e-3},
            wall_ms / steps, {"gelu": gelu_us, "reductions": red_us})


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=100)
    ap.add_argument("--warmup", type=int, default=5)
    ap.add_argument("--all", action="store_true", help="also the graph executor, movement, BERT and MatMul lines")
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline leg")
    ap.add_argument("--no-configs", action="store_true", help="headline only (no per_config array)")
    ap.add_argument("--traffic", choices=("live", "profile", "none"), default="live",
                    help="live: two rocprofv3 counter passes over --probe; profile: the committed summary")
    ap.add_argument("--eager", action="store_true", help="time ordinary launches instead of HIP graphs")
    ap.add_argument("--probe", action="store_true", help=argparse.SUPPRESS)
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
    # one dedicated stream for the library's launches and the timing events: torch's default stream is the
    # null stream, for which the library would launch on its own blocking stream, and every event recorded
    # on the null stream would then serialise against it (tens of us between kernels)
    stream = torch.cuda.Stream()
    torch.cuda.set_stream(stream)
    set_stream(stream.cuda_stream)
    if args.probe:
        run_probe(torch, HIP, DeviceTensor, args.steps)
        return

    host = host_info(torch)
    log("host: " + json.dumps(host))
    W = Workloads(torch, HIP, DeviceTensor, args.steps)
    torch.cuda.synchronize()

    # ---- headline: C5 ----
    ms, per, wall, per_step = headline_c5(torch, W, args.steps, args.warmup)
    gbs = C5_STEP_BYTES / (ms * 1e-3) / 1e9
    gelu_gbs = GELU_BYTES / (per["gelu"] * 1e-3) / 1e9
    log(f"C5 step {ms * 1e3:.1f} us ({gbs:.0f} GB/s): GELU {per['gelu'] * 1e3:.1f} us, ReduceSum(axis 1) + "
        f"ReduceMean(all) {per['reductions'] * 1e3:.1f} us; host wall {wall * 1e3:.1f} us/step")
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
        "data": "synthetic, seeded torch generator on the device: X ~ N(0,1), Y ~ U(-1,1) (BASELINE configs[4])",
        "config": {"workload": "C5 large memory-bound sweep: Erf-GELU subgraph (5 ONNX ops, one fused kernel) on "
                               "X[32,2048,3072] f32, ReduceSum(axis=1) and ReduceMean(all) on Y[256,4096,256] f32",
                   "algorithmic_bytes_per_step": C5_STEP_BYTES,
                   "elements_per_s": round((W.X5.numel() + 2 * W.Yb.numel()) / (ms * 1e-3), 1),
                   "per_op_us": {"gelu": round(per["gelu"] * 1e3, 2),
                                 "reduce_sum_axis1 + reduce_mean_all": round(per["reductions"] * 1e3, 2)},
                   "per_step_us": {"gelu": spread(per_step["gelu"]),
                                   "reduce_sum_axis1 + reduce_mean_all": spread(per_step["reductions"])},
                   "per_step_us_list": {"gelu": [round(v, 1) for v in per_step["gelu"]],
                                        "reduce_sum_axis1 + reduce_mean_all": [round(v, 1) for v in per_step["reductions"]]},
                   "timing": "K eager steps on one dedicated stream (the library's launch stream), HIP events "
                             "recorded on it before and after every GELU launch and after the last step"},
        "roofline": {"bound": "hbm", "achieved": round(gelu_gbs, 2), "peak": PEAK_HBM_GBS, "unit": "GB/s",
                     "frac": round(gelu_gbs / PEAK_HBM_GBS, 4), "traffic": None, "kernel": "lx::k_map_tab<lx::GeluOp, 4, 2>",
                     "kernel_us": round(per["gelu"] * 1e3, 2), "algorithmic_bytes_per_launch": GELU_BYTES},
        "host": host,
    }

    # ---- every BASELINE config op ----
    per_config = []
    if not args.no_configs:
        for sp in W.specs:
            if sp["timing"] == "eager":
                ms_op = wall_time(torch, sp["fn"], sp["k"], 8)
            else:
                ms_op = graph_time(torch, sp["fn"], sp["k"], 3, set_stream, reps=5)
            g = sp["algorithmic_bytes"] / (ms_op * 1e-3) / 1e9
            d = {"config": sp["config"], "op": sp["op"], "kernels": sp["kernels"], "us": round(ms_op * 1e3, 2),
                 "GB/s": round(g, 1), "frac": round(g / PEAK_HBM_GBS, 4),
                 "elements_per_s": round(sp["elements"] / (ms_op * 1e-3), 1),
                 "algorithmic_bytes": sp["algorithmic_bytes"],
                 "timing": f"host wall clock per eager call, median of 5 blocks of {sp['k']} calls" if sp["timing"] == "eager" else
                           f"HIP-graph replay of {sp['k']} launches over {sp['sets']} buffer set(s)"}
            log(json.dumps(d))
            per_config.append(d)
        ceil = {}
        for name, nb, ne, fn, sets, k in W.ceilings:
            ms_c = graph_time(torch, fn, k, 3, set_stream, reps=5)
            ceil[name] = {"us": round(ms_c * 1e3, 2), "GB/s": round(nb / (ms_c * 1e-3) / 1e9, 1),
                          "frac": round(nb / (ms_c * 1e-3) / 1e9 / PEAK_HBM_GBS, 4)}
            log(name, json.dumps(ceil[name]))
        out["ceilings"] = ceil

    # ---- HBM traffic per launch (rocprofv3 counters) ----
    if args.traffic == "live":
        torch.cuda.synchronize()
        per_t, calib, clock = live_traffic(W.specs, args.steps)
        if clock is not None:
            out["roofline"]["clock"] = clock
        if per_t is None:
            log(f"live traffic unavailable: {calib}")
            out["roofline"]["traffic"] = profile_traffic()
            out["roofline"]["traffic_source"] = f"committed profile (live pass failed: {calib})"
        else:
            for i, sp in enumerate(W.specs):
                fb, wb_, names = per_t[i]
                if sp["op"].startswith("GELU"):
                    out["roofline"]["traffic"] = int(fb + wb_)
                    out["roofline"]["traffic_over_algorithmic"] = round((fb + wb_) / GELU_BYTES, 4)
                if i < len(per_config):
                    per_config[i]["traffic_bytes"] = int(fb + wb_)
                    per_config[i]["traffic_over_algorithmic"] = round((fb + wb_) / sp["algorithmic_bytes"], 4)
                    per_config[i]["fetch_bytes"], per_config[i]["write_bytes"] = int(fb), int(wb_)
                    per_config[i]["kernel_names"] = names
            out["roofline"]["traffic_source"] = ("live: rocprofv3 --pmc FETCH_SIZE / WRITE_SIZE passes over "
                                                 "bench.py --probe, scaled by a 256 MiB copy")
            out["traffic_calibration"] = calib
    elif args.traffic == "profile":
        out["roofline"]["traffic"] = profile_traffic()
        out["roofline"]["traffic_source"] = "committed profile"

    # ---- CPU legs ----
    if not args.no_cpu:
        cpu = cpu_ops()
        for d in per_config:
            c = cpu.get((d["config"], d["op"]))
            if c is None:
                continue
            sec, sample = c
            d["cpu_baseline"] = {"us": round(sec * 1e6, 1), "elements_per_s": round(d["elements_per_s"] * d["us"] * 1e-6 / sec, 1),
                                 "GB/s": round(d["algorithmic_bytes"] / sec / 1e9, 4), "cores": 1, "kind": "port",
                                 "sample": sample}
            d["gpu_speedup"] = round(sec * 1e6 / d["us"], 1)
        c5 = [cpu[("C5", sp["op"])] for sp in W.specs if sp["config"] == "C5"]
        sec = sum(c[0] for c in c5)
        out["cpu_baseline"] = {"value": round(C5_STEP_BYTES / sec / 1e9, 4), "unit": "GB/s", "cores": 1, "kind": "port",
                               "sample": "oracle (C restatement of the reference's CPU algorithm, 1 thread) on 1/32 of "
                                         "X (GELU, 5 ops) and 1/16 of Y (ReduceSum axis 1 by transpose + serial folds, "
                                         "ReduceMean by one serial fold), about 4 s each, scaled to the full step: "
                                         f"{sec:.2f} s per step",
                               "host_cores_total": host["host_cores_total"], "host_cpu": host["host_cpu"]}
    out["per_config"] = per_config

    if args.all:
        res = bench_extras(torch, HIP, DeviceTensor, set_stream, args.steps, args.warmup, W)
        os.makedirs(os.path.join(ROOT, "gpurun_out"), exist_ok=True)
        with open(os.path.join(ROOT, "gpurun_out", "bench_configs.json"), "w") as f:
            json.dump(per_config + res, f, indent=1)
    print(json.dumps(out), flush=True)


if __name__ == "__main__":
    main()
