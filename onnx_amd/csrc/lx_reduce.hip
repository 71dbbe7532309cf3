// lx_reduce.hip -- gfx950 reductions (ReduceSum / ReduceMean / ReduceMax) and
// the fused LayerNorm subgraph.
//
// Replaces the C# reductions (TensorOps.cs:1561-1891), which transpose the
// tensor so that the reduced axes are innermost (Transpose, 1358-1407) and then
// fold each slice serially.  Here the tensor is read in place as
// [outer, r, inner]:
//   inner == 1 : one wave64 per row (butterfly reduce), or a split of long rows
//                over many blocks followed by a finishing pass;
//   inner  > 1 : column tiles coalesced along inner, row slices combined in
//                LDS, optional split of r over blocks plus a finishing pass.
// Every combination order is fixed, so results are run-to-run deterministic.
// Integer sums wrap (two's complement); ReduceMax keeps the reference's seed
// of 0 (TensorOps.cs:1820): max(0, max_j x_j), NaN elements never win.
#include <type_traits>

#include "lx_device.h"
#include "lx_kernels.h"

#pragma clang fp contract(off)

namespace lx {

constexpr int kRBlock = 256;

template <typename T> struct AccOf { using A = T; };
template <> struct AccOf<int32_t> { using A = uint32_t; };
template <> struct AccOf<int64_t> { using A = uint64_t; };

template <int OP, typename T>
struct Red {
    using A = typename AccOf<T>::A;
    __device__ __forceinline__ static A ident() { return A(0); }
    // ReduceMean for int32 / int64 / double divides each element by R first
    // (TensorOps.cs:1723-1724, 1777-1778).
    __device__ __forceinline__ static A load(T x, int pre, int64_t R) {
        if constexpr (OP == kMean && !std::is_same<T, float>::value) {
            if (pre) {
                if constexpr (std::is_same<T, double>::value) return x / (double)R;
                else if constexpr (std::is_same<T, int32_t>::value) return (A)(x / (int32_t)R);
                else return (A)(x / R);
            }
        }
        return (A)x;
    }
    __device__ __forceinline__ static A comb(A a, A b) {
        if constexpr (OP == kMax) return b > a ? b : a;
        else return a + b;
    }
    // ReduceMean float: sum, then divide by (float)R (TensorOps.cs:1747-1751).
    __device__ __forceinline__ static T fin(A a, int post, int64_t R) {
        if constexpr (OP == kMean && std::is_same<T, float>::value) {
            if (post) return a / (float)R;
        }
        return (T)a;
    }
};

template <int OP, typename T>
__device__ __forceinline__ typename Red<OP, T>::A block_reduce(typename Red<OP, T>::A v) {
    using R = Red<OP, T>;
    using A = typename R::A;
    __shared__ A part[kRBlock / 64];
    v = wave_reduce(v, [](A x, A y) { return R::comb(x, y); });
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
    if (lane == 0) part[wave] = v;
    __syncthreads();
    A t = R::ident();
    if (threadIdx.x == 0) {
        t = part[0];
#pragma unroll
        for (int w = 1; w < kRBlock / 64; w++) t = R::comb(t, part[w]);
    }
    return t;  // valid in thread 0
}

// A row of r elements starting at element s0 of a 16-byte aligned x, read with whole aligned vectors: its
// head (the (-s0) mod V elements before the first 16-byte boundary), nv vectors, and its tail (the fewer
// than V elements after them).  Rows whose length is a multiple of V start aligned (head and tail empty).
template <int V>
__device__ __forceinline__ int64_t row_head(int64_t s0, int64_t r) {
    const int64_t h = (V - (s0 & (V - 1))) & (V - 1);
    return h < r ? h : r;
}

// inner == 1, one wave per row.
template <int OP, typename T, int V>
__global__ __launch_bounds__(kRBlock) void k_reduce_rows_wave(const T *__restrict__ x, T *__restrict__ y, int64_t rows,
                                                              int64_t r, int pre, int post, int64_t R) {
    using RD = Red<OP, T>;
    using A = typename RD::A;
    const int lane = threadIdx.x & 63;
    // the wave's index from lane 0: the row's address arithmetic runs once per wave on the scalar unit
    const int64_t row = (int64_t)blockIdx.x * (kRBlock / 64) + __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    if (row >= rows) return;
    const int64_t s0 = row * r, head = row_head<V>(s0, r);
    const T *p = x + s0 + head;
    A acc = RD::ident();
    const int64_t nv = (r - head) / V;
    // the head and tail elements (fewer than 2V, lane l < head column l, lane head <= l < ne column nv*V + l),
    // loaded before the vectors so the row costs one memory round trip
    const bool has_e = lane < r - nv * V;
    T xe = T(0);
    if (has_e) xe = x[s0 + (lane < head ? lane : nv * V + lane)];
    int64_t j = lane;
    for (; j + 64 * 3 < nv; j += 64 * 4) {
        Vec<T, V> v0 = vload_nt<T, V>(p + j * V);
        Vec<T, V> v1 = vload_nt<T, V>(p + (j + 64) * V);
        Vec<T, V> v2 = vload_nt<T, V>(p + (j + 128) * V);
        Vec<T, V> v3 = vload_nt<T, V>(p + (j + 192) * V);
#pragma unroll
        for (int k = 0; k < V; k++) acc = RD::comb(acc, RD::load(v0.v[k], pre, R));
#pragma unroll
        for (int k = 0; k < V; k++) acc = RD::comb(acc, RD::load(v1.v[k], pre, R));
#pragma unroll
        for (int k = 0; k < V; k++) acc = RD::comb(acc, RD::load(v2.v[k], pre, R));
#pragma unroll
        for (int k = 0; k < V; k++) acc = RD::comb(acc, RD::load(v3.v[k], pre, R));
    }
    for (; j < nv; j += 64) {
        Vec<T, V> v0 = vload_nt<T, V>(p + j * V);
#pragma unroll
        for (int k = 0; k < V; k++) acc = RD::comb(acc, RD::load(v0.v[k], pre, R));
    }
    if (has_e) acc = RD::comb(acc, RD::load(xe, pre, R));
    acc = wave_reduce(acc, [](A a, A b) { return RD::comb(a, b); });
    if (lane == 0) y[row] = RD::fin(acc, post, R);
}

// inner == 1, short rows (at most 64 whole vectors plus head and tail): L lanes per row (a power of two),
// 64 / L rows per wave at a time, two rows per group in flight; the row split of k_reduce_rows_wave
// within each group of L lanes.
template <int OP, typename T, int V, int L>
__global__ __launch_bounds__(kRBlock) void k_reduce_rows_group(const T *__restrict__ x, T *__restrict__ y,
                                                               int64_t rows, int64_t r, int pre, int post,
                                                               int64_t R) {
    using RD = Red<OP, T>;
    using A = typename RD::A;
    constexpr int RW = 64 / L;
    const int lane = threadIdx.x & 63, gl = lane & (L - 1);
    const int64_t W = (int64_t)gridDim.x * (kRBlock / 64) * RW;
    int64_t row = ((int64_t)blockIdx.x * (kRBlock / 64) + (threadIdx.x >> 6)) * RW + lane / L;
    // one row's whole vector (lane gl < nv) and extra element (gl < r - nv*V) of this lane
    auto load = [&](int64_t rw, Vec<T, V> &v, T &e, bool &hv, bool &he) {
        const int64_t s0 = rw * r, head = row_head<V>(s0, r), nv = (r - head) / V;
        hv = gl < nv;
        he = gl < r - nv * V;
        if (hv) v = vload_nt<T, V>(x + s0 + head + (int64_t)gl * V);
        if (he) e = x[s0 + (gl < head ? gl : nv * V + gl)];
    };
    for (; row < rows; row += 2 * W) {
        const int64_t row2 = row + W;
        Vec<T, V> v0, v1;
        T e0 = T(0), e1 = T(0);
        bool hv0, he0, hv1 = false, he1 = false;
        load(row, v0, e0, hv0, he0);
        if (row2 < rows) load(row2, v1, e1, hv1, he1);
        A a0 = RD::ident(), a1 = RD::ident();
        if (hv0) {
#pragma unroll
            for (int k = 0; k < V; k++) a0 = RD::comb(a0, RD::load(v0.v[k], pre, R));
        }
        if (he0) a0 = RD::comb(a0, RD::load(e0, pre, R));
        if (hv1) {
#pragma unroll
            for (int k = 0; k < V; k++) a1 = RD::comb(a1, RD::load(v1.v[k], pre, R));
        }
        if (he1) a1 = RD::comb(a1, RD::load(e1, pre, R));
        a0 = group_reduce<L>(a0, [](A p, A q) { return RD::comb(p, q); });
        a1 = group_reduce<L>(a1, [](A p, A q) { return RD::comb(p, q); });
        if (gl == 0) {
            y[row] = RD::fin(a0, post, R);
            if (row2 < rows) y[row2] = RD::fin(a1, post, R);
        }
    }
}

// inner == 1, long rows: grid (nchunks, rows).  The row is cut into tiles of
// 4 x 256 vectors; block c takes tiles c, c + nchunks, ... and each lane loads
// the 4 vectors t, t+256, t+512, t+768 of a tile together, so at any moment
// the grid streams one contiguous front of the row.
template <int OP, typename T, int V>
__global__ __launch_bounds__(kRBlock) void k_reduce_rows_split(const T *__restrict__ x,
                                                               typename Red<OP, T>::A *__restrict__ partial,
                                                               T *__restrict__ y, int64_t r, int nchunks, int pre,
                                                               int post, int64_t R) {
    using RD = Red<OP, T>;
    using A = typename RD::A;
    constexpr int64_t kTile = 4 * kRBlock;
    const int64_t row = blockIdx.y;
    const int c = blockIdx.x;
    const int64_t s0 = row * r, head = row_head<V>(s0, r);
    const T *p = x + s0 + head;
    const int64_t nv = (r - head) / V;
    const int64_t step = (int64_t)nchunks * kTile;
    // one accumulator per vector component: V independent chains of four combines per tile instead of one
    // chain of 4 V, so the adds of a tile finish before the next tile's loads return
    A accv[V];
#pragma unroll
    for (int k = 0; k < V; k++) accv[k] = RD::ident();
    int64_t j = (int64_t)c * kTile + threadIdx.x;
    for (; j + 3 * kRBlock < nv; j += step) {
        Vec<T, V> a0 = vload_nt<T, V>(p + j * V);
        Vec<T, V> a1 = vload_nt<T, V>(p + (j + kRBlock) * V);
        Vec<T, V> a2 = vload_nt<T, V>(p + (j + 2 * kRBlock) * V);
        Vec<T, V> a3 = vload_nt<T, V>(p + (j + 3 * kRBlock) * V);
#pragma unroll
        for (int k = 0; k < V; k++) {
            accv[k] = RD::comb(accv[k], RD::load(a0.v[k], pre, R));
            accv[k] = RD::comb(accv[k], RD::load(a1.v[k], pre, R));
            accv[k] = RD::comb(accv[k], RD::load(a2.v[k], pre, R));
            accv[k] = RD::comb(accv[k], RD::load(a3.v[k], pre, R));
        }
    }
    // the partial tile at the end of the row (j points into it for one block)
    for (; j < nv; j += kRBlock) {
        Vec<T, V> a0 = vload_nt<T, V>(p + j * V);
#pragma unroll
        for (int k = 0; k < V; k++) accv[k] = RD::comb(accv[k], RD::load(a0.v[k], pre, R));
    }
    A acc = accv[0];
#pragma unroll
    for (int k = 1; k < V; k++) acc = RD::comb(acc, accv[k]);
    // block 0 takes the head and the tail elements (fewer than 2V): lane l < head column l, lane
    // head <= l < ne column nv*V + l
    if (c == 0 && threadIdx.x < r - nv * V) acc = RD::comb(acc, RD::load(x[s0 + (threadIdx.x < head ? threadIdx.x : nv * V + threadIdx.x)], pre, R));
    acc = block_reduce<OP, T>(acc);
    if (nchunks == 1) {
        if (threadIdx.x == 0) y[row] = RD::fin(acc, post, R);
        return;
    }
    if (threadIdx.x == 0) partial[row * nchunks + c] = acc;
}

// Finishing pass of the split row reduction: one block per row folds the
// row's partials (each lane a fixed stride of them, then the block tree).
// One wave per row folds the row's partials: each lane loads kFinishPer of them at once (one memory
// round trip for up to 64 * kFinishPer partials), folds them in chunk order, and the wave combines the
// lanes.  A 256-lane block whose lanes loaded their partials one dependent load at a time and combined
// the waves through LDS made the C5 ReduceMean (512 partials) up to 0.8 us slower.
constexpr int kFinishPer = 8;
template <int OP, typename T>
__global__ __launch_bounds__(64) void k_reduce_rows_finish(const typename Red<OP, T>::A *__restrict__ partial,
                                                           T *__restrict__ y, int nchunks, int post, int64_t R) {
    using RD = Red<OP, T>;
    using A = typename RD::A;
    const int64_t row = blockIdx.x;
    const A *p = partial + row * nchunks;
    const int lane = threadIdx.x;
    A t = RD::ident();
    for (int q0 = 0; q0 < nchunks; q0 += 64 * kFinishPer) {
        A v[kFinishPer];
#pragma unroll
        for (int u = 0; u < kFinishPer; u++) {
            const int q = q0 + u * 64 + lane;
            v[u] = q < nchunks ? p[q] : RD::ident();
        }
#pragma unroll
        for (int u = 0; u < kFinishPer; u++) t = RD::comb(t, v[u]);
    }
    t = wave_reduce(t, [](A a, A b) { return RD::comb(a, b); });
    if (lane == 0) y[row] = RD::fin(t, post, R);
}

// inner > 1: grid (column tiles * outer, rsplit).  ct lanes cover ct column
// vectors; 256/ct row slices.  Rows are taken in groups of nrs consecutive
// rows, group g going to split g % rsplit, so the splits sweep the slab
// together.  Slices are combined in LDS; with rsplit > 1 each split writes a
// partial and k_reduce_cols_finish folds them in split order.  UN: row vectors
// each lane loads before folding them (in row order, so the fold is the same
// for every UN).
template <int OP, typename T, int V, int UN, int B>
__global__ __launch_bounds__(B) void k_reduce_cols(const T *__restrict__ x,
                                                         typename Red<OP, T>::A *__restrict__ partial,
                                                         T *__restrict__ y, int64_t outer, int64_t r, int64_t inner,
                                                         int ct, int rsplit, int pre, int post, int64_t R) {
    using RD = Red<OP, T>;
    using A = typename RD::A;
    __shared__ A sm[B * V];
    const int t = threadIdx.x;
    const int cvt = t % ct, rs = t / ct, nrs = B / ct;
    const int64_t inner_v = inner / V;
    const int64_t tiles = (inner_v + ct - 1) / ct;
    const int64_t o = (int64_t)blockIdx.x / tiles;
    const int64_t tile = (int64_t)blockIdx.x - o * tiles;
    const int64_t cv = tile * ct + cvt;
    const int s = blockIdx.y;
    const int64_t G = (int64_t)nrs * rsplit;  // row stride between this split's groups
    A acc[V];
#pragma unroll
    for (int k = 0; k < V; k++) acc[k] = RD::ident();
    if (cv < inner_v) {
        const T *p = x + (o * r) * inner + cv * V;
        int64_t j = (int64_t)s * nrs + rs;
        for (; j + (UN - 1) * G < r; j += UN * G) {
            Vec<T, V> a[UN];
#pragma unroll
            for (int u = 0; u < UN; u++) a[u] = vload_nt<T, V>(p + (j + u * G) * inner);
#pragma unroll
            for (int u = 0; u < UN; u++) {
#pragma unroll
                for (int k = 0; k < V; k++) acc[k] = RD::comb(acc[k], RD::load(a[u].v[k], pre, R));
            }
        }
        for (; j < r; j += G) {
            Vec<T, V> a0 = vload_nt<T, V>(p + j * inner);
#pragma unroll
            for (int k = 0; k < V; k++) acc[k] = RD::comb(acc[k], RD::load(a0.v[k], pre, R));
        }
    }
#pragma unroll
    for (int k = 0; k < V; k++) sm[(rs * ct + cvt) * V + k] = acc[k];
    __syncthreads();
    A tot[V];
    if (rs == 0) {
#pragma unroll
        for (int k = 0; k < V; k++) tot[k] = sm[cvt * V + k];
        for (int q = 1; q < nrs; q++) {
#pragma unroll
            for (int k = 0; k < V; k++) tot[k] = RD::comb(tot[k], sm[(q * ct + cvt) * V + k]);
        }
    }
    const int64_t out = o * inner + cv * V;
    if (rsplit == 1) {
        if (rs == 0 && cv < inner_v) {
#pragma unroll
            for (int k = 0; k < V; k++) y[out + k] = RD::fin(tot[k], post, R);
        }
        return;
    }
    if (rs == 0 && cv < inner_v) {
#pragma unroll
        for (int k = 0; k < V; k++) partial[(int64_t)s * outer * inner + out + k] = tot[k];
    }
}

template <int OP, typename T>
__global__ __launch_bounds__(kRBlock) void k_reduce_cols_finish(const typename Red<OP, T>::A *__restrict__ partial,
                                                                T *__restrict__ y, int64_t nout, int rsplit, int post,
                                                                int64_t R) {
    using RD = Red<OP, T>;
    using A = typename RD::A;
    for (int64_t i = (int64_t)blockIdx.x * kRBlock + threadIdx.x; i < nout; i += (int64_t)gridDim.x * kRBlock) {
        A acc = partial[i];
        for (int q = 1; q < rsplit; q++) acc = RD::comb(acc, partial[(int64_t)q * nout + i]);
        y[i] = RD::fin(acc, post, R);
    }
}

// ---------------------------------------------------------------------------
// Host-side planning of one reduction pass.
// ---------------------------------------------------------------------------
static int64_t ceil_div(int64_t a, int64_t b) { return (a + b - 1) / b; }

struct RedPlan {
    int kind;  // 0 wave rows, 1 split rows, 2 cols
    int nchunks;
    int ct;
    int rsplit;
    int block;   // cols: lanes per block (256 or 512)
    int64_t ws;  // partial bytes
};

static constexpr int64_t kTargetBlocks = 2048;
// a column reduction with fewer blocks than this splits its rows into slices (up to kTargetBlocks blocks in
// all, folded by a second launch); each lane keeps kColsUnroll row vectors in flight.  C5's [256,4096,256]
// axis 1 has 512 blocks: unsplit with eight vectors in flight it reads at 7.0 TB/s in one launch (152.8 us),
// against 155.2 us for four slices, four vectors and the folding launch (sixteen vectors: 236 us, the
// registers no longer fit)
static constexpr int64_t kColsSplitBelow = 512;
static constexpr int kColsUnroll = 8;
// blocks over all rows of a split row reduction: 512 (two per CU) read a 1 GiB row at 7.1 TB/s on MI355X,
// against 6.9 with 1024 and 6.8 with 2048; the finishing pass stays a separate launch (a last-block finish
// inside this launch, one device-scope release fence per block, took 20 us longer)
static constexpr int64_t kSplitRowBlocks = 512;

template <typename A>
static RedPlan plan_reduce(int64_t outer, int64_t r, int64_t inner, int V) {
    RedPlan p{};
    if (inner == 1) {
        const int64_t rows = outer;
        if (r <= 8192 || rows >= kTargetBlocks) {
            p.kind = 0;
            return p;
        }
        int64_t nch = ceil_div(kSplitRowBlocks, rows);
        int64_t maxch = ceil_div(r / V, (int64_t)kRBlock * 4);  // >= 4 vectors per lane
        if (nch > maxch) nch = maxch;
        if (nch < 1) nch = 1;
        p.kind = 1;
        p.nchunks = (int)nch;
        p.ws = nch > 1 ? rows * nch * (int64_t)sizeof(A) : 0;
        return p;
    }
    const int64_t inner_v = inner / V > 0 ? inner / V : 1;
    // at most 512 bytes of a row per tile: 32 column vectors of 16 bytes, so a wave covers two rows (C4's
    // int64 [64,256,4096] axis 1: 96 -> 82 us against 64-wide tiles; 16-wide tiles slow C5).  Rows of at most
    // 64 vectors (1 KB) are taken whole by one tile: C5's float [256,4096,256] 155.8 -> 150.7 us and int32 of
    // the same shape 155.8 -> 150.8 us against two 512-byte tiles, unsplit although that leaves one block per
    // CU.  Single elements (an inner axis that is not a multiple of the vector width): 1 KB of a row per tile,
    // 256 floats ([4128,255,255] axis 1: 271 us with 128-float tiles, 217)
    const bool whole = V > 1 && inner_v <= 64;
    const int ct_max = V == 1 ? 1024 / (int)sizeof(A) : whole ? 64 : 512 / (V * (int)sizeof(A));
    int ct = 1;
    while (ct < ct_max && ct < inner_v) ct <<= 1;
    const int64_t tiles = ceil_div(inner_v, ct);
    const int64_t base = tiles * outer;
    // wide rows (more than 64 vectors) over 256 or more reduced rows: 512-lane blocks, sixteen row slices
    // per tile (C4 int64 82.6 -> 80.0 us, int32 [32,512,8192] 82.5 -> 80.8 us, float [64,1024,1024] 40.8 ->
    // 40.2 us; over 64 reduced rows they were 31% slower)
    p.block = (!whole && V > 1 && r >= 256) ? 512 : kRBlock;
    const int nrs = p.block / ct;
    int64_t rsplit = 1;
    if (base < (whole ? 256 : kColsSplitBelow)) {
        rsplit = ceil_div(kTargetBlocks, base);
        int64_t maxs = ceil_div(r, (int64_t)nrs * 16);  // >= 16 rows per slice
        if (rsplit > maxs) rsplit = maxs;
        if (rsplit > 65535) rsplit = 65535;
        // the partials of every split stay within kReducePartialBytes (a slice fewer at most: [255,1024,256]
        // axis 1 takes 8 slices instead of 9), the bound the allocation-free entry point's scratch relies on
        const int64_t cap = kReducePartialBytes / (outer * inner * (int64_t)sizeof(A));
        if (rsplit > cap) rsplit = cap;
        if (rsplit < 1) rsplit = 1;
    }
    p.kind = 2;
    p.ct = ct;
    p.rsplit = (int)rsplit;
    p.ws = rsplit > 1 ? rsplit * outer * inner * (int64_t)sizeof(A) : 0;
    return p;
}

template <int OP, typename T, int V>
static hipError_t reduce_typed_v(const ReduceArgs &a, hipStream_t s) {
    using A = typename Red<OP, T>::A;
    const T *x = (const T *)a.x;
    T *y = (T *)a.y;
    RedPlan p = plan_reduce<A>(a.outer, a.r, a.inner, V);
    if (p.ws > a.ws_bytes) return hipErrorInvalidValue;
    A *ws = (A *)a.workspace;
    if (p.kind == 0) {
        // short rows: L lanes per row, enough for its whole vectors and its head and tail elements (none
        // when r is a multiple of V: every row then starts aligned)
        const int64_t ne_max = a.r % V == 0 ? 0 : (a.r < 2 * V - 2 ? a.r : 2 * V - 2);
        int L = 1;
        while (L < a.r / V || L < ne_max) L <<= 1;
        if (L <= 64) {
            const int64_t per_block = (int64_t)(kRBlock / 64) * (64 / L) * 2;
            int64_t g = ceil_div(a.outer, per_block);
            if (g > (1 << 20)) g = 1 << 20;
#define LX_RG_CASE(N)                                                                                           \
    case N:                                                                                                     \
        hipLaunchKernelGGL((k_reduce_rows_group<OP, T, V, N>), dim3((unsigned)g), dim3(kRBlock), 0, s, x, y, a.outer, \
                           a.r, a.pre_div, a.post_div, a.r_total);                                              \
        break;
            switch (L) {
                LX_RG_CASE(1) LX_RG_CASE(2) LX_RG_CASE(4) LX_RG_CASE(8) LX_RG_CASE(16) LX_RG_CASE(32) LX_RG_CASE(64)
            default: return hipErrorInvalidValue;
            }
#undef LX_RG_CASE
            return hipGetLastError();
        }
        int g = (int)ceil_div(a.outer, kRBlock / 64);
        hipLaunchKernelGGL((k_reduce_rows_wave<OP, T, V>), dim3(g), dim3(kRBlock), 0, s, x, y, a.outer, a.r,
                           a.pre_div, a.post_div, a.r_total);
    } else if (p.kind == 1) {
        hipLaunchKernelGGL((k_reduce_rows_split<OP, T, V>), dim3(p.nchunks, (unsigned)a.outer), dim3(kRBlock), 0, s, x,
                           ws, y, a.r, p.nchunks, a.pre_div, a.post_div, a.r_total);
        if (p.nchunks > 1)
            hipLaunchKernelGGL((k_reduce_rows_finish<OP, T>), dim3((unsigned)a.outer), dim3(64), 0, s, ws, y,
                               p.nchunks, a.post_div, a.r_total);
    } else {
        const int64_t tiles = ceil_div(a.inner / V, p.ct);
        // the same bytes in flight per lane for every vector width: 8 rows of 16-byte vectors, 32 of floats
        constexpr int UN = kColsUnroll * VecWidth<T>::value / V;
        if (p.block == 512)
            hipLaunchKernelGGL((k_reduce_cols<OP, T, V, UN, 512>), dim3((unsigned)(tiles * a.outer), (unsigned)p.rsplit),
                               dim3(512), 0, s, x, ws, y, a.outer, a.r, a.inner, p.ct, p.rsplit, a.pre_div,
                               a.post_div, a.r_total);
        else
            hipLaunchKernelGGL((k_reduce_cols<OP, T, V, UN, kRBlock>), dim3((unsigned)(tiles * a.outer), (unsigned)p.rsplit),
                               dim3(kRBlock), 0, s, x, ws, y, a.outer, a.r, a.inner, p.ct, p.rsplit, a.pre_div,
                               a.post_div, a.r_total);
        if (p.rsplit > 1) {
            const int64_t nout = a.outer * a.inner;
            int64_t g = ceil_div(nout, kRBlock);
            if (g > 8192) g = 8192;
            hipLaunchKernelGGL((k_reduce_cols_finish<OP, T>), dim3((unsigned)g), dim3(kRBlock), 0, s, ws, y, nout,
                               p.rsplit, a.post_div, a.r_total);
        }
    }
    return hipGetLastError();
}

template <int OP, typename T>
static hipError_t reduce_typed(const ReduceArgs &a, hipStream_t s) {
    if (a.vec > 1) return reduce_typed_v<OP, T, VecWidth<T>::value>(a, s);
    return reduce_typed_v<OP, T, 1>(a, s);
}

template <typename T>
static hipError_t reduce_by_op(const ReduceArgs &a, hipStream_t s) {
    switch (a.op) {
    case kSum: return reduce_typed<kSum, T>(a, s);
    case kMean: return reduce_typed<kMean, T>(a, s);
    case kMax:
        if constexpr (std::is_floating_point<T>::value) return reduce_typed<kMax, T>(a, s);
        return hipErrorInvalidValue;
    default: return hipErrorInvalidValue;
    }
}

hipError_t launch_reduce(const ReduceArgs &a, hipStream_t s) {
    if (a.outer * a.inner == 0) return hipSuccess;
    if (a.inner > 1 && a.outer * ((a.inner + 63) / 64) > 0x7fffffffll) return hipErrorInvalidValue;  // grid.x limit
    switch (a.dtype) {
    case kFloat: return reduce_by_op<float>(a, s);
    case kDouble: return reduce_by_op<double>(a, s);
    case kInt32: return reduce_by_op<int32_t>(a, s);
    case kInt64: return reduce_by_op<int64_t>(a, s);
    default: return hipErrorInvalidValue;
    }
}

int64_t reduce_workspace_bytes(int dtype, int64_t outer, int64_t r, int64_t inner, int vec) {
    const int64_t asz = (dtype == kFloat || dtype == kInt32) ? 4 : 8;
    RedPlan p = (asz == 4) ? plan_reduce<float>(outer, r, inner, vec) : plan_reduce<double>(outer, r, inner, vec);
    return p.ws;
}


// ---------------------------------------------------------------------------
// Fused LayerNorm subgraph over rows of length r, one wave per row, the row
// held in registers (NV float4 per lane).  Each ONNX node keeps its float32
// rounding:  mean = sum(x)/(float)r;  d = x - mean;  p = d*d (Pow 2);
// var = sum(p)/(float)r;  ve = var + eps;  sd = sqrtf(ve);  n = d / sd;
// m = n * gamma;  y = m + beta.  Only the two sums run in a different order
// from the reference's serial fold.
// ---------------------------------------------------------------------------
// One row per 64-thread block (4096 blocks for C2): measured 3% faster on
// MI355X than four rows per 256-thread block.  gamma and beta are loaded after
// the reductions: loading them with the row was 15% slower (4.2 against
// 4.9 TB/s on C2), every wave reading the same 6 KB at the same moment.
constexpr int kLnBlock = 64;

// The row sums run over DPP lane moves (wave_reduce_dpp): C2 5.09 -> 5.01 us against the shuffle butterfly.
// The row arithmetic is ln_row_finish (lx_device.h).
template <int NV>
__global__ __launch_bounds__(kLnBlock) void k_layernorm(const float *__restrict__ x, const float *__restrict__ gamma,
                                                       const float *__restrict__ beta, float eps,
                                                       float *__restrict__ y, int64_t rows, int r) {
    const int lane = threadIdx.x & 63;
    const int64_t row = (int64_t)blockIdx.x * (kLnBlock / 64) + (threadIdx.x >> 6);
    if (row >= rows) return;
    const float *p = x + row * (int64_t)r;
    float *q = y + row * (int64_t)r;
    Vec<float, 4> v[NV];
#pragma unroll
    for (int c = 0; c < NV; c++) {
        const int col = (c * 64 + lane) * 4;
        if (col < r) v[c] = vload_nt<float, 4>(p + col);
        else v[c] = Vec<float, 4>{{0.0f, 0.0f, 0.0f, 0.0f}};
    }
    ln_row_finish<NV>(v, r, lane, gamma, beta, eps, q);
}

template <int L>
__device__ __forceinline__ float lanes_sum(float v) {
    if constexpr (L == 64) return wave_reduce_dpp(v, [](float a, float b) { return a + b; });
    else return group_reduce<L>(v, [](float a, float b) { return a + b; });
}

// LayerNorm rows of any length up to 256 NV + 3 and short rows: L lanes per row (64 / L rows per wave at
// a time), the row split into an unaligned head, whole 16-byte vectors and a tail (head and tail one
// element per lane: lane l < head column l, lane head <= l < ne column nv*4 + l), the same node-by-node
// rounding as k_layernorm.  gamma and beta are read by vectors where the row's first whole vector falls
// on a 16-byte boundary of the row (head 0, as every row when r is a multiple of 4), element by element
// otherwise.
template <int NV, int L>
__global__ __launch_bounds__(kRBlock) void k_layernorm_rag(const float *__restrict__ x,
                                                           const float *__restrict__ gamma,
                                                           const float *__restrict__ beta, float eps,
                                                           float *__restrict__ y, int64_t rows, int r) {
    constexpr int RW = 64 / L;
    const int lane = threadIdx.x & 63, gl = lane & (L - 1);
    const int64_t W = (int64_t)gridDim.x * (kRBlock / 64) * RW;
    for (int64_t row = ((int64_t)blockIdx.x * (kRBlock / 64) + (threadIdx.x >> 6)) * RW + lane / L; row < rows;
         row += W) {
        const int64_t s0 = row * (int64_t)r;
        const int head = (int)row_head<4>(s0, r);
        const int nv = (r - head) / 4, ne = r - nv * 4;
        const bool he = gl < ne;
        const int ec = gl < head ? gl : nv * 4 + gl;
        const float *p = x + s0 + head;
        Vec<float, 4> v[NV];
        float e = 0.0f;
#pragma unroll
        for (int c = 0; c < NV; c++)
            if (c * L + gl < nv) v[c] = vload_nt<float, 4>(p + (c * L + gl) * 4);
        if (he) e = x[s0 + ec];
        float s = 0.0f;
#pragma unroll
        for (int c = 0; c < NV; c++)
            if (c * L + gl < nv) s = s + ((v[c].v[0] + v[c].v[1]) + (v[c].v[2] + v[c].v[3]));
        if (he) s = s + e;
        s = lanes_sum<L>(s);
        const float fr = (float)r;
        const float mean = s / fr;
        float s2 = 0.0f;
#pragma unroll
        for (int c = 0; c < NV; c++) {
            if (c * L + gl < nv) {
#pragma unroll
                for (int k = 0; k < 4; k++) v[c].v[k] = v[c].v[k] - mean;
                float p0 = v[c].v[0] * v[c].v[0], p1 = v[c].v[1] * v[c].v[1];
                float p2 = v[c].v[2] * v[c].v[2], p3 = v[c].v[3] * v[c].v[3];
                s2 = s2 + ((p0 + p1) + (p2 + p3));
            }
        }
        if (he) {
            e = e - mean;
            s2 = s2 + e * e;
        }
        s2 = lanes_sum<L>(s2);
        const float var = s2 / fr;
        const float ve = var + eps;
        const float sd = __builtin_sqrtf(ve);
        const float rsd = 1.0f / sd;
        float *q = y + s0 + head;
        const float *ga = gamma + head, *be = beta + head;
#pragma unroll
        for (int c = 0; c < NV; c++) {
            const int vi = c * L + gl;
            if (vi < nv) {
                Vec<float, 4> g, b, o;
                if (head == 0) {
                    g = vload<float, 4>(ga + vi * 4);
                    b = vload<float, 4>(be + vi * 4);
                } else {
#pragma unroll
                    for (int k = 0; k < 4; k++) {
                        g.v[k] = ga[vi * 4 + k];
                        b.v[k] = be[vi * 4 + k];
                    }
                }
#pragma unroll
                for (int k = 0; k < 4; k++) {
                    float nrm = div_by_row_lx(v[c].v[k], sd, rsd);
                    float m = nrm * g.v[k];
                    o.v[k] = m + b.v[k];
                }
                vstore_nt<float, 4>(q + vi * 4, o);
            }
        }
        if (he) {
            float nrm = div_by_row_lx(e, sd, rsd);
            float m = nrm * gamma[ec];
            y[s0 + ec] = m + beta[ec];
        }
    }
}

// Rows of 1 to 4099 elements (whole vectors of at most 16 per lane of a wave, plus head and tail).
bool layernorm_supported(int64_t r) { return r >= 1 && r / 4 <= 1024; }

template <int NV, int L>
static void launch_layernorm_rag(const float *x, const float *gamma, const float *beta, float eps, float *y,
                                 int64_t rows, int r, hipStream_t s) {
    int64_t g = ceil_div(rows, (int64_t)(kRBlock / 64) * (64 / L));
    if (g > (1 << 20)) g = 1 << 20;
    hipLaunchKernelGGL((k_layernorm_rag<NV, L>), dim3((unsigned)g), dim3(kRBlock), 0, s, x, gamma, beta, eps, y, rows,
                       r);
}

hipError_t launch_layernorm(const float *x, const float *gamma, const float *beta, float eps, float *y, int64_t rows,
                            int64_t r, hipStream_t s) {
    if (rows == 0) return hipSuccess;
    if (!layernorm_supported(r)) return hipErrorInvalidValue;
    const int ri = (int)r;
    if (r % 4 != 0 || r < 256) {
        // short rows: L lanes per row; other rows of any length: a wave per row
        const int64_t ne_max = r % 4 == 0 ? 0 : (r < 6 ? r : 6);
        int L = 1;
        while (L < r / 4 || L < ne_max) L <<= 1;
        switch (L) {
        case 1: launch_layernorm_rag<1, 1>(x, gamma, beta, eps, y, rows, ri, s); break;
        case 2: launch_layernorm_rag<1, 2>(x, gamma, beta, eps, y, rows, ri, s); break;
        case 4: launch_layernorm_rag<1, 4>(x, gamma, beta, eps, y, rows, ri, s); break;
        case 8: launch_layernorm_rag<1, 8>(x, gamma, beta, eps, y, rows, ri, s); break;
        case 16: launch_layernorm_rag<1, 16>(x, gamma, beta, eps, y, rows, ri, s); break;
        case 32: launch_layernorm_rag<1, 32>(x, gamma, beta, eps, y, rows, ri, s); break;
        default: {
            const int nvw = (int)ceil_div(r / 4, 64);
            switch (nvw) {
            case 1: launch_layernorm_rag<1, 64>(x, gamma, beta, eps, y, rows, ri, s); break;
            case 2: launch_layernorm_rag<2, 64>(x, gamma, beta, eps, y, rows, ri, s); break;
            case 3: case 4: launch_layernorm_rag<4, 64>(x, gamma, beta, eps, y, rows, ri, s); break;
            case 5: case 6: case 7: case 8: launch_layernorm_rag<8, 64>(x, gamma, beta, eps, y, rows, ri, s); break;
            default: launch_layernorm_rag<16, 64>(x, gamma, beta, eps, y, rows, ri, s); break;
            }
        }
        }
        return hipGetLastError();
    }
    const int nv = (int)ceil_div(r, 256);
    const int g = (int)ceil_div(rows, kLnBlock / 64);
#define LX_LN_CASE(N) \
    case N: hipLaunchKernelGGL((k_layernorm<N>), dim3(g), dim3(kLnBlock), 0, s, x, gamma, beta, eps, y, rows, ri); break;
    switch (nv) {
        LX_LN_CASE(1) LX_LN_CASE(2) LX_LN_CASE(3) LX_LN_CASE(4) LX_LN_CASE(5) LX_LN_CASE(6) LX_LN_CASE(7) LX_LN_CASE(8)
        LX_LN_CASE(9) LX_LN_CASE(10) LX_LN_CASE(11) LX_LN_CASE(12) LX_LN_CASE(13) LX_LN_CASE(14) LX_LN_CASE(15)
        LX_LN_CASE(16)
    default: return hipErrorInvalidValue;
    }
#undef LX_LN_CASE
    return hipGetLastError();
}

}  // namespace lx
