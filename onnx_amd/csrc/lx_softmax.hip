// lx_softmax.hip -- gfx950 Softmax, optionally fused with a broadcast additive
// mask (the Add node that precedes attention softmax).
//
// Reference composite (TensorOps.cs:1312-1330), five passes and three
// temporaries on the CPU:
//   m = ReduceMax(x, axis) (seed 0)   d = x - m   e = MathF.Exp(d)
//   s = ReduceSum(e, axis)            y = e / s   (true division)
// Here: one wave64 per row with the row in registers (rows up to 2048 floats),
// or one block per row with the row in registers (up to 65536 floats), x read
// once and y written once; rows of any length with 16-byte accesses (an
// unaligned head and a tail held one element per lane).  The exponential is
// bit-identical to the host expf (expf_lx), the sums run over lane moves.
// Only the order of the sum differs from the reference.  Other shapes (axis
// not innermost, longer rows, unaligned storage) take three-pass kernels.
#include <algorithm>
#include <type_traits>

#include "lx_device.h"
#include "lx_kernels.h"

#pragma clang fp contract(off)

namespace lx {

constexpr int kSBlock = 256;
constexpr int64_t kSoftmaxMaxBlocks = 16384;  // 65536 waves; each loops over its share of rows

// argument x - max is <= 0 (or NaN): the early-out-free expf applies
template <typename T>
__device__ __forceinline__ T exp_elem(T d, const ExpTable &tab) {
    if constexpr (std::is_same<T, float>::value) return expf_nonpos_lx(d, tab);
    else return ::exp(d);
}

// x / sv for a power of two sv whose reciprocal is a normal number equals x * (1 / sv) for every x:
// both are the correctly rounded value of the same real number.  Returns whether sv is such a
// power of two, and its exact reciprocal.
__device__ __forceinline__ bool exact_pow2_recip(float sv, float *r) {
    const uint32_t b = __builtin_bit_cast(uint32_t, sv), e = (b >> 23) & 0xffu;
    if ((b & 0x7fffffu) != 0 || e < 1 || e > 253) return false;
    *r = __builtin_bit_cast(float, (b & 0x80000000u) | ((254u - e) << 23));
    return true;
}
__device__ __forceinline__ bool exact_pow2_recip(double sv, double *r) {
    const uint64_t b = __builtin_bit_cast(uint64_t, sv), e = (b >> 52) & 0x7ffu;
    if ((b & 0xfffffffffffffull) != 0 || e < 1 || e > 2045) return false;
    *r = __builtin_bit_cast(double, (b & 0x8000000000000000ull) | ((2046ull - e) << 52));
    return true;
}

// the row's max / sum across the wave: DPP lane moves for float (kSoftmaxDpp), the shuffle butterfly otherwise
constexpr bool kSoftmaxDpp = true;
template <typename T, typename F>
__device__ __forceinline__ T row_reduce(T v, F f) {
    if constexpr (std::is_same<T, float>::value && kSoftmaxDpp) return wave_reduce_dpp(v, f);
    else return wave_reduce(v, f);
}

// ReduceMax's step with the seed-0 accumulator (TensorOps.cs:1820-1827): keep m unless v > m.  For float
// the IEEE maxNum instruction gives the same Softmax: a quiet NaN v never wins either way, a signalling
// NaN may win the max but then its row is NaN throughout in both cases (its exponential enters the sum),
// and the sign of a zero maximum is invisible in x - max.
template <typename T>
__device__ __forceinline__ T row_max(T m, T v) {
    if constexpr (std::is_same<T, float>::value) return __builtin_fmaxf(m, v);
    else return v > m ? v : m;
}

template <typename T>
__device__ __forceinline__ T div_row(T e, T s, T rs) {
    if constexpr (std::is_same<T, float>::value) return div_by_row_lx(e, s, rs);
    else return e / s;
}

// Mask row offset: the row index decomposed over the mask's row axes
// (innermost first).  NOUT >= 0 is the compile-time axis count, -1 = runtime.
template <int NOUT>
__device__ __forceinline__ int64_t mask_row_offset(uint32_t row, const NdLayout &L) {
    int64_t off = 0;
    if constexpr (NOUT >= 0) {
#pragma unroll
        for (int d = 0; d < NOUT; d++) {
            uint32_t q = fdiv(row, L.odiv[d]);
            off += (int64_t)(row - q * L.odiv[d].d) * L.a_str[d];
            row = q;
        }
    } else {
        for (int d = 0; d < L.nouter; d++) {
            uint32_t q = fdiv(row, L.odiv[d]);
            off += (int64_t)(row - q * L.odiv[d].d) * L.a_str[d];
            row = q;
        }
    }
    return off;
}

// Loads one row's vectors (and, with a mask, the mask vectors it adds): the
// mask loads go first so that a wave waiting for them never waits for loads
// issued after them.
template <typename T, int V, int NV, int NOUT, bool FULL>
__device__ __forceinline__ void softmax_row_load(const T *__restrict__ x, int64_t row, int r, int lane,
                                                 const T *__restrict__ mask, int mask_inner, const NdLayout &mrows,
                                                 Vec<T, V> (&xv)[NV], Vec<T, V> (&mv)[NV]) {
    if constexpr (NOUT != 0) {
        const T *m = mask + mask_row_offset<NOUT>((uint32_t)row, mrows);
#pragma unroll
        for (int c = 0; c < NV; c++) {
            const int col = (c * 64 + lane) * V;
            if (FULL || col < r) {
                if (mask_inner) {
                    mv[c] = vload<T, V>(m + col);
                } else {
                    const T m0 = m[0];
#pragma unroll
                    for (int k = 0; k < V; k++) mv[c].v[k] = m0;
                }
            }
        }
    }
#pragma unroll
    for (int c = 0; c < NV; c++) {
        const int col = (c * 64 + lane) * V;
        if (FULL || col < r) xv[c] = vload_nt<T, V>(x + row * (int64_t)r + col);
    }
}

// One row held in registers by one wave: the optional Div / Mul by a scalar, the mask add, the seed-0 max,
// the exponentials and their sum, and the division; y's row written with streaming stores.  cur holds the
// row (and mcur its mask vectors) as softmax_row_load left them.
template <typename T, int V, int NV, int NOUT, bool FULL, bool NTS = true>
__device__ __forceinline__ void softmax_row_body(Vec<T, V> (&cur)[NV], const Vec<T, V> (&mcur)[NV], T *__restrict__ q,
                                                 int r, int lane, bool has_scale, T sv, T sf, bool smul,
                                                 const ExpTable &tab) {
    constexpr bool MASK = NOUT != 0;
    if (has_scale) {  // the Div (or Mul) node before the mask Add: the same IEEE operation per element
#pragma unroll
        for (int c = 0; c < NV; c++) {
            const int col = (c * 64 + lane) * V;
            if (FULL || col < r) {
#pragma unroll
                for (int k = 0; k < V; k++) cur[c].v[k] = smul ? cur[c].v[k] * sf : cur[c].v[k] / sv;
            }
        }
    }
    if constexpr (MASK) {
#pragma unroll
        for (int c = 0; c < NV; c++) {
            const int col = (c * 64 + lane) * V;
            if (FULL || col < r) {
#pragma unroll
                for (int k = 0; k < V; k++) cur[c].v[k] = cur[c].v[k] + mcur[c].v[k];
            }
        }
    }
    // ReduceMax with seed 0 (TensorOps.cs:1820-1827)
    T mx = T(0);
#pragma unroll
    for (int c = 0; c < NV; c++) {
        const int col = (c * 64 + lane) * V;
        if (FULL || col < r) {
#pragma unroll
            for (int k = 0; k < V; k++) mx = row_max<T>(mx, cur[c].v[k]);
        }
    }
    mx = row_reduce<T>(mx, [](T a, T b) { return row_max<T>(a, b); });
    T sum = T(0);
#pragma unroll
    for (int c = 0; c < NV; c++) {
        const int col = (c * 64 + lane) * V;
        if (FULL || col < r) {
#pragma unroll
            for (int k = 0; k < V; k++) {
                cur[c].v[k] = exp_elem<T>(cur[c].v[k] - mx, tab);
                sum = sum + cur[c].v[k];
            }
        }
    }
    sum = row_reduce<T>(sum, [](T a, T b) { return a + b; });
    const T rs = T(1) / sum;
#pragma unroll
    for (int c = 0; c < NV; c++) {
        const int col = (c * 64 + lane) * V;
        if (FULL || col < r) {
            Vec<T, V> o;
#pragma unroll
            for (int k = 0; k < V; k++) o.v[k] = div_row<T>(cur[c].v[k], sum, rs);
            if constexpr (NTS) vstore_nt<T, V>(q + col, o);
            else vstore<T, V>(q + col, o);
        }
    }
}

// Rows of length r <= 64*V*NV held in registers, one wave per row at a time.
// Each wave walks rows w, w + W, ... (W = all waves of the grid) and loads the
// next row (and its mask vectors) while it finishes the current one.  NOUT:
// mask row axes (0 = no mask; see mask_row_offset).  FULL: r == 64*V*NV, every
// lane holds NV whole vectors (no per-vector bounds, one straight-line body).
// Rows of exactly 256 or 512 floats go to k_softmax_row1 instead (C3 on MI355X,
// interleaved in one process: Softmax 64.0 -> 60.5 us, Add mask + Softmax
// 63.9 -> 61.0 us, with its ordinary stores; on 400 MB of rows of 768 and 1024
// floats it was 2-10% slower than this kernel); this kernel takes the other
// row lengths.
template <typename T, int V, int NV, int NOUT, bool FULL>
__global__ __launch_bounds__(kSBlock) void k_softmax_wave(const T *__restrict__ x, T *__restrict__ y, int64_t rows,
                                                          int r, const T *__restrict__ mask, int mask_inner,
                                                          NdLayout mrows, const T *__restrict__ scale, int scale_div) {
    constexpr bool MASK = NOUT != 0;
    __shared__ ExpTable tab;
    if constexpr (std::is_same<T, float>::value) {
        exp_table_fill(tab);
        __syncthreads();
    }
    const int lane = threadIdx.x & 63;
    const int64_t W = (int64_t)gridDim.x * (kSBlock / 64);
    // the wave's index, read from lane 0 so the row and everything derived from it (the mask row offset,
    // the row's base addresses) are computed once per wave on the scalar unit
    int64_t row = (int64_t)blockIdx.x * (kSBlock / 64) + __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    if (row >= rows) return;
    Vec<T, V> cur[NV], nxt[NV], mcur[NV], mnxt[NV];
    const T sv = scale ? scale[0] : T(1);
    // a division by a power of two runs as the multiplication by its exact reciprocal
    T sf = sv;
    const bool smul = !scale_div || exact_pow2_recip(sv, &sf);
    softmax_row_load<T, V, NV, NOUT, FULL>(x, row, r, lane, mask, mask_inner, mrows, cur, mcur);
    for (; row < rows; row += W) {
        const int64_t next = row + W;
        if (next < rows) softmax_row_load<T, V, NV, NOUT, FULL>(x, next, r, lane, mask, mask_inner, mrows, nxt, mnxt);
        softmax_row_body<T, V, NV, NOUT, FULL>(cur, mcur, y + row * (int64_t)r, r, lane, scale != nullptr, sv, sf,
                                               smul, tab);
#pragma unroll
        for (int c = 0; c < NV; c++) {
            cur[c] = nxt[c];
            if constexpr (MASK) mcur[c] = mnxt[c];
        }
    }
}

// The same rows, one row per one-wave block and no loop: the block issues its row's loads, then fills its
// own expf table (exp_table_fill_wave), so no barrier stands between its start and its loads, and the wave
// ends right after its stores.  The output goes out with ordinary stores, measured faster here than
// streaming ones.  row0: the first row of this launch (launches of at most kMaxRowBlocks).
constexpr int64_t kMaxRowBlocks = 1ll << 24;
template <typename T, int V, int NV, int NOUT, bool FULL>
__global__ __launch_bounds__(64) void k_softmax_row1(const T *__restrict__ x, T *__restrict__ y, int64_t row0,
                                                     int r, const T *__restrict__ mask, int mask_inner,
                                                     NdLayout mrows, const T *__restrict__ scale, int scale_div) {
    __shared__ ExpTable tab;
    const int lane = threadIdx.x;
    const int64_t row = row0 + blockIdx.x;
    Vec<T, V> cur[NV], mcur[NV];
    softmax_row_load<T, V, NV, NOUT, FULL>(x, row, r, lane, mask, mask_inner, mrows, cur, mcur);
    if constexpr (std::is_same<T, float>::value) exp_table_fill_wave(tab);
    const T sv = scale ? scale[0] : T(1);
    T sf = sv;
    const bool smul = !scale_div || exact_pow2_recip(sv, &sf);
    softmax_row_body<T, V, NV, NOUT, FULL, false>(cur, mcur, y + row * (int64_t)r, r, lane, scale != nullptr, sv, sf,
                                                  smul, tab);
}

// ---------------------------------------------------------------------------
// Rows of any length with 16-byte accesses.  A row starting at element s0 of
// x splits into its head (the head = (-s0) mod V elements before its first
// 16-byte boundary), nvb whole aligned vectors, and its tail (the fewer than V
// elements after them).  Head and tail, ne = r - nvb*V <= 2V - 2 elements, are
// held one element per lane in lanes 0 .. ne-1: lane l < head holds column l,
// lane head <= l < ne holds column nvb*V + l.  y has x's layout, so the same
// split addresses the output.
// ---------------------------------------------------------------------------
struct RagRow {
    int head, nvb, ne;
};

template <int V>
__device__ __forceinline__ RagRow rag_row(int64_t s0, int r) {
    int head = (int)((V - (s0 & (V - 1))) & (V - 1));
    if (head > r) head = r;
    const int nvb = (r - head) / V;
    return {head, nvb, r - nvb * V};
}

template <int V>
__device__ __forceinline__ int rag_col(const RagRow &g, int lane) {
    return lane < g.head ? lane : g.nvb * V + lane;
}

// The row's elements: vector c of lane l is whole vector c*S + l (S = lanes of the row: 64 for a wave,
// the block size for a block), the lane's extra element as above.
template <typename T, int V, int NV, int S>
__device__ __forceinline__ void rag_load(const T *__restrict__ x, int64_t s0, const RagRow &g, int lane,
                                         Vec<T, V> (&v)[NV], T &e) {
    const T *p = x + s0 + g.head;
#pragma unroll
    for (int c = 0; c < NV; c++)
        if (c * S + lane < g.nvb) v[c] = vload_nt<T, V>(p + (int64_t)(c * S + lane) * V);
    if (lane < g.ne) e = x[s0 + rag_col<V>(g, lane)];
}

// x / scale or x * scale (the Div / Mul node), then + mask (the Add node), element by element.  A mask
// row contiguous along the row is read by vectors when it is 16-byte aligned at the row's first whole
// vector, by elements otherwise.
template <typename T, int V, int NV, int S>
__device__ __forceinline__ void rag_scale_mask(Vec<T, V> (&v)[NV], T &e, const RagRow &g, int lane, bool scaled,
                                               bool smul, T sf, T sv, const T *m, int mask_inner) {
    if (scaled) {
#pragma unroll
        for (int c = 0; c < NV; c++)
            if (c * S + lane < g.nvb) {
#pragma unroll
                for (int k = 0; k < V; k++) v[c].v[k] = smul ? v[c].v[k] * sf : v[c].v[k] / sv;
            }
        e = smul ? e * sf : e / sv;
    }
    if (!m) return;
    if (!mask_inner) {
        const T m0 = m[0];
#pragma unroll
        for (int c = 0; c < NV; c++)
            if (c * S + lane < g.nvb) {
#pragma unroll
                for (int k = 0; k < V; k++) v[c].v[k] = v[c].v[k] + m0;
            }
        e = e + m0;
        return;
    }
    const T *mb = m + g.head;
    const bool al = ((uintptr_t)mb & 15) == 0;
#pragma unroll
    for (int c = 0; c < NV; c++) {
        const int vi = c * S + lane;
        if (vi < g.nvb) {
            Vec<T, V> mv;
            if (al) {
                mv = vload<T, V>(mb + (int64_t)vi * V);
            } else {
#pragma unroll
                for (int k = 0; k < V; k++) mv.v[k] = mb[(int64_t)vi * V + k];
            }
#pragma unroll
            for (int k = 0; k < V; k++) v[c].v[k] = v[c].v[k] + mv.v[k];
        }
    }
    if (lane < g.ne) e = e + m[rag_col<V>(g, lane)];
}

// max (seed 0) of the lane's elements, their exponentials x - max in place and the lane's sum of them
template <typename T, int V, int NV, int S>
__device__ __forceinline__ T rag_lane_max(const Vec<T, V> (&v)[NV], T e, const RagRow &g, int lane) {
    T mx = T(0);
#pragma unroll
    for (int c = 0; c < NV; c++)
        if (c * S + lane < g.nvb) {
#pragma unroll
            for (int k = 0; k < V; k++) mx = row_max<T>(mx, v[c].v[k]);
        }
    if (lane < g.ne) mx = row_max<T>(mx, e);
    return mx;
}

template <typename T, int V, int NV, int S>
__device__ __forceinline__ T rag_lane_exp_sum(Vec<T, V> (&v)[NV], T &e, T mx, const RagRow &g, int lane,
                                              const ExpTable &tab) {
    T sum = T(0);
#pragma unroll
    for (int c = 0; c < NV; c++)
        if (c * S + lane < g.nvb) {
#pragma unroll
            for (int k = 0; k < V; k++) {
                v[c].v[k] = exp_elem<T>(v[c].v[k] - mx, tab);
                sum = sum + v[c].v[k];
            }
        }
    if (lane < g.ne) {
        e = exp_elem<T>(e - mx, tab);
        sum = sum + e;
    }
    return sum;
}

template <typename T, int V, int NV, int S>
__device__ __forceinline__ void rag_store(T *__restrict__ y, int64_t s0, const RagRow &g, int lane,
                                          const Vec<T, V> (&v)[NV], T e, T sum, T rs) {
    T *q = y + s0 + g.head;
#pragma unroll
    for (int c = 0; c < NV; c++)
        if (c * S + lane < g.nvb) {
            Vec<T, V> o;
#pragma unroll
            for (int k = 0; k < V; k++) o.v[k] = div_row<T>(v[c].v[k], sum, rs);
            vstore_nt<T, V>(q + (int64_t)(c * S + lane) * V, o);
        }
    if (lane < g.ne) y[s0 + rag_col<V>(g, lane)] = div_row<T>(e, sum, rs);
}

// Row per wave for rows whose length is not a multiple of V (or whose mask is not 16-byte aligned), up to
// 64*V*NV + V - 1 elements: the walk of k_softmax_wave, rows split as above.
template <typename T, int V, int NV, int NOUT>
__global__ __launch_bounds__(kSBlock) void k_softmax_wave_rag(const T *__restrict__ x, T *__restrict__ y,
                                                              int64_t rows, int r, const T *__restrict__ mask,
                                                              int mask_inner, NdLayout mrows,
                                                              const T *__restrict__ scale, int scale_div) {
    __shared__ ExpTable tab;
    if constexpr (std::is_same<T, float>::value) {
        exp_table_fill(tab);
        __syncthreads();
    }
    const int lane = threadIdx.x & 63;
    const int64_t W = (int64_t)gridDim.x * (kSBlock / 64);
    int64_t row = (int64_t)blockIdx.x * (kSBlock / 64) + __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    if (row >= rows) return;
    const T sv = scale ? scale[0] : T(1);
    T sf = sv;
    const bool smul = !scale_div || exact_pow2_recip(sv, &sf);
    Vec<T, V> cur[NV], nxt[NV];
    T ecur = T(0), enxt = T(0);
    RagRow gc = rag_row<V>(row * (int64_t)r, r), gn = gc;
    rag_load<T, V, NV, 64>(x, row * (int64_t)r, gc, lane, cur, ecur);
    for (; row < rows; row += W) {
        const int64_t next = row + W, s0 = row * (int64_t)r;
        if (next < rows) {
            gn = rag_row<V>(next * (int64_t)r, r);
            rag_load<T, V, NV, 64>(x, next * (int64_t)r, gn, lane, nxt, enxt);
        }
        const T *m = nullptr;
        if constexpr (NOUT != 0) m = mask + mask_row_offset<NOUT>((uint32_t)row, mrows);
        rag_scale_mask<T, V, NV, 64>(cur, ecur, gc, lane, scale != nullptr, smul, sf, sv, m, mask_inner);
        T mx = rag_lane_max<T, V, NV, 64>(cur, ecur, gc, lane);
        mx = row_reduce<T>(mx, [](T a, T b) { return row_max<T>(a, b); });
        T sum = rag_lane_exp_sum<T, V, NV, 64>(cur, ecur, mx, gc, lane, tab);
        sum = row_reduce<T>(sum, [](T a, T b) { return a + b; });
        rag_store<T, V, NV, 64>(y, s0, gc, lane, cur, ecur, sum, T(1) / sum);
#pragma unroll
        for (int c = 0; c < NV; c++) cur[c] = nxt[c];
        ecur = enxt;
        gc = gn;
    }
}

// Short rows (at most 32 whole vectors plus head and tail): L lanes per row (a power of two below 64),
// 64 / L rows per wave at a time, where one row per wave would leave most lanes idle.  Each group of L
// lanes walks its rows like the wave of k_softmax_wave_rag (next row loaded while the current one is
// finished), with the same row split, scale and mask.
template <typename T, int V, int L, int NOUT>
__global__ __launch_bounds__(kSBlock) void k_softmax_group(const T *__restrict__ x, T *__restrict__ y,
                                                           int64_t rows, int r, const T *__restrict__ mask,
                                                           int mask_inner, NdLayout mrows,
                                                           const T *__restrict__ scale, int scale_div) {
    __shared__ ExpTable tab;
    if constexpr (std::is_same<T, float>::value) {
        exp_table_fill(tab);
        __syncthreads();
    }
    constexpr int RW = 64 / L;  // rows per wave
    const int lane = threadIdx.x & 63, gl = lane & (L - 1);
    const int64_t W = (int64_t)gridDim.x * (kSBlock / 64) * RW;
    int64_t row = ((int64_t)blockIdx.x * (kSBlock / 64) + (threadIdx.x >> 6)) * RW + lane / L;
    if (row >= rows) return;
    const T sv = scale ? scale[0] : T(1);
    T sf = sv;
    const bool smul = !scale_div || exact_pow2_recip(sv, &sf);
    Vec<T, V> cur[1], nxt[1];
    T ecur = T(0), enxt = T(0);
    RagRow gc = rag_row<V>(row * (int64_t)r, r), gn = gc;
    rag_load<T, V, 1, L>(x, row * (int64_t)r, gc, gl, cur, ecur);
    for (; row < rows; row += W) {
        const int64_t next = row + W, s0 = row * (int64_t)r;
        if (next < rows) {
            gn = rag_row<V>(next * (int64_t)r, r);
            rag_load<T, V, 1, L>(x, next * (int64_t)r, gn, gl, nxt, enxt);
        }
        const T *m = nullptr;
        if constexpr (NOUT != 0) m = mask + mask_row_offset<NOUT>((uint32_t)row, mrows);
        rag_scale_mask<T, V, 1, L>(cur, ecur, gc, gl, scale != nullptr, smul, sf, sv, m, mask_inner);
        T mx = rag_lane_max<T, V, 1, L>(cur, ecur, gc, gl);
        mx = group_reduce<L>(mx, [](T a, T b) { return row_max<T>(a, b); });
        T sum = rag_lane_exp_sum<T, V, 1, L>(cur, ecur, mx, gc, gl, tab);
        sum = group_reduce<L>(sum, [](T a, T b) { return a + b; });
        rag_store<T, V, 1, L>(y, s0, gc, gl, cur, ecur, sum, T(1) / sum);
        cur[0] = nxt[0];
        ecur = enxt;
        gc = gn;
    }
}

// max or sum over the block, the same value returned to every lane: the waves' values through LDS,
// folded in wave order (deterministic)
template <typename T, int B, typename F>
__device__ __forceinline__ T block_allreduce(T v, T *red, F f) {
    v = row_reduce<T>(v, f);
    if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = v;
    __syncthreads();
    T t = red[0];
#pragma unroll
    for (int w = 1; w < B / 64; w++) t = f(t, red[w]);
    __syncthreads();  // red is written again by the next reduction
    return t;
}

// inner == 1, rows longer than a wave holds (up to B*V*NV + V - 1 elements): one block of B lanes per row,
// the row in registers, so x is read once and y written once; rows split as above.
template <typename T, int V, int NV, int B, bool MASK>
__global__ __launch_bounds__(B) void k_softmax_rows(const T *__restrict__ x, T *__restrict__ y, int64_t rows, int r,
                                                    const T *__restrict__ mask, int mask_inner, NdLayout mrows,
                                                    const T *__restrict__ scale, int scale_div) {
    __shared__ ExpTable tab;
    __shared__ T red[B / 64];
    if constexpr (std::is_same<T, float>::value) {
        exp_table_fill(tab);
        __syncthreads();
    }
    const int tid = threadIdx.x;
    const T sv = scale ? scale[0] : T(1);
    T sf = sv;
    const bool smul = !scale_div || exact_pow2_recip(sv, &sf);
    for (int64_t row = blockIdx.x; row < rows; row += gridDim.x) {
        const int64_t s0 = row * (int64_t)r;
        const RagRow g = rag_row<V>(s0, r);
        Vec<T, V> v[NV];
        T e = T(0);
        rag_load<T, V, NV, B>(x, s0, g, tid, v, e);
        const T *m = nullptr;
        if constexpr (MASK) m = mask + mask_row_offset<-1>((uint32_t)row, mrows);
        rag_scale_mask<T, V, NV, B>(v, e, g, tid, scale != nullptr, smul, sf, sv, m, mask_inner);
        T mx = rag_lane_max<T, V, NV, B>(v, e, g, tid);
        mx = block_allreduce<T, B>(mx, red, [](T a, T b) { return row_max<T>(a, b); });
        T sum = rag_lane_exp_sum<T, V, NV, B>(v, e, mx, g, tid, tab);
        sum = block_allreduce<T, B>(sum, red, [](T a, T b) { return a + b; });
        rag_store<T, V, NV, B>(y, s0, g, tid, v, e, sum, T(1) / sum);
    }
}

// inner == 1, long rows: one block per row, three passes over the row.
template <typename T>
__global__ __launch_bounds__(kSBlock) void k_softmax_block(const T *__restrict__ x, T *__restrict__ y, int64_t r) {
    __shared__ ExpTable tab;
    __shared__ T red[kSBlock / 64];
    if constexpr (std::is_same<T, float>::value) exp_table_fill(tab);
    __syncthreads();
    const int64_t row = blockIdx.x;
    const T *p = x + row * r;
    T *q = y + row * r;
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
    T mx = T(0);
    for (int64_t j = threadIdx.x; j < r; j += kSBlock) mx = p[j] > mx ? p[j] : mx;
    mx = wave_reduce(mx, [](T a, T b) { return b > a ? b : a; });
    if (lane == 0) red[wave] = mx;
    __syncthreads();
    mx = red[0];
    for (int w = 1; w < kSBlock / 64; w++) mx = red[w] > mx ? red[w] : mx;
    __syncthreads();
    T s = T(0);
    for (int64_t j = threadIdx.x; j < r; j += kSBlock) s = s + exp_elem<T>(p[j] - mx, tab);
    s = wave_reduce(s, [](T a, T b) { return a + b; });
    if (lane == 0) red[wave] = s;
    __syncthreads();
    s = red[0];
    for (int w = 1; w < kSBlock / 64; w++) s = s + red[w];
    for (int64_t j = threadIdx.x; j < r; j += kSBlock) q[j] = exp_elem<T>(p[j] - mx, tab) / s;
}

// inner > 1: one thread per (outer, inner) column, coalesced along inner.
// The sum runs serially along the axis, in the reference's order.
template <typename T>
__global__ __launch_bounds__(kSBlock) void k_softmax_cols(const T *__restrict__ x, T *__restrict__ y, int64_t outer,
                                                          int64_t r, int64_t inner) {
    __shared__ ExpTable tab;
    if constexpr (std::is_same<T, float>::value) exp_table_fill(tab);
    __syncthreads();
    const int64_t ncol = outer * inner;
    for (int64_t c = (int64_t)blockIdx.x * kSBlock + threadIdx.x; c < ncol; c += (int64_t)gridDim.x * kSBlock) {
        const int64_t o = c / inner, i = c - o * inner;
        const T *p = x + o * r * inner + i;
        T *q = y + o * r * inner + i;
        T mx = T(0);
        for (int64_t j = 0; j < r; j++) {
            T v = p[j * inner];
            mx = v > mx ? v : mx;
        }
        T s = T(0);
        for (int64_t j = 0; j < r; j++) s = s + exp_elem<T>(p[j * inner] - mx, tab);
        for (int64_t j = 0; j < r; j++) q[j * inner] = exp_elem<T>(p[j * inner] - mx, tab) / s;
    }
}

template <typename T, int V, int NOUT>
static hipError_t softmax_wave_launch(const SoftmaxArgs &a, hipStream_t s) {
    const int r = (int)a.r;
    const int nv = (r + 64 * V - 1) / (64 * V);
    int64_t g = (a.outer + kSBlock / 64 - 1) / (kSBlock / 64);
    if (g > kSoftmaxMaxBlocks) g = kSoftmaxMaxBlocks;
    const T *x = (const T *)a.x;
    T *y = (T *)a.y;
    const T *m = (const T *)a.mask;
    const bool full = r == nv * 64 * V;
#define LX_SM_ROW1(N, F)                                                                                        \
    for (int64_t r0 = 0; r0 < a.outer; r0 += kMaxRowBlocks)                                                     \
        hipLaunchKernelGGL((k_softmax_row1<T, V, (N <= 2 ? N : 2), NOUT, F>), dim3((unsigned)std::min(kMaxRowBlocks, a.outer - r0)), \
                           dim3(64), 0, s, x, y, r0, r, m, a.mask_inner, a.mask_rows, (const T *)a.scale, a.scale_div);
#define LX_SM_CASE(N)                                                                                           \
    case N:                                                                                                     \
        if (full && N <= 2) {                                                                                   \
            LX_SM_ROW1(N, true)                                                                                 \
        } else if (full && N <= 4) {                                                                            \
            hipLaunchKernelGGL((k_softmax_wave<T, V, N, NOUT, (N <= 4)>), dim3((unsigned)g), dim3(kSBlock), 0, s, x, y, \
                               a.outer, r, m, a.mask_inner, a.mask_rows, (const T *)a.scale, a.scale_div);      \
        } else {                                                                                                \
            hipLaunchKernelGGL((k_softmax_wave<T, V, N, NOUT, false>), dim3((unsigned)g), dim3(kSBlock), 0, s, x, y,  \
                               a.outer, r, m, a.mask_inner, a.mask_rows, (const T *)a.scale, a.scale_div);      \
        }                                                                                                       \
        break;
    switch (nv) {
        LX_SM_CASE(1) LX_SM_CASE(2) LX_SM_CASE(3) LX_SM_CASE(4) LX_SM_CASE(5) LX_SM_CASE(6) LX_SM_CASE(7) LX_SM_CASE(8)
    default: return hipErrorInvalidValue;
    }
#undef LX_SM_CASE
#undef LX_SM_ROW1
    return hipGetLastError();
}

template <typename T, int V, bool MASK>
static hipError_t softmax_wave_dispatch(const SoftmaxArgs &a, hipStream_t s) {
    if constexpr (!MASK) return softmax_wave_launch<T, V, 0>(a, s);
    switch (a.mask_rows.nouter) {
    case 1: return softmax_wave_launch<T, V, 1>(a, s);
    case 2: return softmax_wave_launch<T, V, 2>(a, s);
    case 3: return softmax_wave_launch<T, V, 3>(a, s);
    default: return softmax_wave_launch<T, V, -1>(a, s);
    }
}

template <typename T, int V, int NOUT>
static hipError_t softmax_rag_launch(const SoftmaxArgs &a, hipStream_t s) {
    const int r = (int)a.r;
    int nv = (int)((r / V + 63) / 64);
    if (nv < 1) nv = 1;
    int64_t g = (a.outer + kSBlock / 64 - 1) / (kSBlock / 64);
    if (g > kSoftmaxMaxBlocks) g = kSoftmaxMaxBlocks;
    const T *x = (const T *)a.x;
    T *y = (T *)a.y;
    const T *m = (const T *)a.mask;
#define LX_SMR_CASE(N)                                                                                             \
    case N:                                                                                                        \
        hipLaunchKernelGGL((k_softmax_wave_rag<T, V, N, NOUT>), dim3((unsigned)g), dim3(kSBlock), 0, s, x, y, a.outer, \
                           r, m, a.mask_inner, a.mask_rows, (const T *)a.scale, a.scale_div);                      \
        break;
    switch (nv) {
        LX_SMR_CASE(1) LX_SMR_CASE(2) LX_SMR_CASE(3) LX_SMR_CASE(4) LX_SMR_CASE(5) LX_SMR_CASE(6) LX_SMR_CASE(7) LX_SMR_CASE(8)
    default: return hipErrorInvalidValue;
    }
#undef LX_SMR_CASE
    return hipGetLastError();
}

template <typename T, int V>
static hipError_t softmax_rag_dispatch(const SoftmaxArgs &a, hipStream_t s) {
    if (!a.mask) return softmax_rag_launch<T, V, 0>(a, s);
    switch (a.mask_rows.nouter) {
    case 1: return softmax_rag_launch<T, V, 1>(a, s);
    case 2: return softmax_rag_launch<T, V, 2>(a, s);
    case 3: return softmax_rag_launch<T, V, 3>(a, s);
    default: return softmax_rag_launch<T, V, -1>(a, s);
    }
}

template <typename T, int V, int NOUT>
static hipError_t softmax_group_launch(const SoftmaxArgs &a, int L, hipStream_t s) {
    const int64_t per_block = (int64_t)(kSBlock / 64) * (64 / L);  // rows a block takes at a time
    int64_t g = (a.outer + per_block - 1) / per_block;
    if (g > kSoftmaxMaxBlocks) g = kSoftmaxMaxBlocks;
    const T *x = (const T *)a.x;
    T *y = (T *)a.y;
    const T *m = (const T *)a.mask;
#define LX_SMG_CASE(N)                                                                                             \
    case N:                                                                                                        \
        hipLaunchKernelGGL((k_softmax_group<T, V, N, NOUT>), dim3((unsigned)g), dim3(kSBlock), 0, s, x, y, a.outer,   \
                           (int)a.r, m, a.mask_inner, a.mask_rows, (const T *)a.scale, a.scale_div);               \
        break;
    switch (L) {
        LX_SMG_CASE(1) LX_SMG_CASE(2) LX_SMG_CASE(4) LX_SMG_CASE(8) LX_SMG_CASE(16) LX_SMG_CASE(32)
    default: return hipErrorInvalidValue;
    }
#undef LX_SMG_CASE
    return hipGetLastError();
}

template <typename T, int V>
static hipError_t softmax_group_dispatch(const SoftmaxArgs &a, int L, hipStream_t s) {
    if (!a.mask) return softmax_group_launch<T, V, 0>(a, L, s);
    switch (a.mask_rows.nouter) {
    case 1: return softmax_group_launch<T, V, 1>(a, L, s);
    case 2: return softmax_group_launch<T, V, 2>(a, L, s);
    case 3: return softmax_group_launch<T, V, 3>(a, L, s);
    default: return softmax_group_launch<T, V, -1>(a, L, s);
    }
}

template <typename T, int V, int NV, int B>
static hipError_t softmax_rows_launch(const SoftmaxArgs &a, hipStream_t s) {
    const int64_t g = a.outer < (1 << 20) ? a.outer : (1 << 20);
    const T *x = (const T *)a.x;
    T *y = (T *)a.y;
    constexpr bool kMaskable = NV * V * (int)sizeof(T) <= 128;  // registers for the mask add
    if (a.mask) {
        if constexpr (kMaskable)
            hipLaunchKernelGGL((k_softmax_rows<T, V, NV, B, true>), dim3((unsigned)g), dim3(B), 0, s, x, y, a.outer,
                               (int)a.r, (const T *)a.mask, a.mask_inner, a.mask_rows, (const T *)a.scale,
                               a.scale_div);
        else
            return hipErrorInvalidValue;
    } else {
        hipLaunchKernelGGL((k_softmax_rows<T, V, NV, B, false>), dim3((unsigned)g), dim3(B), 0, s, x, y, a.outer,
                           (int)a.r, (const T *)nullptr, 0, a.mask_rows, (const T *)a.scale, a.scale_div);
    }
    return hipGetLastError();
}

// ---------------------------------------------------------------------------
// Attention heads (launch_attention): one block per batch.
// ---------------------------------------------------------------------------
typedef float v16f __attribute__((ext_vector_type(16)));

// Scores, Softmax and context of one head, in T x T tiles (T = 32 or 64) with NT lanes.  Q, K and V are first
// staged in LDS with zeros past their rows and columns (every load issued before the first is waited for; Q, K
// and the scores in rows padded by one float against bank conflicts).  Each of the first (T / 32)^2 waves then
// runs one 32x32 part of the product as the MatMul's register-staged kernel runs the 32x32 quarters of its 64x64
// tiles: K in steps of 16 (zeros past K), MFMA j of a step taking k = j from lanes 0-31 and k = 8 + j from lanes
// 32-63, as B^T A^T (lane l % 32 holds row l % 32 of A and column l % 32 of B), so acc[q] is C[row l % 32][column
// 8 (q / 4) + 4 (l / 32) + q % 4].  The zeros make every product past the operands +0, as the kernel's zero
// loads do.  The scores go to LDS; each row splits into head, whole vectors and tail by its flat offset in the
// dense scores tensor, as k_softmax_group<V = 4, L> splits it in memory, and is scaled, masked, reduced over its
// L lanes and divided by the same functions in the same lanes, in place; the context then reads the
// probabilities (+0 past the keys) from LDS.  T = 64 takes 16 waves (the Softmax's 64 rows in one pass); T = 32,
// for heads of at most 32, takes 4 waves and a quarter of the LDS, so that many heads run at once.

// a rows x cols strided matrix into a T x T LDS tile of rows of ld floats, zeros past rows and cols: lane t takes
// column t % 64 (of the first T) of rows t / 64 + (NT / 64) u.  attn_load issues the loads into x, attn_store
// writes them, so that the loads of all three operands are in flight together.
template <int T, int NT>
__device__ __forceinline__ void attn_load(float (&x)[T / (NT / 64)], const float *__restrict__ src, int rows, int cols,
                                          int64_t rs, int64_t cs) {
    constexpr int RP = NT / 64, U = T / RP;  // rows per pass, passes
    static_assert(U * RP == T, "whole rows per pass");
    const int c = threadIdx.x & 63, r0 = threadIdx.x >> 6;
    const float *p = src + (int64_t)c * cs + (int64_t)r0 * rs;
#pragma unroll
    for (int u = 0; u < U; u++) x[u] = (c < T && c < cols && r0 + RP * u < rows) ? p[(int64_t)(RP * u) * rs] : 0.f;
}
template <int T, int NT>
__device__ __forceinline__ void attn_store(const float (&x)[T / (NT / 64)], float *__restrict__ dst, int ld) {
    constexpr int RP = NT / 64, U = T / RP;
    const int c = threadIdx.x & 63, r0 = threadIdx.x >> 6;
    if (c >= T) return;
#pragma unroll
    for (int u = 0; u < U; u++) dst[(r0 + RP * u) * ld + c] = x[u];
}

template <int T, int NT, int L, int NOUT>
__global__ __launch_bounds__(NT) void k_attention(AttentionArgs a) {
    static_assert((T == 32 || T == 64) && NT % 64 == 0 && NT / 64 >= (T / 32) * (T / 32), "a wave per 32x32 part");
    constexpr int LD = T + 1;  // padded LDS row of Q, K and the scores
    __shared__ ExpTable tab;
    __shared__ float qs[T * LD];  // Q [S][D]
    __shared__ float ks[T * LD];  // K as rows of keys [SK][D]
    __shared__ float vs[T * T];   // V [SK][DV]
    __shared__ float ps[T * LD];  // scores, then probabilities [S][SK]
    const int t = threadIdx.x, l = t & 63, w = t >> 6;
    const int64_t z = blockIdx.x;
    int64_t qo = 0, ko = 0, vo = 0, yo = 0;
    {
        int64_t b = z;
        for (int d = a.nbatch - 1; d >= 0; d--) {
            const int64_t i = b % a.bdims[d];
            b /= a.bdims[d];
            qo += i * a.q_bstr[d];
            ko += i * a.k_bstr[d];
            vo += i * a.v_bstr[d];
            yo += i * a.y_bstr[d];
        }
    }
    const int S = a.s, SK = a.sk, D = a.d, DV = a.dv;
    // this lane's Softmax row (every row in one pass: NT / 64 waves of 64 / L rows cover T rows) and its mask
    // elements, loaded with Q, K and V: the mask add below reads them as rag_scale_mask reads them
    constexpr int RW = 64 / L;  // rows per wave
    static_assert((NT / 64) * RW >= T, "one Softmax pass");
    const int gl = l & (L - 1), i = w * RW + l / L;
    const int64_t row = z * S + i;
    const RagRow g = rag_row<4>(row * SK, SK);
    float mv[4] = {0.f, 0.f, 0.f, 0.f}, me = 0.f;
    if (NOUT != 0 && i < S) {
        const float *m = a.mask + mask_row_offset<NOUT>((uint32_t)row, a.mask_rows);
        if (!a.mask_inner) {
            mv[0] = m[0];
        } else {
            if (gl < g.nvb) {
#pragma unroll
                for (int k = 0; k < 4; k++) mv[k] = m[g.head + 4 * gl + k];
            }
            if (gl < g.ne) me = m[rag_col<4>(g, gl)];
        }
    }
    // K's element (kk, j) of the product's right operand is key j's element kk
    float xq[T / (NT / 64)], xk[T / (NT / 64)], xv[T / (NT / 64)];
    attn_load<T, NT>(xq, a.q + qo, S, D, a.q_rs, a.q_cs);
    attn_load<T, NT>(xk, a.k + ko, SK, D, a.k_cs, a.k_rs);
    attn_load<T, NT>(xv, a.v + vo, SK, DV, a.v_rs, a.v_cs);
    attn_store<T, NT>(xq, qs, LD);
    attn_store<T, NT>(xk, ks, LD);
    attn_store<T, NT>(xv, vs, T);
    exp_table_fill(tab);
    __syncthreads();

    // the first (T / 32)^2 waves: one 32x32 part each of the T x T products
    constexpr int P = T / 32, NP = P * P;
    const int wr = 32 * (w / P % P), wc = 32 * (w % P);
    const int r = wr + (l & 31), c = wc + (l & 31), h = l >> 5;
    if (w < NP) {
        v16f acc;
#pragma unroll
        for (int q = 0; q < 16; q++) acc[q] = 0.f;
        const float *qa = qs + r * LD + 8 * h, *kb = ks + c * LD + 8 * h;
        for (int kt = 0; kt < D; kt += 16)
#pragma unroll
            for (int j = 0; j < 8; j++) acc = __builtin_amdgcn_mfma_f32_32x32x2f32(kb[kt + j], qa[kt + j], acc, 0, 0, 0);
        float *pr = ps + r * LD + wc + 4 * h;
#pragma unroll
        for (int q = 0; q < 16; q++) pr[8 * (q / 4) + q % 4] = acc[q];
    }
    __syncthreads();

    const float sv = a.scale ? a.scale[0] : 1.f;
    float sf = sv;
    const bool smul = !a.scale_div || exact_pow2_recip(sv, &sf);
    if (i < S) {
        float *pr = ps + i * LD;
        Vec<float, 4> v[1];
        float e = 0.f;
        if (gl < g.nvb) {
#pragma unroll
            for (int k = 0; k < 4; k++) v[0].v[k] = pr[g.head + 4 * gl + k];
        }
        if (gl < g.ne) e = pr[rag_col<4>(g, gl)];
        // rag_scale_mask's scale, then its mask add with the elements loaded above
        rag_scale_mask<float, 4, 1, L>(v, e, g, gl, a.scale != nullptr, smul, sf, sv, nullptr, 0);
        if constexpr (NOUT != 0) {
            if (!a.mask_inner) {
                if (gl < g.nvb) {
#pragma unroll
                    for (int k = 0; k < 4; k++) v[0].v[k] = v[0].v[k] + mv[0];
                }
                e = e + mv[0];
            } else {
                if (gl < g.nvb) {
#pragma unroll
                    for (int k = 0; k < 4; k++) v[0].v[k] = v[0].v[k] + mv[k];
                }
                if (gl < g.ne) e = e + me;
            }
        }
        float mx = rag_lane_max<float, 4, 1, L>(v, e, g, gl);
        mx = group_reduce<L>(mx, [](float x, float y) { return row_max<float>(x, y); });
        float sum = rag_lane_exp_sum<float, 4, 1, L>(v, e, mx, g, gl, tab);
        sum = group_reduce<L>(sum, [](float x, float y) { return x + y; });
        const float rs = 1.f / sum;
        if (gl < g.nvb) {
#pragma unroll
            for (int k = 0; k < 4; k++) pr[g.head + 4 * gl + k] = div_row<float>(v[0].v[k], sum, rs);
        }
        if (gl < g.ne) pr[rag_col<4>(g, gl)] = div_row<float>(e, sum, rs);
    }
    __syncthreads();

    if (w < NP && wr < S && wc < DV) {
        v16f acc;
#pragma unroll
        for (int q = 0; q < 16; q++) acc[q] = 0.f;
        const float *pa = ps + r * LD + 8 * h, *vb = vs + 8 * h * T + c;
        for (int kt = 0; kt < SK; kt += 16)
#pragma unroll
            for (int j = 0; j < 8; j++) acc = __builtin_amdgcn_mfma_f32_32x32x2f32(vb[(kt + j) * T], pa[kt + j], acc, 0, 0, 0);
        float *Y = a.y + yo + (int64_t)r * a.y_rs;
        if (r < S) {
#pragma unroll
            for (int q = 0; q < 16; q++) {
                const int col = wc + 8 * (q / 4) + 4 * h + q % 4;
                if (col < DV) Y[col * a.y_cs] = acc[q];
            }
        }
    }
}

template <int T, int NT, int NOUT>
static hipError_t attention_launch(const AttentionArgs &a, int L, hipStream_t s) {
    const dim3 g((unsigned)a.batch), blk(NT);
    switch (L) {
    case 1: hipLaunchKernelGGL((k_attention<T, NT, 1, NOUT>), g, blk, 0, s, a); break;
    case 2: hipLaunchKernelGGL((k_attention<T, NT, 2, NOUT>), g, blk, 0, s, a); break;
    case 4: hipLaunchKernelGGL((k_attention<T, NT, 4, NOUT>), g, blk, 0, s, a); break;
    case 8: hipLaunchKernelGGL((k_attention<T, NT, 8, NOUT>), g, blk, 0, s, a); break;
    case 16:
        if constexpr (T == 64) {
            hipLaunchKernelGGL((k_attention<T, NT, 16, NOUT>), g, blk, 0, s, a);
            break;
        }
        return hipErrorInvalidValue;
    default: return hipErrorInvalidValue;
    }
    return hipGetLastError();
}

template <int NOUT>
static hipError_t attention_size(const AttentionArgs &a, int L, hipStream_t s) {
    if (a.s <= 32 && a.sk <= 32 && a.d <= 32 && a.dv <= 32) return attention_launch<32, 256, NOUT>(a, L, s);
    return attention_launch<64, 1024, NOUT>(a, L, s);
}

hipError_t launch_attention(const AttentionArgs &a, hipStream_t s) {
    if (a.s < 1 || a.sk < 1 || a.d < 1 || a.dv < 1 || a.s > kAttentionMax || a.sk > kAttentionMax ||
        a.d > kAttentionMax || a.dv > kAttentionMax || a.batch < 1 || a.batch > 0x7fffffff)
        return hipErrorInvalidValue;
    // the lanes per row softmax_typed gives rows of sk floats in 16-byte aligned tensors
    const int nvr = a.sk / 4, ne_max = a.sk % 4 == 0 ? 0 : (a.sk < 6 ? a.sk : 6);
    int L = 1;
    while (L < nvr || L < ne_max) L <<= 1;
    if (!a.mask) return attention_size<0>(a, L, s);
    switch (a.mask_rows.nouter) {
    case 1: return attention_size<1>(a, L, s);
    case 2: return attention_size<2>(a, L, s);
    case 3: return attention_size<3>(a, L, s);
    default: return attention_size<-1>(a, L, s);
    }
}

// Whole 16-byte vectors a row-in-registers kernel holds at most: blocks of 1024 lanes with 16 vectors each
// for float rows, 8 each for double rows and rows with a mask or scale (16 spill registers there).
constexpr int64_t kSoftmaxRowVecs = 1024 * 16, kSoftmaxRowVecsMasked = 1024 * 8;

template <typename T>
static hipError_t softmax_typed(const SoftmaxArgs &a, hipStream_t s) {
    constexpr int VW = VecWidth<T>::value;
    if (a.inner == 1 && a.outer < (1ll << 31)) {
        if (a.vec > 1) {
            // x and y 16-byte aligned: rows held in registers, 16-byte accesses
            const int64_t nvr = a.r / VW;
            // short rows: L lanes per row, enough for its whole vectors and its head and tail elements
            // (none when r is a multiple of VW: every row then starts aligned)
            const int64_t ne_max = a.r % VW == 0 ? 0 : (a.r < 2 * VW - 2 ? a.r : 2 * VW - 2);
            int L = 1;
            while (L < nvr || L < ne_max) L <<= 1;
            if (L <= 32) return softmax_group_dispatch<T, VW>(a, L, s);
            const bool mask_al = !a.mask || !a.mask_inner || ((uintptr_t)a.mask & 15) == 0;
            if (a.r % VW == 0 && mask_al && a.r <= 64 * VW * 8) {
                if (a.mask) return softmax_wave_dispatch<T, VW, true>(a, s);
                return softmax_wave_dispatch<T, VW, false>(a, s);
            }
            if (nvr <= 64 * 8) return softmax_rag_dispatch<T, VW>(a, s);
            if (nvr <= 256 * 4) return softmax_rows_launch<T, VW, 4, 256>(a, s);
            if (nvr <= 256 * 8) return softmax_rows_launch<T, VW, 8, 256>(a, s);
            if (nvr <= kSoftmaxRowVecsMasked) return softmax_rows_launch<T, VW, 8, 1024>(a, s);
            if constexpr (std::is_same<T, float>::value)
                if (nvr <= kSoftmaxRowVecs && !a.mask && !a.scale) return softmax_rows_launch<T, VW, 16, 1024>(a, s);
        } else if (a.r <= 64 * 8) {
            if (a.mask) return softmax_wave_dispatch<T, 1, true>(a, s);
            return softmax_wave_dispatch<T, 1, false>(a, s);
        }
    }
    if (a.mask || a.scale) return hipErrorInvalidValue;  // the host falls back to Div / Add + Softmax
    if (a.inner == 1) {
        hipLaunchKernelGGL((k_softmax_block<T>), dim3((unsigned)a.outer), dim3(kSBlock), 0, s, (const T *)a.x, (T *)a.y,
                           a.r);
    } else {
        int64_t ncol = a.outer * a.inner;
        int64_t g = (ncol + kSBlock - 1) / kSBlock;
        if (g > 8192) g = 8192;
        hipLaunchKernelGGL((k_softmax_cols<T>), dim3((unsigned)g), dim3(kSBlock), 0, s, (const T *)a.x, (T *)a.y,
                           a.outer, a.r, a.inner);
    }
    return hipGetLastError();
}

// True when launch_softmax can apply the mask inside the kernel.
bool softmax_mask_fusable(int dtype, int64_t r, int64_t inner, int64_t outer, int vec) {
    const int vw = dtype == kFloat ? 4 : 2;
    if (inner != 1 || outer >= (1ll << 31)) return false;
    return (vec > 1 && r / vw <= kSoftmaxRowVecsMasked) || r <= 64 * 8;
}

hipError_t launch_softmax(const SoftmaxArgs &a, hipStream_t s) {
    if (a.outer * a.r * a.inner == 0) return hipSuccess;
    if (a.dtype == kFloat) return softmax_typed<float>(a, s);
    if (a.dtype == kDouble) return softmax_typed<double>(a, s);
    return hipErrorInvalidValue;
}

}  // namespace lx
