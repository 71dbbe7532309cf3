// lx_softmax.hip -- gfx950 Softmax, optionally fused with a broadcast additive
// mask (the Add node that precedes attention softmax).
//
// Reference composite (TensorOps.cs:1312-1330), five passes and three
// temporaries on the CPU:
//   m = ReduceMax(x, axis) (seed 0)   d = x - m   e = MathF.Exp(d)
//   s = ReduceSum(e, axis)            y = e / s   (true division)
// Here: one wave64 per row with the row in registers (rows up to 2048 floats),
// the exponential bit-identical to the host expf (expf_lx), the sum as a
// wave butterfly.  Only the order of the sum differs from the reference.
// Other shapes (axis not innermost, long rows) take a three-pass kernel.
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

// Rows of length r <= 64*V*NV held in registers, one wave per row at a time.
// Each wave walks rows w, w + W, ... (W = all waves of the grid) and loads the
// next row (and its mask vectors) while it finishes the current one.  NOUT:
// mask row axes (0 = no mask; see mask_row_offset).  FULL: r == 64*V*NV, every
// lane holds NV whole vectors (no per-vector bounds, one straight-line body).
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
        if (scale) {  // the Div (or Mul) node before the mask Add: the same IEEE operation per element
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
        T *q = y + row * (int64_t)r;
#pragma unroll
        for (int c = 0; c < NV; c++) {
            const int col = (c * 64 + lane) * V;
            if (FULL || col < r) {
                Vec<T, V> o;
#pragma unroll
                for (int k = 0; k < V; k++) o.v[k] = div_row<T>(cur[c].v[k], sum, rs);
                vstore_nt<T, V>(q + col, o);
            }
        }
#pragma unroll
        for (int c = 0; c < NV; c++) {
            cur[c] = nxt[c];
            if constexpr (MASK) mcur[c] = mnxt[c];
        }
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
#define LX_SM_CASE(N)                                                                                           \
    case N:                                                                                                     \
        if (full && N <= 4)                                                                                     \
            hipLaunchKernelGGL((k_softmax_wave<T, V, N, NOUT, (N <= 4)>), dim3((unsigned)g), dim3(kSBlock), 0, s, x, y, \
                               a.outer, r, m, a.mask_inner, a.mask_rows, (const T *)a.scale, a.scale_div);      \
        else                                                                                                    \
            hipLaunchKernelGGL((k_softmax_wave<T, V, N, NOUT, false>), dim3((unsigned)g), dim3(kSBlock), 0, s, x, y,  \
                               a.outer, r, m, a.mask_inner, a.mask_rows, (const T *)a.scale, a.scale_div);      \
        break;
    switch (nv) {
        LX_SM_CASE(1) LX_SM_CASE(2) LX_SM_CASE(3) LX_SM_CASE(4) LX_SM_CASE(5) LX_SM_CASE(6) LX_SM_CASE(7) LX_SM_CASE(8)
    default: return hipErrorInvalidValue;
    }
#undef LX_SM_CASE
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

template <typename T>
static hipError_t softmax_typed(const SoftmaxArgs &a, hipStream_t s) {
    constexpr int VW = VecWidth<T>::value;
    const bool wave_ok = a.inner == 1 && a.r <= 64 * VW * 8 && a.outer < (1ll << 31);
    if (wave_ok) {
        if (a.vec > 1 && a.r % VW == 0) {
            if (a.mask) return softmax_wave_dispatch<T, VW, true>(a, s);
            return softmax_wave_dispatch<T, VW, false>(a, s);
        }
        if (a.r <= 64 * 8) {
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
    if (inner != 1 || outer >= (1ll << 31) || r > 64 * vw * 8) return false;
    return (vec > 1 && r % vw == 0) || r <= 64 * 8;
}

hipError_t launch_softmax(const SoftmaxArgs &a, hipStream_t s) {
    if (a.outer * a.r * a.inner == 0) return hipSuccess;
    if (a.dtype == kFloat) return softmax_typed<float>(a, s);
    if (a.dtype == kDouble) return softmax_typed<double>(a, s);
    return hipErrorInvalidValue;
}

}  // namespace lx
