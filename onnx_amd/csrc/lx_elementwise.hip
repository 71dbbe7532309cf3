// lx_elementwise.hip -- gfx950 kernels for the binary / unary / cast operators
// and the fused GELU subgraph.
//
// Replaces the C# elementwise engines Apply / VectorizedApply
// (TensorOps.cs:18-123) and the broadcast materialisation ToDenseTensor
// (Tensor.cs:1605-1613): broadcast operands are read in place through stride-0
// addressing instead of being copied.
//
// Memory-bound design: every lane moves 16 bytes per access (dwordx4) with
// nontemporal loads and stores, and the grid covers the whole array with one
// vector per lane (measured faster on MI355X than grid-stride loops with
// several loads in flight per lane).
#include <algorithm>
#include <limits>
#include <type_traits>

#include "lx_device.h"
#include "lx_kernels.h"

#pragma clang fp contract(off)

namespace lx {

constexpr int kBlock = 256;
constexpr int kMaxBlocks = 1 << 24;  // beyond this the kernels loop
constexpr int kDivVecsPerLane = 4;  // integer Div: vectors loaded per lane before computing
// integer Div by a divisor constant along the outermost axis: rows per lane sharing one reciprocal, and
// lanes per block, by element size (C4 [64,1,4096] / [1,256,4096] on MI355X, kernel time over 100 launches
// in one process: int64 86.5 us with 4 rows in 256-lane blocks, 84.3 with 2 rows, 82.1 with 2 rows in
// 128-lane blocks; int32 43.6 us with 4 rows, 44.4 with 2, 43.8 with 2 in 128-lane blocks)
template <typename T> constexpr int kDivRowsPerLane = sizeof(T) == 8 ? 2 : 4;
template <typename T> constexpr int kDivRowsBlock = sizeof(T) == 8 ? 128 : kBlock;
// Cast: two vectors per lane for arrays of [2^16, 2^22) vectors (a 25 MB float copy: 5.75 -> 4.86 us on
// MI355X); one per lane above (an 805 MB int64 -> float Cast: 125 us with one, 132 us with two)
constexpr int64_t kCastTwoMin = 1 << 16, kCastTwoMax = 1 << 22;
// Arrays of kTileUMin to kTileUMax vectors (8 to 32 MB of floats) run as one-wave tiles of 4 x 64 vectors:
// measured on MI355X (graph replays over rotating buffers), C2's [8,512,768] - [8,512,1] 5.9 -> 5.2 us and
// * gamma[768] 6.1 -> 5.4 us against tiles of 2 x 64, a 17 MB copy 6.9 -> 6.1-6.5 us against two vectors per
// lane in 256-lane blocks; outside the window four vectors per lane were slower (8 MB +14%, 67 MB +3%, 400 MB
// +4%: too few blocks below it, too little overlap above).
constexpr int64_t kTileUMin = 1 << 19, kTileUMax = 1 << 21;

template <int CODE> struct CType;
template <> struct CType<kFloat> { using T = float; };
template <> struct CType<kDouble> { using T = double; };
template <> struct CType<kUInt8> { using T = uint8_t; };
template <> struct CType<kInt8> { using T = int8_t; };
template <> struct CType<kUInt16> { using T = uint16_t; };
template <> struct CType<kInt16> { using T = int16_t; };
template <> struct CType<kInt32> { using T = int32_t; };
template <> struct CType<kUInt32> { using T = uint32_t; };
template <> struct CType<kInt64> { using T = int64_t; };
template <> struct CType<kUInt64> { using T = uint64_t; };
template <> struct CType<kBool> { using T = uint8_t; };

static inline int grid_for(int64_t work_items, int per_block) {
    int64_t g = (work_items + per_block - 1) / per_block;
    if (g < 1) g = 1;
    if (g > kMaxBlocks) g = kMaxBlocks;
    return (int)g;
}

__global__ void k_reset_errs(ErrFlags *e) {
    if (threadIdx.x == 0) {
        e->first_dbz = ~0ull;
        e->first_ovf = ~0ull;
    }
}

template <typename T>
__global__ __launch_bounds__(kBlock) void k_fill(T *y, int64_t n, T v) {
    for (int64_t i = (int64_t)blockIdx.x * kBlock + threadIdx.x; i < n; i += (int64_t)gridDim.x * kBlock) y[i] = v;
}

hipError_t launch_fill(void *y, int64_t n, int esize, uint64_t bits, hipStream_t s) {
    if (n == 0) return hipSuccess;
    int g = grid_for(n, kBlock);
    switch (esize) {
    case 1: hipLaunchKernelGGL(k_fill<uint8_t>, dim3(g), dim3(kBlock), 0, s, (uint8_t *)y, n, (uint8_t)bits); break;
    case 2: hipLaunchKernelGGL(k_fill<uint16_t>, dim3(g), dim3(kBlock), 0, s, (uint16_t *)y, n, (uint16_t)bits); break;
    case 4: hipLaunchKernelGGL(k_fill<uint32_t>, dim3(g), dim3(kBlock), 0, s, (uint32_t *)y, n, (uint32_t)bits); break;
    case 8: hipLaunchKernelGGL(k_fill<uint64_t>, dim3(g), dim3(kBlock), 0, s, (uint64_t *)y, n, (uint64_t)bits); break;
    default: return hipErrorInvalidValue;
    }
    return hipGetLastError();
}

hipError_t launch_reset_errs(ErrFlags *e, hipStream_t s) {
    hipLaunchKernelGGL(k_reset_errs, dim3(1), dim3(64), 0, s, e);
    return hipGetLastError();
}

// One block: every lane copies its words and fences at system scope, the block
// meets, then lane 0 stores the sequence number with release semantics.
// reset (null, or src itself): each word is set to all ones after it has been
// copied, by the thread that read it -- the cleared state of an error record,
// so the next check on the stream needs no reset launch of its own.  A record of at
// most kPublishFew words (an error record) is copied by lane 0 alone, whose release
// store then orders its own copies: no fence or barrier of the other lanes.
constexpr int64_t kPublishFew = 4;
__global__ __launch_bounds__(kBlock) void k_publish(const uint64_t *src, int64_t n, uint64_t *__restrict__ dst,
                                                    uint64_t *seq_dst, uint64_t seq, uint64_t *reset) {
    if (n <= kPublishFew) {
        if (threadIdx.x == 0) {
            for (int64_t i = 0; i < n; i++) {
                dst[i] = src[i];
                if (reset) reset[i] = ~0ull;
            }
            __hip_atomic_store(seq_dst, seq, __ATOMIC_RELEASE, __HIP_MEMORY_SCOPE_SYSTEM);
        }
        return;
    }
    for (int64_t i = threadIdx.x; i < n; i += kBlock) {
        dst[i] = src[i];
        if (reset) reset[i] = ~0ull;
    }
    __threadfence_system();
    __syncthreads();
    if (threadIdx.x == 0) __hip_atomic_store(seq_dst, seq, __ATOMIC_RELEASE, __HIP_MEMORY_SCOPE_SYSTEM);
}

hipError_t launch_publish(const uint64_t *src, int64_t n, uint64_t *dst, uint64_t *seq_dst, uint64_t seq,
                          uint64_t *reset, hipStream_t s) {
    hipLaunchKernelGGL(k_publish, dim3(1), dim3(n <= kPublishFew ? 64 : kBlock), 0, s, src, n, dst, seq_dst, seq, reset);
    return hipGetLastError();
}

constexpr int kDivScanU = 2;      // vectors per lane, all loaded before any is tested
constexpr int kDivScanBlock = 1024;

// Eager integer Div whose divisor is much smaller than its output: the divisor alone decides whether the
// call can throw (a zero divides by zero, and for signed types a minus one can overflow against MIN).
// Each block ORs what its lanes find (bit 0: a zero, bit 1: a minus one) and stores (seq << 2) | bits into
// its own slot of mapped host memory with one relaxed system-scope store: the verdict is the stored word
// itself, so no fence orders anything before it, and no block waits for another.  The loads are ordinary
// (cacheable): the quotient kernel queued behind reads the same divisor.
template <typename T>
__global__ __launch_bounds__(kDivScanBlock) void k_div_scan(const T *__restrict__ b, int64_t n, int vec,
                                                     uint64_t *slots, uint64_t seq) {
    constexpr int V = 16 / (int)sizeof(T);
    constexpr bool kSigned = std::is_signed<T>::value;
    bool zero = false, minus1 = false;
    const int64_t nv = vec ? n / V : 0;
    // kDivScanU vectors per lane issued before any is tested, in 1024-lane blocks: the scan is one round
    // trip of many waves, not a chain of them (C4's 8 MB int64 divisor is one step of 256 blocks; with
    // 256-lane blocks and eight rounds of loads it took 6.5 us, with 256-lane blocks and eight vectors
    // per lane about 4)
    const int64_t step = (int64_t)gridDim.x * kDivScanBlock * kDivScanU;
    for (int64_t i0 = (int64_t)blockIdx.x * kDivScanBlock * kDivScanU + threadIdx.x; i0 < nv; i0 += step) {
        Vec<T, V> v[kDivScanU];
#pragma unroll
        for (int u = 0; u < kDivScanU; u++)
            if (i0 + u * kDivScanBlock < nv) v[u] = vload<T, V>(b + (i0 + u * kDivScanBlock) * V);
#pragma unroll
        for (int u = 0; u < kDivScanU; u++) {
            if (i0 + u * kDivScanBlock < nv) {
#pragma unroll
                for (int k = 0; k < V; k++) {
                    zero = zero || v[u].v[k] == (T)0;
                    if constexpr (kSigned) minus1 = minus1 || v[u].v[k] == (T)-1;
                }
            }
        }
    }
    const int64_t stride = (int64_t)gridDim.x * kDivScanBlock;
    for (int64_t i = nv * V + (int64_t)blockIdx.x * kDivScanBlock + threadIdx.x; i < n; i += stride) {
        zero = zero || b[i] == (T)0;
        if constexpr (kSigned) minus1 = minus1 || b[i] == (T)-1;
    }
    __shared__ uint32_t waves[kDivScanBlock / 64];
    const uint32_t w = (__ballot(zero) ? 1u : 0u) | (__ballot(minus1) ? 2u : 0u);
    if ((threadIdx.x & 63) == 0) waves[threadIdx.x >> 6] = w;
    __syncthreads();
    if (threadIdx.x == 0) {
        uint32_t all = 0;
#pragma unroll
        for (int i = 0; i < kDivScanBlock / 64; i++) all |= waves[i];
        __hip_atomic_store(slots + blockIdx.x, (seq << 2) | all, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM);
    }
}

int div_scan_blocks(int64_t n, int esize) {
    const int64_t vecs = (n * esize + 15) / 16;
    const int64_t g = (vecs + kDivScanBlock * kDivScanU - 1) / (kDivScanBlock * kDivScanU);
    return (int)std::max<int64_t>(1, std::min<int64_t>(g, kScanSlots));
}

hipError_t launch_div_scan(int dtype, const void *b, int64_t n, int vec, uint64_t *slots, uint64_t seq,
                           hipStream_t s) {
    switch (dtype) {
    case kInt32:
        hipLaunchKernelGGL(k_div_scan<int32_t>, dim3(div_scan_blocks(n, 4)), dim3(kDivScanBlock), 0, s, (const int32_t *)b, n,
                           vec, slots, seq);
        break;
    case kInt64:
        hipLaunchKernelGGL(k_div_scan<int64_t>, dim3(div_scan_blocks(n, 8)), dim3(kDivScanBlock), 0, s, (const int64_t *)b, n,
                           vec, slots, seq);
        break;
    case kUInt8:
        hipLaunchKernelGGL(k_div_scan<uint8_t>, dim3(div_scan_blocks(n, 1)), dim3(kDivScanBlock), 0, s, (const uint8_t *)b, n,
                           vec, slots, seq);
        break;
    default: return hipErrorInvalidValue;
    }
    return hipGetLastError();
}

// Eager Gather whose indices are far fewer than its output's elements: whether every index lies in
// [-dim, dim) -- the only way the call can fail once its shapes are checked -- from the indices alone, with
// the same per-block slots and store as k_div_scan (bit 0: an index out of range).
template <typename I>
__global__ __launch_bounds__(kDivScanBlock) void k_index_scan(const I *__restrict__ idx, int64_t n, int64_t dim,
                                                              uint64_t *slots, uint64_t seq) {
    constexpr int U = 8;  // indices per lane, all loaded before any is tested
    bool out = false;
    const int64_t step = (int64_t)gridDim.x * kDivScanBlock * U;
    for (int64_t i0 = (int64_t)blockIdx.x * kDivScanBlock * U + threadIdx.x; i0 < n; i0 += step) {
        I v[U];
#pragma unroll
        for (int u = 0; u < U; u++) v[u] = i0 + u * kDivScanBlock < n ? idx[i0 + u * kDivScanBlock] : (I)0;
#pragma unroll
        for (int u = 0; u < U; u++) out = out || (int64_t)v[u] < -dim || (int64_t)v[u] >= dim;
    }
    __shared__ uint32_t waves[kDivScanBlock / 64];
    const uint32_t w = __ballot(out) ? 1u : 0u;
    if ((threadIdx.x & 63) == 0) waves[threadIdx.x >> 6] = w;
    __syncthreads();
    if (threadIdx.x == 0) {
        uint32_t all = 0;
#pragma unroll
        for (int i = 0; i < kDivScanBlock / 64; i++) all |= waves[i];
        __hip_atomic_store(slots + blockIdx.x, (seq << 2) | all, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM);
    }
}

int index_scan_blocks(int64_t n) {
    const int64_t g = (n + kDivScanBlock * 8 - 1) / (kDivScanBlock * 8);
    return (int)std::max<int64_t>(1, std::min<int64_t>(g, kScanSlots));
}

hipError_t launch_index_scan(int idx_dtype, const void *idx, int64_t n, int64_t dim, uint64_t *slots, uint64_t seq,
                             hipStream_t s) {
    if (idx_dtype == kInt32)
        hipLaunchKernelGGL(k_index_scan<int32_t>, dim3(index_scan_blocks(n)), dim3(kDivScanBlock), 0, s,
                           (const int32_t *)idx, n, dim, slots, seq);
    else if (idx_dtype == kInt64)
        hipLaunchKernelGGL(k_index_scan<int64_t>, dim3(index_scan_blocks(n)), dim3(kDivScanBlock), 0, s,
                           (const int64_t *)idx, n, dim, slots, seq);
    else
        return hipErrorInvalidValue;
    return hipGetLastError();
}

// ---------------------------------------------------------------------------
// Binary element operation with C# semantics.
//   float/double: IEEE-754 round to nearest even (TensorOps.cs:241-297).
//   byte: (byte)(l op r) after int promotion (TensorOps.cs:235, 253, 271, 289).
//   int32/int64: unchecked two's-complement wrap, '/' truncates; x/0 and
//   MIN/-1 record the element index (DivideByZero / Overflow exceptions).
// ---------------------------------------------------------------------------
template <int OP, typename T>
__device__ __forceinline__ T bin_apply(T l, T r, uint64_t idx, ErrFlags *e) {
    if constexpr (std::is_floating_point<T>::value) {
        if constexpr (OP == kAdd) return l + r;
        else if constexpr (OP == kSub) return l - r;
        else if constexpr (OP == kMul) return l * r;
        else if constexpr (OP == kDiv) return l / r;
        else return pow_lx(l, r);
    } else if constexpr (sizeof(T) == 1) {
        int li = l, ri = r;
        if constexpr (OP == kAdd) return (T)(li + ri);
        else if constexpr (OP == kSub) return (T)(li - ri);
        else if constexpr (OP == kMul) return (T)(li * ri);
        else {
            if (ri == 0) {
                atomicMin(&e->first_dbz, (unsigned long long)idx);
                return 0;
            }
            return (T)(li / ri);
        }
    } else {
        using U = typename std::make_unsigned<T>::type;
        if constexpr (OP == kAdd) return (T)((U)l + (U)r);
        else if constexpr (OP == kSub) return (T)((U)l - (U)r);
        else if constexpr (OP == kMul) return (T)((U)l * (U)r);
        else {
            if (r == 0) {
                atomicMin(&e->first_dbz, (unsigned long long)idx);
                return 0;
            }
            if (l == std::numeric_limits<T>::min() && r == (T)-1) {
                atomicMin(&e->first_ovf, (unsigned long long)idx);
                return 0;
            }
            if constexpr (sizeof(T) == 4) {
                return l / r;
            } else {
                // both operands inside int32: divide the magnitudes in 32 bits,
                // apply the sign in 64 (so -2^31 / -1 = 2^31 stays exact)
                if (l == (T)(int32_t)l && r == (T)(int32_t)r) {
                    const uint32_t ua = l < 0 ? (uint32_t)(-l) : (uint32_t)l;
                    const uint32_t ub = r < 0 ? (uint32_t)(-r) : (uint32_t)r;
                    const int64_t q = (int64_t)(ua / ub);
                    return ((l < 0) != (r < 0)) ? (T)(-q) : (T)q;
                }
                return l / r;
            }
        }
    }
}

// The V elements of one vector.  Integer division (int32, int64): when every
// divisor in the vector is nonzero, no pair is MIN / -1 and every int64 operand
// lies inside int32, the quotients come from the branch-free double-precision
// division; any other vector takes the element-wise path with its error records.
template <int OP, typename T, int V>
__device__ __forceinline__ Vec<T, V> bin_apply_vec(const Vec<T, V> &va, const Vec<T, V> &vb, uint64_t idx0,
                                                   ErrFlags *e) {
    Vec<T, V> vy;
    if constexpr (OP == kDiv && std::is_integral<T>::value && sizeof(T) >= 4) {
        bool plain = true;
#pragma unroll
        for (int k = 0; k < V; k++) {
            const T l = va.v[k], r = vb.v[k];
            plain = plain && r != 0 && !(l == (T)std::numeric_limits<int32_t>::min() && r == (T)-1);
            if constexpr (sizeof(T) == 8) plain = plain && l == (T)(int32_t)l && r == (T)(int32_t)r;
        }
        if (plain) {
#pragma unroll
            for (int k = 0; k < V; k++) vy.v[k] = (T)sdiv32_lx((int32_t)va.v[k], (int32_t)vb.v[k]);
            return vy;
        }
    }
#pragma unroll
    for (int k = 0; k < V; k++) vy.v[k] = bin_apply<OP, T>(va.v[k], vb.v[k], idx0 + k, e);
    return vy;
}

// SAME / SCALAR_A / SCALAR_B: dense output walk with 16-byte vectors.
template <int OP, typename T, int LAYOUT, int V>
__global__ __launch_bounds__(kBlock) void k_binary_flat(const T *__restrict__ a, const T *__restrict__ b,
                                                        T *__restrict__ y, int64_t n, ErrFlags *errs) {
    const int64_t nv = n / V;
    T sa = T(), sb = T();
    if constexpr (LAYOUT == kScalarA) sa = a[0];
    if constexpr (LAYOUT == kScalarB) sb = b[0];
    for (int64_t i = (int64_t)blockIdx.x * kBlock + threadIdx.x; i < nv; i += (int64_t)gridDim.x * kBlock) {
        Vec<T, V> va, vb;
        if constexpr (LAYOUT != kScalarA) va = vload_nt<T, V>(a + i * V);
        else {
#pragma unroll
            for (int k = 0; k < V; k++) va.v[k] = sa;
        }
        if constexpr (LAYOUT != kScalarB) vb = vload_nt<T, V>(b + i * V);
        else {
#pragma unroll
            for (int k = 0; k < V; k++) vb.v[k] = sb;
        }
        vstore_nt<T, V>(y + i * V, bin_apply_vec<OP, T, V>(va, vb, (uint64_t)(i * V), errs));
    }
    const int64_t tail = n - nv * V;
    if (blockIdx.x == 0 && (int64_t)threadIdx.x < tail) {
        int64_t i = nv * V + threadIdx.x;
        T l = (LAYOUT == kScalarA) ? sa : a[i];
        T r = (LAYOUT == kScalarB) ? sb : b[i];
        y[i] = bin_apply<OP, T>(l, r, (uint64_t)i, errs);
    }
}

// The same layouts on mid-sized arrays (kTileUMin to kTileUMax vectors): one-wave blocks over tiles of
// 64 * U vectors, all loaded before any is computed, no loop.  tile0: the first tile of this launch.
template <int OP, typename T, int LAYOUT, int V, int U>
__global__ __launch_bounds__(64) void k_binary_flat_tile(const T *__restrict__ a, const T *__restrict__ b,
                                                         T *__restrict__ y, int64_t n, int64_t tile0, ErrFlags *errs) {
    const int64_t nv = n / V;
    T sa = T(), sb = T();
    if constexpr (LAYOUT == kScalarA) sa = a[0];
    if constexpr (LAYOUT == kScalarB) sb = b[0];
    const int64_t i0 = (tile0 + blockIdx.x) * (64 * U) + threadIdx.x;
    Vec<T, V> va[U], vb[U];
#pragma unroll
    for (int u = 0; u < U; u++) {
        const int64_t i = i0 + u * 64;
        if (i < nv) {
            if constexpr (LAYOUT != kScalarA) va[u] = vload_nt<T, V>(a + i * V);
            if constexpr (LAYOUT != kScalarB) vb[u] = vload_nt<T, V>(b + i * V);
        }
    }
#pragma unroll
    for (int u = 0; u < U; u++) {
        const int64_t i = i0 + u * 64;
        if (i < nv) {
            if constexpr (LAYOUT == kScalarA) {
#pragma unroll
                for (int k = 0; k < V; k++) va[u].v[k] = sa;
            }
            if constexpr (LAYOUT == kScalarB) {
#pragma unroll
                for (int k = 0; k < V; k++) vb[u].v[k] = sb;
            }
            vstore_nt<T, V>(y + i * V, bin_apply_vec<OP, T, V>(va[u], vb[u], (uint64_t)(i * V), errs));
        }
    }
    const int64_t tail = n - nv * V;
    if (tile0 + blockIdx.x == 0 && (int64_t)threadIdx.x < tail) {
        const int64_t i = nv * V + threadIdx.x;
        const T l = (LAYOUT == kScalarA) ? sa : a[i];
        const T r = (LAYOUT == kScalarB) ? sb : b[i];
        y[i] = bin_apply<OP, T>(l, r, (uint64_t)i, errs);
    }
}

// General broadcast: output row-major [rows, inner]; operands addressed via
// per-axis strides (0 on broadcast axes).  AIN/BIN: innermost axis contiguous
// (1) or broadcast (0) for A/B.  32-bit vector index with fast division.
// a_nt / b_nt: the operand is read exactly once (no broadcast axis), so it is
// streamed with nontemporal loads; broadcast operands are re-read and must stay
// cacheable.  U vectors per lane, a grid stride apart, all loaded before any is
// computed: ops with many instructions per element (integer Div) keep more
// bytes in flight per wave.
template <typename T, int AIN, int BIN, int V>
__device__ __forceinline__ void nd_load(const T *__restrict__ a, const T *__restrict__ b, uint32_t v,
                                        const NdLayout &L, int a_nt, int b_nt, Vec<T, V> &va, Vec<T, V> &vb) {
    uint32_t row = fdiv(v, L.inner_v);
    uint32_t cv = v - row * L.inner_v.d;
    int64_t ao = 0, bo = 0;
    uint32_t rr = row;
#pragma unroll
    for (int d = 0; d < kMaxOuter; d++) {
        if (d < L.nouter) {
            uint32_t q = fdiv(rr, L.odiv[d]);
            uint32_t id = rr - q * L.odiv[d].d;
            ao += (int64_t)id * L.a_str[d];
            bo += (int64_t)id * L.b_str[d];
            rr = q;
        }
    }
    const int64_t col = (int64_t)cv * V;
    if constexpr (AIN) va = a_nt ? vload_nt<T, V>(a + ao + col) : vload<T, V>(a + ao + col);
    else {
        T s = a[ao];
#pragma unroll
        for (int k = 0; k < V; k++) va.v[k] = s;
    }
    if constexpr (BIN) vb = b_nt ? vload_nt<T, V>(b + bo + col) : vload<T, V>(b + bo + col);
    else {
        T s = b[bo];
#pragma unroll
        for (int k = 0; k < V; k++) vb.v[k] = s;
    }
}

template <int OP, typename T, int AIN, int BIN, int V, int U>
__global__ __launch_bounds__(kBlock) void k_binary_nd(const T *__restrict__ a, const T *__restrict__ b,
                                                      T *__restrict__ y, uint32_t nv, NdLayout L, int a_nt, int b_nt,
                                                      ErrFlags *errs) {
    const uint32_t stride = gridDim.x * kBlock;
    for (uint32_t v0 = blockIdx.x * kBlock + threadIdx.x; v0 < nv; v0 += stride * U) {
        Vec<T, V> va[U], vb[U];
#pragma unroll
        for (int u = 0; u < U; u++)
            if (u == 0 || v0 + u * stride < nv) nd_load<T, AIN, BIN, V>(a, b, v0 + u * stride, L, a_nt, b_nt, va[u], vb[u]);
#pragma unroll
        for (int u = 0; u < U; u++) {
            const uint32_t v = v0 + u * stride;
            if (u == 0 || v < nv)
                vstore_nt<T, V>(y + (int64_t)v * V, bin_apply_vec<OP, T, V>(va[u], vb[u], (uint64_t)v * V, errs));
        }
    }
}

// Broadcast ops with an operand read once, on large arrays: one-wave blocks over tiles of 64 * U vectors
// (vector u of lane l at tile * 64 * U + u * 64 + l), all U loaded before any is computed, no loop, so a
// wave ends right after its streaming stores.  Measured on MI355X against k_binary_nd's 256-lane blocks,
// interleaved in one process: C3 mask Add 62.7 -> 62.2 us, C2's per-row Sub / Div and gamma Mul on
// [8,512,768] 6.3 -> 5.8-6.1 us, 400 MB of x * gamma[1536] 126.2 -> 125.5 us and [1,96] + [N,96]
// 127.5 -> 122.4 us, C3 in double 65.1 -> 62.3 us.  Ordinary stores lost up to 8% on the re-read row
// operands (x * gamma).  Outputs built only from re-read broadcast operands (C4) ran 35% slower in
// one-wave blocks; for 8-byte elements they take B = 128 lanes, one vector each (int64 [64,1,4096] +
// [1,256,4096]: 76.4-79 -> 75.3-75.9 us against k_binary_nd's 256-lane grid-stride loop; 64 lanes 116 us,
// 128 x 2 vectors 79 us; 4-byte elements lost 1 us and stay with k_binary_nd).  tile0: the first tile
// of this launch.
template <int OP, typename T, int AIN, int BIN, int V, int U, int B = 64>
__global__ __launch_bounds__(B) void k_binary_tile(const T *__restrict__ a, const T *__restrict__ b,
                                                   T *__restrict__ y, uint32_t nv, uint32_t tile0, NdLayout L,
                                                   int a_nt, int b_nt, ErrFlags *errs) {
    const uint32_t v0 = (tile0 + blockIdx.x) * (uint32_t)(B * U) + threadIdx.x;
    Vec<T, V> va[U], vb[U];
#pragma unroll
    for (int u = 0; u < U; u++)
        if (v0 + u * B < nv) nd_load<T, AIN, BIN, V>(a, b, v0 + u * B, L, a_nt, b_nt, va[u], vb[u]);
#pragma unroll
    for (int u = 0; u < U; u++) {
        const uint32_t v = v0 + u * B;
        if (v < nv) vstore_nt<T, V>(y + (int64_t)v * V, bin_apply_vec<OP, T, V>(va[u], vb[u], (uint64_t)v * V, errs));
    }
}

// Integer Div whose divisor does not vary along the outermost output axis (b
// stride 0 there, as in [64,1,4096] / [1,256,4096]).  Lane t takes divisor
// vector vr = t mod rest (rest = vectors per outermost index) and the U
// outermost indices r = (t / rest) * U + u: the reciprocals of the divisor
// (seed and Newton step, most of the division's instructions) are computed
// once for U quotients.  Same arithmetic, fallback and error records per
// element as k_binary_nd.
template <typename T, int AIN, int BIN, int V, int U, int B = kBlock>
__global__ __launch_bounds__(B) void k_div_rows(const T *__restrict__ a, const T *__restrict__ b,
                                                     T *__restrict__ y, uint32_t lanes, FastDiv rest,
                                                     uint32_t R, NdLayout L, int a_nt, int b_nt, ErrFlags *errs) {
    const int top = L.nouter - 1;
    const int64_t a_top = L.a_str[top];
    for (uint32_t t = blockIdx.x * B + threadIdx.x; t < lanes; t += gridDim.x * B) {
        const uint32_t chunk = fdiv(t, rest);
        const uint32_t vr = t - chunk * rest.d;
        const uint32_t row = fdiv(vr, L.inner_v);
        const uint32_t cv = vr - row * L.inner_v.d;
        int64_t ao = 0, bo = 0;
        uint32_t rr = row;
#pragma unroll
        for (int d = 0; d < kMaxOuter - 1; d++) {
            if (d < top) {
                uint32_t q = fdiv(rr, L.odiv[d]);
                uint32_t id = rr - q * L.odiv[d].d;
                ao += (int64_t)id * L.a_str[d];
                bo += (int64_t)id * L.b_str[d];
                rr = q;
            }
        }
        const int64_t col = (int64_t)cv * V;
        Vec<T, V> vb;
        if constexpr (BIN) vb = b_nt ? vload_nt<T, V>(b + bo + col) : vload<T, V>(b + bo + col);
        else {
            const T sv = b[bo];
#pragma unroll
            for (int k = 0; k < V; k++) vb.v[k] = sv;
        }
        const uint32_t r0 = chunk * U;
        Vec<T, V> va[U];
#pragma unroll
        for (int u = 0; u < U; u++) {
            if (u == 0 || r0 + u < R) {
                const T *ap = a + ao + (int64_t)(r0 + u) * a_top;
                if constexpr (AIN) va[u] = a_nt ? vload_nt<T, V>(ap + col) : vload<T, V>(ap + col);
                else {
                    const T sv = ap[0];
#pragma unroll
                    for (int k = 0; k < V; k++) va[u].v[k] = sv;
                }
            }
        }
        bool bplain = true;
        double yr[V];
#pragma unroll
        for (int k = 0; k < V; k++) {
            const T r = vb.v[k];
            bplain = bplain && r != 0;
            if constexpr (sizeof(T) == 8) bplain = bplain && r == (T)(int32_t)r;
            yr[k] = sdiv32_recip_lx((int32_t)r);
        }
#pragma unroll
        for (int u = 0; u < U; u++) {
            if (u == 0 || r0 + u < R) {
                const uint32_t v = (r0 + u) * rest.d + vr;
                bool plain = bplain;
#pragma unroll
                for (int k = 0; k < V; k++) {
                    const T l = va[u].v[k], r = vb.v[k];
                    plain = plain && !(l == (T)std::numeric_limits<int32_t>::min() && r == (T)-1);
                    if constexpr (sizeof(T) == 8) plain = plain && l == (T)(int32_t)l;
                }
                Vec<T, V> vy;
                if (plain) {
#pragma unroll
                    for (int k = 0; k < V; k++) vy.v[k] = (T)sdiv32_quot((int32_t)va[u].v[k], yr[k]);
                } else {
#pragma unroll
                    for (int k = 0; k < V; k++)
                        vy.v[k] = bin_apply<kDiv, T>(va[u].v[k], vb.v[k], (uint64_t)v * V + k, errs);
                }
                vstore_nt<T, V>(y + (int64_t)v * V, vy);
            }
        }
    }
}

// Same as k_binary_nd for more than 2^31 vectors: 64-bit index arithmetic.
template <int OP, typename T, int AIN, int BIN, int V>
__global__ __launch_bounds__(kBlock) void k_binary_nd64(const T *__restrict__ a, const T *__restrict__ b,
                                                        T *__restrict__ y, int64_t nv, NdLayout L,
                                                        BinArgs big, ErrFlags *errs) {
    for (int64_t v = (int64_t)blockIdx.x * kBlock + threadIdx.x; v < nv; v += (int64_t)gridDim.x * kBlock) {
        int64_t row = v / big.nd_inner_vn;
        int64_t cv = v - row * big.nd_inner_vn;
        int64_t ao = 0, bo = 0, rr = row;
        for (int d = 0; d < L.nouter; d++) {
            int64_t q = rr / big.nd_osize[d];
            int64_t id = rr - q * big.nd_osize[d];
            ao += id * L.a_str[d];
            bo += id * L.b_str[d];
            rr = q;
        }
        const int64_t col = cv * V;
        Vec<T, V> va, vb;
#pragma unroll
        for (int k = 0; k < V; k++) {
            va.v[k] = AIN ? a[ao + col + k] : a[ao];
            vb.v[k] = BIN ? b[bo + col + k] : b[bo];
        }
        vstore<T, V>(y + v * V, bin_apply_vec<OP, T, V>(va, vb, (uint64_t)(v * V), errs));
    }
}

// kNd outputs whose inner axis is not a multiple of V (every pointer 16-byte aligned, n < 2^31): the
// output is walked in whole 16-byte vectors of its flat index.  An operand without broadcast axes has the
// output's layout and is read by vectors at the same flat index (flat = 1); a broadcast operand element by
// element: the vector's first element decomposed into (row, column), the next ones stepped along the row,
// the row's operand offsets decomposed again where the vector crosses into the next row.  The n mod V
// last elements are taken by lanes of block 0.  L.inner_v holds the inner length in elements.
template <int OP, typename T, int AIN, int BIN, int V>
__global__ __launch_bounds__(kBlock) void k_binary_rag(const T *__restrict__ a, const T *__restrict__ b,
                                                       T *__restrict__ y, uint32_t nvec, uint32_t n, NdLayout L,
                                                       int a_flat, int b_flat, ErrFlags *errs) {
    const uint32_t inner = L.inner_v.d;
    auto offsets = [&](uint32_t row, int64_t &ao, int64_t &bo) {
        ao = 0;
        bo = 0;
#pragma unroll
        for (int d = 0; d < kMaxOuter; d++) {
            if (d < L.nouter) {
                const uint32_t q = fdiv(row, L.odiv[d]);
                const uint32_t id = row - q * L.odiv[d].d;
                ao += (int64_t)id * L.a_str[d];
                bo += (int64_t)id * L.b_str[d];
                row = q;
            }
        }
    };
    for (uint32_t v = blockIdx.x * kBlock + threadIdx.x; v < nvec; v += gridDim.x * kBlock) {
        const uint32_t f = v * V;
        Vec<T, V> va, vb;
        if (a_flat) va = vload_nt<T, V>(a + f);
        if (b_flat) vb = vload_nt<T, V>(b + f);
        if (!a_flat || !b_flat) {
            uint32_t row = fdiv(f, L.inner_v);
            uint32_t col = f - row * inner;
            int64_t ao, bo;
            offsets(row, ao, bo);
#pragma unroll
            for (int k = 0; k < V; k++) {
                if (!a_flat) va.v[k] = AIN ? a[ao + col] : a[ao];
                if (!b_flat) vb.v[k] = BIN ? b[bo + col] : b[bo];
                if (++col == inner) {
                    col = 0;
                    offsets(++row, ao, bo);
                }
            }
        }
        vstore_nt<T, V>(y + f, bin_apply_vec<OP, T, V>(va, vb, (uint64_t)f, errs));
    }
    const uint32_t done = nvec * V;
    if (blockIdx.x == 0 && threadIdx.x < n - done) {
        const uint32_t f = done + threadIdx.x;
        const uint32_t row = fdiv(f, L.inner_v), col = f - row * inner;
        int64_t ao, bo;
        offsets(row, ao, bo);
        const T l = a_flat ? a[f] : (AIN ? a[ao + col] : a[ao]);
        const T r = b_flat ? b[f] : (BIN ? b[bo + col] : b[bo]);
        y[f] = bin_apply<OP, T>(l, r, (uint64_t)f, errs);
    }
}

template <int OP, typename T>
static hipError_t binary_rag(const BinArgs &A, ErrFlags *errs, hipStream_t s) {
    constexpr int V = VecWidth<T>::value;
    const T *a = (const T *)A.a;
    const T *b = (const T *)A.b;
    T *y = (T *)A.y;
    const uint32_t n = (uint32_t)A.n, nvec = n / V;
    const int g = grid_for(nvec > 0 ? nvec : 1, kBlock);
    switch (A.a_inner * 2 + A.b_inner) {
    case 3: hipLaunchKernelGGL((k_binary_rag<OP, T, 1, 1, V>), dim3(g), dim3(kBlock), 0, s, a, b, y, nvec, n, A.nd, A.a_once, A.b_once, errs); break;
    case 2: hipLaunchKernelGGL((k_binary_rag<OP, T, 1, 0, V>), dim3(g), dim3(kBlock), 0, s, a, b, y, nvec, n, A.nd, A.a_once, A.b_once, errs); break;
    case 1: hipLaunchKernelGGL((k_binary_rag<OP, T, 0, 1, V>), dim3(g), dim3(kBlock), 0, s, a, b, y, nvec, n, A.nd, A.a_once, A.b_once, errs); break;
    default: hipLaunchKernelGGL((k_binary_rag<OP, T, 0, 0, V>), dim3(g), dim3(kBlock), 0, s, a, b, y, nvec, n, A.nd, A.a_once, A.b_once, errs); break;
    }
    return hipGetLastError();
}

template <int OP, typename T, int V, int TU, int B = 64>
static hipError_t binary_tiles(const BinArgs &A, int key, int64_t nv, ErrFlags *errs, hipStream_t s) {
    const T *a = (const T *)A.a;
    const T *b = (const T *)A.b;
    T *y = (T *)A.y;
    const int64_t ntiles = (nv + B * TU - 1) / (B * TU);
    for (int64_t t0 = 0; t0 < ntiles; t0 += kMaxBlocks) {
        const int g = (int)std::min<int64_t>(kMaxBlocks, ntiles - t0);
        switch (key) {
        case 3: hipLaunchKernelGGL((k_binary_tile<OP, T, 1, 1, V, TU, B>), dim3(g), dim3(B), 0, s, a, b, y, (uint32_t)nv, (uint32_t)t0, A.nd, A.a_once, A.b_once, errs); break;
        case 2: hipLaunchKernelGGL((k_binary_tile<OP, T, 1, 0, V, TU, B>), dim3(g), dim3(B), 0, s, a, b, y, (uint32_t)nv, (uint32_t)t0, A.nd, A.a_once, A.b_once, errs); break;
        case 1: hipLaunchKernelGGL((k_binary_tile<OP, T, 0, 1, V, TU, B>), dim3(g), dim3(B), 0, s, a, b, y, (uint32_t)nv, (uint32_t)t0, A.nd, A.a_once, A.b_once, errs); break;
        default: hipLaunchKernelGGL((k_binary_tile<OP, T, 0, 0, V, TU, B>), dim3(g), dim3(B), 0, s, a, b, y, (uint32_t)nv, (uint32_t)t0, A.nd, A.a_once, A.b_once, errs); break;
        }
    }
    return hipGetLastError();
}

template <int OP, typename T, int V>
static hipError_t binary_typed_v(const BinArgs &A, ErrFlags *errs, hipStream_t s) {
    const T *a = (const T *)A.a;
    const T *b = (const T *)A.b;
    T *y = (T *)A.y;
    if (A.layout != kNd && A.n / V >= kTileUMin && A.n / V < kTileUMax) {
        const int64_t ntiles = (A.n / V + 255) / 256;
        for (int64_t t0 = 0; t0 < ntiles; t0 += kMaxBlocks) {
            const int g = (int)std::min<int64_t>(kMaxBlocks, ntiles - t0);
            switch (A.layout) {
            case kSame: hipLaunchKernelGGL((k_binary_flat_tile<OP, T, kSame, V, 4>), dim3(g), dim3(64), 0, s, a, b, y, A.n, t0, errs); break;
            case kScalarA: hipLaunchKernelGGL((k_binary_flat_tile<OP, T, kScalarA, V, 4>), dim3(g), dim3(64), 0, s, a, b, y, A.n, t0, errs); break;
            default: hipLaunchKernelGGL((k_binary_flat_tile<OP, T, kScalarB, V, 4>), dim3(g), dim3(64), 0, s, a, b, y, A.n, t0, errs); break;
            }
        }
        return hipGetLastError();
    }
    if (A.layout != kNd) {
        int64_t nv = A.n / V;
        int g = grid_for(nv > 0 ? nv : 1, kBlock);
        switch (A.layout) {
        case kSame: hipLaunchKernelGGL((k_binary_flat<OP, T, kSame, V>), dim3(g), dim3(kBlock), 0, s, a, b, y, A.n, errs); break;
        case kScalarA: hipLaunchKernelGGL((k_binary_flat<OP, T, kScalarA, V>), dim3(g), dim3(kBlock), 0, s, a, b, y, A.n, errs); break;
        default: hipLaunchKernelGGL((k_binary_flat<OP, T, kScalarB, V>), dim3(g), dim3(kBlock), 0, s, a, b, y, A.n, errs); break;
        }
        return hipGetLastError();
    }
    // With an operand streamed once, two vectors per lane: the index
    // decomposition and the NdLayout argument loads are amortised (C3 mask Add
    // on MI355X: 68 us with one vector per lane, 62 us with two, slower again
    // with four; [8,512,768] - [8,512,1]: 5.98 -> 5.81 us).  Outputs built only
    // from re-read broadcast operands (C4), and small launch-latency-bound
    // arrays (C1, below 2^16 vectors), run fastest with one per lane.
    const int64_t nv = A.n / V;
    const bool two = (A.a_once || A.b_once) && nv >= (1 << 16);
    const int key = A.a_inner * 2 + A.b_inner;
    if (nv < (1ll << 31)) {
        constexpr int U = (OP == kDiv && std::is_integral<T>::value && sizeof(T) >= 4) ? kDivVecsPerLane : 1;
        if constexpr (U > 1) {
            // divisor constant along the outermost axis: one reciprocal per U quotients
            const int top = A.nd.nouter - 1;
            if (nv >= (1 << 20) && top >= 0 && A.nd.b_str[top] == 0 && A.nd.odiv[top].d >= 2 &&
                nv % A.nd.odiv[top].d == 0) {
                constexpr int UR = kDivRowsPerLane<T>;
                const uint32_t R = A.nd.odiv[top].d;
                const int64_t rest = nv / R;
                const int64_t lanes = rest * ((R + UR - 1) / UR);
                const FastDiv fr = make_fastdiv((uint32_t)rest);
                constexpr int BR = kDivRowsBlock<T>;
                const int g = grid_for(lanes, BR);
                switch (key) {
                case 3: hipLaunchKernelGGL((k_div_rows<T, 1, 1, V, UR, BR>), dim3(g), dim3(BR), 0, s, a, b, y, (uint32_t)lanes, fr, R, A.nd, A.a_once, A.b_once, errs); break;
                case 2: hipLaunchKernelGGL((k_div_rows<T, 1, 0, V, UR, BR>), dim3(g), dim3(BR), 0, s, a, b, y, (uint32_t)lanes, fr, R, A.nd, A.a_once, A.b_once, errs); break;
                case 1: hipLaunchKernelGGL((k_div_rows<T, 0, 1, V, UR, BR>), dim3(g), dim3(BR), 0, s, a, b, y, (uint32_t)lanes, fr, R, A.nd, A.a_once, A.b_once, errs); break;
                default: hipLaunchKernelGGL((k_div_rows<T, 0, 0, V, UR, BR>), dim3(g), dim3(BR), 0, s, a, b, y, (uint32_t)lanes, fr, R, A.nd, A.a_once, A.b_once, errs); break;
                }
                return hipGetLastError();
            }
        }
        if (U == 1 && two) {
            if (nv >= kTileUMin && nv < kTileUMax) return binary_tiles<OP, T, V, 4>(A, key, nv, errs, s);
            return binary_tiles<OP, T, V, 2>(A, key, nv, errs, s);
        }
        if (U == 1 && sizeof(T) == 8 && nv >= (1 << 20)) return binary_tiles<OP, T, V, 1, 128>(A, key, nv, errs, s);
        const int64_t lanes = (U > 1 && nv >= (1 << 20)) ? (nv + U - 1) / U : two ? (nv + 1) / 2 : nv;
        const int g = grid_for(lanes, kBlock);
        switch (key) {
        case 3: hipLaunchKernelGGL((k_binary_nd<OP, T, 1, 1, V, U>), dim3(g), dim3(kBlock), 0, s, a, b, y, (uint32_t)nv, A.nd, A.a_once, A.b_once, errs); break;
        case 2: hipLaunchKernelGGL((k_binary_nd<OP, T, 1, 0, V, U>), dim3(g), dim3(kBlock), 0, s, a, b, y, (uint32_t)nv, A.nd, A.a_once, A.b_once, errs); break;
        case 1: hipLaunchKernelGGL((k_binary_nd<OP, T, 0, 1, V, U>), dim3(g), dim3(kBlock), 0, s, a, b, y, (uint32_t)nv, A.nd, A.a_once, A.b_once, errs); break;
        default: hipLaunchKernelGGL((k_binary_nd<OP, T, 0, 0, V, U>), dim3(g), dim3(kBlock), 0, s, a, b, y, (uint32_t)nv, A.nd, A.a_once, A.b_once, errs); break;
        }
    } else {
        const int g = grid_for(two ? (nv + 1) / 2 : nv, kBlock);
        switch (key) {
        case 3: hipLaunchKernelGGL((k_binary_nd64<OP, T, 1, 1, V>), dim3(g), dim3(kBlock), 0, s, a, b, y, nv, A.nd, A, errs); break;
        case 2: hipLaunchKernelGGL((k_binary_nd64<OP, T, 1, 0, V>), dim3(g), dim3(kBlock), 0, s, a, b, y, nv, A.nd, A, errs); break;
        case 1: hipLaunchKernelGGL((k_binary_nd64<OP, T, 0, 1, V>), dim3(g), dim3(kBlock), 0, s, a, b, y, nv, A.nd, A, errs); break;
        default: hipLaunchKernelGGL((k_binary_nd64<OP, T, 0, 0, V>), dim3(g), dim3(kBlock), 0, s, a, b, y, nv, A.nd, A, errs); break;
        }
    }
    return hipGetLastError();
}

template <int OP, typename T>
static hipError_t binary_typed(const BinArgs &A, ErrFlags *errs, hipStream_t s) {
    if (A.layout == kNd && A.rag) return binary_rag<OP, T>(A, errs, s);
    if (A.vec > 1) return binary_typed_v<OP, T, VecWidth<T>::value>(A, errs, s);
    return binary_typed_v<OP, T, 1>(A, errs, s);
}

template <typename T>
static hipError_t binary_by_op(const BinArgs &A, ErrFlags *errs, hipStream_t s) {
    switch (A.op) {
    case kAdd: return binary_typed<kAdd, T>(A, errs, s);
    case kSub: return binary_typed<kSub, T>(A, errs, s);
    case kMul: return binary_typed<kMul, T>(A, errs, s);
    case kDiv: return binary_typed<kDiv, T>(A, errs, s);
    case kPow:
        if constexpr (std::is_floating_point<T>::value) return binary_typed<kPow, T>(A, errs, s);
        return hipErrorInvalidValue;
    default: return hipErrorInvalidValue;
    }
}

hipError_t launch_binary(const BinArgs &A, ErrFlags *errs, hipStream_t s) {
    if (A.n == 0) return hipSuccess;
    switch (A.dtype) {
    case kFloat: return binary_by_op<float>(A, errs, s);
    case kDouble: return binary_by_op<double>(A, errs, s);
    case kUInt8: return binary_by_op<uint8_t>(A, errs, s);
    case kInt32: return binary_by_op<int32_t>(A, errs, s);
    case kInt64: return binary_by_op<int64_t>(A, errs, s);
    default: return hipErrorInvalidValue;
    }
}

// Float maps that look up the expf table (the GELU subgraph, Erf, Exp): one wave per block.  A block takes
// tiles of 64 * U consecutive vectors of V floats, vector u of lane l at tile * 64 * U + u * 64 + l, and
// loads all U before computing any; the wave copies the table into its own LDS slot after issuing its
// first tile's loads (exp_table_fill_wave), so the table's latency hides under them and no block barrier
// delays them.  Straight-line code, one tile per block (as a loop over tiles the same kernel ran 4-12%
// slower).  Measured
// on the C5 GELU (X[32,2048,3072], MI355X): 272.5 -> 246.6 us against four vectors per lane in a
// grid-stride loop of 256-lane blocks with a block-shared table, 247.3 us at U = 1, 251.4 at U = 4,
// 250.6 with two-wave blocks; a plain copy of the same bytes in one-wave blocks takes 243.3 us.
constexpr int kTabMapU = 2;

template <typename F, int V, int U>
__global__ __launch_bounds__(64) void k_map_tab(const float *__restrict__ x, float *__restrict__ y, int64_t n,
                                                int64_t tile0, uint32_t whole, F f) {
    __shared__ ExpTable tab;
    const int lane = threadIdx.x;
    const int64_t nv = n / V;
    const int64_t v0 = (tile0 + blockIdx.x) * (64 * U);
    // the wave's issue priority raised from its first instruction: waves already running win arbitration
    // over those just dispatched, so the waves holding loaded data finish first (C5 GELU on MI355X,
    // interleaved in one process: 250.5 -> 248.4 us mean of nine pairs; raised only for the loads 256 us,
    // only for the arithmetic 253 us)
    __builtin_amdgcn_s_setprio(3);
    Vec<float, V> vx[U];
    if (blockIdx.x < whole) {
        // a whole tile (the launch's first `whole` blocks, a scalar test): the tile's base is uniform (scalar registers) and each lane adds one 32-bit byte
        // offset, the vectors u > 0 lying at immediate offsets from it, so no lane computes a 64-bit
        // address or a bounds test
        const char *xt = reinterpret_cast<const char *>(x + v0 * V);
        char *yt = reinterpret_cast<char *>(y + v0 * V);
        const uint32_t off = (uint32_t)lane * (uint32_t)(V * sizeof(float));
#pragma unroll
        for (int u = 0; u < U; u++)
            vx[u] = vload_nt<float, V>(reinterpret_cast<const float *>(xt + off + u * 64 * V * sizeof(float)));
        exp_table_fill_wave(tab);
#pragma unroll
        for (int u = 0; u < U; u++) {
            Vec<float, V> vy;
#pragma unroll
            for (int k = 0; k < V; k++) vy.v[k] = f(vx[u].v[k], tab);
            vstore_nt<float, V>(reinterpret_cast<float *>(yt + off + u * 64 * V * sizeof(float)), vy);
        }
    } else {
        const int64_t i0 = v0 + lane;
#pragma unroll
        for (int u = 0; u < U; u++)
            if (i0 + u * 64 < nv) vx[u] = vload_nt<float, V>(x + (i0 + u * 64) * V);
        exp_table_fill_wave(tab);
#pragma unroll
        for (int u = 0; u < U; u++) {
            const int64_t i = i0 + u * 64;
            if (i < nv) {
                Vec<float, V> vy;
#pragma unroll
                for (int k = 0; k < V; k++) vy.v[k] = f(vx[u].v[k], tab);
                vstore_nt<float, V>(y + i * V, vy);
            }
        }
    }
    const int64_t tail = n - nv * V;
    if (tile0 + blockIdx.x == 0 && (int64_t)lane < tail) {
        const int64_t i = nv * V + lane;
        y[i] = f(x[i], tab);
    }
}

// One launch per kMaxBlocks tiles (a loop inside the kernel over further tiles made every wave wait for
// its stores before ending: 262 against 243 us at U = 1).
template <typename F>
static hipError_t launch_map_tab(const float *x, float *y, int64_t n, int vec, F f, hipStream_t s) {
    if (n == 0) return hipSuccess;
    const int V = vec > 1 ? 4 : 1;
    const int64_t ntiles = (n / V + 64 * kTabMapU - 1) / (64 * kTabMapU);
    for (int64_t t0 = 0; t0 < (ntiles > 0 ? ntiles : 1); t0 += kMaxBlocks) {
        const int g = (int)std::max<int64_t>(1, std::min<int64_t>(kMaxBlocks, ntiles - t0));
        const uint32_t whole = (uint32_t)std::max<int64_t>(0, std::min<int64_t>(g, (n / V) / (64 * kTabMapU) - t0));
        if (V == 4) hipLaunchKernelGGL((k_map_tab<F, 4, kTabMapU>), dim3(g), dim3(64), 0, s, x, y, n, t0, whole, f);
        else hipLaunchKernelGGL((k_map_tab<F, 1, kTabMapU>), dim3(g), dim3(64), 0, s, x, y, n, t0, whole, f);
    }
    return hipGetLastError();
}

// ---------------------------------------------------------------------------
// Unary: Sqrt (correctly rounded, TensorOps.cs:315-317), Erf (MathOps.cs:988),
// Neg (TensorOps.cs:299-301), Exp (MathF.Exp), Square (Pow with exponent 2).
// ---------------------------------------------------------------------------
template <int OP, typename T>
__device__ __forceinline__ T un_apply(T x, const ExpTable &tab) {
    if constexpr (OP == kSqrt) {
        if constexpr (std::is_same<T, float>::value) return __builtin_sqrtf(x);
        else return __builtin_sqrt(x);
    } else if constexpr (OP == kNeg) return -x;
    else if constexpr (OP == kSquare) return x * x;
    else if constexpr (OP == kErf) {
        if constexpr (std::is_same<T, float>::value) return erf_fast_lx(x, tab);
        else return erf_lx((double)x);
    } else {
        if constexpr (std::is_same<T, float>::value) return expf_lx(x, tab);
        else return ::exp((double)x);
    }
}

// Unary maps that need no expf table (float Erf and Exp run in k_map_tab); tab is never read here.
template <int OP, typename T, int V>
__global__ __launch_bounds__(kBlock) void k_unary(const T *__restrict__ x, T *__restrict__ y, int64_t n) {
    static_assert(!((OP == kErf || OP == kExp) && std::is_same<T, float>::value), "float Erf / Exp use k_map_tab");
    __shared__ ExpTable tab;
    const int64_t nv = n / V;
    for (int64_t i = (int64_t)blockIdx.x * kBlock + threadIdx.x; i < nv; i += (int64_t)gridDim.x * kBlock) {
        Vec<T, V> vx = vload_nt<T, V>(x + i * V), vy;
#pragma unroll
        for (int k = 0; k < V; k++) vy.v[k] = un_apply<OP, T>(vx.v[k], tab);
        vstore_nt<T, V>(y + i * V, vy);
    }
    const int64_t tail = n - nv * V;
    if (blockIdx.x == 0 && (int64_t)threadIdx.x < tail) {
        int64_t i = nv * V + threadIdx.x;
        y[i] = un_apply<OP, T>(x[i], tab);
    }
}

// Chains that stage the expf table in a block-shared LDS copy pay one table
// fill and barrier per block: they run a grid-stride loop over
// kTabVecsPerThread vectors per lane (measured on MI355X with the C5 GELU
// chain in this form: 294 us with one vector per lane, 260 us with four).
constexpr int kTabVecsPerThread = 4;

static inline int64_t lane_work(int64_t vectors, bool uses_table) {
    if (vectors < 1) vectors = 1;
    return uses_table ? (vectors + kTabVecsPerThread - 1) / kTabVecsPerThread : vectors;
}

template <int OP>
struct UnaryTabOp {
    __device__ __forceinline__ float operator()(float x, const ExpTable &tab) const { return un_apply<OP, float>(x, tab); }
};

template <int OP, typename T>
static hipError_t unary_typed(const void *x, void *y, int64_t n, int vec, hipStream_t s) {
    constexpr bool kTab = (OP == kErf || OP == kExp) && std::is_same<T, float>::value;
    if constexpr (kTab) {
        return launch_map_tab((const float *)x, (float *)y, n, vec, UnaryTabOp<OP>(), s);
    } else {
        if (vec > 1) {
            constexpr int V = VecWidth<T>::value;
            int g = grid_for(n / V > 0 ? n / V : 1, kBlock);
            hipLaunchKernelGGL((k_unary<OP, T, V>), dim3(g), dim3(kBlock), 0, s, (const T *)x, (T *)y, n);
        } else {
            int g = grid_for(n > 0 ? n : 1, kBlock);
            hipLaunchKernelGGL((k_unary<OP, T, 1>), dim3(g), dim3(kBlock), 0, s, (const T *)x, (T *)y, n);
        }
        return hipGetLastError();
    }
}

template <typename T>
static hipError_t unary_by_op(int op, const void *x, void *y, int64_t n, int vec, hipStream_t s) {
    switch (op) {
    case kSqrt: return unary_typed<kSqrt, T>(x, y, n, vec, s);
    case kErf: return unary_typed<kErf, T>(x, y, n, vec, s);
    case kNeg: return unary_typed<kNeg, T>(x, y, n, vec, s);
    case kExp: return unary_typed<kExp, T>(x, y, n, vec, s);
    case kSquare: return unary_typed<kSquare, T>(x, y, n, vec, s);
    default: return hipErrorInvalidValue;
    }
}

hipError_t launch_unary(int op, int dtype, const void *x, void *y, int64_t n, int vec, hipStream_t s) {
    if (n == 0) return hipSuccess;
    if (dtype == kFloat) return unary_by_op<float>(op, x, y, n, vec, s);
    if (dtype == kDouble) return unary_by_op<double>(op, x, y, n, vec, s);
    return hipErrorInvalidValue;
}

// ---------------------------------------------------------------------------
// Cast: ITensor.Cast<U> = Convert.ChangeType per element (ITensor.cs:161-170),
// i.e. System.Convert rules:
//   -> Bool: v != 0;  Bool -> number: 1 / 0
//   integer -> integer: must be representable, else OverflowException
//   float/double -> Int32/Int16/UInt16/SByte/Byte: round half to even inside
//     [-2147483648.5, 2147483647.5) (Convert.ToInt32(double)), then the range
//   float/double -> UInt32: (-0.5, 4294967295.5), round half to even
//   float/double -> Int64/UInt64: checked((long)Math.Round(v))
//   integer -> float/double: one round-to-nearest-even conversion
//   double -> float: (float)v
// ---------------------------------------------------------------------------
template <int DST>
__device__ __forceinline__ bool int_fits(int64_t v) {
    switch (DST) {
    case kInt32: return v >= INT32_MIN && v <= INT32_MAX;
    case kInt16: return v >= INT16_MIN && v <= INT16_MAX;
    case kUInt16: return v >= 0 && v <= 65535;
    case kInt8: return v >= -128 && v <= 127;
    case kUInt8: return v >= 0 && v <= 255;
    case kUInt32: return v >= 0 && v <= 4294967295ll;
    default: return true;
    }
}

template <int SRC, int DST>
__device__ __forceinline__ typename CType<DST>::T cast_apply(typename CType<SRC>::T v, bool &ovf) {
    using D = typename CType<DST>::T;
    constexpr bool kSrcFloat = (SRC == kFloat || SRC == kDouble);
    if constexpr (SRC == DST) {
        return v;
    } else if constexpr (DST == kBool) {
        return (D)(v != 0);
    } else if constexpr (DST == kFloat || DST == kDouble) {
        if constexpr (SRC == kBool) return v ? (D)1 : (D)0;
        else return (D)v;
    } else if constexpr (kSrcFloat) {
        double d = (double)v;
        if constexpr (DST == kInt64) {
            double r = __builtin_rint(d);
            if (!(r >= -9223372036854775808.0 && r < 9223372036854775808.0)) { ovf = true; return 0; }
            return (D)(int64_t)r;
        } else if constexpr (DST == kUInt64) {
            double r = __builtin_rint(d);
            if (!(r > -1.0 && r < 18446744073709551616.0)) { ovf = true; return 0; }
            return (D)(uint64_t)(r < 0.0 ? 0.0 : r);
        } else if constexpr (DST == kUInt32) {
            if (!(d > -0.5 && d < 4294967295.5)) { ovf = true; return 0; }
            return (D)(uint32_t)(int64_t)__builtin_rint(d);
        } else {
            if (!(d >= -2147483648.5 && d < 2147483647.5)) { ovf = true; return 0; }
            int64_t iv = (int64_t)__builtin_rint(d);
            if (!int_fits<DST>(iv)) { ovf = true; return 0; }
            return (D)iv;
        }
    } else if constexpr (SRC == kUInt64) {
        uint64_t u = v;
        if constexpr (DST == kInt64) {
            if (u > (uint64_t)INT64_MAX) { ovf = true; return 0; }
            return (D)u;
        } else {
            if (u > (uint64_t)INT64_MAX || !int_fits<DST>((int64_t)u)) { ovf = true; return 0; }
            return (D)u;
        }
    } else {
        int64_t iv = (int64_t)v;  // Bool, UInt8, Int8, UInt16, Int16, Int32, UInt32, Int64
        if constexpr (DST == kUInt64) {
            if (iv < 0) { ovf = true; return 0; }
            return (D)iv;
        } else {
            if (!int_fits<DST>(iv)) { ovf = true; return 0; }
            return (D)iv;
        }
    }
}

// A block takes U * kBlock consecutive vectors, lane t the vectors t, t + kBlock, ...,
// all loaded before any is converted.
template <int SRC, int DST, int E, int U, int B = kBlock, bool NTS = true>
__global__ __launch_bounds__(B) void k_cast(const typename CType<SRC>::T *__restrict__ x,
                                            typename CType<DST>::T *__restrict__ y, int64_t n, ErrFlags *errs) {
    using S = typename CType<SRC>::T;
    using D = typename CType<DST>::T;
    const int64_t nv = n / E;
    bool ovf = false;
    for (int64_t i0 = (int64_t)blockIdx.x * B * U + threadIdx.x; i0 < nv; i0 += (int64_t)gridDim.x * B * U) {
        Vec<S, E> vx[U];
#pragma unroll
        for (int u = 0; u < U; u++)
            if (u == 0 || i0 + u * B < nv) vx[u] = vload_nt<S, E>(x + (i0 + u * B) * E);
#pragma unroll
        for (int u = 0; u < U; u++) {
            if (u == 0 || i0 + u * B < nv) {
                Vec<D, E> vy;
#pragma unroll
                for (int k = 0; k < E; k++) vy.v[k] = cast_apply<SRC, DST>(vx[u].v[k], ovf);
                if constexpr (NTS) vstore_nt<D, E>(y + (i0 + u * B) * E, vy);
                else vstore<D, E>(y + (i0 + u * B) * E, vy);
            }
        }
    }
    const int64_t tail = n - nv * E;
    if (blockIdx.x == 0 && (int64_t)threadIdx.x < tail) {
        int64_t i = nv * E + threadIdx.x;
        y[i] = cast_apply<SRC, DST>(x[i], ovf);
    }
    if (ovf) atomicMin(&errs->first_ovf, 0ull);
}

// Mid-sized casts (kTileUMin to kTileUMax vectors): one-wave blocks over tiles of 64 * 4 vectors, all four
// loaded before any is converted, no loop.  tile0: the first tile of this launch.
template <int SRC, int DST, int E, int U>
__global__ __launch_bounds__(64) void k_cast_tile(const typename CType<SRC>::T *__restrict__ x,
                                                  typename CType<DST>::T *__restrict__ y, int64_t n, int64_t tile0,
                                                  ErrFlags *errs) {
    using S = typename CType<SRC>::T;
    using D = typename CType<DST>::T;
    const int64_t nv = n / E;
    bool ovf = false;
    const int64_t i0 = (tile0 + blockIdx.x) * (64 * U) + threadIdx.x;
    Vec<S, E> vx[U];
#pragma unroll
    for (int u = 0; u < U; u++)
        if (i0 + u * 64 < nv) vx[u] = vload_nt<S, E>(x + (i0 + u * 64) * E);
#pragma unroll
    for (int u = 0; u < U; u++) {
        if (i0 + u * 64 < nv) {
            Vec<D, E> vy;
#pragma unroll
            for (int k = 0; k < E; k++) vy.v[k] = cast_apply<SRC, DST>(vx[u].v[k], ovf);
            vstore_nt<D, E>(y + (i0 + u * 64) * E, vy);
        }
    }
    const int64_t tail = n - nv * E;
    if (tile0 + blockIdx.x == 0 && (int64_t)threadIdx.x < tail) {
        const int64_t i = nv * E + threadIdx.x;
        y[i] = cast_apply<SRC, DST>(x[i], ovf);
    }
    if (ovf) atomicMin(&errs->first_ovf, 0ull);
}

template <int SRC, int DST>
static hipError_t cast_typed(const void *x, void *y, int64_t n, int vec, ErrFlags *errs, hipStream_t s) {
    using S = typename CType<SRC>::T;
    using D = typename CType<DST>::T;
    constexpr int E = 16 / (sizeof(S) < sizeof(D) ? sizeof(S) : sizeof(D));  // 16 bytes on the narrower side
    if (vec > 1 && n / E >= kTileUMin && n / E < kTileUMax) {
        const int64_t ntiles = (n / E + 255) / 256;
        for (int64_t t0 = 0; t0 < ntiles; t0 += kMaxBlocks) {
            const int g = (int)std::min<int64_t>(kMaxBlocks, ntiles - t0);
            hipLaunchKernelGGL((k_cast_tile<SRC, DST, E, 4>), dim3(g), dim3(64), 0, s, (const S *)x, (D *)y, n, t0, errs);
        }
    } else if (vec > 1 && n / E >= kCastTwoMin && n / E < kCastTwoMax) {
        int g = grid_for((n / E + 1) / 2, kBlock);
        hipLaunchKernelGGL((k_cast<SRC, DST, E, 2>), dim3(g), dim3(kBlock), 0, s, (const S *)x, (D *)y, n, errs);
    } else if (vec > 1 && n / E >= kCastTwoMax && sizeof(S) == sizeof(D)) {
        // large same-width casts: one-wave blocks (1 GiB float copy 329.6 -> 322.6 us on MI355X)
        int g = grid_for(n / E, 64);
        hipLaunchKernelGGL((k_cast<SRC, DST, E, 1, 64>), dim3(g), dim3(64), 0, s, (const S *)x, (D *)y, n, errs);
    } else if (vec > 1 && n / E >= kCastTwoMax && sizeof(S) > sizeof(D)) {
        // large narrowing casts: ordinary stores (C4 int64 -> float32 129.4 -> 121.5 us against streaming
        // stores; 123.4 us in one-wave blocks)
        int g = grid_for(n / E, kBlock);
        hipLaunchKernelGGL((k_cast<SRC, DST, E, 1, kBlock, false>), dim3(g), dim3(kBlock), 0, s, (const S *)x, (D *)y, n, errs);
    } else if (vec > 1) {
        int g = grid_for(n / E > 0 ? n / E : 1, kBlock);
        hipLaunchKernelGGL((k_cast<SRC, DST, E, 1>), dim3(g), dim3(kBlock), 0, s, (const S *)x, (D *)y, n, errs);
    } else {
        int g = grid_for(n, kBlock);
        hipLaunchKernelGGL((k_cast<SRC, DST, 1, 1>), dim3(g), dim3(kBlock), 0, s, (const S *)x, (D *)y, n, errs);
    }
    return hipGetLastError();
}

template <int SRC>
static hipError_t cast_to(int dst, const void *x, void *y, int64_t n, int vec, ErrFlags *errs, hipStream_t s) {
    switch (dst) {
    case kFloat: return cast_typed<SRC, kFloat>(x, y, n, vec, errs, s);
    case kDouble: return cast_typed<SRC, kDouble>(x, y, n, vec, errs, s);
    case kUInt8: return cast_typed<SRC, kUInt8>(x, y, n, vec, errs, s);
    case kInt8: return cast_typed<SRC, kInt8>(x, y, n, vec, errs, s);
    case kUInt16: return cast_typed<SRC, kUInt16>(x, y, n, vec, errs, s);
    case kInt16: return cast_typed<SRC, kInt16>(x, y, n, vec, errs, s);
    case kInt32: return cast_typed<SRC, kInt32>(x, y, n, vec, errs, s);
    case kUInt32: return cast_typed<SRC, kUInt32>(x, y, n, vec, errs, s);
    case kInt64: return cast_typed<SRC, kInt64>(x, y, n, vec, errs, s);
    case kUInt64: return cast_typed<SRC, kUInt64>(x, y, n, vec, errs, s);
    case kBool: return cast_typed<SRC, kBool>(x, y, n, vec, errs, s);
    default: return hipErrorInvalidValue;
    }
}

hipError_t launch_cast(int src, int dst, const void *x, void *y, int64_t n, int vec, ErrFlags *errs,
                       hipStream_t s) {
    if (n == 0) return hipSuccess;
    switch (src) {
    case kFloat: return cast_to<kFloat>(dst, x, y, n, vec, errs, s);
    case kDouble: return cast_to<kDouble>(dst, x, y, n, vec, errs, s);
    case kUInt8: return cast_to<kUInt8>(dst, x, y, n, vec, errs, s);
    case kInt8: return cast_to<kInt8>(dst, x, y, n, vec, errs, s);
    case kUInt16: return cast_to<kUInt16>(dst, x, y, n, vec, errs, s);
    case kInt16: return cast_to<kInt16>(dst, x, y, n, vec, errs, s);
    case kInt32: return cast_to<kInt32>(dst, x, y, n, vec, errs, s);
    case kUInt32: return cast_to<kUInt32>(dst, x, y, n, vec, errs, s);
    case kInt64: return cast_to<kInt64>(dst, x, y, n, vec, errs, s);
    case kUInt64: return cast_to<kUInt64>(dst, x, y, n, vec, errs, s);
    case kBool: return cast_to<kBool>(dst, x, y, n, vec, errs, s);
    default: return hipErrorInvalidValue;
    }
}

// ---------------------------------------------------------------------------
// Fused GELU subgraph, one rounding per ONNX node:
//   a = x / 1.4142135f (Div), e = Erf(a), b = e + 1f (Add), c = x * b (Mul),
//   y = c * 0.5f (Mul)
// ---------------------------------------------------------------------------
struct GeluOp {
    __device__ __forceinline__ float operator()(float x, const ExpTable &tab) const { return gelu_erf_lx(x, tab); }
};

hipError_t launch_gelu_erf(const float *x, float *y, int64_t n, int vec, hipStream_t s) {
    return launch_map_tab(x, y, n, vec, GeluOp(), s);
}

// ---------------------------------------------------------------------------
// Elementwise chain: a linear sequence of float32 Add/Sub/Mul/Div/Pow/Sqrt/Erf
// nodes in one pass (the graph runtime's fusion of elementwise chains).  Each
// instruction calls the same device routine as the separate operator, so the
// result is bit-identical to running the nodes one by one.  The instruction
// list is uniform across the launch: the switch below does not diverge.
// ---------------------------------------------------------------------------
// the operands are ordered by selects rather than by two copies of the op: the division
// and power sequences are long, and a smaller kernel starts faster on a cold instruction cache
template <int OP, int V>
__device__ __forceinline__ void chain_bin(Vec<float, V> &acc, const Vec<float, V> &x, bool x_left) {
#pragma unroll
    for (int k = 0; k < V; k++) {
        const float l = x_left ? x.v[k] : acc.v[k];
        const float r = x_left ? acc.v[k] : x.v[k];
        acc.v[k] = bin_apply<OP, float>(l, r, 0, nullptr);
    }
}

// one instruction; op and x_left are uniform, so each branch is taken by the whole
// wave.  ERF / POW: whether the chain holds those instructions (their code is large
// and its registers would cost occupancy in the chains that do not).
template <int V, bool ERF, bool POW>
__device__ __forceinline__ void chain_step(int op, Vec<float, V> &acc, const Vec<float, V> &x, bool x_left,
                                           const ExpTable &tab) {
    switch (op) {
    case kAdd: chain_bin<kAdd, V>(acc, x, x_left); break;
    case kSub: chain_bin<kSub, V>(acc, x, x_left); break;
    case kMul: chain_bin<kMul, V>(acc, x, x_left); break;
    case kDiv: chain_bin<kDiv, V>(acc, x, x_left); break;
    case kPow:
        if constexpr (POW) chain_bin<kPow, V>(acc, x, x_left);
        break;
    case kChainUnary + kSqrt:
#pragma unroll
        for (int k = 0; k < V; k++) acc.v[k] = un_apply<kSqrt, float>(acc.v[k], tab);
        break;
    default:
        if constexpr (ERF) {
#pragma unroll
            for (int k = 0; k < V; k++) acc.v[k] = un_apply<kErf, float>(acc.v[k], tab);
        }
        break;
    }
}

// NIN: inputs held in registers (n_in <= NIN)
extern __shared__ ExpTable chain_lds[];  // the expf table of chains with Erf (dynamic LDS: none otherwise)

// One vector of every input of the chain (inputs with a broadcast inner axis: their one element across
// the vector).
template <int V, int NIN>
__device__ __forceinline__ void chain_load(const ChainArgs &A, uint32_t v, Vec<float, V> (&x)[NIN]) {
    const uint32_t row = fdiv(v, A.inner_v);
    const uint32_t cv = v - row * A.inner_v.d;
    int64_t off[NIN];
#pragma unroll
    for (int j = 0; j < NIN; j++) off[j] = 0;
    uint32_t rr = row;
    for (int d = 0; d < A.nouter; d++) {
        const uint32_t q = fdiv(rr, A.odiv[d]);
        const int64_t id = rr - q * A.odiv[d].d;
#pragma unroll
        for (int j = 0; j < NIN; j++)
            if (j < A.n_in) off[j] += id * A.str[j][d];
        rr = q;
    }
    const int64_t col = (int64_t)cv * V;
#pragma unroll
    for (int j = 0; j < NIN; j++) {
        if (j < A.n_in) {
            if ((A.inner_mode >> j) & 1) {
                // ordinary loads: streaming loads measured slower here (C3-sized Add -> Mul
                // chain 106 against 86 us on MI355X)
                x[j] = vload<float, V>(A.in[j] + off[j] + col);
            } else {
                const float sv = A.in[j][off[j]];
#pragma unroll
                for (int k = 0; k < V; k++) x[j].v[k] = sv;
            }
        }
    }
}

// The chain's instructions over one vector of inputs.
template <int V, int NIN, bool ERF, bool POW>
__device__ __forceinline__ Vec<float, V> chain_eval(const ChainArgs &A, const Vec<float, V> (&x)[NIN],
                                                    const ExpTable &tab) {
    Vec<float, V> acc = x[0];
    for (int i = 0; i < A.n_ops; i++) {
        const int o = A.operand[i];
        const int j = o < 0 ? -o - 1 : o;
        Vec<float, V> xj = x[0];
#pragma unroll
        for (int jj = 1; jj < NIN; jj++)
            if (jj == j) xj = x[jj];
        chain_step<V, ERF, POW>(A.op[i], acc, xj, o < 0, tab);
    }
    return acc;
}

// Small chains: a grid-stride loop in 256-lane blocks, one vector per lane.
template <int V, int NIN, bool ERF, bool POW>
__global__ __launch_bounds__(kBlock) void k_chain(ChainArgs A) {
    ExpTable &tab = chain_lds[0];
    if constexpr (ERF) {
        exp_table_fill(tab);
        __syncthreads();
    }
    for (uint32_t v = blockIdx.x * kBlock + threadIdx.x; v < A.nv; v += gridDim.x * kBlock) {
        Vec<float, V> x[NIN];
        chain_load<V, NIN>(A, v, x);
        vstore_nt<float, V>(A.y + (int64_t)v * V, chain_eval<V, NIN, ERF, POW>(A, x, tab));
    }
}

// Chains of 2^16 or more vectors: one-wave blocks over tiles of 64 * U vectors, every input of all U loaded
// before any is computed, no loop; a chain with Erf fills the wave's own expf table after its loads.
// Interleaved in one process on MI355X against k_chain: C3-sized Add mask -> Mul scalar 78.5 -> 69.8 us,
// C2-sized Sub row -> Mul gamma 8.3 -> 7.0 us; on C1's 12,288 vectors it was slower (2.6 -> 3.6 us), so
// small chains stay with k_chain.  tile0: the first tile of this launch.
constexpr int64_t kChainTileMin = 1 << 16;
template <int V, int NIN, bool ERF, bool POW, int U>
__global__ __launch_bounds__(64) void k_chain_tile(ChainArgs A, uint32_t tile0) {
    __shared__ ExpTable tab;
    const uint32_t v0 = (tile0 + blockIdx.x) * (64u * U) + threadIdx.x;
    Vec<float, V> x[U][NIN];
#pragma unroll
    for (int u = 0; u < U; u++)
        if (v0 + u * 64 < A.nv) chain_load<V, NIN>(A, v0 + u * 64, x[u]);
    if constexpr (ERF) exp_table_fill_wave(tab);
#pragma unroll
    for (int u = 0; u < U; u++) {
        const uint32_t v = v0 + u * 64;
        if (v < A.nv) vstore_nt<float, V>(A.y + (int64_t)v * V, chain_eval<V, NIN, ERF, POW>(A, x[u], tab));
    }
}

template <int V, int NIN>
static void launch_chain_v(const ChainArgs &A, int g, bool pow, hipStream_t s) {
    const size_t lds = sizeof(ExpTable);
    if (A.nv >= kChainTileMin) {
        constexpr int U = 2;
        const int64_t ntiles = ((int64_t)A.nv + 64 * U - 1) / (64 * U);
        for (int64_t t0 = 0; t0 < ntiles; t0 += kMaxBlocks) {
            const int gt = (int)std::min<int64_t>(kMaxBlocks, ntiles - t0);
            if (A.uses_erf && pow) hipLaunchKernelGGL((k_chain_tile<V, NIN, true, true, U>), dim3(gt), dim3(64), 0, s, A, (uint32_t)t0);
            else if (A.uses_erf) hipLaunchKernelGGL((k_chain_tile<V, NIN, true, false, U>), dim3(gt), dim3(64), 0, s, A, (uint32_t)t0);
            else if (pow) hipLaunchKernelGGL((k_chain_tile<V, NIN, false, true, U>), dim3(gt), dim3(64), 0, s, A, (uint32_t)t0);
            else hipLaunchKernelGGL((k_chain_tile<V, NIN, false, false, U>), dim3(gt), dim3(64), 0, s, A, (uint32_t)t0);
        }
        return;
    }
    if (A.uses_erf && pow) hipLaunchKernelGGL((k_chain<V, NIN, true, true>), dim3(g), dim3(kBlock), lds, s, A);
    else if (A.uses_erf) hipLaunchKernelGGL((k_chain<V, NIN, true, false>), dim3(g), dim3(kBlock), lds, s, A);
    else if (pow) hipLaunchKernelGGL((k_chain<V, NIN, false, true>), dim3(g), dim3(kBlock), 0, s, A);
    else hipLaunchKernelGGL((k_chain<V, NIN, false, false>), dim3(g), dim3(kBlock), 0, s, A);
}

hipError_t launch_chain(const ChainArgs &A, hipStream_t s) {
    if (A.nv == 0) return hipSuccess;
    bool pow = false;
    for (int i = 0; i < A.n_ops; i++) pow = pow || A.op[i] == kPow;
    // small chains with the expf table: several vectors per lane, so the table fill is paid once per four
    const int64_t work = A.uses_erf ? lane_work(A.nv, true) : A.nv;
    const int g = grid_for(work, kBlock);
    if (A.vec == 4) {
        if (A.n_in <= 2) launch_chain_v<4, 2>(A, g, pow, s);
        else if (A.n_in <= 4) launch_chain_v<4, 4>(A, g, pow, s);
        else launch_chain_v<4, 8>(A, g, pow, s);
    } else {
        if (A.n_in <= 2) launch_chain_v<1, 2>(A, g, pow, s);
        else if (A.n_in <= 4) launch_chain_v<1, 4>(A, g, pow, s);
        else launch_chain_v<1, 8>(A, g, pow, s);
    }
    return hipGetLastError();
}

}  // namespace lx
