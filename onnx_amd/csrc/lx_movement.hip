// lx_movement.hip -- data movement on gfx950: Transpose, Slice, Concat and
// broadcast expansion as one strided view copy, Gather as an indexed row copy.
// All HBM-bound: every element is read once and written once.
//
// View copy: the axes are collapsed on the host wherever both views stay
// contiguous across them; when the innermost axis is contiguous in source and
// destination the copy moves 16-byte vectors, four per lane.  When the
// destination's innermost axis is not the source's (a transpose that moves the
// innermost axis), 64x64 tiles (32x32 for shapes that do not divide by 4) go
// through LDS so that both the reads and the writes run along contiguous
// addresses.  Concat moves up to eight inputs in one launch.
#include <hip/hip_runtime.h>

#include <cstring>

#include "lx_device.h"
#include "lx_kernels.h"
#include "lx_plan.h"

namespace lx {

constexpr int kMBlock = 256;

// uint32 decomposition of an outer index over up to 7 axes (innermost first)
struct OuterDecomp {
    int32_t n;
    int32_t pad;
    FastDiv div[7];
    int64_t src_str[7];
    int64_t dst_str[7];
};

// Copies rows of L elements (L = dims[rank-1]); each lane moves kRowsU
// vectors of V contiguous elements, all loads issued before the stores.  Row
// strides come from the outer decomposition.  Ordinary loads with streaming
// stores: on MI355X a 25 MB strided copy runs at 5.1 TB/s that way against
// 4.5 TB/s with streaming loads and 3.5 TB/s with ordinary stores; two
// vectors per lane is as fast as four and faster than eight.
constexpr int kRowsU = 2;

template <typename T, int V>
__device__ __forceinline__ void row_offsets(uint32_t v, const FastDiv &lv, const OuterDecomp &od, int64_t src_in,
                                            int64_t dst_in, int64_t src_base, int64_t dst_base, int64_t *so,
                                            int64_t *d_o) {
    uint32_t row = fdiv(v, lv);
    const uint32_t cv = v - row * lv.d;
    int64_t s = src_base, d = dst_base;
#pragma unroll
    for (int k = 0; k < 7; k++) {
        if (k < od.n) {
            const uint32_t q = fdiv(row, od.div[k]);
            const uint32_t id = row - q * od.div[k].d;
            s += (int64_t)id * od.src_str[k];
            d += (int64_t)id * od.dst_str[k];
            row = q;
        }
    }
    const int64_t e = (int64_t)cv * V;
    *so = s + (V > 1 ? e : e * src_in);
    *d_o = d + (V > 1 ? e : e * dst_in);
}

template <typename T, int V>
__global__ __launch_bounds__(kMBlock) void k_view_rows(const T *__restrict__ src, T *__restrict__ dst, uint32_t nvec,
                                                       FastDiv lv, int64_t src_in, int64_t dst_in, OuterDecomp od,
                                                       int64_t src_base, int64_t dst_base) {
    for (uint32_t base = blockIdx.x * (kMBlock * kRowsU); base < nvec; base += gridDim.x * (kMBlock * kRowsU)) {
        Vec<T, V> r[kRowsU];
        int64_t dof[kRowsU];
#pragma unroll
        for (int u = 0; u < kRowsU; u++) {
            const uint32_t v = base + u * kMBlock + threadIdx.x;
            if (v < nvec) {
                int64_t so;
                row_offsets<T, V>(v, lv, od, src_in, dst_in, src_base, dst_base, &so, &dof[u]);
                if constexpr (V > 1) r[u] = vload<T, V>(src + so);
                else r[u].v[0] = src[so];
            }
        }
#pragma unroll
        for (int u = 0; u < kRowsU; u++) {
            const uint32_t v = base + u * kMBlock + threadIdx.x;
            if (v < nvec) {
                if constexpr (V > 1) vstore_nt<T, V>(dst + dof[u], r[u]);
                else dst[dof[u]] = r[u].v[0];
            }
        }
    }
}

// 64x64 tiles of the plane (dst innermost axis l, src-contiguous axis q), four
// elements per access on both sides: a lane reads 4 consecutive q of one l
// from the source and writes 4 consecutive l of one q to the destination,
// the transposition going through LDS (row pitch 65 elements: the column
// reads of a wave touch each bank at most twice).  Needs nq, nl, the two
// plane strides and both bases divisible by 4 and 4-element-aligned pointers.
template <typename T>
__global__ __launch_bounds__(kMBlock) void k_view_tiled4(const T *__restrict__ src, T *__restrict__ dst, int64_t nl,
                                                         int64_t nq, int64_t src_l, int64_t dst_q, OuterDecomp od,
                                                         int64_t src_base, int64_t dst_base, uint32_t z0) {
    __shared__ T tile[64][65];
    uint32_t row = blockIdx.z + z0;
    int64_t so = src_base, d_o = dst_base;
    for (int d = 0; d < od.n; d++) {
        const uint32_t q = fdiv(row, od.div[d]);
        const uint32_t id = row - q * od.div[d].d;
        so += (int64_t)id * od.src_str[d];
        d_o += (int64_t)id * od.dst_str[d];
        row = q;
    }
    const int64_t l0 = (int64_t)blockIdx.x * 64, q0 = (int64_t)blockIdx.y * 64;
    const int ta = threadIdx.x % 16, tb = threadIdx.x / 16;  // 16 x 16
    Vec<T, 4> r[4];
#pragma unroll
    for (int k = 0; k < 4; k++) {  // source rows l0 + tb + 16k, elements q0 + 4ta .. +3
        const int64_t l = l0 + tb + 16 * k, q = q0 + 4 * ta;
        if (l < nl && q < nq) r[k] = vload<T, 4>(src + so + q + l * src_l);
    }
#pragma unroll
    for (int k = 0; k < 4; k++) {
        const int64_t l = l0 + tb + 16 * k, q = q0 + 4 * ta;
        if (l < nl && q < nq) {
#pragma unroll
            for (int j = 0; j < 4; j++) tile[tb + 16 * k][4 * ta + j] = r[k].v[j];
        }
    }
    __syncthreads();
#pragma unroll
    for (int k = 0; k < 4; k++) {  // destination rows q0 + tb + 16k, elements l0 + 4ta .. +3
        const int64_t q = q0 + tb + 16 * k, l = l0 + 4 * ta;
        if (l < nl && q < nq) {
            Vec<T, 4> w;
#pragma unroll
            for (int j = 0; j < 4; j++) w.v[j] = tile[4 * ta + j][tb + 16 * k];
            vstore_nt<T, 4>(dst + d_o + l + q * dst_q, w);
        }
    }
}

// 32x32 tiles of the plane (dst innermost axis, src-contiguous axis q); the
// remaining axes are walked by blockIdx.z through the outer decomposition.
template <typename T>
__global__ __launch_bounds__(kMBlock) void k_view_tiled(const T *__restrict__ src, T *__restrict__ dst, int64_t nl,
                                                        int64_t nq, int64_t src_l, int64_t dst_q, OuterDecomp od,
                                                        int64_t src_base, int64_t dst_base, uint32_t z0) {
    __shared__ T tile[32][33];
    uint32_t row = blockIdx.z + z0;
    int64_t so = src_base, d_o = dst_base;
    for (int d = 0; d < od.n; d++) {
        const uint32_t q = fdiv(row, od.div[d]);
        const uint32_t id = row - q * od.div[d].d;
        so += (int64_t)id * od.src_str[d];
        d_o += (int64_t)id * od.dst_str[d];
        row = q;
    }
    const int64_t l0 = (int64_t)blockIdx.x * 32, q0 = (int64_t)blockIdx.y * 32;
    const int tx = threadIdx.x % 32, ty = threadIdx.x / 32;  // 32 x 8
    // read along q (contiguous in src): tile[q][l]
#pragma unroll
    for (int k = 0; k < 32; k += 8) {
        const int64_t q = q0 + tx, l = l0 + ty + k;
        if (q < nq && l < nl) tile[tx][ty + k] = src[so + q + l * src_l];
    }
    __syncthreads();
    // write along l (contiguous in dst)
#pragma unroll
    for (int k = 0; k < 32; k += 8) {
        const int64_t l = l0 + tx, q = q0 + ty + k;
        if (q < nq && l < nl) dst[d_o + l + q * dst_q] = tile[ty + k][tx];
    }
}

template <typename T>
static hipError_t view_copy_typed(const T *src, T *dst, const ViewCopyArgs &a0, hipStream_t s) {
    // collapse size-1 axes and axes contiguous in both views
    ViewCopyArgs a;
    a.rank = 0;
    a.src_base = a0.src_base;
    a.dst_base = a0.dst_base;
    int64_t total = 1;
    for (int k = 0; k < a0.rank; k++) {
        total *= a0.dims[k];
        if (a0.dims[k] == 1) continue;
        if (a.rank > 0 && a.src_str[a.rank - 1] == a0.src_str[k] * a0.dims[k] &&
            a.dst_str[a.rank - 1] == a0.dst_str[k] * a0.dims[k]) {
            a.dims[a.rank - 1] *= a0.dims[k];
            a.src_str[a.rank - 1] = a0.src_str[k];
            a.dst_str[a.rank - 1] = a0.dst_str[k];
            continue;
        }
        a.dims[a.rank] = a0.dims[k];
        a.src_str[a.rank] = a0.src_str[k];
        a.dst_str[a.rank] = a0.dst_str[k];
        a.rank++;
    }
    if (total == 0) return hipSuccess;
    if (a.rank == 0) {
        a.rank = 1;
        a.dims[0] = 1;
        a.src_str[0] = a.dst_str[0] = 1;
    }
    const int r = a.rank;
    // tiled transpose: the dst innermost axis is not contiguous in src, another axis is
    int qax = -1;
    if (a.dst_str[r - 1] == 1 && a.src_str[r - 1] != 1)
        for (int k = 0; k < r - 1; k++)
            if (a.src_str[k] == 1) qax = k;
    OuterDecomp od;
    memset(&od, 0, sizeof od);
    if (qax >= 0) {
        int64_t nz = 1;
        for (int k = r - 2, n = 0; k >= 0; k--) {
            if (k == qax) continue;
            od.div[n] = make_fastdiv((uint32_t)a.dims[k]);
            od.src_str[n] = a.src_str[k];
            od.dst_str[n] = a.dst_str[k];
            n++;
            od.n = n;
            nz *= a.dims[k];
        }
        if (nz < (1ll << 31) && a.dims[r - 1] < (1ll << 31) && a.dims[qax] < (1ll << 31) && r - 2 <= 7) {
            const int64_t nl = a.dims[r - 1], nq = a.dims[qax];
            bool v4 = nl % 4 == 0 && nq % 4 == 0 && a.src_str[r - 1] % 4 == 0 && a.dst_str[qax] % 4 == 0 &&
                      a.src_base % 4 == 0 && a.dst_base % 4 == 0 && (uintptr_t)src % (4 * sizeof(T)) == 0 &&
                      (uintptr_t)dst % (4 * sizeof(T)) == 0;
            for (int k = 0; k < od.n; k++)
                if (od.src_str[k] % 4 || od.dst_str[k] % 4) v4 = false;
            const int tw = v4 ? 64 : 32;
            const dim3 blk(kMBlock);
            for (int64_t z0 = 0; z0 < nz; z0 += 65535) {
                const unsigned nzb = (unsigned)(nz - z0 < 65535 ? nz - z0 : 65535);
                const dim3 g((unsigned)((nl + tw - 1) / tw), (unsigned)((nq + tw - 1) / tw), nzb);
                if (v4)
                    hipLaunchKernelGGL(k_view_tiled4<T>, g, blk, 0, s, src, dst, nl, nq, a.src_str[r - 1],
                                       a.dst_str[qax], od, a.src_base, a.dst_base, (uint32_t)z0);
                else
                    hipLaunchKernelGGL(k_view_tiled<T>, g, blk, 0, s, src, dst, nl, nq, a.src_str[r - 1],
                                       a.dst_str[qax], od, a.src_base, a.dst_base, (uint32_t)z0);
            }
            return hipGetLastError();
        }
    }
    // row copy
    constexpr int VW = 16 / sizeof(T) > 0 ? 16 / sizeof(T) : 1;
    const int64_t L = a.dims[r - 1];
    const bool vec = VW > 1 && a.src_str[r - 1] == 1 && a.dst_str[r - 1] == 1 && L % VW == 0 &&
                     (a.src_base % VW == 0) && (a.dst_base % VW == 0) && ((uintptr_t)src % 16 == 0) &&
                     ((uintptr_t)dst % 16 == 0) && [&] {
                         for (int k = 0; k < r - 1; k++)
                             if (a.src_str[k] % VW || a.dst_str[k] % VW) return false;
                         return true;
                     }();
    const int64_t V = vec ? VW : 1;
    const int64_t nvec = total / V;
    if (nvec >= (1ll << 31) || r - 1 > 7) return hipErrorInvalidValue;  // host rejects beforehand
    for (int k = r - 2, n = 0; k >= 0; k--, n++) {
        od.div[n] = make_fastdiv((uint32_t)a.dims[k]);
        od.src_str[n] = a.src_str[k];
        od.dst_str[n] = a.dst_str[k];
        od.n = n + 1;
    }
    const FastDiv lv = make_fastdiv((uint32_t)(L / V));
    int64_t g = (nvec + kMBlock * kRowsU - 1) / (kMBlock * kRowsU);
    if (g > 65536 * 4) g = 65536 * 4;
    if (vec)
        hipLaunchKernelGGL((k_view_rows<T, VW>), dim3((unsigned)g), dim3(kMBlock), 0, s, src, dst, (uint32_t)nvec, lv,
                           a.src_str[r - 1], a.dst_str[r - 1], od, a.src_base, a.dst_base);
    else
        hipLaunchKernelGGL((k_view_rows<T, 1>), dim3((unsigned)g), dim3(kMBlock), 0, s, src, dst, (uint32_t)nvec, lv,
                           a.src_str[r - 1], a.dst_str[r - 1], od, a.src_base, a.dst_base);
    return hipGetLastError();
}

hipError_t launch_view_copy(int esize, const void *src, void *dst, const ViewCopyArgs &a, hipStream_t s) {
    switch (esize) {
    case 1: return view_copy_typed<uint8_t>((const uint8_t *)src, (uint8_t *)dst, a, s);
    case 2: return view_copy_typed<uint16_t>((const uint16_t *)src, (uint16_t *)dst, a, s);
    case 4: return view_copy_typed<uint32_t>((const uint32_t *)src, (uint32_t *)dst, a, s);
    case 8: return view_copy_typed<uint64_t>((const uint64_t *)src, (uint64_t *)dst, a, s);
    default: return hipErrorInvalidValue;
    }
}

// ---------------------------------------------------------------------------
// Concat: input i is a row-major [outer, len_i] block (len_i = dims_i[axis] x
// the elements after the axis) that lands in columns [off_i, off_i + len_i) of
// the [outer, total] output.  The blocks of one input are contiguous in
// blockIdx.x; the input is picked by a wave-uniform search and selected from
// the argument block without dynamic indexing.
// ---------------------------------------------------------------------------
struct ConcatArgs {
    int32_t n;
    uint32_t pad;
    const void *src[kConcatMax];
    uint32_t block0[kConcatMax + 1];  // first block of input i
    uint32_t nvec[kConcatMax];        // outer * len_i / V
    FastDiv lenv[kConcatMax];         // len_i / V
    int64_t off[kConcatMax];          // column offset, elements
    int64_t total;                    // output row length, elements
};

template <typename T, int V>
__global__ __launch_bounds__(kMBlock) void k_concat(T *__restrict__ dst, ConcatArgs a) {
    const uint32_t bx = blockIdx.x;
    const T *src = nullptr;
    uint32_t b = 0, nvec = 0;
    FastDiv lenv{1, 0, 0, 0};
    int64_t off = 0;
#pragma unroll
    for (int k = 0; k < kConcatMax; k++) {
        if (k < a.n && bx >= a.block0[k] && bx < a.block0[k + 1]) {
            src = (const T *)a.src[k];
            b = bx - a.block0[k];
            nvec = a.nvec[k];
            lenv = a.lenv[k];
            off = a.off[k];
        }
    }
    const uint32_t base = b * (kMBlock * kRowsU);
    Vec<T, V> r[kRowsU];
#pragma unroll
    for (int u = 0; u < kRowsU; u++) {
        const uint32_t v = base + u * kMBlock + threadIdx.x;
        if (v < nvec) r[u] = vload<T, V>(src + (int64_t)v * V);
    }
#pragma unroll
    for (int u = 0; u < kRowsU; u++) {
        const uint32_t v = base + u * kMBlock + threadIdx.x;
        if (v < nvec) {
            const uint32_t row = fdiv(v, lenv), col = v - row * lenv.d;
            vstore_nt<T, V>(dst + (int64_t)row * a.total + off + (int64_t)col * V, r[u]);
        }
    }
}

template <typename T>
static hipError_t concat_typed(T *dst, int64_t outer, int64_t total, const ConcatPart *parts, int n, hipStream_t s) {
    constexpr int VW = 16 / sizeof(T) > 0 ? 16 / sizeof(T) : 1;
    bool vec = VW > 1 && total % VW == 0 && (uintptr_t)dst % 16 == 0;
    for (int i = 0; i < n; i++)
        if (parts[i].len % VW || parts[i].off % VW || (uintptr_t)parts[i].src % 16) vec = false;
    const int V = vec ? VW : 1;
    for (int i0 = 0; i0 < n; i0 += kConcatMax) {
        ConcatArgs a;
        memset(&a, 0, sizeof a);
        a.total = total;
        uint32_t blocks = 0;
        for (int i = i0; i < n && a.n < kConcatMax; i++) {
            const int64_t nv = outer * parts[i].len / V;
            if (nv == 0) continue;
            if (nv >= (1ll << 31)) return hipErrorInvalidValue;  // the host rejects it beforehand
            const int k = a.n++;
            a.src[k] = parts[i].src;
            a.block0[k] = blocks;
            a.nvec[k] = (uint32_t)nv;
            a.lenv[k] = make_fastdiv((uint32_t)(parts[i].len / V));
            a.off[k] = parts[i].off;
            blocks += (uint32_t)((nv + kMBlock * kRowsU - 1) / (kMBlock * kRowsU));
        }
        a.block0[a.n] = blocks;
        if (a.n == 0) continue;
        if (vec)
            hipLaunchKernelGGL((k_concat<T, VW>), dim3(blocks), dim3(kMBlock), 0, s, dst, a);
        else
            hipLaunchKernelGGL((k_concat<T, 1>), dim3(blocks), dim3(kMBlock), 0, s, dst, a);
    }
    return hipGetLastError();
}

hipError_t launch_concat(int esize, void *dst, int64_t outer, int64_t total, const ConcatPart *parts, int n,
                         hipStream_t s) {
    switch (esize) {
    case 1: return concat_typed<uint8_t>((uint8_t *)dst, outer, total, parts, n, s);
    case 2: return concat_typed<uint16_t>((uint16_t *)dst, outer, total, parts, n, s);
    case 4: return concat_typed<uint32_t>((uint32_t *)dst, outer, total, parts, n, s);
    case 8: return concat_typed<uint64_t>((uint64_t *)dst, outer, total, parts, n, s);
    default: return hipErrorInvalidValue;
    }
}

// ---------------------------------------------------------------------------
// Gather: kRowsU vectors of V contiguous elements of output rows per lane;
// output row (o, i) copies data row (o, idx[i]).
// ---------------------------------------------------------------------------
template <typename T, typename I, int V>
__global__ __launch_bounds__(kMBlock) void k_gather(const T *__restrict__ data, const I *__restrict__ idx,
                                                    T *__restrict__ out, uint32_t nvec, FastDiv inner_v, FastDiv nidx,
                                                    int64_t inner, int64_t dim, ErrFlags *errs) {
    for (uint32_t base = blockIdx.x * (kMBlock * kRowsU); base < nvec; base += gridDim.x * (kMBlock * kRowsU)) {
        Vec<T, V> r[kRowsU];
        bool ok[kRowsU];
#pragma unroll
        for (int u = 0; u < kRowsU; u++) {
            const uint32_t v = base + u * kMBlock + threadIdx.x;
            ok[u] = false;
            if (v < nvec) {
                const uint32_t rowi = fdiv(v, inner_v), cv = v - rowi * inner_v.d;
                const uint32_t o = fdiv(rowi, nidx), i = rowi - o * nidx.d;
                int64_t k = (int64_t)idx[i];
                if (k < 0) k += dim;  // HandleNegativeAxisOrIndex
                if (k < 0 || k >= dim) {
                    atomicMin(&errs->first_ovf, (unsigned long long)rowi * inner + (unsigned long long)cv * V);
                } else {
                    ok[u] = true;
                    r[u] = vload<T, V>(data + ((int64_t)o * dim + k) * inner + (int64_t)cv * V);
                }
            }
        }
#pragma unroll
        for (int u = 0; u < kRowsU; u++) {
            const uint32_t v = base + u * kMBlock + threadIdx.x;
            if (ok[u]) vstore_nt<T, V>(out + (int64_t)v * V, r[u]);
        }
    }
}

template <typename T, typename I>
static hipError_t gather_typed(const T *data, const I *idx, T *out, int64_t outer, int64_t nidx, int64_t inner,
                               int64_t dim, ErrFlags *errs, hipStream_t s) {
    constexpr int VW = 16 / sizeof(T) > 0 ? 16 / sizeof(T) : 1;
    const bool vec = VW > 1 && inner % VW == 0 && ((uintptr_t)data % 16 == 0) && ((uintptr_t)out % 16 == 0);
    const int64_t V = vec ? VW : 1;
    const int64_t nvec = outer * nidx * (inner / V);
    if (nvec == 0) return hipSuccess;
    if (nvec >= (1ll << 31)) return hipErrorInvalidValue;  // the host rejects it beforehand
    int64_t g = (nvec + kMBlock * kRowsU - 1) / (kMBlock * kRowsU);
    if (g > 65536 * 4) g = 65536 * 4;
    const FastDiv iv = make_fastdiv((uint32_t)(inner / V)), nd = make_fastdiv((uint32_t)nidx);
    if (vec)
        hipLaunchKernelGGL((k_gather<T, I, VW>), dim3((unsigned)g), dim3(kMBlock), 0, s, data, idx, out,
                           (uint32_t)nvec, iv, nd, inner, dim, errs);
    else
        hipLaunchKernelGGL((k_gather<T, I, 1>), dim3((unsigned)g), dim3(kMBlock), 0, s, data, idx, out,
                           (uint32_t)nvec, iv, nd, inner, dim, errs);
    return hipGetLastError();
}

template <typename T>
static hipError_t gather_by_index(int idx_dtype, const void *data, const void *idx, void *out, int64_t outer,
                                  int64_t nidx, int64_t inner, int64_t dim, ErrFlags *errs, hipStream_t s) {
    if (idx_dtype == kInt32)
        return gather_typed<T, int32_t>((const T *)data, (const int32_t *)idx, (T *)out, outer, nidx, inner, dim, errs, s);
    if (idx_dtype == kInt64)
        return gather_typed<T, int64_t>((const T *)data, (const int64_t *)idx, (T *)out, outer, nidx, inner, dim, errs, s);
    return hipErrorInvalidValue;
}

hipError_t launch_gather(int esize, int idx_dtype, const void *data, const void *idx, void *out, int64_t outer,
                         int64_t nidx, int64_t inner, int64_t dim, ErrFlags *errs, hipStream_t s) {
    switch (esize) {
    case 1: return gather_by_index<uint8_t>(idx_dtype, data, idx, out, outer, nidx, inner, dim, errs, s);
    case 2: return gather_by_index<uint16_t>(idx_dtype, data, idx, out, outer, nidx, inner, dim, errs, s);
    case 4: return gather_by_index<uint32_t>(idx_dtype, data, idx, out, outer, nidx, inner, dim, errs, s);
    case 8: return gather_by_index<uint64_t>(idx_dtype, data, idx, out, outer, nidx, inner, dim, errs, s);
    default: return hipErrorInvalidValue;
    }
}

}  // namespace lx
