// lx_matmul.hip -- MatMul on gfx950 (Tensor<T>.MatMul, TensorOps.cs:504-806,
// via CPUExecutionProvider.MatMul, CPUExecutionProvider.cs:359-378).
//
// float : v_mfma_f32_32x32x2f32 (fp32 products, fp32 accumulation -- the
//         reference's float32 arithmetic, summed in a different order).
//         block tiles from 64x64 to 128x128 (128x96 for N = 768) chosen per
//         shape, K step 16, four waves, double-buffered LDS fed from
//         registers one K step ahead.
// double: v_mfma_f64_16x16x4f64, 64x64 block tile, four waves of 32x32.
// int32 : exact two's-complement multiply-add on the VALU (no int32 MFMA),
//         16x16 LDS tiles.
// Batches: the leading (broadcast) axes are decomposed per block with
// per-operand element strides, 0 on broadcast axes (no materialisation).
// Layout of the MFMA operands and results checked on the device:
//   32x32x2 f32: a lane l = A[l%32][l/32], b = B[l/32][l%32],
//                acc[r] = C[8*(r/4) + 4*(l/32) + r%4][l%32]
//   16x16x4 f64: a = A[l%16][l/16], b = B[l/16][l%16], acc[r] = C[l/16 + 4r][l%16]
#include <hip/hip_runtime.h>

#include "lx_device.h"
#include "lx_kernels.h"

namespace lx {

typedef float v16f __attribute__((ext_vector_type(16)));
typedef double v4d __attribute__((ext_vector_type(4)));

// per-block batch offsets of A, B and C
__device__ __forceinline__ void batch_offsets(int64_t b, const MatMulArgs &p, int64_t *ao, int64_t *bo) {
    int64_t a = 0, c = 0;
    for (int d = p.nbatch - 1; d >= 0; d--) {
        const int64_t i = b % p.bdims[d];
        b /= p.bdims[d];
        a += i * p.a_bstr[d];
        c += i * p.b_bstr[d];
    }
    *ao = a;
    *bo = c;
}

// ---------------------------------------------------------------------------
// float: MFMA 32x32x2
// ---------------------------------------------------------------------------

// BM x BN block tile, four waves in a WM x WN grid, each wave (BM/WM) x (BN/WN)
// = MT x NT MFMA tiles of 32x32.  K steps of 16, double-buffered in LDS with k
// as the outer index (A transposed to [k][m], B as [k][n]), so the lanes of a
// fragment read 32 consecutive floats.  Register-only loops of this MFMA reach
// about 144 TF/s on MI355X; the 128x128 tile runs large GEMMs at 127-131 TF/s.
constexpr int kFBK = 16, kFPad = 4;

template <int BM, int BN, int WM, int WN, bool VEC, bool GELU>
__global__ __launch_bounds__(WM * WN * 64) void k_matmul_f32(const float *__restrict__ A, const float *__restrict__ B,
                                                             float *__restrict__ C, MatMulArgs p) {
    constexpr int NTHR = WM * WN * 64;               // threads of the block
    constexpr int WTM = BM / WM, WTN = BN / WN;      // wave tile
    constexpr int MT = WTM / 32, NT = WTN / 32;      // MFMA tiles per wave
    static_assert((WM * WN == 4 || WM * WN == 8) && MT * 32 == WTM && NT * 32 == WTN, "waves of whole 32x32 tiles");
    constexpr int AV = BM * kFBK / 4, BV = BN * kFBK / 4;  // float4 of A and of B per K step
    constexpr int LA = (AV + NTHR - 1) / NTHR, LB = (BV + NTHR - 1) / NTHR;
    constexpr int BQ = BN / 4;                       // float4 per B row
    __shared__ float As[2][kFBK][BM + kFPad];
    __shared__ float Bs[2][kFBK][BN + kFPad];
    __shared__ ExpTable tab;  // the GELU epilogue's exponential (filled before the first barrier)
    if constexpr (GELU) exp_table_fill(tab);
    const int M = p.m, N = p.n, K = p.k;
    const int t = threadIdx.x, l = t & 63, w = t >> 6;
    const int row0 = blockIdx.y * BM, col0 = blockIdx.x * BN;
    int64_t ao, bo;
    batch_offsets(p.batch_base + blockIdx.z, p, &ao, &bo);
    const float *Ab = A + ao;
    const float *Bb = B + bo;
    float *Cb = C + (p.batch_base + blockIdx.z) * (int64_t)M * N;

    // global -> register staging one K step ahead: float4 e = t + NTHR h of the step's
    // A tile (row e / KQ, k 4 (e % KQ)) and B tile (k row e / BQ, column 4 (e % BQ))
    constexpr int KQ = kFBK / 4;                     // float4 per A row of a K step
    float4 ra[LA], rb[LB];
    auto load = [&](int k0) {
#pragma unroll
        for (int h = 0; h < LA; h++) {
            const int e = t + NTHR * h;
            if (AV % NTHR != 0 && e >= AV) continue;
            const int r = row0 + e / KQ, kk = k0 + (e % KQ) * 4;
            if constexpr (VEC) {
                ra[h] = (r < M && kk < K) ? *reinterpret_cast<const float4 *>(Ab + (int64_t)r * K + kk)
                                          : make_float4(0.f, 0.f, 0.f, 0.f);
            } else {
                float v[4];
#pragma unroll
                for (int q = 0; q < 4; q++) v[q] = (r < M && kk + q < K) ? Ab[(int64_t)r * K + kk + q] : 0.f;
                ra[h] = make_float4(v[0], v[1], v[2], v[3]);
            }
        }
#pragma unroll
        for (int h = 0; h < LB; h++) {
            const int e = t + NTHR * h;
            if (BV % NTHR != 0 && e >= BV) continue;
            const int kb = k0 + e / BQ, c = col0 + (e % BQ) * 4;
            if constexpr (VEC) {
                rb[h] = (kb < K && c < N) ? *reinterpret_cast<const float4 *>(Bb + (int64_t)kb * N + c)
                                          : make_float4(0.f, 0.f, 0.f, 0.f);
            } else {
                float v[4];
#pragma unroll
                for (int q = 0; q < 4; q++) v[q] = (kb < K && c + q < N) ? Bb[(int64_t)kb * N + c + q] : 0.f;
                rb[h] = make_float4(v[0], v[1], v[2], v[3]);
            }
        }
    };
    auto store = [&](int buf) {
#pragma unroll
        for (int h = 0; h < LA; h++) {
            const int e = t + NTHR * h;
            if (AV % NTHR != 0 && e >= AV) continue;
            const int r = e / KQ, kk = (e % KQ) * 4;
            As[buf][kk + 0][r] = ra[h].x;
            As[buf][kk + 1][r] = ra[h].y;
            As[buf][kk + 2][r] = ra[h].z;
            As[buf][kk + 3][r] = ra[h].w;
        }
#pragma unroll
        for (int h = 0; h < LB; h++) {
            const int e = t + NTHR * h;
            if (BV % NTHR != 0 && e >= BV) continue;
            *reinterpret_cast<float4 *>(&Bs[buf][e / BQ][(e % BQ) * 4]) = rb[h];
        }
    };

    const int wr = (w / WN) * WTM, wc = (w % WN) * WTN;  // this wave's sub-tile
    v16f acc[MT][NT];
#pragma unroll
    for (int i = 0; i < MT; i++)
#pragma unroll
        for (int j = 0; j < NT; j++)
#pragma unroll
            for (int r = 0; r < 16; r++) acc[i][j][r] = 0.f;

    const int nk = (K + kFBK - 1) / kFBK;
    load(0);
    store(0);
    __syncthreads();
    int buf = 0;
    for (int kt = 0; kt < nk; kt++) {
        if (kt + 1 < nk) load((kt + 1) * kFBK);
#pragma unroll
        for (int kk = 0; kk < kFBK; kk += 2) {
            const int kr = kk + l / 32;
            float a[MT], b[NT];
#pragma unroll
            for (int i = 0; i < MT; i++) a[i] = As[buf][kr][wr + 32 * i + (l % 32)];
#pragma unroll
            for (int j = 0; j < NT; j++) b[j] = Bs[buf][kr][wc + 32 * j + (l % 32)];
#pragma unroll
            for (int i = 0; i < MT; i++)
#pragma unroll
                for (int j = 0; j < NT; j++)
                    acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x2f32(a[i], b[j], acc[i][j], 0, 0, 0);
        }
        if (kt + 1 < nk) store(buf ^ 1);
        __syncthreads();
        buf ^= 1;
    }
    const float *Rb = p.res ? p.res + (p.batch_base + blockIdx.z) * (int64_t)M * N : nullptr;
    const float *Bias = p.bias ? p.bias + (p.batch_base + blockIdx.z) * p.bias_bstr : nullptr;
#pragma unroll
    for (int i = 0; i < MT; i++)
#pragma unroll
        for (int j = 0; j < NT; j++) {
            const int c = col0 + wc + 32 * j + (l % 32);
            if (c >= N) continue;
            const float bc = Bias ? Bias[c] : 0.0f;
#pragma unroll
            for (int r = 0; r < 16; r++) {
                const int row = row0 + wr + 32 * i + 8 * (r / 4) + 4 * (l / 32) + (r % 4);
                if (row < M) {
                    float v = acc[i][j][r];
                    if (Bias) v = v + bc;
                    if (Rb) v = v + Rb[(int64_t)row * N + c];
                    if constexpr (GELU) v = gelu_erf_lx(v, tab);
                    Cb[(int64_t)row * N + c] = v;
                }
            }
        }
}

template <int BM, int BN, int WM, int WN>
static void launch_f32(const float *a, const float *b, float *c, const MatMulArgs &p, bool vec, hipStream_t s) {
    dim3 g((p.n + BN - 1) / BN, (p.m + BM - 1) / BM, (unsigned)p.batch);
    const dim3 blk(WM * WN * 64);
    if (p.gelu) {
        if (vec) hipLaunchKernelGGL((k_matmul_f32<BM, BN, WM, WN, true, true>), g, blk, 0, s, a, b, c, p);
        else hipLaunchKernelGGL((k_matmul_f32<BM, BN, WM, WN, false, true>), g, blk, 0, s, a, b, c, p);
    } else {
        if (vec) hipLaunchKernelGGL((k_matmul_f32<BM, BN, WM, WN, true, false>), g, blk, 0, s, a, b, c, p);
        else hipLaunchKernelGGL((k_matmul_f32<BM, BN, WM, WN, false, false>), g, blk, 0, s, a, b, c, p);
    }
}

// ---------------------------------------------------------------------------
// double: MFMA 16x16x4
// ---------------------------------------------------------------------------
constexpr int kDBM = 64, kDBN = 64, kDBK = 16, kDPad = 2;

__global__ __launch_bounds__(256) void k_matmul_f64(const double *__restrict__ A, const double *__restrict__ B,
                                                    double *__restrict__ C, MatMulArgs p) {
    __shared__ double As[kDBK][kDBM + kDPad];
    __shared__ double Bs[kDBK][kDBN + kDPad];
    const int M = p.m, N = p.n, K = p.k;
    const int t = threadIdx.x, l = t & 63, w = t >> 6;
    const int row0 = blockIdx.y * kDBM, col0 = blockIdx.x * kDBN;
    int64_t ao, bo;
    batch_offsets(p.batch_base + blockIdx.z, p, &ao, &bo);
    const double *Ab = A + ao;
    const double *Bb = B + bo;
    double *Cb = C + (p.batch_base + blockIdx.z) * (int64_t)M * N;
    const int wr = (w >> 1) * 32, wc = (w & 1) * 32;
    v4d acc[2][2];
#pragma unroll
    for (int i = 0; i < 2; i++)
#pragma unroll
        for (int j = 0; j < 2; j++)
#pragma unroll
            for (int r = 0; r < 4; r++) acc[i][j][r] = 0.0;
    for (int k0 = 0; k0 < K; k0 += kDBK) {
        // 64x16 A and 16x64 B tiles: four elements of each per thread
#pragma unroll
        for (int h = 0; h < 4; h++) {
            const int e = t + 256 * h;
            const int ar = e / kDBK, ak = e % kDBK;
            As[ak][ar] = (row0 + ar < M && k0 + ak < K) ? Ab[(int64_t)(row0 + ar) * K + k0 + ak] : 0.0;
            const int bk = e / kDBN, bc = e % kDBN;
            Bs[bk][bc] = (k0 + bk < K && col0 + bc < N) ? Bb[(int64_t)(k0 + bk) * N + col0 + bc] : 0.0;
        }
        __syncthreads();
#pragma unroll
        for (int kk = 0; kk < kDBK; kk += 4) {
            const int kr = kk + l / 16;
            double a0 = As[kr][wr + (l % 16)], a1 = As[kr][wr + 16 + (l % 16)];
            double b0 = Bs[kr][wc + (l % 16)], b1 = Bs[kr][wc + 16 + (l % 16)];
            acc[0][0] = __builtin_amdgcn_mfma_f64_16x16x4f64(a0, b0, acc[0][0], 0, 0, 0);
            acc[0][1] = __builtin_amdgcn_mfma_f64_16x16x4f64(a0, b1, acc[0][1], 0, 0, 0);
            acc[1][0] = __builtin_amdgcn_mfma_f64_16x16x4f64(a1, b0, acc[1][0], 0, 0, 0);
            acc[1][1] = __builtin_amdgcn_mfma_f64_16x16x4f64(a1, b1, acc[1][1], 0, 0, 0);
        }
        __syncthreads();
    }
#pragma unroll
    for (int i = 0; i < 2; i++)
#pragma unroll
        for (int j = 0; j < 2; j++) {
            const int c = col0 + wc + 16 * j + (l % 16);
            if (c >= N) continue;
#pragma unroll
            for (int r = 0; r < 4; r++) {
                const int row = row0 + wr + 16 * i + l / 16 + 4 * r;
                if (row < M) Cb[(int64_t)row * N + c] = acc[i][j][r];
            }
        }
}

// ---------------------------------------------------------------------------
// int32: exact wrapping multiply-add (C# unchecked int arithmetic)
// ---------------------------------------------------------------------------
__global__ __launch_bounds__(256) void k_matmul_i32(const int32_t *__restrict__ A, const int32_t *__restrict__ B,
                                                    int32_t *__restrict__ C, MatMulArgs p) {
    __shared__ uint32_t As[16][17], Bs[16][17];
    const int M = p.m, N = p.n, K = p.k;
    const int tx = threadIdx.x % 16, ty = threadIdx.x / 16;
    const int row = blockIdx.y * 16 + ty, col = blockIdx.x * 16 + tx;
    int64_t ao, bo;
    batch_offsets(p.batch_base + blockIdx.z, p, &ao, &bo);
    const int32_t *Ab = A + ao;
    const int32_t *Bb = B + bo;
    uint32_t acc = 0;
    for (int k0 = 0; k0 < K; k0 += 16) {
        As[ty][tx] = (row < M && k0 + tx < K) ? (uint32_t)Ab[(int64_t)row * K + k0 + tx] : 0u;
        Bs[ty][tx] = (k0 + ty < K && col < N) ? (uint32_t)Bb[(int64_t)(k0 + ty) * N + col] : 0u;
        __syncthreads();
#pragma unroll
        for (int k = 0; k < 16; k++) acc += As[ty][k] * Bs[k][tx];
        __syncthreads();
    }
    if (row < M && col < N) C[(p.batch_base + blockIdx.z) * (int64_t)M * N + (int64_t)row * N + col] = (int32_t)acc;
}

// ---------------------------------------------------------------------------
// dense copy of a strided view (the broadcast operands of MatMul's rank-1 case)
// ---------------------------------------------------------------------------
struct StridedView {
    int32_t rank;
    int64_t dims[8];
    int64_t strides[8];
};

template <typename T>
__global__ __launch_bounds__(256) void k_strided_copy(const T *__restrict__ x, T *__restrict__ y, int64_t n,
                                                      StridedView v) {
    for (int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x; i < n; i += (int64_t)gridDim.x * 256) {
        int64_t r = i, off = 0;
        for (int d = v.rank - 1; d >= 0; d--) {
            off += (r % v.dims[d]) * v.strides[d];
            r /= v.dims[d];
        }
        y[i] = x[off];
    }
}

hipError_t launch_strided_copy(int esize, const void *x, void *y, int rank, const int64_t *dims, const int64_t *strides,
                               hipStream_t s) {
    StridedView v;
    v.rank = rank;
    int64_t n = 1;
    for (int d = 0; d < rank; d++) {
        v.dims[d] = dims[d];
        v.strides[d] = strides[d];
        n *= dims[d];
    }
    if (n == 0) return hipSuccess;
    int64_t g = (n + 255) / 256;
    if (g > 65536) g = 65536;
    if (esize == 4)
        hipLaunchKernelGGL(k_strided_copy<uint32_t>, dim3((unsigned)g), dim3(256), 0, s, (const uint32_t *)x, (uint32_t *)y, n, v);
    else if (esize == 8)
        hipLaunchKernelGGL(k_strided_copy<uint64_t>, dim3((unsigned)g), dim3(256), 0, s, (const uint64_t *)x, (uint64_t *)y, n, v);
    else
        return hipErrorInvalidValue;
    return hipGetLastError();
}

hipError_t launch_matmul(int dtype, const void *a, const void *b, void *c, const MatMulArgs &p0, hipStream_t s) {
    if (p0.m == 0 || p0.n == 0 || p0.batch == 0) return hipSuccess;
    // grid z holds at most 65535 batches: larger batch counts take several launches
    if (p0.batch > 65535) {
        for (int64_t b0 = 0; b0 < p0.batch; b0 += 65535) {
            MatMulArgs q = p0;
            q.batch_base = p0.batch_base + b0;
            q.batch = p0.batch - b0 < 65535 ? p0.batch - b0 : 65535;
            hipError_t e = launch_matmul(dtype, a, b, c, q, s);
            if (e != hipSuccess) return e;
        }
        return hipSuccess;
    }
    const MatMulArgs &p = p0;
    if (dtype == kFloat) {
        bool vec = (p.k % 4 == 0) && (p.n % 4 == 0) && (((uintptr_t)a | (uintptr_t)b) % 16 == 0);
        for (int d = 0; d < p.nbatch; d++) vec = vec && (p.a_bstr[d] % 4 == 0) && (p.b_bstr[d] % 4 == 0);
        // block tile: among the tiles that give each of the 256 CUs two or more blocks (a lone block
        // per CU leaves its barrier and load latencies unhidden: measured 93 against 104 TF/s for
        // [4096,3072]x[3072,768]), the one whose busiest CU has the least work -- ceil(blocks / 256)
        // blocks, each costing its area over the tile's relative efficiency; 64x64 when none does
        const float *fa = (const float *)a, *fb = (const float *)b;
        float *fc = (float *)c;
        struct Tile {
            int bm, bn;
            double eff;
        };
        // (eight-wave 256x128 / 128x256 tiles measured 129.6 against 126.3 TFLOP/s at 4096^3 and far
        // slower wherever they leave fewer than two blocks per CU: not worth a candidate)
        static const Tile cand[] = {{128, 128, 1.0}, {128, 96, 0.93}, {96, 128, 0.93},
                                    {128, 64, 0.85}, {64, 128, 0.85}, {64, 64, 0.65}};
        constexpr int kCand = (int)(sizeof(cand) / sizeof(cand[0]));
        int best = 5;
        double best_cost = 0;
        for (int i = 0; i < kCand; i++) {
            const int64_t blocks =
                (int64_t)((p.m + cand[i].bm - 1) / cand[i].bm) * ((p.n + cand[i].bn - 1) / cand[i].bn) * p.batch;
            if (blocks < 512) continue;
            const double cost = (double)((blocks + 255) / 256) * cand[i].bm * cand[i].bn / cand[i].eff;
            if (best == 5 || cost < best_cost) {
                best = i;
                best_cost = cost;
            }
        }
        // a short K (at most 64, attention scores): the epilogue outweighs the K loop, and 64x64 tiles run
        // faster than the large ones ([16,12,512,64]x[16,12,64,512]: 70 against 66 TFLOP/s)
        if (p.k <= 64) best = 5;
        switch (best) {
        case 0: launch_f32<128, 128, 2, 2>(fa, fb, fc, p, vec, s); break;
        case 1: launch_f32<128, 96, 4, 1>(fa, fb, fc, p, vec, s); break;
        case 2: launch_f32<96, 128, 1, 4>(fa, fb, fc, p, vec, s); break;
        case 3: launch_f32<128, 64, 2, 2>(fa, fb, fc, p, vec, s); break;
        case 4: launch_f32<64, 128, 2, 2>(fa, fb, fc, p, vec, s); break;
        default: launch_f32<64, 64, 2, 2>(fa, fb, fc, p, vec, s); break;
        }
    } else if (dtype == kDouble) {
        dim3 g((p.n + kDBN - 1) / kDBN, (p.m + kDBM - 1) / kDBM, (unsigned)p.batch);
        hipLaunchKernelGGL(k_matmul_f64, g, dim3(256), 0, s, (const double *)a, (const double *)b, (double *)c, p);
    } else if (dtype == kInt32) {
        dim3 g((p.n + 15) / 16, (p.m + 15) / 16, (unsigned)p.batch);
        hipLaunchKernelGGL(k_matmul_i32, g, dim3(256), 0, s, (const int32_t *)a, (const int32_t *)b, (int32_t *)c, p);
    } else {
        return hipErrorInvalidValue;
    }
    return hipGetLastError();
}

}  // namespace lx
