// lx_matmul.hip -- MatMul on gfx950 (Tensor<T>.MatMul, TensorOps.cs:504-806,
// via CPUExecutionProvider.MatMul, CPUExecutionProvider.cs:359-378).
//
// float : v_mfma_f32_32x32x2f32 (fp32 products, fp32 accumulation -- the
//         reference's float32 arithmetic, summed in a different order, the
//         same order in both kernels).  K a multiple of 64 with aligned
//         operands: a ring of LDS stages filled by direct-to-LDS loads two or
//         three K steps ahead (k_matmul_f32_dl); otherwise double-buffered LDS
//         fed from registers one K step ahead (k_matmul_f32).  Block tiles
//         from 64x64 to 128x128 chosen per shape, K step 16, four waves.
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

#include <algorithm>
#include <type_traits>
#include <utility>

#include "lx_device.h"
#include "lx_kernels.h"

namespace lx {

typedef float v16f __attribute__((ext_vector_type(16)));
typedef double v4d __attribute__((ext_vector_type(4)));
typedef float v4f __attribute__((ext_vector_type(4)));

// per-block batch offsets of A, B and C
__device__ __forceinline__ void batch_offsets(int64_t b, const MatMulArgs &p, int64_t *ao, int64_t *bo,
                                              int64_t *co) {
    int64_t a = 0, bb = 0, c = 0;
    for (int d = p.nbatch - 1; d >= 0; d--) {
        const int64_t i = b % p.bdims[d];
        b /= p.bdims[d];
        a += i * p.a_bstr[d];
        bb += i * p.b_bstr[d];
        c += i * p.c_bstr[d];
    }
    *ao = a;
    *bo = bb;
    *co = c;
}

// ---------------------------------------------------------------------------
// float: MFMA 32x32x2
// ---------------------------------------------------------------------------

// Bias / residual / GELU epilogue and store of a wave's MT x NT tiles of 32x32 results (rows r0.., columns
// c0..) into the batch's C at offset co.  The MFMA ran as B^T A^T, so acc[i][j][q] = C[r0 + 32 i + l % 32][c0 +
// 32 j + 8 (q / 4) + 4 (l / 32) + q % 4]: each lane holds four consecutive columns of one row per group of four
// results (one 16-byte store).  The residual and the bias rows are dense.
template <int MT, int NT, bool VEC, bool GELU>
__device__ __forceinline__ void mm_epilogue(const v16f (&acc)[MT][NT], float *__restrict__ C, const MatMulArgs &p,
                                            int64_t co, int r0, int c0, int l, const ExpTable &tab) {
    const int M = p.m, N = p.n;
    const int64_t bz = p.batch_base + blockIdx.z;
    float *Cb = C + co;
    const float *Rb = p.res ? p.res + bz * (int64_t)M * N : nullptr;
    const float *Bias = p.bias ? p.bias + bz * p.bias_bstr : nullptr;
#pragma unroll
    for (int i = 0; i < MT; i++) {
        const int row = r0 + 32 * i + (l % 32);
        if (row >= M) continue;
        float *Cr = Cb + (int64_t)row * p.ldc;
        const float *Rr = Rb ? Rb + (int64_t)row * N : nullptr;
#pragma unroll
        for (int j = 0; j < NT; j++)
#pragma unroll
            for (int q = 0; q < 4; q++) {
                const int c = c0 + 32 * j + 8 * q + 4 * (l / 32);
                float v[4] = {acc[i][j][4 * q], acc[i][j][4 * q + 1], acc[i][j][4 * q + 2], acc[i][j][4 * q + 3]};
                if (VEC && c + 3 < N) {
                    if (Bias) {
                        const float4 bc = *reinterpret_cast<const float4 *>(Bias + c);
                        v[0] = v[0] + bc.x; v[1] = v[1] + bc.y; v[2] = v[2] + bc.z; v[3] = v[3] + bc.w;
                    }
                    if (Rr) {
                        const float4 rc = *reinterpret_cast<const float4 *>(Rr + c);
                        v[0] = v[0] + rc.x; v[1] = v[1] + rc.y; v[2] = v[2] + rc.z; v[3] = v[3] + rc.w;
                    }
                    if constexpr (GELU) {
#pragma unroll
                        for (int e = 0; e < 4; e++) v[e] = gelu_erf_lx(v[e], tab);
                    }
                    *reinterpret_cast<float4 *>(Cr + c) = make_float4(v[0], v[1], v[2], v[3]);
                } else {
#pragma unroll
                    for (int e = 0; e < 4; e++) {
                        if (c + e >= N) break;
                        float x = v[e];
                        if (Bias) x = x + Bias[c + e];
                        if (Rr) x = x + Rr[c + e];
                        if constexpr (GELU) x = gelu_erf_lx(x, tab);
                        Cr[c + e] = x;
                    }
                }
            }
    }
}

// Store of a wave's raw accumulators (no epilogue) into the partial product P (a dense M x N matrix, N a multiple
// of 4), in mm_epilogue's layout.
template <int MT, int NT>
__device__ __forceinline__ void mm_store_part(const v16f (&acc)[MT][NT], float *__restrict__ P, int M, int N, int r0,
                                              int c0, int l) {
#pragma unroll
    for (int i = 0; i < MT; i++) {
        const int row = r0 + 32 * i + (l % 32);
        if (row >= M) continue;
        float *Pr = P + (int64_t)row * N;
#pragma unroll
        for (int j = 0; j < NT; j++)
#pragma unroll
            for (int q = 0; q < 4; q++) {
                const int c = c0 + 32 * j + 8 * q + 4 * (l / 32);
                if (c < N)
                    *reinterpret_cast<v4f *>(Pr + c) =
                        v4f{acc[i][j][4 * q], acc[i][j][4 * q + 1], acc[i][j][4 * q + 2], acc[i][j][4 * q + 3]};
            }
    }
}

// C = epilogue(P[0] + P[1] + ... + P[split - 1]) over the split partial products of a launch's batches, summed in
// that order, then the bias, residual and GELU of mm_epilogue, each rounded as there: 16 bytes per lane.
template <bool GELU>
__global__ __launch_bounds__(256) void k_matmul_split_sum(float *__restrict__ C, MatMulArgs p) {
    __shared__ ExpTable tab;
    if constexpr (GELU) {
        exp_table_fill(tab);
        __syncthreads();
    }
    const int64_t mn = (int64_t)p.m * p.n, nq = mn / 4;
    const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
    if (i >= nq * p.batch) return;
    const int64_t zb = i / nq, e = (i - zb * nq) * 4;  // batch of this launch, element of its matrix
    const int64_t stride = p.batch * mn;                // between the partials of two K ranges
    const float *P = p.part + zb * mn + e;
    // the bias and residual loaded with the partials, one memory latency for all (added after them, as before)
    const int64_t bz = p.batch_base + zb;
    const float4 bc = p.bias ? *reinterpret_cast<const float4 *>(p.bias + bz * p.bias_bstr + e % p.n)
                             : make_float4(0.f, 0.f, 0.f, 0.f);
    const float4 rc = p.res ? *reinterpret_cast<const float4 *>(p.res + bz * mn + e) : make_float4(0.f, 0.f, 0.f, 0.f);
    // the partials eight at a time, all eight loads in flight before the first add (one memory latency per
    // eight, not one per partial); the adds in range order
    constexpr int kChunk = 8;
    v4f v = *reinterpret_cast<const v4f *>(P);
    for (int s0 = 1; s0 < p.split; s0 += kChunk) {
        v4f x[kChunk];
#pragma unroll
        for (int c = 0; c < kChunk; c++)
            if (s0 + c < p.split) x[c] = *reinterpret_cast<const v4f *>(P + (s0 + c) * stride);
#pragma unroll
        for (int c = 0; c < kChunk; c++)
            if (s0 + c < p.split) {
                v[0] = v[0] + x[c][0]; v[1] = v[1] + x[c][1]; v[2] = v[2] + x[c][2]; v[3] = v[3] + x[c][3];
            }
    }
    if (p.bias) {
        v[0] = v[0] + bc.x; v[1] = v[1] + bc.y; v[2] = v[2] + bc.z; v[3] = v[3] + bc.w;
    }
    if (p.res) {
        v[0] = v[0] + rc.x; v[1] = v[1] + rc.y; v[2] = v[2] + rc.z; v[3] = v[3] + rc.w;
    }
    if constexpr (GELU) {
#pragma unroll
        for (int k = 0; k < 4; k++) v[k] = gelu_erf_lx(v[k], tab);
    }
    int64_t ao, bo, co;
    batch_offsets(bz, p, &ao, &bo, &co);
    const int64_t row = e / p.n;
    *reinterpret_cast<float4 *>(C + co + row * p.ldc + (e - row * p.n)) = make_float4(v[0], v[1], v[2], v[3]);
}

// k_matmul_split_sum for a product whose rows are then normalised (the decomposed LayerNorm after a projection and
// its residual): one wave per row, lane l holding the vectors c * 64 + l as k_layernorm does; each element summed
// over the partials in range order with the bias and residual exactly as in k_matmul_split_sum, then the row
// normalised by ln_row_finish into y (dense, the product's shape).  Bit for bit k_matmul_split_sum followed by
// k_layernorm, without the product's round trip through memory.
template <int NV>
__global__ __launch_bounds__(64) void k_matmul_split_sum_ln(const float *__restrict__ gamma, const float *__restrict__ beta,
                                                             float eps, float *__restrict__ y, MatMulArgs p) {
    const int lane = threadIdx.x;
    const int64_t rg = blockIdx.x, zb = rg / p.m, row = rg - zb * p.m;  // row of the launch's batch zb
    const int N = p.n;
    const int64_t mn = (int64_t)p.m * N, stride = p.batch * mn, bz = p.batch_base + zb;
    constexpr int kChunk = 8;
    // the bias, residual, gamma and beta vectors loaded with the partials, one memory latency for all
    Vec<float, 4> v[NV], gv[NV], bv[NV];
    float4 bcv[NV], rcv[NV];
#pragma unroll
    for (int c = 0; c < NV; c++) {
        const int col = (c * 64 + lane) * 4;
        if (col >= N) continue;
        gv[c] = vload<float, 4>(gamma + col);
        bv[c] = vload<float, 4>(beta + col);
        if (p.bias) bcv[c] = *reinterpret_cast<const float4 *>(p.bias + bz * p.bias_bstr + col);
        if (p.res) rcv[c] = *reinterpret_cast<const float4 *>(p.res + bz * mn + row * N + col);
    }
#pragma unroll
    for (int c = 0; c < NV; c++) {
        const int col = (c * 64 + lane) * 4;
        v[c] = Vec<float, 4>{{0.0f, 0.0f, 0.0f, 0.0f}};
        if (col >= N) continue;
        const float *P = p.part + zb * mn + row * N + col;
        v4f a = *reinterpret_cast<const v4f *>(P);
        for (int s0 = 1; s0 < p.split; s0 += kChunk) {
            v4f x[kChunk];
#pragma unroll
            for (int q = 0; q < kChunk; q++)
                if (s0 + q < p.split) x[q] = *reinterpret_cast<const v4f *>(P + (s0 + q) * stride);
#pragma unroll
            for (int q = 0; q < kChunk; q++)
                if (s0 + q < p.split) {
                    a[0] = a[0] + x[q][0]; a[1] = a[1] + x[q][1]; a[2] = a[2] + x[q][2]; a[3] = a[3] + x[q][3];
                }
        }
        if (p.bias) {
            const float4 bc = bcv[c];
            a[0] = a[0] + bc.x; a[1] = a[1] + bc.y; a[2] = a[2] + bc.z; a[3] = a[3] + bc.w;
        }
        if (p.res) {
            const float4 rc = rcv[c];
            a[0] = a[0] + rc.x; a[1] = a[1] + rc.y; a[2] = a[2] + rc.z; a[3] = a[3] + rc.w;
        }
        v[c] = Vec<float, 4>{{a[0], a[1], a[2], a[3]}};
    }
    ln_row_finish<NV>(v, N, lane, gamma, beta, eps, y + bz * mn + row * N, gv, bv);
}

// BM x BN block tile, four waves in a WM x WN grid, each wave (BM/WM) x (BN/WN)
// = MT x NT MFMA tiles of 32x32.  K steps of 16, double-buffered in LDS with k
// as the outer index (A transposed to [k][m], B as [k][n]), so the lanes of a
// fragment read 32 consecutive floats.  The kernel for K not a multiple of 64,
// unaligned operands, K <= 64, N <= 64 and 128x96 tiles beyond one per CU.
constexpr int kFBK = 16, kFPad = 4;

// BT: B stored by columns (element (k, n) at n * ldb + k: a transposed view), loaded as A is, along K, and
// written into the same LDS layout, so the MFMAs and their sums are those of a row-major B.
template <int BM, int BN, int WM, int WN, bool VEC, bool GELU, bool BT = false>
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
    int64_t ao, bo, co;
    batch_offsets(p.batch_base + blockIdx.z, p, &ao, &bo, &co);
    const float *Ab = A + ao;
    const float *Bb = B + bo;
    const int64_t lda = p.lda, ldb = p.ldb;

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
                ra[h] = (r < M && kk < K) ? *reinterpret_cast<const float4 *>(Ab + (int64_t)r * lda + kk)
                                          : make_float4(0.f, 0.f, 0.f, 0.f);
            } else {
                float v[4];
#pragma unroll
                for (int q = 0; q < 4; q++) v[q] = (r < M && kk + q < K) ? Ab[(int64_t)r * lda + kk + q] : 0.f;
                ra[h] = make_float4(v[0], v[1], v[2], v[3]);
            }
        }
#pragma unroll
        for (int h = 0; h < LB; h++) {
            const int e = t + NTHR * h;
            if (BV % NTHR != 0 && e >= BV) continue;
            if constexpr (BT) {  // column col0 + e / KQ, k 4 (e % KQ) of the step
                const int c = col0 + e / KQ, kk = k0 + (e % KQ) * 4;
                if constexpr (VEC) {
                    rb[h] = (c < N && kk < K) ? *reinterpret_cast<const float4 *>(Bb + (int64_t)c * ldb + kk)
                                              : make_float4(0.f, 0.f, 0.f, 0.f);
                } else {
                    float v[4];
#pragma unroll
                    for (int q = 0; q < 4; q++) v[q] = (c < N && kk + q < K) ? Bb[(int64_t)c * ldb + kk + q] : 0.f;
                    rb[h] = make_float4(v[0], v[1], v[2], v[3]);
                }
                continue;
            }
            const int kb = k0 + e / BQ, c = col0 + (e % BQ) * 4;
            if constexpr (VEC) {
                rb[h] = (kb < K && c < N) ? *reinterpret_cast<const float4 *>(Bb + (int64_t)kb * ldb + c)
                                          : make_float4(0.f, 0.f, 0.f, 0.f);
            } else {
                float v[4];
#pragma unroll
                for (int q = 0; q < 4; q++) v[q] = (kb < K && c + q < N) ? Bb[(int64_t)kb * ldb + c + q] : 0.f;
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
            if constexpr (BT) {
                const int c = e / KQ, kk = (e % KQ) * 4;
                Bs[buf][kk + 0][c] = rb[h].x;
                Bs[buf][kk + 1][c] = rb[h].y;
                Bs[buf][kk + 2][c] = rb[h].z;
                Bs[buf][kk + 3][c] = rb[h].w;
            } else {
                *reinterpret_cast<float4 *>(&Bs[buf][e / BQ][(e % BQ) * 4]) = rb[h];
            }
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
        // MFMA j of the step takes k = j from lanes 0-31 and k = 8 + j from lanes 32-63, the order of the
        // direct-load kernel below: every float MatMul sums its products in one order, whichever kernel runs it
#pragma unroll
        for (int j = 0; j < kFBK / 2; j++) {
            const int kr = 8 * (l / 32) + j;
            float a[MT], b[NT];
#pragma unroll
            for (int i = 0; i < MT; i++) a[i] = As[buf][kr][wr + 32 * i + (l % 32)];
#pragma unroll
            for (int jn = 0; jn < NT; jn++) b[jn] = Bs[buf][kr][wc + 32 * jn + (l % 32)];
#pragma unroll
            for (int i = 0; i < MT; i++)
#pragma unroll
                for (int jn = 0; jn < NT; jn++)
                    acc[i][jn] = __builtin_amdgcn_mfma_f32_32x32x2f32(b[jn], a[i], acc[i][jn], 0, 0, 0);
        }
        if (kt + 1 < nk) store(buf ^ 1);
        __syncthreads();
        buf ^= 1;
    }
    mm_epilogue<MT, NT, VEC, GELU>(acc, C, p, co, row0 + wr, col0 + wc, l, tab);
}

// Direct-to-LDS pipeline for K a multiple of 64 and 16-byte aligned operands.  Each K step of 16 is one stage of a
// four-stage ring in LDS, filled by global_load_lds_dwordx4 (16 bytes per lane straight into LDS, no register
// staging) three steps ahead of the MFMAs, with one barrier per step; each wave reads its fragments of a stage one
// step before it multiplies them.  Stage layout:
//   A: BM rows of the step's 16 floats (four 16-byte chunks per row, chunk c of row r at slot c ^ swz(r));
//   B: the step's rows 0-7, then 128 bytes on, rows 8-15, each row BN floats.
// The K order within a step is permuted: MFMA j (j = 0..7) takes k = j from lanes 0-31 and k = 8 + j from lanes
// 32-63, so a lane's A operands for the whole step are eight consecutive floats of its row (two 16-byte reads).
// Rows past M and columns past N read a clamped in-range address (their results are not stored).
__device__ __forceinline__ int dl_swz(int r) { return ((r >> 1) ^ (r >> 3)) & 3; }

// global_load_lds_dwordx4: the lane's 16 bytes at g land in LDS at lds + 16 * lane (lds uniform over the wave).
// Written as inline asm so that the compiler does not track these LDS writes: it would otherwise wait for every
// outstanding direct load before LDS reads of the other stages.  The kernel orders them itself: a stage is read
// only after an s_waitcnt vmcnt that covers its loads and a barrier.  (Loads the compiler does not count only
// make its own vmcnt waits longer.)  The LDS address goes in M0 (set by the compiler, an operand of the asm),
// which takes one wait state before the load.
__device__ __forceinline__ void load_to_lds16(const float *g, char *lds) {
#if defined(__HIP_DEVICE_COMPILE__)
    const uint32_t m0 = (uint32_t)(uintptr_t)(__attribute__((address_space(3))) char *)lds;
    __asm__ volatile("s_nop 0\n\tglobal_load_lds_dwordx4 %1, off" ::"{m0}"(m0), "v"(g) : "memory");
#else
    (void)g;
    (void)lds;
#endif
}
// no instruction is scheduled across this point
__device__ __forceinline__ void sched_fence() {
#if defined(__HIP_DEVICE_COMPILE__)
    __builtin_amdgcn_sched_barrier(0);
#endif
}

// f(integral_constant<int, i>) for i = R0 .. R1 - 1, in order
template <int R0, typename F, int... Is>
__device__ __forceinline__ void static_for_impl(F &&f, std::integer_sequence<int, Is...>) {
    (f(std::integral_constant<int, R0 + Is>()), ...);
}
template <int R0, int R1, typename F>
__device__ __forceinline__ void static_for(F &&f) {
    if constexpr (R1 > R0) static_for_impl<R0>(f, std::make_integer_sequence<int, R1 - R0>());
}

// s_waitcnt vmcnt(n) lgkmcnt(0), then s_barrier: this wave's direct loads but the last n have landed and its LDS
// reads are done before any wave passes.  (A __syncthreads would wait for every outstanding direct load.)
template <int N>
__device__ __forceinline__ void wait_vmcnt_barrier() {
    static_assert(N >= 0 && N < 64, "vmcnt range");
    __builtin_amdgcn_s_waitcnt((N & 15) | ((N >> 4) << 14) | (7 << 4));
#if defined(__HIP_DEVICE_COMPILE__)
    __asm__ volatile("s_barrier" ::: "memory");
#endif
}

// SPLIT: block z = batch * p.split + r computes the partial product of the r-th of p.split equal K ranges (whole
// passes of four steps) into p.part, without the epilogue (k_matmul_split_sum applies it).
template <int BM, int BN, int WM, int WN, int S, int WMIN, int WMAX, bool GELU, bool SPLIT = false>
__global__ __launch_bounds__(WM * WN * 64) __attribute__((amdgpu_waves_per_eu(WMIN, WMAX))) void k_matmul_f32_dl(const float *__restrict__ A, const float *__restrict__ B,
                                                                float *__restrict__ C, MatMulArgs p) {
    constexpr int NW = WM * WN;
    constexpr int WTM = BM / WM, WTN = BN / WN, MT = WTM / 32, NT = WTN / 32;
    static_assert(MT * 32 == WTM && NT * 32 == WTN && S >= 2 && S <= 4, "waves of whole 32x32 tiles");
    constexpr int A_BYTES = BM * 64, B_HALF = BN * 32, B_HI = A_BYTES + B_HALF + 128;
    constexpr int STAGE = A_BYTES + 2 * B_HALF + 128;
    static_assert(A_BYTES % 1024 == 0 && B_HALF % 1024 == 0, "whole wave loads");
    constexpr int LA = A_BYTES / 1024, LBH = B_HALF / 1024, NL = LA + 2 * LBH;
    constexpr int L = (NL + NW - 1) / NW;  // wave loads per wave per stage (the last one repeated when uneven)
    // one LDS variable per stage: the compiler then knows that the reads of one stage do not wait for the
    // direct loads still landing in the others
    __shared__ __attribute__((aligned(1024))) char sm0[STAGE];
    __shared__ __attribute__((aligned(1024))) char sm1[STAGE];
    __shared__ __attribute__((aligned(1024))) char sm2[STAGE];
    __shared__ __attribute__((aligned(1024))) char sm3[STAGE];
    auto stage_mem = [&](auto sidx) -> char * {
        constexpr int sx = decltype(sidx)::value;
        if constexpr (sx == 0) return sm0;
        else if constexpr (sx == 1) return sm1;
        else if constexpr (sx == 2) return sm2;
        else return sm3;
    };
    __shared__ ExpTable tab;
    if constexpr (GELU) exp_table_fill(tab);
    const int M = p.m, N = p.n, K = p.k;
    const int l = threadIdx.x & 63;
    const int w = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int row0 = blockIdx.y * BM, col0 = blockIdx.x * BN;
    // the batch of this launch and, split, the K range: steps [k0, k0 + nk) of 16
    const int zb = SPLIT ? (int)blockIdx.z / p.split : (int)blockIdx.z;
    const int nk = SPLIT ? K / 16 / p.split : K / 16;
    const int k0 = SPLIT ? ((int)blockIdx.z - zb * p.split) * nk * 16 : 0;
    int64_t ao, bo, co;
    batch_offsets(p.batch_base + zb, p, &ao, &bo, &co);

    // this wave's loads: a per-lane source address (advanced by `inc` floats per step) and an LDS offset
    const float *src[L];
    int64_t inc[L];
    int dst[L];
#pragma unroll
    for (int j = 0; j < L; j++) {
        const int i = min(w + NW * j, NL - 1);
        if (i < LA) {
            const int q = 64 * i + l, r = q >> 2, c = (q & 3) ^ dl_swz(r);
            src[j] = A + ao + (int64_t)min(row0 + r, M - 1) * p.lda + k0 + 4 * c;
            inc[j] = 16;
            dst[j] = 1024 * i;
        } else {
            const int h = (i - LA) / LBH, wl = (i - LA) % LBH, q = 64 * wl + l;
            const int k = 8 * h + q / (BN / 4), c = col0 + 4 * (q % (BN / 4));
            src[j] = B + bo + (int64_t)(k0 + k) * p.ldb + min(c, N - 4);
            inc[j] = 16 * p.ldb;
            dst[j] = A_BYTES + h * (B_HALF + 128) + 1024 * wl;
        }
    }
    auto issue = [&](auto sidx, int kt) {
        char *base = stage_mem(sidx);
#pragma unroll
        for (int j = 0; j < L; j++)
            load_to_lds16(src[j] + kt * inc[j], base + dst[j]);
    };

    // fragment offsets within a stage
    const int wr = (w / WN) * WTM, wc = (w % WN) * WTN, h = l / 32;
    int aoff[MT][2], boff[NT];
#pragma unroll
    for (int i = 0; i < MT; i++) {
        const int r = wr + 32 * i + (l % 32);
#pragma unroll
        for (int e = 0; e < 2; e++) aoff[i][e] = r * 64 + 16 * ((2 * h + e) ^ dl_swz(r));
    }
#pragma unroll
    for (int j = 0; j < NT; j++) boff[j] = (h ? B_HI : A_BYTES) + 4 * (wc + 32 * j + (l % 32));

    v16f acc[MT][NT];
#pragma unroll
    for (int i = 0; i < MT; i++)
#pragma unroll
        for (int j = 0; j < NT; j++)
#pragma unroll
            for (int r = 0; r < 16; r++) acc[i][j][r] = 0.f;

    // Step t: wait for this wave's loads of step t + 1 (the S - 3 later steps' loads stay outstanding); barrier
    // (every wave's loads of step t + 1 are visible, and stage (t - 1) % S, read during step t - 2, is free);
    // issue step t + S - 1 into that stage; read step t + 1's fragments; run step t's MFMAs on the fragments read
    // during step t - 1.  No read latency lies between the barrier and the first MFMA.  The LDS reads are
    // ordinary loads, waited for by the compiler; the direct loads are invisible to it (load_to_lds16).
    // two fragment sets, the current step's and the next's, swapping roles from step to step (no copies)
    v4f af0[MT][2], af1[MT][2];
    float bf0[NT][8], bf1[NT][8];
    auto read_all = [&](auto sidx, v4f (&ra)[MT][2], float (&rb)[NT][8]) {
        const char *stg = stage_mem(sidx);
#pragma unroll
        for (int i = 0; i < MT; i++) {
            ra[i][0] = *reinterpret_cast<const v4f *>(stg + aoff[i][0]);
            ra[i][1] = *reinterpret_cast<const v4f *>(stg + aoff[i][1]);
        }
#pragma unroll
        for (int j = 0; j < NT; j++)
#pragma unroll
            for (int kk = 0; kk < 8; kk++) rb[j][kk] = *reinterpret_cast<const float *>(stg + boff[j] + kk * BN * 4);
    };
    auto step = [&](auto sidx, int t, const v4f (&caf)[MT][2], const float (&cbf)[NT][8], v4f (&naf)[MT][2],
                    float (&nbf)[NT][8]) {
        constexpr int sx = decltype(sidx)::value;
        wait_vmcnt_barrier<(S - 3) * L>();
        // the MFMAs of k pair kk, then a slice of the next stage's fragment reads (the direct loads after the first
        // pair): the reads' latency hides under the MFMAs that follow, and the fences keep this order
        const char *nst = stage_mem(std::integral_constant<int, (sx + 1) % S>());
        constexpr int R = 2 * MT + 8 * NT;  // fragment reads per stage
        auto read_one = [&](auto rc) {
            constexpr int r = decltype(rc)::value;
            if constexpr (r < 2 * MT) {
                naf[r / 2][r % 2] = *reinterpret_cast<const v4f *>(nst + aoff[r / 2][r % 2]);
            } else {
                constexpr int j = (r - 2 * MT) / 8, kk = (r - 2 * MT) % 8;
                nbf[j][kk] = *reinterpret_cast<const float *>(nst + boff[j] + kk * BN * 4);
            }
        };
        static_for<0, 8>([&](auto kc) {
            constexpr int kk = decltype(kc)::value;
#pragma unroll
            for (int i = 0; i < MT; i++)
#pragma unroll
                for (int j = 0; j < NT; j++)
                    acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x2f32(cbf[j][kk], caf[i][kk / 4][kk % 4], acc[i][j], 0, 0, 0);
            sched_fence();
            if constexpr (kk == 0) {
                // past the last step the ring re-loads step nk - 1 into a stage no later step reads: every
                // step then issues the same loads, and the wait above is the same count everywhere
                issue(std::integral_constant<int, (sx + S - 1) % S>(), min(t + S - 1, nk - 1));
            } else if constexpr (kk <= 6) {
                static_for<(kk - 1) * R / 6, kk * R / 6>(read_one);
            }
            sched_fence();
        });
    };
    issue(std::integral_constant<int, 0>(), 0);
    issue(std::integral_constant<int, 1>(), min(1, nk - 1));
    issue(std::integral_constant<int, 2>(), min(2, nk - 1));
    static_assert(S == 4, "fragments a step ahead need the loads two steps ahead; four steps per loop pass");
    wait_vmcnt_barrier<(S - 2) * L>();
    read_all(std::integral_constant<int, 0>(), af0, bf0);
    // K is a multiple of 64: whole passes of four steps, each fragment set in the same registers on every pass
    for (int t = 0; t < nk; t += S) {
        step(std::integral_constant<int, 0>(), t, af0, bf0, af1, bf1);
        step(std::integral_constant<int, 1>(), t + 1, af1, bf1, af0, bf0);
        step(std::integral_constant<int, 2>(), t + 2, af0, bf0, af1, bf1);
        step(std::integral_constant<int, 3>(), t + 3, af1, bf1, af0, bf0);
    }
    // the ring's last loads land before the wave can end (the block's LDS is then handed to another block)
    __builtin_amdgcn_s_waitcnt((7 << 4) | (15 << 8));
    if constexpr (SPLIT)
        mm_store_part<MT, NT>(acc, p.part + ((int64_t)(blockIdx.z - zb * p.split) * p.batch + zb) * M * N, M, N,
                              row0 + wr, col0 + wc, l);
    else
        mm_epilogue<MT, NT, true, GELU>(acc, C, p, co, row0 + wr, col0 + wc, l, tab);
}

template <int BM, int BN, int WM, int WN, int WMIN, int WMAX>
static void launch_f32_dl(const float *a, const float *b, float *c, const MatMulArgs &p, hipStream_t s) {
    dim3 g((p.n + BN - 1) / BN, (p.m + BM - 1) / BM, (unsigned)p.batch);
    const dim3 blk(WM * WN * 64);
    if (p.gelu) hipLaunchKernelGGL((k_matmul_f32_dl<BM, BN, WM, WN, 4, WMIN, WMAX, true>), g, blk, 0, s, a, b, c, p);
    else hipLaunchKernelGGL((k_matmul_f32_dl<BM, BN, WM, WN, 4, WMIN, WMAX, false>), g, blk, 0, s, a, b, c, p);
}

// Split K (p.split ranges, p.part holding the partials): 64x64 tiles, then the ordered sum with the epilogue.
static void launch_f32_split(const float *a, const float *b, float *c, const MatMulArgs &p, hipStream_t s) {
    dim3 g((p.n + 63) / 64, (p.m + 63) / 64, (unsigned)(p.batch * p.split));
    hipLaunchKernelGGL((k_matmul_f32_dl<64, 64, 2, 2, 4, 3, 8, false, true>), g, dim3(256), 0, s, a, b, c, p);
    const int64_t nq = (int64_t)p.m * p.n / 4 * p.batch;
    const dim3 gs((unsigned)((nq + 255) / 256));
    if (p.gelu) hipLaunchKernelGGL(k_matmul_split_sum<true>, gs, dim3(256), 0, s, c, p);
    else hipLaunchKernelGGL(k_matmul_split_sum<false>, gs, dim3(256), 0, s, c, p);
}

template <int BM, int BN, int WM, int WN>
static void launch_f32(const float *a, const float *b, float *c, const MatMulArgs &p, bool vec, hipStream_t s) {
    dim3 g((p.n + BN - 1) / BN, (p.m + BM - 1) / BM, (unsigned)p.batch);
    const dim3 blk(WM * WN * 64);
    if (p.bt) {  // a transposed view of B, without an epilogue
        if (vec) hipLaunchKernelGGL((k_matmul_f32<BM, BN, WM, WN, true, false, true>), g, blk, 0, s, a, b, c, p);
        else hipLaunchKernelGGL((k_matmul_f32<BM, BN, WM, WN, false, false, true>), g, blk, 0, s, a, b, c, p);
        return;
    }
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
// BM x BN block tile, four waves in a 2 x 2 grid, each (BM / 2) x (BN / 2) = MT x NT MFMA tiles of 16x16.  K steps
// of 16, double-buffered in LDS with k as the outer index (A transposed to [k][m], B as [k][n]), fed from
// registers one step ahead; VEC: 16-byte loads (k, n, the row and batch strides even, the operands 16-byte
// aligned).  Each dot product is summed in K order, four products per MFMA.
constexpr int kDBK = 16, kDPad = 2;

template <int BM, int BN, bool VEC>
__global__ __launch_bounds__(256) void k_matmul_f64(const double *__restrict__ A, const double *__restrict__ B,
                                                    double *__restrict__ C, MatMulArgs p) {
    constexpr int WTM = BM / 2, WTN = BN / 2, MT = WTM / 16, NT = WTN / 16;
    constexpr int AV = BM * kDBK / 2, BV = BN * kDBK / 2;  // 16-byte pairs of A and of B per K step
    static_assert(AV % 256 == 0 && BV % 256 == 0 && MT * 16 == WTM && NT * 16 == WTN, "whole tiles and loads");
    constexpr int LA = AV / 256, LB = BV / 256;
    constexpr int KQ = kDBK / 2, BQ = BN / 2;              // pairs per A row and per B row of a step
    __shared__ double As[2][kDBK][BM + kDPad];
    __shared__ double Bs[2][kDBK][BN + kDPad];
    const int M = p.m, N = p.n, K = p.k;
    const int t = threadIdx.x, l = t & 63, w = t >> 6;
    const int row0 = blockIdx.y * BM, col0 = blockIdx.x * BN;
    int64_t ao, bo, co;
    batch_offsets(p.batch_base + blockIdx.z, p, &ao, &bo, &co);
    const double *Ab = A + ao;
    const double *Bb = B + bo;
    double *Cb = C + co;
    const int64_t lda = p.lda, ldb = p.ldb;
    double2 ra[LA], rb[LB];
    auto load = [&](int k0) {
#pragma unroll
        for (int h = 0; h < LA; h++) {
            const int e = t + 256 * h;
            const int r = row0 + e / KQ, kk = k0 + (e % KQ) * 2;
            if constexpr (VEC) {
                ra[h] = (r < M && kk < K) ? *reinterpret_cast<const double2 *>(Ab + (int64_t)r * lda + kk)
                                          : make_double2(0.0, 0.0);
            } else {
                ra[h].x = (r < M && kk < K) ? Ab[(int64_t)r * lda + kk] : 0.0;
                ra[h].y = (r < M && kk + 1 < K) ? Ab[(int64_t)r * lda + kk + 1] : 0.0;
            }
        }
#pragma unroll
        for (int h = 0; h < LB; h++) {
            const int e = t + 256 * h;
            const int kb = k0 + e / BQ, c = col0 + (e % BQ) * 2;
            if constexpr (VEC) {
                rb[h] = (kb < K && c < N) ? *reinterpret_cast<const double2 *>(Bb + (int64_t)kb * ldb + c)
                                          : make_double2(0.0, 0.0);
            } else {
                rb[h].x = (kb < K && c < N) ? Bb[(int64_t)kb * ldb + c] : 0.0;
                rb[h].y = (kb < K && c + 1 < N) ? Bb[(int64_t)kb * ldb + c + 1] : 0.0;
            }
        }
    };
    auto store = [&](int buf) {
#pragma unroll
        for (int h = 0; h < LA; h++) {
            const int e = t + 256 * h;
            const int r = e / KQ, kk = (e % KQ) * 2;
            As[buf][kk][r] = ra[h].x;
            As[buf][kk + 1][r] = ra[h].y;
        }
#pragma unroll
        for (int h = 0; h < LB; h++) {
            const int e = t + 256 * h;
            *reinterpret_cast<double2 *>(&Bs[buf][e / BQ][(e % BQ) * 2]) = rb[h];
        }
    };
    const int wr = (w >> 1) * WTM, wc = (w & 1) * WTN;
    v4d acc[MT][NT];
#pragma unroll
    for (int i = 0; i < MT; i++)
#pragma unroll
        for (int j = 0; j < NT; j++)
#pragma unroll
            for (int r = 0; r < 4; r++) acc[i][j][r] = 0.0;
    const int nk = (K + kDBK - 1) / kDBK;
    load(0);
    store(0);
    __syncthreads();
    int buf = 0;
    for (int kt = 0; kt < nk; kt++) {
        if (kt + 1 < nk) load((kt + 1) * kDBK);
#pragma unroll
        for (int kk = 0; kk < kDBK; kk += 4) {
            const int kr = kk + l / 16;
            double a[MT], b[NT];
#pragma unroll
            for (int i = 0; i < MT; i++) a[i] = As[buf][kr][wr + 16 * i + (l % 16)];
#pragma unroll
            for (int j = 0; j < NT; j++) b[j] = Bs[buf][kr][wc + 16 * j + (l % 16)];
#pragma unroll
            for (int i = 0; i < MT; i++)
#pragma unroll
                for (int j = 0; j < NT; j++) acc[i][j] = __builtin_amdgcn_mfma_f64_16x16x4f64(a[i], b[j], acc[i][j], 0, 0, 0);
        }
        if (kt + 1 < nk) store(buf ^ 1);
        __syncthreads();
        buf ^= 1;
    }
#pragma unroll
    for (int i = 0; i < MT; i++)
#pragma unroll
        for (int j = 0; j < NT; j++) {
            const int c = col0 + wc + 16 * j + (l % 16);
            if (c >= N) continue;
#pragma unroll
            for (int r = 0; r < 4; r++) {
                const int row = row0 + wr + 16 * i + l / 16 + 4 * r;
                if (row < M) Cb[(int64_t)row * p.ldc + c] = acc[i][j][r];
            }
        }
}

template <int BM, int BN>
static void launch_f64(const double *a, const double *b, double *c, const MatMulArgs &p, hipStream_t s) {
    bool vec = p.k % 2 == 0 && p.n % 2 == 0 && p.lda % 2 == 0 && p.ldb % 2 == 0 &&
               (((uintptr_t)a | (uintptr_t)b) % 16 == 0);
    for (int d = 0; d < p.nbatch; d++) vec = vec && p.a_bstr[d] % 2 == 0 && p.b_bstr[d] % 2 == 0;
    const dim3 g((p.n + BN - 1) / BN, (p.m + BM - 1) / BM, (unsigned)p.batch);
    if (vec) hipLaunchKernelGGL((k_matmul_f64<BM, BN, true>), g, dim3(256), 0, s, a, b, c, p);
    else hipLaunchKernelGGL((k_matmul_f64<BM, BN, false>), g, dim3(256), 0, s, a, b, c, p);
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
    int64_t ao, bo, co;
    batch_offsets(p.batch_base + blockIdx.z, p, &ao, &bo, &co);
    const int32_t *Ab = A + ao;
    const int32_t *Bb = B + bo;
    uint32_t acc = 0;
    for (int k0 = 0; k0 < K; k0 += 16) {
        As[ty][tx] = (row < M && k0 + tx < K) ? (uint32_t)Ab[(int64_t)row * p.lda + k0 + tx] : 0u;
        Bs[ty][tx] = (k0 + ty < K && col < N) ? (uint32_t)Bb[(int64_t)(k0 + ty) * p.ldb + col] : 0u;
        __syncthreads();
#pragma unroll
        for (int k = 0; k < 16; k++) acc += As[ty][k] * Bs[k][tx];
        __syncthreads();
    }
    if (row < M && col < N) C[co + (int64_t)row * p.ldc + col] = (int32_t)acc;
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

// VEC: 16-byte loads of A and B and 16-byte epilogue accesses of C, the residual and the bias
static bool f32_vec(const void *a, const void *b, const void *c, const MatMulArgs &p) {
    bool vec = (p.k % 4 == 0) && (p.n % 4 == 0) &&
               (((uintptr_t)a | (uintptr_t)b | (uintptr_t)c | (uintptr_t)p.res | (uintptr_t)p.bias) % 16 == 0) &&
               p.bias_bstr % 4 == 0 && p.lda % 4 == 0 && p.ldb % 4 == 0 && p.ldc % 4 == 0;
    for (int d = 0; d < p.nbatch; d++)
        vec = vec && (p.a_bstr[d] % 4 == 0) && (p.b_bstr[d] % 4 == 0) && (p.c_bstr[d] % 4 == 0);
    return vec;
}

// K ranges of a float product on the direct-load kernel's terms (16-byte operands, K a multiple of 64): with
// T tiles of 64x64 over the batch (ceil(m / 64) ceil(n / 64) per matrix), the most ranges, each a whole number
// of passes of 64, that divide K / 64 into equal parts and keep T times the ranges within 256 blocks (one per
// CU); 1 when T alone reaches 128 or K is a single pass.  A product of few tiles otherwise leaves
// most CUs idle while its blocks each walk the whole of K ([8,1536] x [1536,384]: 6 blocks).  With
// split_per_matrix, T counts one matrix's tiles (and a batch above kMatMulSplitBatch does not split), so
// that each matrix of a grouped launch splits as it does alone.
static int f32_split(const MatMulArgs &p, bool vec) {
    if (!vec || p.k % 64 != 0) return 1;
    const int64_t per = (((int64_t)p.m + 63) / 64) * (((int64_t)p.n + 63) / 64);
    if (p.split_per_matrix && p.batch > kMatMulSplitBatch) return 1;
    const int64_t tiles = p.split_per_matrix ? per : per * p.batch;
    if (tiles >= 128) return 1;
    const int steps = p.k / 64;
    int best = 1;
    for (int r = 2; r <= steps; r++)
        if (steps % r == 0 && tiles * r <= 256) best = r;
    return best;
}

bool matmul_ln_fusable(int dtype, const void *a, const void *b, const void *c, const MatMulArgs &p) {
    return dtype == kFloat && !p.gelu && !p.bt && p.n % 4 == 0 && p.n >= 256 && p.n <= 4096 &&
           matmul_part_bytes(dtype, a, b, c, p) > 0;
}

hipError_t launch_matmul_ln(const void *a, const void *b, void *y, const MatMulArgs &p0, const float *gamma,
                            const float *beta, float eps, hipStream_t s) {
    if (!matmul_ln_fusable(kFloat, a, b, y, p0) || !p0.part) return hipErrorInvalidValue;
    MatMulArgs p = p0;
    p.split = f32_split(p, f32_vec(a, b, y, p));
    const dim3 g((p.n + 63) / 64, (p.m + 63) / 64, (unsigned)(p.batch * p.split));
    hipLaunchKernelGGL((k_matmul_f32_dl<64, 64, 2, 2, 4, 3, 8, false, true>), g, dim3(256), 0, s, (const float *)a,
                       (const float *)b, (float *)y, p);
    const dim3 gr((unsigned)(p.batch * p.m));
    float *fy = (float *)y;
    switch ((p.n + 255) / 256) {
#define LX_MM_LN_CASE(NV) \
    case NV: hipLaunchKernelGGL(k_matmul_split_sum_ln<NV>, gr, dim3(64), 0, s, gamma, beta, eps, fy, p); break;
        LX_MM_LN_CASE(1) LX_MM_LN_CASE(2) LX_MM_LN_CASE(3) LX_MM_LN_CASE(4) LX_MM_LN_CASE(5) LX_MM_LN_CASE(6)
        LX_MM_LN_CASE(7) LX_MM_LN_CASE(8) LX_MM_LN_CASE(9) LX_MM_LN_CASE(10) LX_MM_LN_CASE(11) LX_MM_LN_CASE(12)
        LX_MM_LN_CASE(13) LX_MM_LN_CASE(14) LX_MM_LN_CASE(15) LX_MM_LN_CASE(16)
#undef LX_MM_LN_CASE
    default: return hipErrorInvalidValue;
    }
    return hipGetLastError();
}

int64_t matmul_part_bytes(int dtype, const void *a, const void *b, const void *c, const MatMulArgs &p) {
    if (dtype != kFloat || p.m == 0 || p.n == 0 || p.batch == 0) return 0;
    const int r = f32_split(p, f32_vec(a, b, c, p));
    return r > 1 ? (int64_t)r * p.batch * p.m * p.n * (int64_t)sizeof(float) : 0;
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
        const bool vec = f32_vec(a, b, c, p);
        const float *fa = (const float *)a, *fb = (const float *)b;
        float *fc = (float *)c;
        const int split = f32_split(p, vec);
        if (split > 1) {
            if (!p.part || p.bt) return hipErrorInvalidValue;  // the caller sizes it with matmul_part_bytes
            MatMulArgs q = p;
            q.split = split;
            launch_f32_split(fa, fb, fc, q, s);
            return hipGetLastError();
        }
        // block tile: among the tiles that give each of the 256 CUs two or more blocks (a lone block
        // per CU leaves its barrier and load latencies unhidden: measured 93 against 104 TF/s for
        // [4096,3072]x[3072,768]), the one whose busiest CU has the least work -- ceil(blocks / 256)
        // blocks, each costing its area over the tile's relative efficiency; 64x64 when none does
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
        // The direct-load kernel (K a multiple of 64, 16-byte aligned operands) for every shape but short K
        // (attention scores, K = 64: the register-staged kernel 81 against 78 TFLOP/s); both kernels sum in one
        // order, so the choice never changes a result.  Tile: the least cost, where a tile config that holds r
        // blocks per CU at once (its LDS and its occupancy hint) runs ceil(tiles / (256 r)) rounds, each as long
        // as min(r, tiles per CU) of its tiles, each costing its area over a measured efficiency.  128x128 runs
        // with at most two waves per SIMD (accumulators in AGPRs: 135 TFLOP/s at 4096^3 against 104 with them in
        // VGPRs for three waves), 128x96 with one or two, the smaller tiles with three or more.  One 128x96 tile
        // per CU over a long K (at least 2048) keeps that tile: its lone wave per SIMD runs the longest
        // uninterrupted MFMA stream ([4096,3072]x[3072,768]: 133 against 126 TFLOP/s for 64x64).
        // N of at most 32 (the attention context of 32-wide heads): 128x32 tiles, four waves of 32x32
        // ([8,12,512,512]x[8,12,512,32]: 65 against 43 TFLOP/s for the register-staged kernel's 64x64)
        // (B by columns, p.bt: the register-staged kernel only, never split -- the host checks)
        if (!p.bt && vec && p.k % 64 == 0 && p.k > 64 && p.n <= 32 && p.m >= 64) {
            launch_f32_dl<128, 32, 4, 1, 1, 2>(fa, fb, fc, p, s);
            return hipGetLastError();
        }
        if (!p.bt && vec && p.k % 64 == 0 && p.k > 64 && p.n >= 64 && p.m >= 64) {
            struct DTile {
                int bm, bn, resident;
                double eff;
            };
            static const DTile dcand[] = {{128, 128, 2, 1.0}, {128, 96, 2, 0.9}, {64, 64, 4, 0.97}, {128, 64, 3, 0.95}};
            auto tiles_of = [&](const DTile &c) {
                return (int64_t)((p.m + c.bm - 1) / c.bm) * ((p.n + c.bn - 1) / c.bn) * p.batch;
            };
            int dt = 0;
            double bc = 0;
            for (int i = 0; i < 4; i++) {
                const int64_t tiles = tiles_of(dcand[i]);
                const int64_t rounds = (tiles + 256 * dcand[i].resident - 1) / (256 * dcand[i].resident);
                const int64_t per_cu = std::min<int64_t>(dcand[i].resident, (tiles + 255) / 256);
                const double cost = (double)(rounds * per_cu) * dcand[i].bm * dcand[i].bn / dcand[i].eff;
                if (i == 0 || cost < bc) {
                    dt = i;
                    bc = cost;
                }
            }
            const int64_t t96 = tiles_of(dcand[1]);
            if (t96 > 192 && t96 <= 256 && p.k >= 2048) dt = 1;
            switch (dt) {
            case 0: launch_f32_dl<128, 128, 2, 2, 1, 2>(fa, fb, fc, p, s); break;
            case 1: launch_f32_dl<128, 96, 4, 1, 1, 2>(fa, fb, fc, p, s); break;
            case 2: launch_f32_dl<64, 64, 2, 2, 3, 8>(fa, fb, fc, p, s); break;
            default: launch_f32_dl<128, 64, 2, 2, 3, 8>(fa, fb, fc, p, s); break;
            }
            return hipGetLastError();
        }
        switch (best) {
        case 0: launch_f32<128, 128, 2, 2>(fa, fb, fc, p, vec, s); break;
        case 1: launch_f32<128, 96, 4, 1>(fa, fb, fc, p, vec, s); break;
        case 2: launch_f32<96, 128, 1, 4>(fa, fb, fc, p, vec, s); break;
        case 3: launch_f32<128, 64, 2, 2>(fa, fb, fc, p, vec, s); break;
        case 4: launch_f32<64, 128, 2, 2>(fa, fb, fc, p, vec, s); break;
        default: launch_f32<64, 64, 2, 2>(fa, fb, fc, p, vec, s); break;
        }
    } else if (dtype == kDouble) {
        // the largest of 128x128, 64x64 and 32x32 tiles that gives every CU a block
        const double *da = (const double *)a, *db = (const double *)b;
        double *dc = (double *)c;
        auto tiles = [&](int t) { return (((int64_t)p.m + t - 1) / t) * (((int64_t)p.n + t - 1) / t) * p.batch; };
        if (tiles(128) >= 256) launch_f64<128, 128>(da, db, dc, p, s);
        else if (tiles(64) >= 256) launch_f64<64, 64>(da, db, dc, p, s);
        else launch_f64<32, 32>(da, db, dc, p, s);
    } else if (dtype == kInt32) {
        dim3 g((p.n + 15) / 16, (p.m + 15) / 16, (unsigned)p.batch);
        hipLaunchKernelGGL(k_matmul_i32, g, dim3(256), 0, s, (const int32_t *)a, (const int32_t *)b, (int32_t *)c, p);
    } else {
        return hipErrorInvalidValue;
    }
    return hipGetLastError();
}

}  // namespace lx
