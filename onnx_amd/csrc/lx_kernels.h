// lx_kernels.h -- internal launch interface between the host layer (lx_api.cpp)
// and the gfx950 kernels (lx_elementwise.hip, lx_reduce.hip, lx_softmax.hip).
// Not part of the public C ABI.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "lx_plan.h"

namespace lx {

// TensorElementType codes (Tensor.cs:31-50)
enum DType : int {
    kFloat = 1, kUInt8 = 2, kInt8 = 3, kUInt16 = 4, kInt16 = 5, kInt32 = 6, kInt64 = 7,
    kBool = 9, kDouble = 11, kUInt32 = 12, kUInt64 = 13
};

enum BinOp : int { kAdd = 0, kSub = 1, kMul = 2, kDiv = 3, kPow = 4 };
enum UnOp : int { kSqrt = 0, kErf = 1, kNeg = 2, kExp = 3, kSquare = 4 };
enum RedOp : int { kSum = 0, kMean = 1, kMax = 2 };

// Binary layouts chosen by the planner.
enum BinLayout : int {
    kSame = 0,      // a[i] op b[i]
    kScalarA = 1,   // a[0] op b[i]
    kScalarB = 2,   // a[i] op b[0]
    kNd = 3         // NdLayout with inner strides given by a_inner / b_inner
};

// Device-side error record: first element index that raised each exception
// (UINT64_MAX = none).  Lives in device memory owned by the host layer.
struct ErrFlags {
    unsigned long long first_dbz;   // DivideByZeroException
    unsigned long long first_ovf;   // OverflowException
};

struct BinArgs {
    int op, dtype, layout;
    int a_inner, b_inner;   // kNd: 1 = contiguous innermost axis, 0 = broadcast
    int a_once, b_once;     // kNd: operand has no broadcast axis (read once: streamed)
    int vec;                // 1 = scalar element access, else 16-byte vectors
    int rag;                // kNd, inner axis not a multiple of the vector width, every pointer 16-byte
                            // aligned, fewer than 2^31 elements: output by 16-byte vectors of the flat index
    const void *a;
    const void *b;
    void *y;
    int64_t n;              // output elements
    NdLayout nd;            // kNd only
    int64_t nd_osize[kMaxOuter];  // outer sizes as int64 (large-index path)
    int64_t nd_inner_vn;          // inner axis in vector units (large-index path)
};

hipError_t launch_reset_errs(ErrFlags *e, hipStream_t s);
// Copies n 64-bit words from device memory into mapped host memory, then writes seq to *seq_dst
// after a system-scope release: the host waits for the sequence number instead of the stream.
// reset: null, or src itself, whose words are then set to all ones once copied.
hipError_t launch_publish(const uint64_t *src, int64_t n, uint64_t *dst, uint64_t *seq_dst, uint64_t seq,
                          uint64_t *reset, hipStream_t s);
// Eager integer Div: scans the divisor b (n elements of dtype, 16-byte vectors when vec) for 0 and, for
// signed types, -1; block i stores (seq << 2) | bits (bit 0: a zero, bit 1: a minus one) into slots[i] of
// mapped host memory (kScanSlots of them).  div_scan_blocks gives the number of blocks (slots) a launch uses.
constexpr int kScanSlots = 256;
int div_scan_blocks(int64_t n, int esize);
hipError_t launch_div_scan(int dtype, const void *b, int64_t n, int vec, uint64_t *slots, uint64_t seq,
                           hipStream_t s);
// Eager Gather: scans n indices (Int32 / Int64) for a value outside [-dim, dim); block i stores
// (seq << 2) | bit into slots[i] (bit 0: an index out of range); index_scan_blocks gives the blocks used.
int index_scan_blocks(int64_t n);
hipError_t launch_index_scan(int idx_dtype, const void *idx, int64_t n, int64_t dim, uint64_t *slots, uint64_t seq,
                             hipStream_t s);
hipError_t launch_binary(const BinArgs &args, ErrFlags *errs, hipStream_t s);
hipError_t launch_unary(int op, int dtype, const void *x, void *y, int64_t n, int vec, hipStream_t s);
hipError_t launch_cast(int src, int dst, const void *x, void *y, int64_t n, int vec, ErrFlags *errs,
                       hipStream_t s);
hipError_t launch_gelu_erf(const float *x, float *y, int64_t n, int vec, hipStream_t s);
// Reads `bytes` (16-byte vectors) with nontemporal loads, one word per block into out (at most max_blocks).
hipError_t launch_read_probe(const void *src, int64_t bytes, uint32_t *out, int64_t max_blocks, hipStream_t s);

// Elementwise chain (float32): acc = in[0], then per instruction k
//   binary op[k] in BinOp:   acc = acc op in[j]   (operand[k] = j >= 0)
//                            acc = in[j] op acc   (operand[k] = -(j + 1))
//   unary  op[k] = kChainUnary + UnOp (Sqrt, Erf): acc = op(acc)
// each op rounded as the separate operator rounds it.  Output row-major
// [rows, inner]; input j is addressed by its per-axis strides str[j][d] over
// the outer axes and, along the inner axis, contiguously (bit j of inner_mode)
// or broadcast.
constexpr int kChainMaxIn = 8, kChainMaxOps = 16, kChainUnary = 16;
struct ChainArgs {
    int32_t n_in, n_ops;
    int32_t inner_mode;
    int32_t uses_erf;
    int32_t vec;             // 4 = 16-byte vectors, 1 = scalars
    int32_t nouter;
    uint32_t nv;             // output vectors
    uint32_t pad;
    FastDiv odiv[kMaxOuter]; // outer axis sizes, innermost first
    FastDiv inner_v;         // inner axis in vector units
    int64_t str[kChainMaxIn][kMaxOuter];
    const float *in[kChainMaxIn];
    float *y;
    int8_t op[kChainMaxOps];
    int8_t operand[kChainMaxOps];
};
hipError_t launch_chain(const ChainArgs &args, hipStream_t s);
// y[i] = value (bit pattern of one element of esize bytes), used for empty reductions.
hipError_t launch_fill(void *y, int64_t n, int esize, uint64_t bits, hipStream_t s);

// Reduction of x viewed as [outer, r, inner] (row-major) into y[outer, inner].
//   pre_div : divide every element by R_total before accumulating (ReduceMean int/double)
//   post_div: divide the result by (float)R_total (ReduceMean float)
// workspace: device scratch of ws_bytes (partials of split reductions).
struct ReduceArgs {
    int op, dtype;
    const void *x;
    void *y;
    int64_t outer, r, inner;
    int pre_div, post_div;
    int64_t r_total;
    int vec;
    void *workspace;
    int64_t ws_bytes;
};
hipError_t launch_reduce(const ReduceArgs &args, hipStream_t s);
// Bytes of workspace launch_reduce needs for these sizes and vector width
// (vec = 1 or the 16-byte element count, as in ReduceArgs::vec).
// The most partial bytes a reduction pass's plan uses (column splits are capped to it; split rows need
// far less): the size of the allocation-free entry point's partials.
constexpr int64_t kReducePartialBytes = 2 << 20;
int64_t reduce_workspace_bytes(int dtype, int64_t outer, int64_t r, int64_t inner, int vec);

// Softmax of x viewed as [outer, r, inner] along r, with an optional additive
// mask (already planned against x as an NdLayout over [outer*inner rows, r]).
struct SoftmaxArgs {
    int dtype;
    const void *x;
    void *y;
    int64_t outer, r, inner;
    int vec;
    const void *mask;        // nullptr = no mask (only for inner == 1)
    int mask_inner;          // 1 = mask contiguous along r, 0 = broadcast along r
    NdLayout mask_rows;      // row -> mask offset (nouter axes over the rows)
    const void *scale;       // nullptr, or one element: x / scale (scale_div) or x * scale, before the mask
    int scale_div;
};
hipError_t launch_softmax(const SoftmaxArgs &args, hipStream_t s);
bool softmax_mask_fusable(int dtype, int64_t r, int64_t inner, int64_t outer, int vec);

// Attention heads of at most kAttentionMax rows, keys and columns (Float): per batch, the scores Q K (Q [s, d],
// K as the product's right operand [d, sk]), their Softmax along the keys with SoftmaxArgs' scale and mask, and
// the context P V (V [sk, dv]) into y, in one launch -- bit for bit the two MatMul launches and the Softmax
// launch it replaces (the same MFMA sequence per output as the 64x64 register-staged MatMul kernel, the same
// lanes per row and reduction order as the grouped Softmax kernel).  Element (i, j) of an operand is at
// i * rs + j * cs past its batch's offset; batches decompose row-major over bdims.
constexpr int kAttentionMax = 64;
struct AttentionArgs {
    const float *q, *k, *v;
    float *y;
    int32_t s, sk, d, dv;
    int32_t nbatch;
    int64_t batch;
    int64_t bdims[kMaxOuter], q_bstr[kMaxOuter], k_bstr[kMaxOuter], v_bstr[kMaxOuter], y_bstr[kMaxOuter];
    int64_t q_rs, q_cs, k_rs, k_cs, v_rs, v_cs, y_rs, y_cs;
    // the Softmax between the products, on the scores as a dense [batch * s, sk] tensor
    const float *mask;
    int32_t mask_inner;
    NdLayout mask_rows;
    const float *scale;
    int32_t scale_div;
};
hipError_t launch_attention(const AttentionArgs &a, hipStream_t s);

// LayerNorm decomposed into its ONNX nodes, rows of length r (1 <= r <= 4099; x, gamma, beta, y 16-byte
// aligned).
hipError_t launch_layernorm(const float *x, const float *gamma, const float *beta, float eps, float *y,
                            int64_t rows, int64_t r, hipStream_t s);
bool layernorm_supported(int64_t r);

// MatMul C[batch][m][n] = A[batch][m][k] * B[batch][k][n], matrices with unit column stride and row strides
// lda / ldb / ldc; batch index decomposed over bdims (outermost first) with per-operand element strides
// (0 on broadcast axes for A and B).
struct MatMulArgs {
    int32_t m, n, k;
    int32_t nbatch;
    int64_t batch;       // batches in this launch (grid z)
    int64_t batch_base;  // index of the launch's first batch
    int64_t bdims[kMaxOuter];
    int64_t a_bstr[kMaxOuter];
    int64_t b_bstr[kMaxOuter];
    int64_t c_bstr[kMaxOuter];
    // row strides (elements) of A, B and C; k, n and n for dense matrices.  C other than dense (a transposed
    // output) only without the epilogue below
    int64_t lda, ldb, ldc;
    // 1: B stored by columns, element (k, n) at n * ldb + k (Float, no epilogue, never split)
    int32_t bt;
    // optional epilogue (Float only): C = (A B + bias[batch * bias_bstr + col]) + res[same index], each
    // add rounded as the separate Add node rounds it
    const float *bias;
    const float *res;
    int64_t bias_bstr;  // 0: one bias row for every batch; n: a bias row per batch (linear batch index)
    // then, when gelu != 0, the ONNX GELU subgraph Div(., sqrt 2) -> Erf -> Add 1 -> Mul . -> Mul 0.5 on
    // each result, every node rounded as it rounds (Float)
    int32_t gelu;
    // Float products with few output tiles split K into equal ranges: each range's partial product goes to
    // part ([split][batch][m][n] floats, matmul_part_bytes of them, supplied by the caller), then a second
    // kernel sums the partials in range order and applies the epilogue.  split is set by launch_matmul.
    int32_t split;
    // 1: the split counts the tiles of one matrix, not of the whole batch, so that each matrix of the launch
    // splits as it would alone (grouped projections, at most kMatMulSplitBatch of them; larger batches then
    // do not split)
    int32_t split_per_matrix;
    float *part;
};
// Bytes of partial products launch_matmul needs in MatMulArgs::part for these operands (0: no split).
constexpr int64_t kMatMulSplitBatch = 16;
int64_t matmul_part_bytes(int dtype, const void *a, const void *b, const void *c, const MatMulArgs &p);
hipError_t launch_matmul(int dtype, const void *a, const void *b, void *c, const MatMulArgs &p, hipStream_t s);
// A split Float product (its epilogue included, no GELU) whose rows of n (a multiple of 4, 256 to 4096) are then
// normalised by the decomposed LayerNorm (gamma and beta rows of n): launch_matmul_ln writes the normalised rows
// into y, bit for bit launch_matmul followed by launch_layernorm on its result, in two launches.
bool matmul_ln_fusable(int dtype, const void *a, const void *b, const void *c, const MatMulArgs &p);
hipError_t launch_matmul_ln(const void *a, const void *b, void *y, const MatMulArgs &p, const float *gamma,
                            const float *beta, float eps, hipStream_t s);

// Data movement (Transpose, Slice, Concat, expand): for every index j of `dims`
//   dst[dst_base + sum_k j_k dst_str[k]] = src[src_base + sum_k j_k src_str[k]]
// (element strides, any sign, 0 on broadcast axes; at most 8 axes, outermost first).
struct ViewCopyArgs {
    int32_t rank;
    int32_t pad;
    int64_t dims[8];
    int64_t src_str[8];
    int64_t dst_str[8];
    int64_t src_base;
    int64_t dst_base;
};
hipError_t launch_view_copy(int esize, const void *src, void *dst, const ViewCopyArgs &a, hipStream_t s);

// Concat of n inputs into a [outer, total] output: input i is a contiguous
// [outer, len] block placed at column off (elements).  Each input's
// outer * len must stay below 2^31 vectors.
constexpr int kConcatMax = 8;
struct ConcatPart {
    const void *src;
    int64_t len;
    int64_t off;
};
hipError_t launch_concat(int esize, void *dst, int64_t outer, int64_t total, const ConcatPart *parts, int n,
                         hipStream_t s);

// Gather: out[o][i][r] = data[o][idx[i] (+dim if negative)][r]; an index outside
// [-dim, dim) records its output position in errs->first_ovf and writes nothing.
// The output must hold fewer than 2^31 vectors.
hipError_t launch_gather(int esize, int idx_dtype, const void *data, const void *idx, void *out, int64_t outer,
                         int64_t nidx, int64_t inner, int64_t dim, ErrFlags *errs, hipStream_t s);

// y[i] = x[offset(i)] for a strided view (strides in elements, 0 on broadcast axes)
hipError_t launch_strided_copy(int esize, const void *x, void *y, int rank, const int64_t *dims, const int64_t *strides,
                               hipStream_t s);

}  // namespace lx
