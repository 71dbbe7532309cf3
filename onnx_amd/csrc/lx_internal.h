// lx_internal.h -- library-internal interface between the C ABI (lx_api.cpp)
// and the graph runtime (lx_graph.cpp, lx_onnx.cpp).
#pragma once

#include <hip/hip_runtime.h>

#include <chrono>
#include <string>

#include "../../include/lonnx.h"

namespace lx {

int api_set_error(int code, const std::string &message);  // sets lx_last_error, returns code

// One operator call for lx_set_op_profiling: constructed at the top of an exported operator, it records
// the call when profiling is on and the call is not nested in another operator or a graph execution (the
// graph entry points hold an OpScope(nullptr), which records nothing and marks what runs inside as nested).
class OpScope {
  public:
    explicit OpScope(const char *op);
    ~OpScope();
    OpScope(const OpScope &) = delete;
    OpScope &operator=(const OpScope &) = delete;

  private:
    bool active_ = false;
    const char *op_ = nullptr;
    hipEvent_t e0_ = nullptr;
    std::chrono::steady_clock::time_point h0_;
};
bool api_initialized();
hipStream_t api_stream();
int64_t api_esize(int dtype);
const char *api_dtype_name(int dtype);

// Deferred device checks (graph executor).  Integer Div, narrowing Cast and Gather check values on
// the device; called alone they read the verdict back at once (one synchronisation).  While a slot
// is set, they record into it instead -- the slot and the kind of check -- and return without
// waiting; the caller reads many slots back in one copy later and turns them into the same status
// and message with api_check_status.
enum CheckKind { kCheckNone = 0, kCheckGather = 1, kCheckDiv = 2, kCheckCast = 3 };
struct DeferredCheck {
    int kind = kCheckNone;
    int dst = 0;  // Cast: the target element type
};
struct ErrFlags;
void api_defer_checks(ErrFlags *slot, DeferredCheck *rec);
// Reads `bytes` (a multiple of 8) of device memory into host memory after the work queued on the
// library stream: the caller returns as soon as the device has written them (no stream-sync wake-up).
int api_read_device(const void *src, size_t bytes, void *dst);
int api_check_status(const DeferredCheck &rec, const ErrFlags &flags);  // sets lx_last_error on failure

// Whether gamma / beta of a decomposed LayerNorm are [1, ..., 1, r] against X (r = X's last dimension,
// rank at most X's): the shapes for which the fused kernel's last-axis affine step equals the Mul / Add
// nodes' broadcast.
bool api_layernorm_affine_fits(const lx_tensor *t, const lx_tensor *X);

// lx_MatMulAdd of one left operand [1, M, K] against G stacked weights [G, K, N] and biases [G, 1, N] (the
// graph's grouped projections): each of the G products splits its K exactly as a product of its own, so each
// slice is bit-identical to that product.  LX_ERR_NOT_SUPPORTED (no message) for G above 16.
int api_matmul_add_grouped(const lx_tensor *A, const lx_tensor *W, const lx_tensor *bias, lx_tensor *Y);

// lx_MatMulAdd (bias, optional residual) then lx_LayerNormDecomposed on its result into Y (empty): when the
// product splits K and every step fits, the split product's ordered sum applies the Adds and the LayerNorm in one
// launch (the product never written), bit for bit the two calls; otherwise the two calls.
int api_matmul_add_layernorm(const lx_tensor *A, const lx_tensor *W, const lx_tensor *bias, const lx_tensor *residual,
                             const lx_tensor *gamma, const lx_tensor *beta, float eps, lx_tensor *Y);

// MatMul of transpose(A, a_perm) and transpose(B, b_perm) (null: the tensor itself), its product stored as
// transpose(product, y_perm) into Y (null: as it is), Float, each permutation keeping the last axis last: the
// kernels read and write the transposed views through their strides, and the result is bit for bit the
// Transpose nodes' and MatMul's.  LX_ERR_NOT_SUPPORTED (no message) for operands it does not take.
int api_matmul_permuted(const lx_tensor *A, const int *a_perm, const lx_tensor *B, const int *b_perm,
                        const int *y_perm, lx_tensor *Y);
// An attention head's scores transpose(Q, q_perm) x transpose(K, k_perm), their Softmax along the last axis
// after the optional scale (x / scale when scale_div, else x * scale) and the additive mask, and the context
// probabilities x transpose(V, v_perm) stored as transpose(context, y_perm) into Y: one launch, bit for bit
// the MatMulPermuted, ScaleAddSoftmax (AddSoftmax without a scale) and MatMulPermuted nodes it replaces.
// Float, equal batch axes, and rows, keys and head widths of at most kAttentionMax; LX_ERR_NOT_SUPPORTED (no
// message) otherwise.
int api_attention(const lx_tensor *Q, const int *q_perm, const lx_tensor *K, const int *k_perm,
                  const lx_tensor *scale, int scale_div, const lx_tensor *mask, int32_t axis, const lx_tensor *V,
                  const int *v_perm, const int *y_perm, lx_tensor *Y);

}  // namespace lx
