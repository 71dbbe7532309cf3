/*
 * lonnx.h -- C ABI of the MI355X (gfx950) device path for the Lokad.Onnx
 * elementwise / broadcast / reduction operators.
 *
 * The ABI is plain C (cdecl, POD structs, no C++ or torch types) so that the
 * unchanged C# operator layer can bind it with [DllImport] exactly as it binds
 * any native library; a Python ctypes binding of the same symbols is what the
 * tests use.  Every operator entry point mirrors one static method of
 * CPUExecutionProvider (src/Lokad.Onnx.Backend/CPUExecutionProvider.cs) with
 * the same argument meaning; the status codes mirror the OpResult factories
 * (src/Lokad.Onnx.Backend/OpResult.cs:34-60) and the exceptions that
 * Node.Execute converts into OpResult.Failure (Node.cs:107-118).
 *
 * Threading: one device per process, one stream at a time (lx_set_stream).
 * Calls are stream ordered; lx_tensor_download synchronises.  The library is
 * not re-entrant across host threads.
 */
#ifndef LONNX_H
#define LONNX_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define LX_MAX_RANK 8

/* Element type codes: TensorElementType (src/Lokad.Onnx.Tensors/Tensor.cs:31-50). */
enum lx_dtype {
    LX_FLOAT = 1, LX_UINT8 = 2, LX_INT8 = 3, LX_UINT16 = 4, LX_INT16 = 5,
    LX_INT32 = 6, LX_INT64 = 7, LX_BOOL = 9, LX_DOUBLE = 11, LX_UINT32 = 12,
    LX_UINT64 = 13
};

/* Status codes returned by every entry point (0 = success). */
enum lx_status {
    LX_OK = 0,
    LX_ERR_MISSING_INPUT = 1,            /* OpResult.MissingInput            (OpResult.cs:46) */
    LX_ERR_WRONG_INPUT_TYPE = 2,         /* OpResult.WrongInputType          (OpResult.cs:50-52) */
    LX_ERR_CANNOT_BROADCAST = 3,         /* OpResult.CannotBroadcast         (OpResult.cs:60) */
    LX_ERR_INPUT_TYPE_NOT_SUPPORTED = 4, /* OpResult.InputTypeNotSupported   (OpResult.cs:40) */
    LX_ERR_NOT_SUPPORTED = 5,            /* OpResult.NotSupported            (OpResult.cs:38) */
    LX_ERR_ATTRIBUTE_NOT_SUPPORTED = 6,  /* OpResult.AttributeNotSupported   (OpResult.cs:42) */
    LX_ERR_WRONG_INPUT_SHAPE = 7,        /* OpResult.WrongInputShape         (OpResult.cs:54-58) */
    LX_ERR_INVALID_ARGUMENT = 8,         /* ArgumentException  -> OpResult.Failure (Node.cs:115-118) */
    LX_ERR_DIVIDE_BY_ZERO = 9,           /* DivideByZeroException -> OpResult.Failure */
    LX_ERR_OVERFLOW = 10,                /* OverflowException -> OpResult.Failure */
    LX_ERR_OUT_OF_MEMORY = 11,           /* hipMalloc failure (device path only) */
    LX_ERR_HIP = 12,                     /* any other HIP runtime error (device path only) */
    LX_ERR_NOT_INITIALIZED = 13,         /* lx_init not called (device path only) */
    LX_ERR_BUFFER_TOO_SMALL = 14         /* caller-provided output storage too small */
};

/*
 * Device tensor handle: the device twin of DenseTensor<T>
 * (src/Lokad.Onnx.Tensors/DenseTensor.cs:31-278): row-major contiguous
 * storage, int64 dims, explicit host/device residency.
 *   data     : device address (from the library's pool by lx_tensor_alloc, or wrapped)
 *   capacity : bytes usable at data
 *   owns     : 1 if lx_tensor_free must release data (back to the pool)
 * Operator outputs: if Y->data is NULL the operator allocates Y (owns = 1);
 * otherwise it writes into Y->data (capacity checked, LX_ERR_BUFFER_TOO_SMALL)
 * and only updates dtype/rank/dims.  Inputs are never modified.
 */
typedef struct lx_tensor {
    int32_t dtype;
    int32_t rank;
    int64_t dims[LX_MAX_RANK];
    void *data;
    int64_t capacity;
    int32_t owns;
    int32_t reserved;
} lx_tensor;

/*
 * Broadcast plan (host only, no device call): ITensor.Broadcast shape rule
 * (src/Lokad.Onnx.Tensors/ITensor.cs:64-120) plus the stride-0 view of
 * BroadcastedTensor (BroadcastedTensor.cs:24-31), with size-1 axes dropped and
 * adjacent axes merged where both operands stay contiguous.
 */
enum lx_plan_kind {
    LX_PLAN_EMPTY = 0,    /* zero output elements */
    LX_PLAN_SAME = 1,     /* both operands dense over the whole output */
    LX_PLAN_SCALAR_A = 2, /* A is one value, B dense */
    LX_PLAN_SCALAR_B = 3, /* B is one value, A dense */
    LX_PLAN_ND = 4        /* general: per-axis strides, 0 on broadcast axes */
};

typedef struct lx_bcast_plan {
    int32_t status;                 /* LX_OK or LX_ERR_CANNOT_BROADCAST */
    int32_t out_rank;               /* rank of the broadcast result */
    int64_t out_dims[LX_MAX_RANK];  /* shape of the broadcast result */
    int32_t kind;                   /* lx_plan_kind */
    int32_t rank;                   /* collapsed rank (>= 1 unless EMPTY) */
    int64_t dims[LX_MAX_RANK];      /* collapsed dims, outermost first */
    int64_t a_strides[LX_MAX_RANK]; /* element strides of A per collapsed axis */
    int64_t b_strides[LX_MAX_RANK]; /* element strides of B per collapsed axis */
    int64_t numel;                  /* output element count */
} lx_bcast_plan;

/* ---- library lifecycle ------------------------------------------------- */
int lx_init(int32_t device);          /* select device, create the library stream and workspace */
int lx_shutdown(void);
const char *lx_last_error(void);      /* message of the last failure on this thread (OpResult.Message) */
const char *lx_version(void);
int lx_set_stream(void *hip_stream);  /* NULL = the library's own stream */
void *lx_get_stream(void);
int lx_synchronize(void);

/* ---- device tensors (residency) ---------------------------------------- */
int64_t lx_dtype_size(int32_t dtype);
int lx_tensor_alloc(int32_t dtype, int32_t rank, const int64_t *dims, lx_tensor *out);
int lx_tensor_wrap(int32_t dtype, int32_t rank, const int64_t *dims, void *device_ptr,
                   int64_t capacity, lx_tensor *out);
int lx_tensor_free(lx_tensor *t);
int lx_tensor_upload(lx_tensor *t, const void *host, int64_t nbytes);         /* host -> device, synchronous */
int lx_tensor_download(const lx_tensor *t, void *host, int64_t nbytes);       /* device -> host, synchronous */
/* Reshape / Unsqueeze alias: same storage, new dims (DenseTensor.cs:231-242). */
int lx_tensor_reshape(const lx_tensor *t, int32_t rank, const int64_t *dims, lx_tensor *out);

/* Device memory pool: released tensor storage is cached per size class and
 * reused by later allocations on the library stream (no reference counterpart:
 * the reference's storage is GC-managed managed arrays, DenseTensor.cs:34-35).
 * lx_pool_trim synchronises and returns every cached block to HIP. */
int lx_pool_trim(void);
int lx_pool_stats(int64_t *live_bytes, int64_t *cached_bytes);

/* ---- planner ------------------------------------------------------------ */
int lx_plan_broadcast(int32_t rank_a, const int64_t *dims_a, int32_t rank_b, const int64_t *dims_b,
                      lx_bcast_plan *plan);

/* ---- operators: CPUExecutionProvider twins ------------------------------ */
/* CPUExecutionProvider.Add (CPUExecutionProvider.cs:82-112).  dtypes: UInt8, Int32, Float, Double,
 * and Int64 (C# unchecked semantics; the reference returns InputTypeNotSupported for Int64). */
int lx_Add(const lx_tensor *A, const lx_tensor *B, lx_tensor *Y);
/* CPUExecutionProvider.Sub (CPUExecutionProvider.cs:114-143). */
int lx_Sub(const lx_tensor *A, const lx_tensor *B, lx_tensor *Y);
/* CPUExecutionProvider.Mul (CPUExecutionProvider.cs:145-175). */
int lx_Mul(const lx_tensor *A, const lx_tensor *B, lx_tensor *Y);
/* CPUExecutionProvider.Div (CPUExecutionProvider.cs:177-206).  UInt8, Float, Double, plus Int32 and
 * Int64 (truncating; x/0 -> LX_ERR_DIVIDE_BY_ZERO, MIN/-1 -> LX_ERR_OVERFLOW). */
int lx_Div(const lx_tensor *A, const lx_tensor *B, lx_tensor *Y);
/* CPUExecutionProvider.Pow (CPUExecutionProvider.cs:208-236).  Float, Double. */
int lx_Pow(const lx_tensor *A, const lx_tensor *B, lx_tensor *Y);
/* CPUExecutionProvider.Sqrt (CPUExecutionProvider.cs:380-396). */
int lx_Sqrt(const lx_tensor *A, lx_tensor *Y);
/* CPUExecutionProvider.Erf (CPUExecutionProvider.cs:398-409); MathOps.Erf (MathOps.cs:988-1034). */
int lx_Erf(const lx_tensor *X, lx_tensor *Y);
/* CPUExecutionProvider.Cast (CPUExecutionProvider.cs:451-476); ITensor.Cast (ITensor.cs:161-170). */
int lx_Cast(const lx_tensor *input, int64_t to, lx_tensor *Y);
/* CPUExecutionProvider.ReduceSum (CPUExecutionProvider.cs:623-640).
 * axes: n_axes < 0 means the axes input is absent; keepdims / noop: < 0 means attribute absent. */
int lx_ReduceSum(const lx_tensor *data, const int64_t *axes, int32_t n_axes, int32_t keepdims,
                 int32_t noop_with_empty_axes, lx_tensor *Y);
/* ReduceSum that allocates nothing (no counterpart in the reference): for callers that cannot call
 * hipMalloc -- code under HIP graph capture, tight serving loops, harnesses that forbid allocation.  Same
 * arguments, validation, results and errors as lx_ReduceSum, except that Y must already hold device storage
 * of sufficient capacity, and that split partials (at most 2 MiB: the planner caps every reduction's splits
 * there, so both entry points run the same plan) and the intermediate of each pass of a
 * multi-pass reduction (at most 1 MiB each) live in a 4 MiB static device array per GPU instead of the
 * library's workspace and pool; a reduction that needs more fails with LX_ERR_NOT_SUPPORTED before
 * anything is launched.  Calls on one GPU share that array: calls that overlap on one GPU (other
 * streams or threads) race. */
int lx_ReduceSum_noalloc(const lx_tensor *data, const int64_t *axes, int32_t n_axes, int32_t keepdims,
                         int32_t noop_with_empty_axes, lx_tensor *Y);
/* CPUExecutionProvider.ReduceMean (CPUExecutionProvider.cs:642-660). */
int lx_ReduceMean(const lx_tensor *data, const int64_t *axes, int32_t n_axes, int32_t keepdims,
                  int32_t noop_with_empty_axes, lx_tensor *Y);
/* CPUExecutionProvider.ReduceMax (CPUExecutionProvider.cs:662-678). */
int lx_ReduceMax(const lx_tensor *data, const int64_t *axes, int32_t n_axes, int32_t keepdims, lx_tensor *Y);
/* CPUExecutionProvider.Softmax (CPUExecutionProvider.cs:680-695); has_axis = 0 means default -1. */
int lx_Softmax(const lx_tensor *input, int32_t axis, int32_t has_axis, lx_tensor *Y);
/* CPUExecutionProvider.MatMul (CPUExecutionProvider.cs:359-378); Tensor<T>.MatMul (TensorOps.cs:504-806)
 * for Int32 (exact, wrapping), Float (fp32 MFMA) and Double (fp64 MFMA), with the reference's batch
 * broadcast and rank-1 rules. */
int lx_MatMul(const lx_tensor *A, const lx_tensor *B, lx_tensor *Y);
/* CPUExecutionProvider.Transpose (CPUExecutionProvider.cs:411-433); Tensor<T>.Transpose (TensorOps.cs:1358-1405).
 * n_perm < 0: perm absent (reversed axes).  Rank <= 1 returns the input itself (a view, owns = 0). */
int lx_Transpose(const lx_tensor *data, const int64_t *perm, int32_t n_perm, lx_tensor *Y);
/* CPUExecutionProvider.Concat (CPUExecutionProvider.cs:477-501); Tensor<T>.Concat (TensorOps.cs:1446-1498).
 * has_axis = 0: axis 0. */
int lx_Concat(const lx_tensor *const *inputs, int32_t n, int32_t axis, int32_t has_axis, lx_tensor *Y);
/* CPUExecutionProvider.Gather (CPUExecutionProvider.cs:516-546); Tensor<T>.Gather (TensorOps.cs:1407-1444).
 * indices: Int32 or Int64 device tensor; negative indices count from the end of the axis once; an
 * index still outside the axis fails like the reference's IndexOutOfRangeException. */
int lx_Gather(const lx_tensor *data, const lx_tensor *indices, int32_t axis, int32_t has_axis, lx_tensor *Y);
/* CPUExecutionProvider.Slice (CPUExecutionProvider.cs:548-600); Tensor<T>.Slice (TensorOps.cs:1500-1531) with
 * SliceIndex.ToSliceDef (SliceIndex.cs:271-324): starts / ends / axes / steps as host arrays (axes, steps may be
 * NULL).  Starts and ends are clamped to [0, dim] after negative wrap-around, as the reference does. */
int lx_Slice(const lx_tensor *data, const int64_t *starts, int32_t n_starts, const int64_t *ends, int32_t n_ends,
             const int64_t *axes, int32_t n_axes, const int64_t *steps, int32_t n_steps, lx_tensor *Y);

/* MatMul(A, B) -> Add(., bias) [-> Add(., residual)] (no single reference counterpart: the
 * CPUExecutionProvider.MatMul and .Add calls of a projection with bias and a residual connection,
 * CPUExecutionProvider.cs:82-113, 359-378).  Float, with bias a row vector of the product's last axis (or
 * one such row per batch, [batch..., 1, n] for a product [batch..., m, n]) and residual of the product's
 * shape: both Adds in the MatMul's epilogue, each rounded as the Add node rounds it; otherwise the MatMul
 * and the Adds run one after the other.  residual may be NULL. */
int lx_MatMulAdd(const lx_tensor *A, const lx_tensor *B, const lx_tensor *bias, const lx_tensor *residual,
                 lx_tensor *Y);
/* MatMul(A, B) -> Add(., bias) -> the ONNX GELU subgraph Div(., sqrt2) -> Erf -> Add 1 -> Mul . -> Mul 0.5
 * (a BERT FFN's first projection; the graph runtime's fusion of those seven nodes).  Float: the Add and
 * the GELU in the MatMul's epilogue, every node rounded as it rounds (bias as for lx_MatMulAdd); otherwise
 * lx_MatMulAdd's path followed by lx_GeluErf. */
int lx_MatMulAddGelu(const lx_tensor *A, const lx_tensor *B, const lx_tensor *bias, lx_tensor *Y);

/* ---- fused subgraphs (one kernel each; every intermediate keeps the float32
 * rounding of the separate ONNX node it replaces) ------------------------- */
/* Div(X, sqrt2) -> Erf -> Add 1 -> Mul X -> Mul 0.5 (the ONNX GELU subgraph;
 * each node runs through CPUExecutionProvider.Div/Erf/Add/Mul in the reference). */
int lx_GeluErf(const lx_tensor *X, lx_tensor *Y);
/* ReduceMean(-1) -> Sub -> Pow 2 -> ReduceMean(-1) -> Add eps -> Sqrt -> Div -> Mul gamma -> Add beta. */
int lx_LayerNormDecomposed(const lx_tensor *X, const lx_tensor *gamma, const lx_tensor *beta, float eps,
                           lx_tensor *Y);
/* Add(S, mask) -> Softmax(axis) with the mask broadcast against S. */
int lx_AddSoftmax(const lx_tensor *S, const lx_tensor *mask, int32_t axis, lx_tensor *Y);
/* Div(S, scale) (divide != 0) or Mul(S, scale) -> [Add(., mask) when mask != NULL] -> Softmax(axis): the
 * scaled attention scores of BERT-class models.  scale is a one-element tensor. */
int lx_ScaleAddSoftmax(const lx_tensor *S, const lx_tensor *scale, int32_t divide, const lx_tensor *mask, int32_t axis,
                       lx_tensor *Y);
/* A linear chain of Float elementwise nodes in one pass (no single reference counterpart: it replaces
 * consecutive CPUExecutionProvider.Add/Sub/Mul/Div/Pow/Sqrt/Erf calls, CPUExecutionProvider.cs:82-236,
 * 380-409, whose intermediates have no other consumer).  acc = inputs[0]; instruction k applies ops[k]:
 *   LX_CHAIN_ADD..LX_CHAIN_POW (0..4): acc = acc op inputs[j] for operands[k] = j >= 0,
 *                                        acc = inputs[j] op acc for operands[k] = -(j + 1);
 *   LX_CHAIN_SQRT (16), LX_CHAIN_ERF (17): acc = op(acc), operands[k] ignored.
 * Each step broadcasts like the separate operator and rounds as it does, so the result is bit-identical
 * to running the nodes one by one.  1..8 inputs, 1..16 instructions, Float only. */
enum { LX_CHAIN_ADD = 0, LX_CHAIN_SUB = 1, LX_CHAIN_MUL = 2, LX_CHAIN_DIV = 3, LX_CHAIN_POW = 4,
       LX_CHAIN_SQRT = 16, LX_CHAIN_ERF = 17 };
int lx_ElementwiseChain(const lx_tensor *const *inputs, int32_t n_in, const int32_t *ops, const int32_t *operands,
                        int32_t n_ops, lx_tensor *Y);

/* ---- operator profiling: the OpStage.Math stage of eager calls ------------------
 * The reference's operators open profiler stages as they go (Profiler.StartOpStage, Profiler.cs:71-80;
 * CPUExecutionProvider.cs:92-103) and its stopwatch closes the last one, Math, when Node.Execute returns
 * (ComputationalGraph.cs:241-243).  On the device a call returns after queueing its kernels, so a host
 * clock would time the launch; these records time the device work instead.  While enabled, every
 * operator call from outside the library (lx_Add ... lx_Slice and the fused operators; not the calls a
 * graph execution makes, which lx_graph_set_profiling covers) appends one record with two HIP events on
 * the library stream, before the call's first launch and after its last.  Nothing waits for them when the
 * call returns: lx_op_profile waits for the record's second event.  Calls on a stream under capture are
 * recorded untimed (math_ms 0).  Records accumulate until lx_op_profile_reset. */
typedef struct lx_call_profile {
    char op[36];         /* the operator, NUL-terminated (Add, ..., LayerNormDecomposed) */
    double math_ms;      /* device time between the call's two events (OpStage.Math); 0 if not timed */
    double host_ms;      /* host time spent in the call: validation, planning, launches (and any readback) */
    double start_ms;     /* device time from the first timed record since the last reset to this one */
} lx_call_profile;
int lx_set_op_profiling(int32_t enabled);
int32_t lx_op_profile_count(void);
int lx_op_profile(int32_t i, lx_call_profile *out);
int lx_op_profile_reset(void);

/* ---- diagnostics (no reference counterpart) ---------------------------------
 * The HBM ceiling a read-only stream reaches on this GPU, the bound of the whole-tensor reductions:
 * reads `bytes` (a multiple of 16, 16-byte aligned) at src with nontemporal 16-byte loads and writes one
 * 32-bit XOR of what each block read to out, which holds out_bytes / 4 words (the launch uses at most
 * that many blocks of 256 lanes, each reading 4 x 4 KiB per grid-stride step).  Stream-ordered. */
int lx_read_probe(const void *src, int64_t bytes, void *out, int64_t out_bytes);

/* ---- graph runtime: ComputationalGraph + Node.Execute on the device -------
 * (src/Lokad.Onnx.Backend/ComputationalGraph.cs, Node.cs, Model.cs).  Graph
 * inputs, initializers, intermediates and outputs stay in HBM for the whole
 * execution; only the caller's uploads and downloads cross PCIe.  Nodes run in
 * the order they were added (the ONNX topological order the reference keeps,
 * Model.cs:56-60) and execution stops at the first failing node
 * (ComputationalGraph.cs:245-250) with lx_last_error naming it. */
typedef struct lx_graph lx_graph;

/* new ComputationalGraph() with Opset[""] = opset (Model.cs:33-37). */
int lx_graph_create(int64_t opset, lx_graph **out);
int lx_graph_free(lx_graph *g);
/* graph.Inputs / graph.Outputs entries from ValueInfoProto (Model.cs:48-50,
 * TensorUtil.cs:62-84); dims < 0 or a symbolic dim are stored as 0 like
 * DimValue of a dim_param. */
int lx_graph_add_input(lx_graph *g, const char *name, int32_t dtype, int32_t rank, const int64_t *dims);
int lx_graph_add_output(lx_graph *g, const char *name);
/* graph.Initializers[name] = TensorProto.ToTensor() (Model.cs:44-47, TensorUtil.cs:14-58); the host
 * bytes (row-major) are uploaded to HBM once, on the first execution if the graph was built before
 * lx_init. */
int lx_graph_add_initializer(lx_graph *g, const char *name, int32_t dtype, int32_t rank, const int64_t *dims,
                             const void *host, int64_t nbytes);
/* NodeProto.ToNode (NodeUtil.cs:25-50): op_type must name an ONNX operator (OpType.cs); the node
 * index is returned through *index for the attribute setters. */
int lx_graph_add_node(lx_graph *g, const char *name, const char *op_type, int32_t n_in, const char *const *inputs,
                      int32_t n_out, const char *const *outputs, int32_t *index);
/* Node.Attributes values (AttributeProto.Value, NodeUtil.cs:9-22). */
int lx_graph_set_attr_int(lx_graph *g, int32_t node, const char *attr, int64_t v);
int lx_graph_set_attr_ints(lx_graph *g, int32_t node, const char *attr, const int64_t *v, int32_t n);
int lx_graph_set_attr_float(lx_graph *g, int32_t node, const char *attr, float v);
int lx_graph_set_attr_floats(lx_graph *g, int32_t node, const char *attr, const float *v, int32_t n);
int lx_graph_set_attr_string(lx_graph *g, int32_t node, const char *attr, const char *v);
int lx_graph_set_attr_tensor(lx_graph *g, int32_t node, const char *attr, int32_t dtype, int32_t rank,
                             const int64_t *dims, const void *host, int64_t nbytes);
/* Model.Parse + Model.Load (Model.cs:14-63) from the bytes of an ONNX ModelProto.  A malformed protobuf,
 * including a name, op type or domain that is not UTF-8 (protobuf string fields are UTF-8), fails with
 * LX_ERR_INVALID_ARGUMENT; a field the reference cannot convert fails with LX_ERR_NOT_SUPPORTED and its message. */
int lx_graph_load_onnx(const void *bytes, int64_t nbytes, lx_graph **out);
/* Pattern fusion (no reference counterpart; the reference runs every node):
 * replaces the GELU subgraph (Div sqrt2 -> Erf -> Add 1 -> Mul x -> Mul 0.5), the decomposed
 * LayerNorm (ReduceMean -> Sub -> Pow 2 -> ReduceMean -> Add eps -> Sqrt -> Div -> Mul -> Add),
 * Add(mask) -> Softmax, Div / Mul by a scalar constant -> Add(mask) -> Softmax, MatMul -> Add(row-vector
 * constant) [-> Add | -> the GELU subgraph], and Transposes that keep the last axis last around a MatMul
 * (read or written as strided views) by the fused kernels when every intermediate has exactly one
 * consumer and is not a graph output; then every linear chain of two or more Float elementwise nodes
 * (Add/Sub/Mul/Div/Pow/Sqrt/Erf) whose intermediates have one consumer by an ElementwiseChain node
 * (lx_ElementwiseChain); then the MatMul -> Add projections of one input as one grouped launch, a
 * projection whose result only a decomposed LayerNorm reads with that LayerNorm, and an attention layer's
 * scores MatMul -> (scaled) masked Softmax -> context MatMul as one launch per execution where every head has
 * at most 64 rows, keys and columns.
 * Results equal the unfused graph's bit for bit where the fused kernels' are stated to.
 * *n_fused = number of fused nodes made. */
int lx_graph_fuse(lx_graph *g, int32_t *n_fused);
/* Capture (no reference counterpart; the reference dispatches every node from the host on every
 * execution): runs lx_graph_execute once with these inputs, then records a second execution into a HIP
 * graph and runs it, so the graph's outputs are those of one execution when it returns.  The record
 * keeps the inputs' device addresses: lx_graph_replay runs every node's kernels again with one launch,
 * on whatever the caller has written into those same input buffers since.  Device checks (Gather
 * indices, integer division, narrowing casts) are read back after each replay and fail it with the
 * failing node's message, as lx_graph_execute does.  A graph whose execution needs a host value of a
 * device-computed tensor (a shape computed on the device), or whose constants change, cannot be
 * captured (LX_ERR_NOT_SUPPORTED).  The device memory of the recorded execution stays reserved until
 * lx_graph_release_capture, lx_graph_free or a change of the graph (lx_graph_add_*, lx_graph_set_attr_*,
 * lx_graph_fuse). */
int lx_graph_capture(lx_graph *g, int32_t n, const char *const *names, const lx_tensor *inputs,
                     int32_t use_initializers);
int lx_graph_replay(lx_graph *g);
int lx_graph_release_capture(lx_graph *g);
/* ComputationalGraph.Execute(userInputs, useInitializers) (ComputationalGraph.cs:199-272) with the
 * inputs given by name (the Dictionary overload, ComputationalGraph.cs:105-130) or, when names is
 * NULL, by position (the ITensor[] overload, 73-103).  Input tensors are borrowed. */
int lx_graph_execute(lx_graph *g, int32_t n, const char *const *names, const lx_tensor *inputs,
                     int32_t use_initializers);
/* ComputationalGraph.ExecuteNode (ComputationalGraph.cs:274-334). */
int lx_graph_execute_node(lx_graph *g, const char *node, int32_t n, const char *const *names,
                          const lx_tensor *inputs, int32_t use_initializers);
/* graph.Outputs[name] after an execution: a view (owns = 0) of device storage the graph keeps
 * until lx_graph_reset, the next execution or lx_graph_free. */
int lx_graph_output(lx_graph *g, const char *name, lx_tensor *out);
/* ComputationalGraph.Reset (ComputationalGraph.cs:336-349): drops intermediates and outputs (their
 * storage returns to the pool). */
int lx_graph_reset(lx_graph *g);
/* ---- node profiling: the device twin of Profiler (src/Lokad.Onnx.Base/Profiler.cs:24-97) ----
 * Profiler.Enabled / StartNodeProfile / StopNodeProfile (ComputationalGraph.cs:241-243), per graph: while
 * enabled, every node an execution runs (the failing one included) appends one record, NodeProfile's
 * NodeId and Op plus the two stages a device node has: math_ms (OpStage.Math), the device time between
 * HIP events recorded on the library stream before and after the node, so the records of one execution
 * add up to its device span, and host_ms, the host time of the node's dispatch (argument validation,
 * broadcast planning and launches: OpStage.ValidateArguments / GraphOrchestration; broadcast copies do
 * not exist on the device).  A profiled execution waits for its last event before it returns.  Captured
 * executions and replays are not profiled.  Records accumulate until lx_graph_profile_reset. */
typedef struct lx_node_profile {
    int64_t node_id;     /* the node's position in the graph as built (a fused node: its last original node) */
    int32_t node_index;  /* its position in the current node list (lx_graph_node_info) */
    char op[36];         /* op type, NUL-terminated (a fused node: its fused op, e.g. LayerNormDecomposed) */
    double math_ms;      /* device time between the node's boundary events (OpStage.Math); 0 if not timed */
    double host_ms;      /* host time of the node's dispatch (OpStage.GraphOrchestration) */
    double start_ms;     /* device time from the execution's first boundary event to this node's start */
} lx_node_profile;
int lx_graph_set_profiling(lx_graph *g, int32_t enabled);
int32_t lx_graph_profile_count(const lx_graph *g);
int lx_graph_profile(const lx_graph *g, int32_t i, lx_node_profile *out);
int lx_graph_profile_reset(lx_graph *g);

/* introspection for callers and tests */
int32_t lx_graph_node_count(const lx_graph *g);
int lx_graph_node_info(const lx_graph *g, int32_t i, char *op_type, int32_t op_len, char *name, int32_t name_len);
int32_t lx_graph_input_count(const lx_graph *g);
int lx_graph_input_info(const lx_graph *g, int32_t i, char *name, int32_t name_len, int32_t *dtype, int32_t *rank,
                        int64_t *dims);
int32_t lx_graph_initializer_count(const lx_graph *g);
int lx_graph_initializer_info(const lx_graph *g, int32_t i, char *name, int32_t name_len, int32_t *dtype,
                              int32_t *rank, int64_t *dims);
int32_t lx_graph_output_count(const lx_graph *g);
int lx_graph_output_name(const lx_graph *g, int32_t i, char *name, int32_t name_len);

#ifdef __cplusplus
}
#endif
#endif /* LONNX_H */
