// HipNative.cs -- P/Invoke declarations of liblonnx_hip.so (include/lonnx.h), one [DllImport] per exported
// symbol.  Belongs in src/Lokad.Onnx.Backend next to CPUExecutionProvider.cs; built with the Backend project
// (AllowUnsafeBlocks).  The layouts below are the C structs' field for field (sequential, natural alignment).
namespace Lokad.Onnx;

using System;
using System.Runtime.InteropServices;

/// <summary>lx_status codes (include/lonnx.h); the texts behind them come from lx_last_error.</summary>
public enum LxStatus
{
    Ok = 0,
    MissingInput = 1,
    WrongInputType = 2,
    CannotBroadcast = 3,
    InputTypeNotSupported = 4,
    NotSupported = 5,
    AttributeNotSupported = 6,
    WrongInputShape = 7,
    InvalidArgument = 8,
    DivideByZero = 9,
    Overflow = 10,
    OutOfMemory = 11,
    Hip = 12,
    NotInitialized = 13,
    BufferTooSmall = 14,
}

/// <summary>lx_tensor: a device tensor handle.  Dtype is the TensorElementType code (Tensor.cs:31-50).</summary>
[StructLayout(LayoutKind.Sequential)]
public unsafe struct LxTensor
{
    public const int MaxRank = 8;
    public int Dtype;
    public int Rank;
    public fixed long Dims[MaxRank];
    public IntPtr Data;          // device address; IntPtr.Zero asks an operator to allocate its output
    public long Capacity;        // bytes usable at Data
    public int Owns;             // 1: lx_tensor_free returns Data to the library's pool
    public int Reserved;
}

/// <summary>lx_bcast_plan: ITensor.Broadcast's shape rule plus the stride-0 view, computed on the host.</summary>
[StructLayout(LayoutKind.Sequential)]
public unsafe struct LxBroadcastPlan
{
    public int Status;
    public int OutRank;
    public fixed long OutDims[LxTensor.MaxRank];
    public int Kind;
    public int Rank;
    public fixed long Dims[LxTensor.MaxRank];
    public fixed long AStrides[LxTensor.MaxRank];
    public fixed long BStrides[LxTensor.MaxRank];
    public long Numel;
}

/// <summary>lx_node_profile: one node of a profiled graph execution (Profiler.NodeProfile).</summary>
[StructLayout(LayoutKind.Sequential)]
public unsafe struct LxNodeProfile
{
    public long NodeId;
    public int NodeIndex;
    public fixed byte Op[36];    // NUL-terminated ASCII
    public double MathMs;        // OpStage.Math: device time between the node's boundary events
    public double HostMs;        // host time of the node's dispatch
    public double StartMs;       // device time from the execution's first boundary event to the node's start

    public string OpName()
    {
        fixed (byte* p = Op) return Marshal.PtrToStringAnsi((IntPtr)p) ?? "";
    }
}

/// <summary>lx_call_profile: one operator call made while lx_set_op_profiling is on (its OpStage.Math stage).</summary>
[StructLayout(LayoutKind.Sequential)]
public unsafe struct LxOpProfile
{
    public fixed byte Op[36];    // NUL-terminated ASCII
    public double MathMs;        // device time between the HIP events around the call's launches
    public double HostMs;        // host time of the call
    public double StartMs;       // device time from the first record since the last reset

    public string OpName()
    {
        fixed (byte* p = Op) return Marshal.PtrToStringAnsi((IntPtr)p) ?? "";
    }
}

internal static unsafe class HipNative
{
    const string Lib = "lonnx_hip";   // liblonnx_hip.so next to the assembly (or on LD_LIBRARY_PATH)

    // ---- library ---------------------------------------------------------------------------------
    [DllImport(Lib)] public static extern int lx_init(int device);
    [DllImport(Lib)] public static extern int lx_shutdown();
    [DllImport(Lib)] public static extern IntPtr lx_last_error();
    [DllImport(Lib)] public static extern IntPtr lx_version();
    [DllImport(Lib)] public static extern int lx_set_stream(IntPtr hipStream);
    [DllImport(Lib)] public static extern int lx_set_op_profiling(int enabled);
    [DllImport(Lib)] public static extern int lx_op_profile_count();
    [DllImport(Lib)] public static extern int lx_op_profile(int i, LxOpProfile* p);
    [DllImport(Lib)] public static extern int lx_op_profile_reset();
    [DllImport(Lib)] public static extern IntPtr lx_get_stream();
    [DllImport(Lib)] public static extern int lx_synchronize();
    [DllImport(Lib)] public static extern long lx_dtype_size(int dtype);

    // ---- tensors ---------------------------------------------------------------------------------
    [DllImport(Lib)] public static extern int lx_tensor_alloc(int dtype, int rank, long* dims, LxTensor* t);
    [DllImport(Lib)] public static extern int lx_tensor_wrap(int dtype, int rank, long* dims, IntPtr devicePtr,
                                                             long capacity, LxTensor* t);
    [DllImport(Lib)] public static extern int lx_tensor_free(LxTensor* t);
    [DllImport(Lib)] public static extern int lx_tensor_upload(LxTensor* t, void* host, long nbytes);
    [DllImport(Lib)] public static extern int lx_tensor_download(LxTensor* t, void* host, long nbytes);
    [DllImport(Lib)] public static extern int lx_tensor_reshape(LxTensor* t, int rank, long* dims, LxTensor* o);
    [DllImport(Lib)] public static extern int lx_pool_trim();
    [DllImport(Lib)] public static extern int lx_pool_stats(long* liveBytes, long* cachedBytes);
    [DllImport(Lib)] public static extern int lx_plan_broadcast(int rankA, long* dimsA, int rankB, long* dimsB,
                                                                LxBroadcastPlan* plan);

    // ---- operators (CPUExecutionProvider's twins) ------------------------------------------------
    [DllImport(Lib)] public static extern int lx_Add(LxTensor* a, LxTensor* b, LxTensor* y);
    [DllImport(Lib)] public static extern int lx_Sub(LxTensor* a, LxTensor* b, LxTensor* y);
    [DllImport(Lib)] public static extern int lx_Mul(LxTensor* a, LxTensor* b, LxTensor* y);
    [DllImport(Lib)] public static extern int lx_Div(LxTensor* a, LxTensor* b, LxTensor* y);
    [DllImport(Lib)] public static extern int lx_Pow(LxTensor* a, LxTensor* b, LxTensor* y);
    [DllImport(Lib)] public static extern int lx_Sqrt(LxTensor* a, LxTensor* y);
    [DllImport(Lib)] public static extern int lx_Erf(LxTensor* x, LxTensor* y);
    [DllImport(Lib)] public static extern int lx_Cast(LxTensor* x, long to, LxTensor* y);
    [DllImport(Lib)] public static extern int lx_ReduceSum(LxTensor* x, long* axes, int nAxes, int keepdims, int noop,
                                                           LxTensor* y);
    [DllImport(Lib)] public static extern int lx_ReduceSum_noalloc(LxTensor* x, long* axes, int nAxes, int keepdims,
                                                                   int noop, LxTensor* y);
    [DllImport(Lib)] public static extern int lx_ReduceMean(LxTensor* x, long* axes, int nAxes, int keepdims, int noop,
                                                            LxTensor* y);
    [DllImport(Lib)] public static extern int lx_ReduceMax(LxTensor* x, long* axes, int nAxes, int keepdims, LxTensor* y);
    [DllImport(Lib)] public static extern int lx_Softmax(LxTensor* x, int axis, int hasAxis, LxTensor* y);
    [DllImport(Lib)] public static extern int lx_MatMul(LxTensor* a, LxTensor* b, LxTensor* y);
    [DllImport(Lib)] public static extern int lx_Transpose(LxTensor* data, long* perm, int nPerm, LxTensor* y);
    [DllImport(Lib)] public static extern int lx_Concat(LxTensor** inputs, int n, int axis, int hasAxis, LxTensor* y);
    [DllImport(Lib)] public static extern int lx_Gather(LxTensor* data, LxTensor* indices, int axis, int hasAxis,
                                                        LxTensor* y);
    [DllImport(Lib)] public static extern int lx_Slice(LxTensor* data, long* starts, int nStarts, long* ends, int nEnds,
                                                       long* axes, int nAxes, long* steps, int nSteps, LxTensor* y);

    // ---- fused subgraphs (one kernel each, every node's float32 rounding kept) ----------------
    [DllImport(Lib)] public static extern int lx_MatMulAdd(LxTensor* a, LxTensor* b, LxTensor* bias, LxTensor* residual,
                                                           LxTensor* y);
    [DllImport(Lib)] public static extern int lx_MatMulAddGelu(LxTensor* a, LxTensor* b, LxTensor* bias, LxTensor* y);
    [DllImport(Lib)] public static extern int lx_GeluErf(LxTensor* x, LxTensor* y);
    [DllImport(Lib)] public static extern int lx_LayerNormDecomposed(LxTensor* x, LxTensor* gamma, LxTensor* beta,
                                                                     float eps, LxTensor* y);
    [DllImport(Lib)] public static extern int lx_AddSoftmax(LxTensor* s, LxTensor* mask, int axis, LxTensor* y);
    [DllImport(Lib)] public static extern int lx_ScaleAddSoftmax(LxTensor* s, LxTensor* scale, int divide, LxTensor* mask,
                                                                 int axis, LxTensor* y);
    [DllImport(Lib)] public static extern int lx_ElementwiseChain(LxTensor** inputs, int nIn, int* ops, int* operands,
                                                                  int nOps, LxTensor* y);

    // ---- diagnostics ---------------------------------------------------------------------------
    [DllImport(Lib)] public static extern int lx_read_probe(IntPtr src, long bytes, IntPtr output, long outBytes);

    // ---- graph runtime (ComputationalGraph / Model on the device) -------------------------------
    [DllImport(Lib)] public static extern int lx_graph_create(long opset, IntPtr* graph);
    [DllImport(Lib)] public static extern int lx_graph_free(IntPtr graph);
    [DllImport(Lib, CharSet = CharSet.Ansi)]
    public static extern int lx_graph_add_input(IntPtr graph, string name, int dtype, int rank, long* dims);
    [DllImport(Lib, CharSet = CharSet.Ansi)] public static extern int lx_graph_add_output(IntPtr graph, string name);
    [DllImport(Lib, CharSet = CharSet.Ansi)]
    public static extern int lx_graph_add_initializer(IntPtr graph, string name, int dtype, int rank, long* dims,
                                                      void* host, long nbytes);
    [DllImport(Lib, CharSet = CharSet.Ansi)]
    public static extern int lx_graph_add_node(IntPtr graph, string name, string opType, int nIn, string[] inputs,
                                               int nOut, string[] outputs, int* index);
    [DllImport(Lib, CharSet = CharSet.Ansi)]
    public static extern int lx_graph_set_attr_int(IntPtr graph, int node, string attr, long v);
    [DllImport(Lib, CharSet = CharSet.Ansi)]
    public static extern int lx_graph_set_attr_ints(IntPtr graph, int node, string attr, long* v, int n);
    [DllImport(Lib, CharSet = CharSet.Ansi)]
    public static extern int lx_graph_set_attr_float(IntPtr graph, int node, string attr, float v);
    [DllImport(Lib, CharSet = CharSet.Ansi)]
    public static extern int lx_graph_set_attr_floats(IntPtr graph, int node, string attr, float* v, int n);
    [DllImport(Lib, CharSet = CharSet.Ansi)]
    public static extern int lx_graph_set_attr_string(IntPtr graph, int node, string attr, string v);
    [DllImport(Lib, CharSet = CharSet.Ansi)]
    public static extern int lx_graph_set_attr_tensor(IntPtr graph, int node, string attr, int dtype, int rank, long* dims,
                                                      void* host, long nbytes);
    [DllImport(Lib)] public static extern int lx_graph_load_onnx(void* bytes, long nbytes, IntPtr* graph);
    [DllImport(Lib)] public static extern int lx_graph_fuse(IntPtr graph, int* nFused);
    [DllImport(Lib, CharSet = CharSet.Ansi)]
    public static extern int lx_graph_capture(IntPtr graph, int n, string[]? names, LxTensor* inputs, int useInitializers);
    [DllImport(Lib)] public static extern int lx_graph_replay(IntPtr graph);
    [DllImport(Lib)] public static extern int lx_graph_release_capture(IntPtr graph);
    [DllImport(Lib, CharSet = CharSet.Ansi)]
    public static extern int lx_graph_execute(IntPtr graph, int n, string[]? names, LxTensor* inputs, int useInitializers);
    [DllImport(Lib, CharSet = CharSet.Ansi)]
    public static extern int lx_graph_execute_node(IntPtr graph, string node, int n, string[]? names, LxTensor* inputs,
                                                   int useInitializers);
    [DllImport(Lib, CharSet = CharSet.Ansi)] public static extern int lx_graph_output(IntPtr graph, string name, LxTensor* t);
    [DllImport(Lib)] public static extern int lx_graph_reset(IntPtr graph);
    [DllImport(Lib)] public static extern int lx_graph_set_profiling(IntPtr graph, int enabled);
    [DllImport(Lib)] public static extern int lx_graph_profile_count(IntPtr graph);
    [DllImport(Lib)] public static extern int lx_graph_profile(IntPtr graph, int i, LxNodeProfile* p);
    [DllImport(Lib)] public static extern int lx_graph_profile_reset(IntPtr graph);
    [DllImport(Lib)] public static extern int lx_graph_node_count(IntPtr graph);
    [DllImport(Lib)] public static extern int lx_graph_node_info(IntPtr graph, int i, byte* opType, int opLen, byte* name,
                                                                 int nameLen);
    [DllImport(Lib)] public static extern int lx_graph_input_count(IntPtr graph);
    [DllImport(Lib)] public static extern int lx_graph_input_info(IntPtr graph, int i, byte* name, int nameLen, int* dtype,
                                                                  int* rank, long* dims);
    [DllImport(Lib)] public static extern int lx_graph_initializer_count(IntPtr graph);
    [DllImport(Lib)] public static extern int lx_graph_initializer_info(IntPtr graph, int i, byte* name, int nameLen,
                                                                        int* dtype, int* rank, long* dims);
    [DllImport(Lib)] public static extern int lx_graph_output_count(IntPtr graph);
    [DllImport(Lib)] public static extern int lx_graph_output_name(IntPtr graph, int i, byte* name, int nameLen);

    public static string LastError() => Marshal.PtrToStringAnsi(lx_last_error()) ?? "";

    /// <summary>Throws with the library's message when a call that cannot fail in normal use fails.</summary>
    public static void Check(int status, string what)
    {
        if (status != 0) throw new InvalidOperationException($"{what} failed ({(LxStatus)status}): {LastError()}");
    }
}
