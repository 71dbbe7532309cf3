// HipExecutionProvider.cs -- the device twin of CPUExecutionProvider (src/Lokad.Onnx.Backend/CPUExecutionProvider.cs):
// the same static operators, signatures, validation order and OpResult failures, running on liblonnx_hip.so.
// Inputs may be host tensors (uploaded for the call) or DeviceTensors (read in place); outputs are DeviceTensors
// that stay in HBM until a caller asks for ToHost()/ToDenseTensor().  Belongs in src/Lokad.Onnx.Backend.
//
// Validation that the reference performs in C# before any arithmetic (null inputs, element-type equality, rank
// checks of index tensors) is repeated here in the same order with the same OpResult factories, so messages that
// name tensors (OpResult.cs:46-58) carry the tensors' names; the library repeats every check itself and reports
// the failures that arise inside the reference's tensor library (broadcast, dtype support, axes, overflow,
// division by zero, indices) with the reference's texts, which Map turns into the same OpResults.
namespace Lokad.Onnx;

using System;
using System.Collections.Generic;
using System.Linq;

using static OpResult;
using CPU = CPUExecutionProvider;

public unsafe class HipExecutionProvider : Runtime
{
    /// <summary>The operators that run on the device; Node.ExecuteHIP sends the others to CPUExecutionProvider on
    /// host copies.</summary>
    public static List<OpType> DeviceOps { get; } = new List<OpType>()
    {
        OpType.Reshape, OpType.Add, OpType.Sub, OpType.Mul, OpType.Div, OpType.Pow, OpType.MatMul, OpType.Sqrt,
        OpType.Erf, OpType.Transpose, OpType.Cast, OpType.Concat, OpType.Shape, OpType.Gather, OpType.Slice,
        OpType.Unsqueeze, OpType.ReduceSum, OpType.ReduceMean, OpType.ReduceMax, OpType.Softmax,
    };

    static bool initialised;

    /// <summary>lx_init on the given device, once per process (the CLI and the interop call it at start-up).</summary>
    public static void Init(int device = 0)
    {
        if (initialised) return;
        HipNative.Check(HipNative.lx_init(device), "lx_init");
        initialised = true;
    }

    #region Marshalling
    /// <summary>The operands of one call on the device: host inputs are uploaded and released after the call.</summary>
    sealed class Args : IDisposable
    {
        readonly List<DeviceTensor> uploaded = new();

        public LxTensor In(ITensor t)
        {
            if (t is DeviceTensor d) return d.Native;
            var u = DeviceTensor.ToDevice(t);
            uploaded.Add(u);
            return u.Native;
        }

        public void Dispose()
        {
            foreach (var u in uploaded) u.Dispose();
        }
    }

    /// <summary>The library's status turned into the OpResult the reference returns for the same failure
    /// (OpResult.cs:34-60; exceptions as Node.Execute wraps them, Node.cs:107-118).</summary>
    static OpResult Map(OpType op, int st, ITensor? a = null, ITensor? b = null, string aName = "A") => (LxStatus)st switch
    {
        LxStatus.CannotBroadcast when a is not null && b is not null => CannotBroadcast(op, a, b),
        LxStatus.InputTypeNotSupported when a is not null => InputTypeNotSupported(op, aName, a),
        LxStatus.NotSupported => NotSupported(op),
        _ => Failure(op, HipNative.LastError()),   // the library formats the reference's message
    };

    static OpResult Done(OpType op, int st, LxTensor y, ITensor? a = null, ITensor? b = null, string aName = "A")
    {
        if (st == 0) return Success(op, DeviceTensor.Own(y));
        if (y.Owns != 0) HipNative.lx_tensor_free(&y);
        return Map(op, st, a, b, aName);
    }

    /// <summary>The values of a small integer tensor (axes, perm, starts, ...), on the host.</summary>
    static long[] Longs(ITensor t)
    {
        var h = t is DeviceTensor d ? d.ToHost() : t;
        return h.ElementType switch
        {
            TensorElementType.Int64 => ((Tensor<long>)h.ToDenseTensor()).ToArray(),
            TensorElementType.Int32 => ((Tensor<int>)h.ToDenseTensor()).ToArray().Select(v => (long)v).ToArray(),
            _ => throw new ArgumentException($"Index tensors must be Int32 or Int64, got {h.ElementType}."),
        };
    }

    #region Profiling
    static bool deviceProfiling;
    static readonly List<(OpProfile Stage, int Record)> pendingMath = new();

    /// <summary>Profiler.StartOpStage(OpStage.Math) (Profiler.cs:71-80) for a call about to run on the device, as
    /// the reference opens it before its arithmetic (CPUExecutionProvider.cs:92-103).  The stopwatch would time
    /// only the launch, so the library records the call's device time between two HIP events
    /// (lx_set_op_profiling) and ResolveDeviceProfile writes it into this stage.</summary>
    static void MathStage()
    {
        if (!Profiler.Enabled) return;
        if (!deviceProfiling)
        {
            HipNative.Check(HipNative.lx_set_op_profiling(1), "lx_set_op_profiling");
            deviceProfiling = true;
        }
        Profiler.StartOpStage(OpStage.Math);
        pendingMath.Add((Profiler.CurrentOpProfile, HipNative.lx_op_profile_count()));
    }

    /// <summary>Writes the device time of every call made since the last resolve into its OpStage.Math record
    /// (waiting for the calls' last events), then clears the library's records.  The graph executor calls it
    /// after its node loop when Profiler.Enabled, before the profile is read.</summary>
    public static void ResolveDeviceProfile()
    {
        foreach (var (stage, record) in pendingMath)
        {
            if (record >= HipNative.lx_op_profile_count()) continue;
            LxOpProfile p;
            HipNative.Check(HipNative.lx_op_profile(record, &p), "lx_op_profile");
            stage.Time = TimeSpan.FromMilliseconds(p.MathMs);
        }
        pendingMath.Clear();
        HipNative.Check(HipNative.lx_op_profile_reset(), "lx_op_profile_reset");
    }
    #endregion

    delegate int BinaryFn(LxTensor* a, LxTensor* b, LxTensor* y);
    delegate int UnaryFn(LxTensor* a, LxTensor* y);

    // CPUExecutionProvider.Add/Sub/Mul/Div/Pow (CPUExecutionProvider.cs:82-236): null checks, element types,
    // then broadcast and dtype support inside the library
    static OpResult Binary(OpType op, ITensor? A, ITensor? B, BinaryFn fn)
    {
        if (A is null) return MissingInput(op, nameof(A));
        if (B is null) return MissingInput(op, nameof(B));
        if (A.ElementType != B.ElementType) return WrongInputType(op, nameof(B), "Input tensors must be of the same type.", B);
        using var args = new Args();
        LxTensor a = args.In(A), b = args.In(B), y = default;
        MathStage();
        return Done(op, fn(&a, &b, &y), y, A, B);
    }

    static OpResult Unary(OpType op, ITensor? X, string name, UnaryFn fn)
    {
        if (X is null) return MissingInput(op, name);
        using var args = new Args();
        LxTensor x = args.In(X), y = default;
        MathStage();
        return Done(op, fn(&x, &y), y, X, null, name);
    }
    #endregion

    #region Operators (CPUExecutionProvider's signatures)
    /// <summary>CPUExecutionProvider.Reshape (CPUExecutionProvider.cs:56-80) with Tensor.Reshape's rule
    /// (TensorOps.cs:1256-1310): a view of the same device storage.</summary>
    public static OpResult Reshape(ITensor? input, ITensor? shape, bool? allow_zero = null)
    {
        var op = OpType.Reshape;
        if (input is null) return MissingInput(op, nameof(input));
        if (shape is null) return MissingInput(op, nameof(shape));
        if (shape.ElementType != TensorElementType.Int64) return WrongInputType(op, nameof(shape), TensorElementType.Int64, shape);
        if (shape.Rank != 1) return Failure(op, "Shape tensors must be of rank 1. (Parameter 'shape')");
        var s = Longs(shape);
        if (s.Any(v => v < -1)) return Failure(op, $"A shape dimension cannot be < -1, got {s.First(v => v < -1)}. (Parameter 'shape')");
        if (s.Count(v => v == -1) > 1) return Failure(op, "At most 1 shape dimension can be -1. (Parameter 'shape')");
        bool allowZero = allow_zero ?? false;
        var dims = new List<int>();
        int unknown = -1;
        long size = 1;
        for (int i = 0; i < s.Length; i++)
        {
            if (s[i] == -1) { unknown = i; dims.Add(-1); }
            else if (s[i] == 0 && !allowZero) { dims.Add(input.Dims[i]); size *= input.Dims[i]; }
            else if (s[i] == 0) dims.Add(0);
            else { dims.Add(checked((int)s[i])); size *= s[i]; }
        }
        long length = input.Dims.Aggregate(1L, (p, d) => p * d);
        if (unknown != -1)
        {
            dims[unknown] = checked((int)(length / size));
            size *= dims[unknown];
        }
        if (size != length)
            return Failure(op, $"The input tensor cannot be reshaped to the requested shape. Input shape:{input.PrintShape()}, " +
                               $"requested shape:{dims.ToArray().Print()} (Parameter 'shape')");
        var d = DeviceTensor.From(input);
        return Success(op, d.Reshape(dims.ToArray()));
    }

    public static OpResult Add(ITensor? A, ITensor? B) => Binary(OpType.Add, A, B, HipNative.lx_Add);

    public static OpResult Sub(ITensor? A, ITensor? B) => Binary(OpType.Sub, A, B, HipNative.lx_Sub);

    public static OpResult Mul(ITensor? A, ITensor? B) => Binary(OpType.Mul, A, B, HipNative.lx_Mul);

    /// <summary>Also Int32 and Int64 (C# semantics: truncation, DivideByZeroException and OverflowException as
    /// failures), which the reference rejects with InputTypeNotSupported.</summary>
    public static OpResult Div(ITensor? A, ITensor? B) => Binary(OpType.Div, A, B, HipNative.lx_Div);

    public static OpResult Pow(ITensor? A, ITensor? B) => Binary(OpType.Pow, A, B, HipNative.lx_Pow);

    public static OpResult MatMul(ITensor? A, ITensor? B)
    {
        var op = OpType.MatMul;
        if (A is null) return MissingInput(op, nameof(A));
        if (B is null) return MissingInput(op, nameof(B));
        using var args = new Args();
        LxTensor a = args.In(A), b = args.In(B), y = default;
        MathStage();
        return Done(op, HipNative.lx_MatMul(&a, &b, &y), y, A, B);
    }

    public static OpResult Sqrt(ITensor? A) => Unary(OpType.Sqrt, A, nameof(A), HipNative.lx_Sqrt);

    public static OpResult Erf(ITensor? X) => Unary(OpType.Erf, X, nameof(X), HipNative.lx_Erf);

    /// <summary>CPUExecutionProvider.Transpose (CPUExecutionProvider.cs:411-433); a tensor of rank 0 or 1 comes
    /// back as itself, as Tensor.Transpose returns its input.</summary>
    public static OpResult Transpose(ITensor? data, int[]? perm = null)
    {
        var op = OpType.Transpose;
        if (data is null) return MissingInput(op, nameof(data));
        using var args = new Args();
        LxTensor x = args.In(data), y = default;
        var p = perm?.Select(v => (long)v).ToArray() ?? new long[1];
        int st;
        MathStage();
        fixed (long* pp = p) st = HipNative.lx_Transpose(&x, pp, perm?.Length ?? -1, &y);
        if (st == 0 && y.Owns == 0) return Success(op, DeviceTensor.From(data));
        return Done(op, st, y, data);
    }

    public static OpResult Constant(object? value)
    {
        var r = CPU.Constant(value);
        return r.Status == OpStatus.Success ? Success(OpType.Constant, DeviceTensor.ToDevice(r.Outputs[0])) : r;
    }

    /// <summary>CPUExecutionProvider.Cast (CPUExecutionProvider.cs:451-476): Convert.ChangeType's rounding and
    /// OverflowException on the device.</summary>
    public static OpResult Cast(ITensor? input, long to)
    {
        var op = OpType.Cast;
        if (input is null) return MissingInput(op, nameof(input));
        using var args = new Args();
        LxTensor x = args.In(input), y = default;
        MathStage();
        return Done(op, HipNative.lx_Cast(&x, to, &y), y, input);
    }

    public static OpResult Concat(ITensor[]? inputs, int? _axis)
    {
        var op = OpType.Concat;
        if (inputs is null) return MissingInput(op, nameof(inputs));
        if (!inputs.All(i => i.ElementType == inputs[0].ElementType))
            return WrongInputType(op, nameof(inputs), inputs[0].ElementType, inputs.First(i => i.ElementType == inputs[0].ElementType),
                                  "All tensors in a concat operation must have the same type.");
        using var args = new Args();
        var ts = new LxTensor[inputs.Length];
        for (int i = 0; i < inputs.Length; i++) ts[i] = args.In(inputs[i]);
        LxTensor y = default;
        int st;
        MathStage();
        fixed (LxTensor* p = ts)
        {
            var ptrs = stackalloc LxTensor*[Math.Max(ts.Length, 1)];
            for (int i = 0; i < ts.Length; i++) ptrs[i] = p + i;
            st = HipNative.lx_Concat(ptrs, ts.Length, _axis ?? 0, 1, &y);
        }
        return Done(op, st, y, inputs.Length > 0 ? inputs[0] : null, null, nameof(inputs));
    }

    /// <summary>Shape needs only the dims: the CPU operator on the device tensor gives a host Int64 vector,
    /// which the consumers of shapes (Reshape, Gather, Concat of shape pieces) read on the host anyway.</summary>
    public static OpResult Shape(ITensor? data, int? _start = null, int? _end = null) => CPU.Shape(data, _start, _end);

    public static OpResult Gather(ITensor? data, ITensor? indices, int? axis = null)
    {
        var op = OpType.Gather;
        if (data is null) return MissingInput(op, nameof(data));
        if (indices is null) return MissingInput(op, nameof(indices));
        if (indices.Rank > data.Rank) return WrongInputShape(op, nameof(indices), data.Rank, indices);
        using var args = new Args();
        LxTensor x = args.In(data), i = args.In(indices), y = default;
        MathStage();
        return Done(op, HipNative.lx_Gather(&x, &i, axis ?? 0, axis.HasValue ? 1 : 0, &y), y, data, null, nameof(data));
    }

    public static OpResult Slice(ITensor? data, ITensor? starts, ITensor? ends, ITensor? axes, ITensor? steps)
    {
        var op = OpType.Slice;
        if (data is null) return MissingInput(op, nameof(data));
        if (starts is null) return MissingInput(op, nameof(starts));
        if (ends is null) return MissingInput(op, nameof(ends));
        if (data.Rank == 0) return WrongInputShape(op, nameof(data), data, "Cannot slice a tensor of rank 0");
        if (starts.Rank != 1) return WrongInputShape(op, nameof(starts), starts, "The rank of the starts tensor must be 1");
        if (starts.Length > data.Rank) return WrongInputShape(op, nameof(starts), starts, "The length of the starts tensor must be less-than or equal to the rank of the data tensor.");
        if (ends.Rank != 1) return WrongInputShape(op, nameof(ends), ends, "The rank of the ends tensor must be 1");
        if (starts.Length != ends.Length) return WrongInputShape(op, nameof(ends), ends, "The ends tensor must be the same length as the start tensor.");
        if (axes is not null && (axes.Rank != 1 || axes.Length != starts.Length)) return WrongInputShape(op, nameof(axes), axes, "The axes tensor must be a rank 1 tensor with the same length as the start tensor.");
        if (steps is not null && (steps.Rank != 1 || steps.Length != starts.Length)) return WrongInputShape(op, nameof(steps), steps, "The steps tensor must be a rank 1 tensor with the same length as the start tensor.");
        long[] s = Longs(starts), e = Longs(ends), a = axes is null ? new long[1] : Longs(axes), p = steps is null ? new long[1] : Longs(steps);
        // ConvertToInt32 of Int64 index tensors (ITensor.cs:172-183) throws OverflowException out of range
        if (s.Concat(e).Concat(axes is null ? Array.Empty<long>() : a).Concat(steps is null ? Array.Empty<long>() : p)
             .Any(v => v < int.MinValue || v > int.MaxValue))
            return Failure(op, "Value was either too large or too small for an Int32.");
        using var args = new Args();
        LxTensor x = args.In(data), y = default;
        int st;
        MathStage();
        fixed (long* ps = s, pe = e, pa = a, pp = p)
            st = HipNative.lx_Slice(&x, ps, s.Length, pe, e.Length, pa, axes is null ? -1 : a.Length, pp,
                                    steps is null ? -1 : p.Length, &y);
        return Done(op, st, y, data, null, nameof(data));
    }

    public static OpResult Unsqueeze(ITensor? data, ITensor? axes)
    {
        var op = OpType.Unsqueeze;
        if (data is null) return MissingInput(op, nameof(data));
        if (axes is null) return MissingInput(op, nameof(axes));
        var ax = Longs(axes);
        if (ax.Any(v => v < int.MinValue || v > int.MaxValue)) return Failure(op, "Value was either too large or too small for an Int32.");
        return Unsqueeze(data, ax.Select(v => (int)v).ToArray());
    }

    /// <summary>ITensor.Unsqueeze (ITensor.cs:185-208) on the device tensor: a Reshape view.</summary>
    public static OpResult Unsqueeze(ITensor? data, int[] axes)
    {
        var op = OpType.Unsqueeze;
        if (data is null) return MissingInput(op, nameof(data));
        if (axes is null) return MissingInput(op, nameof(axes));
        return Success(op, ((ITensor)DeviceTensor.From(data)).Unsqueeze(axes));
    }

    delegate int ReduceFn(LxTensor* x, long* axes, int nAxes, int keepdims, int noop, LxTensor* y);

    static OpResult Reduce(OpType op, ITensor? data, ITensor? axes, int? keepdims, int? noop, ReduceFn fn, bool axesRankCheck)
    {
        if (data is null) return MissingInput(op, nameof(data));
        if (axesRankCheck && axes is not null && axes.Rank != 1) return WrongInputShape(op, nameof(axes), 1, axes);
        var ax = axes is null ? new long[1] : Longs(axes);
        using var args = new Args();
        LxTensor x = args.In(data), y = default;
        int st;
        MathStage();
        fixed (long* pa = ax) st = fn(&x, pa, axes is null ? -1 : ax.Length, keepdims ?? -1, noop ?? -1, &y);
        return Done(op, st, y, data, null, nameof(data));
    }

    /// <summary>CPUExecutionProvider.ReduceSum (CPUExecutionProvider.cs:623-640); also Int64 (wrapping sums).</summary>
    public static OpResult ReduceSum(ITensor? data, ITensor? axes, int? _keep_dims, int? noop_with_empty_axes) =>
        Reduce(OpType.ReduceSum, data, axes, _keep_dims, noop_with_empty_axes, HipNative.lx_ReduceSum, false);

    public static OpResult ReduceMean(ITensor? data, ITensor? axes, int? _keep_dims, int? noop_with_empty_axes) =>
        Reduce(OpType.ReduceMean, data, axes, _keep_dims, noop_with_empty_axes, HipNative.lx_ReduceMean, true);

    public static OpResult ReduceMax(ITensor? data, ITensor? axes, int? _keep_dims)
    {
        var op = OpType.ReduceMax;
        if (data is null) return MissingInput(op, nameof(data));
        if (axes is not null && axes.Rank != 1) return WrongInputShape(op, nameof(axes), 1, axes);
        var ax = axes is null ? new long[1] : Longs(axes);
        using var args = new Args();
        LxTensor x = args.In(data), y = default;
        int st;
        MathStage();
        fixed (long* pa = ax) st = HipNative.lx_ReduceMax(&x, pa, axes is null ? -1 : ax.Length, _keep_dims ?? -1, &y);
        return Done(op, st, y, data, null, nameof(data));
    }

    public static OpResult Softmax(ITensor? input, int? _axis)
    {
        var op = OpType.Softmax;
        if (input is null) return MissingInput(op, nameof(input));
        using var args = new Args();
        LxTensor x = args.In(input), y = default;
        MathStage();
        return Done(op, HipNative.lx_Softmax(&x, _axis ?? -1, _axis.HasValue ? 1 : 0, &y), y, input, null, nameof(input));
    }

    // Conv, Relu and MaxPool are outside the device path: the CPU operators on host copies
    public static OpResult Conv(ITensor? X, ITensor? W, ITensor? B, string? auto_pad = null, int[]? dilations = null,
                                int? group = null, int[]? kernel_shape = null, int[]? pads = null, int[]? strides = null) =>
        CPU.Conv(Host(X), Host(W), Host(B), auto_pad, dilations, group, kernel_shape, pads, strides);

    public static OpResult Relu(ITensor? X) => CPU.Relu(Host(X));

    public static OpResult MaxPool(ITensor? X, string? auto_pad = null, int? ceil_mode = null, int[]? dilations = null,
                                   int[]? kernel_shape = null, int[]? pads = null, int? storage_order = null,
                                   int[]? strides = null) =>
        CPU.MaxPool(Host(X), auto_pad, ceil_mode, dilations, kernel_shape, pads, storage_order, strides);

    static ITensor? Host(ITensor? t) => t is DeviceTensor d ? d.ToHost() : t;
    #endregion

    #region Fused subgraphs (no single reference counterpart: each replaces consecutive operator calls)
    public static OpResult GeluErf(ITensor? X) => Unary(OpType.Erf, X, "A", HipNative.lx_GeluErf);

    public static OpResult LayerNormDecomposed(ITensor? X, ITensor? gamma, ITensor? beta, float eps)
    {
        var op = OpType.ReduceMean;
        if (X is null) return MissingInput(op, "data");
        if (gamma is null) return MissingInput(OpType.Mul, "B");
        if (beta is null) return MissingInput(OpType.Add, "B");
        using var args = new Args();
        LxTensor x = args.In(X), g = args.In(gamma), b = args.In(beta), y = default;
        MathStage();
        return Done(op, HipNative.lx_LayerNormDecomposed(&x, &g, &b, eps, &y), y, X, gamma, "data");
    }

    public static OpResult AddSoftmax(ITensor? S, ITensor? mask, int axis = -1)
    {
        var op = OpType.Softmax;
        if (S is null) return MissingInput(OpType.Add, "A");
        if (mask is null) return MissingInput(OpType.Add, "B");
        using var args = new Args();
        LxTensor s = args.In(S), m = args.In(mask), y = default;
        MathStage();
        return Done(op, HipNative.lx_AddSoftmax(&s, &m, axis, &y), y, S, mask, "input");
    }

    public static OpResult MatMulAdd(ITensor? A, ITensor? B, ITensor? bias, ITensor? residual = null)
    {
        var op = OpType.MatMul;
        if (A is null) return MissingInput(op, nameof(A));
        if (B is null) return MissingInput(op, nameof(B));
        if (bias is null) return MissingInput(OpType.Add, "B");
        using var args = new Args();
        LxTensor a = args.In(A), b = args.In(B), c = args.In(bias), y = default;
        LxTensor r = residual is null ? default : args.In(residual);
        MathStage();
        return Done(op, HipNative.lx_MatMulAdd(&a, &b, &c, residual is null ? null : &r, &y), y, A, B);
    }

    /// <summary>MatMul -> Add bias -> the GELU subgraph (a BERT FFN's first projection) in one launch.</summary>
    public static OpResult MatMulAddGelu(ITensor? A, ITensor? B, ITensor? bias)
    {
        var op = OpType.MatMul;
        if (A is null) return MissingInput(op, nameof(A));
        if (B is null) return MissingInput(op, nameof(B));
        if (bias is null) return MissingInput(OpType.Add, "B");
        using var args = new Args();
        LxTensor a = args.In(A), b = args.In(B), c = args.In(bias), y = default;
        MathStage();
        return Done(op, HipNative.lx_MatMulAddGelu(&a, &b, &c, &y), y, A, B);
    }
    #endregion
}
