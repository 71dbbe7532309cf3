// HipGraph.cs -- a whole ONNX model on the device through the native graph runtime (lx_graph_*): load
// (Model.Load, Model.cs:30-92), optional fusion, execution with every intermediate in HBM (ComputationalGraph.
// Execute, ComputationalGraph.cs:199-272), outputs as DeviceTensors, capture / replay for serving loops, and
// the node profiler mapped onto Profiler.Profile (Profiler.cs:24-97) so `lonnx run --profile` charts device
// runs unchanged.  Belongs in src/Lokad.Onnx.Backend.
namespace Lokad.Onnx;

using System;
using System.Collections.Generic;
using System.IO;
using System.Linq;
using System.Runtime.InteropServices;

public sealed unsafe class HipGraph : IDisposable
{
    IntPtr g;

    HipGraph(IntPtr handle) => g = handle;

    /// <summary>Model.Load on the device: the ModelProto decoded natively, initializers uploaded once.</summary>
    public static HipGraph Load(string path) => Load(File.ReadAllBytes(path));

    public static HipGraph Load(byte[] model)
    {
        HipExecutionProvider.Init();
        IntPtr h;
        fixed (byte* p = model) HipNative.Check(HipNative.lx_graph_load_onnx(p, model.Length, &h), "lx_graph_load_onnx");
        return new HipGraph(h);
    }

    /// <summary>Pattern fusion (GELU, decomposed LayerNorm, mask + Softmax, scaled Softmax, MatMul + bias, elementwise
    /// chains, grouped projections); returns the number of fused nodes.  Results equal the unfused graph's.</summary>
    public int Fuse()
    {
        int n;
        HipNative.Check(HipNative.lx_graph_fuse(g, &n), "lx_graph_fuse");
        return n;
    }

    /// <summary>ComputationalGraph.Execute(userInputs, useInitializers): false with the reference's message in
    /// LastError when a node fails ("Execution of node {c} {n} with op {op} failed: {m}").</summary>
    public bool Execute(IDictionary<string, ITensor> userInputs, bool useInitializers = true)
    {
        var names = userInputs.Keys.ToArray();
        var dev = names.Select(n => DeviceTensor.From(userInputs[n])).ToArray();   // kept alive for the call
        var ts = dev.Select(d => d.Native).ToArray();
        int st;
        fixed (LxTensor* p = ts) st = HipNative.lx_graph_execute(g, ts.Length, names, p, useInitializers ? 1 : 0);
        GC.KeepAlive(dev);
        LastError = st == 0 ? "" : HipNative.LastError();
        return st == 0;
    }

    public string LastError { get; private set; } = "";

    /// <summary>graph.Outputs[name]: a view of storage the graph holds until its next execution or Reset.</summary>
    public DeviceTensor Output(string name)
    {
        LxTensor t;
        HipNative.Check(HipNative.lx_graph_output(g, name, &t), "lx_graph_output");
        return DeviceTensor.Borrow(t).WithName(name);
    }

    public void Reset() => HipNative.Check(HipNative.lx_graph_reset(g), "lx_graph_reset");

    /// <summary>Records one execution into a HIP graph; Replay() then runs it with one launch (inputs rewritten in
    /// place with lx_tensor_upload between replays).</summary>
    public bool Capture(IDictionary<string, DeviceTensor> inputs, bool useInitializers = true)
    {
        var names = inputs.Keys.ToArray();
        var ts = names.Select(n => inputs[n].Native).ToArray();
        int st;
        fixed (LxTensor* p = ts) st = HipNative.lx_graph_capture(g, ts.Length, names, p, useInitializers ? 1 : 0);
        LastError = st == 0 ? "" : HipNative.LastError();
        return st == 0;
    }

    public bool Replay()
    {
        int st = HipNative.lx_graph_replay(g);
        LastError = st == 0 ? "" : HipNative.LastError();
        return st == 0;
    }

    /// <summary>Profiler.Enabled for this graph's executions.</summary>
    public bool Profiling
    {
        set => HipNative.Check(HipNative.lx_graph_set_profiling(g, value ? 1 : 0), "lx_graph_set_profiling");
    }

    /// <summary>The OpType a fused node is charted under (OpType has no members for fused kernels): the op that
    /// dominates its arithmetic.</summary>
    static OpType FusedOp(string name) => name switch
    {
        "GeluErf" => OpType.Erf,
        "LayerNormDecomposed" => OpType.ReduceMean,
        "MatMulAddLayerNorm" => OpType.MatMul,
        "AddSoftmax" or "ScaleAddSoftmax" => OpType.Softmax,
        "Attention" => OpType.MatMul,
        "MatMulAdd" or "MatMulAddGroup" or "MatMulAddGelu" or "MatMulPermuted" => OpType.MatMul,
        _ => OpType.Add,   // ElementwiseChain
    };

    /// <summary>Moves the node records of the profiled executions onto Profiler.Profile as NodeProfiles with a
    /// Math stage (device time) and a GraphOrchestration stage (host dispatch), then clears them.</summary>
    public void PushProfile()
    {
        int n = HipNative.lx_graph_profile_count(g);
        for (int i = 0; i < n; i++)
        {
            LxNodeProfile p;
            HipNative.Check(HipNative.lx_graph_profile(g, i, &p), "lx_graph_profile");
            var name = p.OpName();
            var op = Enum.TryParse<OpType>(name, out var o) ? o : FusedOp(name);
            var np = new NodeProfile() { NodeId = p.NodeId, Op = op };
            np.OpsProfile.Push(new OpProfile() { Stage = OpStage.GraphOrchestration, Time = TimeSpan.FromMilliseconds(p.HostMs) });
            np.OpsProfile.Push(new OpProfile() { Stage = OpStage.Math, Time = TimeSpan.FromMilliseconds(p.MathMs) });
            Profiler.Profile.Push(np);
        }
        HipNative.Check(HipNative.lx_graph_profile_reset(g), "lx_graph_profile_reset");
    }

    public void Dispose()
    {
        if (g != IntPtr.Zero) HipNative.lx_graph_free(g);
        g = IntPtr.Zero;
    }
}
