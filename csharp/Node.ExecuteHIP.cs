// Node.ExecuteHIP.cs -- the HIP twin of Node.ExecuteCPU (src/Lokad.Onnx.Backend/Node.cs:121-181): the same op
// switch, attribute conventions and opset rules, dispatching to HipExecutionProvider.  Belongs in
// src/Lokad.Onnx.Backend beside Node.cs (Node is a partial struct).  Two edits of the reference complete the
// dispatch:
//   CPUExecutionProvider.cs:11-14   public enum ExecutionProvider { CPU, HIP }
//   Node.cs:84-105 (Node.Execute)   var r = provider == ExecutionProvider.CPU ? ExecuteCPU(graph)
//                                         : provider == ExecutionProvider.HIP ? ExecuteHIP(graph)
//                                         : throw new NotSupportedException();
// and ComputationalGraph.Execute / ExecuteNode (ComputationalGraph.cs:242, 316) pass their provider argument to
// node.Execute instead of dropping it.  Exceptions keep the reference's wrapping in Node.Execute (Node.cs:107-118).
namespace Lokad.Onnx;

using static Lokad.Onnx.OpResult;
using HIP = HipExecutionProvider;

public partial struct Node
{
    public OpResult ExecuteHIP(ComputationalGraph graph) => Op switch
    {
        OpType.Reshape => HIP.Reshape(InputTensor(graph, 0), InputTensor(graph, 1), Attr<bool?>("allow_zero")),

        OpType.Add => HIP.Add(InputTensor(graph, 0), InputTensor(graph, 1)),

        OpType.Sub => HIP.Sub(InputTensor(graph, 0), InputTensor(graph, 1)),

        OpType.Mul => HIP.Mul(InputTensor(graph, 0), InputTensor(graph, 1)),

        OpType.Div => HIP.Div(InputTensor(graph, 0), InputTensor(graph, 1)),

        OpType.Pow => HIP.Pow(InputTensor(graph, 0), InputTensor(graph, 1)),

        OpType.Sqrt => HIP.Sqrt(InputTensor(graph, 0)),

        OpType.Conv => HIP.Conv(InputTensor(graph, 0), InputTensor(graph, 1), InputTensor(graph, 2),
            Attr<string>("auto_pad"), Attr<int[]>("dilations"), Attr<int?>("group"), Attr<int[]>("kernel_shape"), Attr<int[]>("pads"), Attr<int[]>("strides")),

        OpType.Relu => HIP.Relu(InputTensor(graph, 0)),

        OpType.Erf => HIP.Erf(InputTensor(graph, 0)),

        OpType.MaxPool => HIP.MaxPool(InputTensor(graph, 0), Attr<string>("auto_pad"), Attr<int?>("ceil_mode"), Ints("dilations"), Ints("kernel_shape"), Ints("pads"), Attr<int?>("storage_order"), Ints("strides")),

        OpType.MatMul => HIP.MatMul(InputTensor(graph, 0), InputTensor(graph, 1)),

        OpType.Transpose => HIP.Transpose(InputTensor(graph, 0), Ints("perm")),

        OpType.Constant => HIP.Constant(OneOfAttr("sparse_value", "value", "value_float", "value_floats", "value_int", "value_ints", "value_string", "value_strings")),

        OpType.Cast => HIP.Cast(InputTensor(graph, 0), RequiredInt("to")),

        OpType.Concat => HIP.Concat(graph.GetInputTensors(Inputs), RequiredInt("axis")),

        OpType.Shape => HIP.Shape(InputTensor(graph, 0), Int("start"), Int("end")),

        OpType.Gather => HIP.Gather(InputTensor(graph, 0), InputTensor(graph, 1), Int("axis")),

        OpType.Slice => HIP.Slice(InputTensor(graph, 0), InputTensor(graph, 1), InputTensor(graph, 2), InputTensor(graph, 3), InputTensor(graph, 4)),

        OpType.Unsqueeze => graph.OpsetVersion() switch
        {
            int v when v >= 13 => HIP.Unsqueeze(InputTensor(graph, 0), InputTensor(graph, 1)),
            _ => HIP.Unsqueeze(InputTensor(graph, 0), RequiredInts("axes")),
        },

        OpType.ReduceSum => HIP.ReduceSum(InputTensor(graph, 0), InputTensor(graph, 1), Int("keepdims"), Int("noop_with_empty_axes")),

        OpType.ReduceMean => graph.OpsetVersion() switch
        {
            int v when v >= 13 => HIP.ReduceMean(InputTensor(graph, 0), InputTensor(graph, 1), Int("keepdims"), Int("noop_with_empty_axes")),
            _ => HIP.ReduceMean(InputTensor(graph, 0), RequiredInts("axes")?.ToTensor<int>(), Int("keepdims"), Int("noop_with_empty_axes")),
        },

        OpType.ReduceMax => HIP.ReduceMax(InputTensor(graph, 0), InputTensor(graph, 1), Int("keepdims")),

        OpType.Softmax => HIP.Softmax(InputTensor(graph, 0), Int("axis")),

        _ => NotSupported(Op)
    };
}
