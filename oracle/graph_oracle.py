"""TEST INFRASTRUCTURE ONLY -- CPU restatement of the reference's graph
executor for the operators of the device path, on numpy arrays through the C
oracle (oracle.py).  Only tests/ import it.

  run(nodes, inputs, initializers, opset) follows ComputationalGraph.Execute
  (src/Lokad.Onnx.Backend/ComputationalGraph.cs:199-272): nodes in list order,
  tensors looked up in Inputs, then Initializers, then IntermediateOutputs
  (ComputationalGraph.cs:39-41), the first failing node stops the run.  The op
  switch follows Node.ExecuteCPU (Node.cs:121-181) and CPUExecutionProvider.

A node is a dict: {"op", "inputs", "outputs", "name", "attrs"}.
"""
import numpy as np

from . import oracle as O

BIN = {"Add": O.ADD, "Sub": O.SUB, "Mul": O.MUL, "Div": O.DIV, "Pow": O.POW}
UN = {"Sqrt": O.SQRT, "Erf": O.ERF}
RED = {"ReduceSum": O.RSUM, "ReduceMean": O.RMEAN, "ReduceMax": O.RMAX}


class GraphFailure(Exception):
    def __init__(self, index, node, cause):
        super().__init__(f"node {index} {node.get('name', '')} ({node['op']}) failed: {cause}")
        self.index, self.node, self.cause = index, node, cause


def _reshape(x, shape):
    """Tensor<T>.Reshape (TensorOps.cs:1256-1310) with allowZero = false."""
    shape = [int(v) for v in np.asarray(shape).reshape(-1)]
    out, unknown, size = [], -1, 1
    for i, v in enumerate(shape):
        if v == -1:
            unknown = i
            out.append(-1)
        elif v == 0:
            out.append(x.shape[i])
            size *= x.shape[i]
        else:
            out.append(v)
            size *= v
    if unknown != -1:
        out[unknown] = x.size // size
    return x.reshape(out)


def _unsqueeze(x, axes):
    """ITensor.Unsqueeze (ITensor.cs:185-208): negative axes relative to the input rank."""
    axes = [a if a >= 0 else x.ndim + a for a in axes]
    ns = [0] * (x.ndim + len(axes))
    for a in axes:
        ns[a] = 1
    it = iter(x.shape)
    ns = [d if d else next(it) for d in ns]
    return x.reshape(ns)


def run_node(node, get, opset):
    op, ins, at = node["op"], node["inputs"], node.get("attrs", {})

    def inp(k):
        return get(ins[k]) if k < len(ins) else None

    if op in BIN:
        return [O.binary(BIN[op], inp(0), inp(1))]
    if op in UN:
        return [O.unary(UN[op], inp(0))]
    if op == "Cast":
        return [O.cast(inp(0), int(at["to"]))]
    if op == "Softmax":
        return [O.softmax(inp(0), int(at.get("axis", -1)))]
    if op in RED:
        if op == "ReduceMean" and opset < 13:
            axes = at["axes"]
        else:
            a = inp(1)
            axes = None if a is None else [int(v) for v in np.asarray(a).reshape(-1)]
        return [O.reduce(RED[op], inp(0), axes, bool(at.get("keepdims", 1)))]
    if op == "Reshape":
        return [_reshape(inp(0), inp(1))]
    if op == "Unsqueeze":
        axes = at["axes"] if opset < 13 else [int(v) for v in np.asarray(inp(1)).reshape(-1)]
        return [_unsqueeze(inp(0), axes)]
    if op == "Constant":
        v = at.get("value", at.get("value_float", at.get("value_floats")))
        return [np.asarray(v, dtype=np.float32) if not isinstance(v, np.ndarray) else v]
    if op == "Shape":
        x = inp(0)
        r = x.ndim
        s, e = at.get("start", 0), at.get("end", r)
        s, e = (s if s >= 0 else r + s), (e if e >= 0 else r + e)
        s, e = min(max(s, 0), r), min(max(e, 0), r)
        return [np.array(x.shape[s:e], dtype=np.int64)]
    if op == "MatMul":
        return [O.matmul(inp(0), inp(1))]
    if op == "Transpose":
        return [O.transpose(inp(0), at.get("perm"))]
    if op == "Concat":
        return [O.concat([get(n) for n in ins], int(at["axis"]))]
    if op == "Gather":
        return [O.gather(inp(0), inp(1), int(at.get("axis", 0)))]
    if op == "Slice":
        def ints(k):
            v = inp(k)
            return None if v is None else [int(t) for t in np.asarray(v).reshape(-1)]
        return [O.slice_(inp(0), ints(1), ints(2), ints(3), ints(4))]
    raise NotImplementedError(op)


def run(nodes, inputs, initializers=None, opset=13):
    """Executes the node list; returns the dict of every tensor produced."""
    initializers = initializers or {}
    values = {}

    def get(name):
        if name in inputs:
            return inputs[name]
        if name in initializers:
            return initializers[name]
        return values[name]

    for i, n in enumerate(nodes):
        try:
            outs = run_node(n, get, opset)
        except O.OracleError as e:
            raise GraphFailure(i + 1, n, e) from e
        for name, v in zip(n["outputs"], outs):
            values[name] = v
    return values
