"""ComputationalGraph and Model twins over the device graph runtime of
include/lonnx.h (lx_graph_*): the reference's graph API
(src/Lokad.Onnx.Backend/ComputationalGraph.cs, Model.cs) with every tensor of
an execution resident in HBM.

    g = Model.Load("model.onnx")          # Model.Load (Model.cs:65-78); initializers uploaded once
    g.Fuse()                              # optional: GELU / LayerNorm / mask+Softmax subgraphs and elementwise chains -> fused kernels
    ok = g.Execute([x], True)             # ComputationalGraph.Execute (ComputationalGraph.cs:199-272)
    y = g.Outputs["output"].to_numpy()

Execute returns False on failure and keeps the message in `LastError`, as the
reference logs it and returns false.
"""
import ctypes
from typing import Dict, List, Optional, Sequence, Union

import numpy as np

from . import _lib as L
from .provider import CODE_OF, DeviceTensor, init


def _b(s: str) -> bytes:
    return s.encode()


def _strs(names: Sequence[str]):
    arr = (ctypes.c_char_p * max(1, len(names)))()
    for i, n in enumerate(names):
        arr[i] = _b(n)
    return arr


def _check(st, what):
    if st != L.OK:
        raise RuntimeError(f"{what} failed ({st}): {L.last_error()}")


class Node:
    """A graph node as the runtime holds it (after fusion, fused nodes appear with op types GeluErf,
    LayerNormDecomposed, AddSoftmax, ScaleAddSoftmax, MatMulAdd, MatMulAddGelu, MatMulAddGroup,
    MatMulPermuted, MatMulAddLayerNorm, Attention and ElementwiseChain)."""

    def __init__(self, name: str, op: str):
        self.Name, self.Op = name, op

    def __repr__(self):
        return f"Node({self.Name!r}, {self.Op!r})"


class ComputationalGraph:
    """Device twin of ComputationalGraph (ComputationalGraph.cs:10-35)."""

    def __init__(self, opset: int = 13, _handle=None):
        self._h = ctypes.c_void_p()
        if _handle is not None:
            self._h = _handle
        else:
            _check(L.lib().lx_graph_create(opset, ctypes.byref(self._h)), "lx_graph_create")
        self.LastError = ""
        self._borrowed = []
        self._captured = []

    # ---- construction (what Model.Load does from a ModelProto) -------------
    def AddInput(self, name: str, dtype, shape):
        _check(L.lib().lx_graph_add_input(self._h, _b(name), CODE_OF[np.dtype(dtype)], len(shape),
                                          L.dims_array(shape)), "lx_graph_add_input")

    def AddOutput(self, name: str):
        _check(L.lib().lx_graph_add_output(self._h, _b(name)), "lx_graph_add_output")

    def AddInitializer(self, name: str, value: np.ndarray):
        a = np.ascontiguousarray(value)
        _check(L.lib().lx_graph_add_initializer(self._h, _b(name), CODE_OF[a.dtype], a.ndim, L.dims_array(a.shape),
                                                ctypes.c_void_p(a.ctypes.data), a.nbytes),
               "lx_graph_add_initializer")

    def AddNode(self, op: str, inputs: Sequence[str], outputs: Sequence[str], name: str = "", **attrs) -> int:
        idx = ctypes.c_int32()
        _check(L.lib().lx_graph_add_node(self._h, _b(name), _b(op), len(inputs), _strs(inputs), len(outputs),
                                         _strs(outputs), ctypes.byref(idx)), "lx_graph_add_node")
        for k, v in attrs.items():
            self.SetAttr(idx.value, k, v)
        return idx.value

    def SetAttr(self, node: int, name: str, v):
        lib, h, k = L.lib(), self._h, _b(name)
        if isinstance(v, (bool, int, np.integer)):
            st = lib.lx_graph_set_attr_int(h, node, k, int(v))
        elif isinstance(v, (float, np.floating)):
            st = lib.lx_graph_set_attr_float(h, node, k, float(v))
        elif isinstance(v, str):
            st = lib.lx_graph_set_attr_string(h, node, k, _b(v))
        elif isinstance(v, np.ndarray):
            a = np.ascontiguousarray(v)
            st = lib.lx_graph_set_attr_tensor(h, node, k, CODE_OF[a.dtype], a.ndim, L.dims_array(a.shape),
                                              ctypes.c_void_p(a.ctypes.data), a.nbytes)
        elif isinstance(v, (list, tuple)) and all(isinstance(x, (int, np.integer)) for x in v):
            arr = (ctypes.c_int64 * max(1, len(v)))(*[int(x) for x in v])
            st = lib.lx_graph_set_attr_ints(h, node, k, arr, len(v))
        elif isinstance(v, (list, tuple)):
            arr = (ctypes.c_float * max(1, len(v)))(*[float(x) for x in v])
            st = lib.lx_graph_set_attr_floats(h, node, k, arr, len(v))
        else:
            raise TypeError(f"attribute {name}: unsupported value {v!r}")
        _check(st, "lx_graph_set_attr")

    # ---- structure -----------------------------------------------------------
    @property
    def Nodes(self) -> List[Node]:
        lib = L.lib()
        out = []
        for i in range(lib.lx_graph_node_count(self._h)):
            op, nm = ctypes.create_string_buffer(128), ctypes.create_string_buffer(512)
            _check(lib.lx_graph_node_info(self._h, i, op, 128, nm, 512), "lx_graph_node_info")
            out.append(Node(nm.value.decode(), op.value.decode()))
        return out

    @property
    def InputInfo(self):
        """[(name, TensorElementType, dims)] of the graph inputs (graph.Inputs)."""
        lib = L.lib()
        res = []
        for i in range(lib.lx_graph_input_count(self._h)):
            nm, dt, rk = ctypes.create_string_buffer(512), ctypes.c_int32(), ctypes.c_int32()
            dims = (ctypes.c_int64 * L.MAX_RANK)()
            _check(lib.lx_graph_input_info(self._h, i, nm, 512, ctypes.byref(dt), ctypes.byref(rk), dims),
                   "lx_graph_input_info")
            res.append((nm.value.decode(), dt.value, tuple(dims[k] for k in range(rk.value))))
        return res

    @property
    def InitializerInfo(self):
        """[(name, TensorElementType, dims)] of graph.Initializers."""
        lib = L.lib()
        res = []
        for i in range(lib.lx_graph_initializer_count(self._h)):
            nm, dt, rk = ctypes.create_string_buffer(512), ctypes.c_int32(), ctypes.c_int32()
            dims = (ctypes.c_int64 * L.MAX_RANK)()
            _check(lib.lx_graph_initializer_info(self._h, i, nm, 512, ctypes.byref(dt), ctypes.byref(rk), dims),
                   "lx_graph_initializer_info")
            res.append((nm.value.decode(), dt.value, tuple(dims[k] for k in range(rk.value))))
        return res

    @property
    def OutputNames(self) -> List[str]:
        lib = L.lib()
        res = []
        for i in range(lib.lx_graph_output_count(self._h)):
            nm = ctypes.create_string_buffer(512)
            _check(lib.lx_graph_output_name(self._h, i, nm, 512), "lx_graph_output_name")
            res.append(nm.value.decode())
        return res

    # ---- profiling (Profiler.Enabled / Profiler.Profile) ---------------------
    def EnableProfiling(self, enabled: bool = True):
        """Per-node timing of later executions (Profiler.Enabled for this graph)."""
        _check(L.lib().lx_graph_set_profiling(self._h, 1 if enabled else 0), "lx_graph_set_profiling")

    @property
    def Profile(self) -> List[dict]:
        """One record per node executed while profiling (Profiler.Profile): node_id, node_index, op,
        math_ms (device time between the node's boundary events), host_ms (its dispatch) and start_ms (device
        time from the execution's first boundary event to the node's start)."""
        lib = L.lib()
        out = []
        for i in range(lib.lx_graph_profile_count(self._h)):
            p = L.LxNodeProfile()
            _check(lib.lx_graph_profile(self._h, i, ctypes.byref(p)), "lx_graph_profile")
            out.append({"node_id": p.node_id, "node_index": p.node_index, "op": p.op.decode(),
                        "math_ms": p.math_ms, "host_ms": p.host_ms, "start_ms": p.start_ms})
        return out

    def ResetProfile(self):
        _check(L.lib().lx_graph_profile_reset(self._h), "lx_graph_profile_reset")

    def Fuse(self) -> int:
        """Replace the GELU, decomposed-LayerNorm and Add+Softmax subgraphs by their
        fused kernels, then linear chains of Float elementwise nodes by one
        ElementwiseChain node each; returns how many fused nodes were made."""
        n = ctypes.c_int32()
        _check(L.lib().lx_graph_fuse(self._h, ctypes.byref(n)), "lx_graph_fuse")
        return n.value

    # ---- execution -------------------------------------------------------------
    @staticmethod
    def _as_device(t):
        return t if isinstance(t, DeviceTensor) else DeviceTensor.from_numpy(np.asarray(t))

    def _pack(self, user_inputs):
        if isinstance(user_inputs, dict):
            names = list(user_inputs.keys())
            tens = [self._as_device(user_inputs[k]) for k in names]
        else:
            names = None
            tens = [self._as_device(t) for t in user_inputs]
        self._borrowed = tens  # the graph borrows them for this execution
        arr = (L.LxTensor * max(1, len(tens)))(*[t.h for t in tens])
        return (_strs(names) if names is not None else None), arr, len(tens)

    def Execute(self, user_inputs: Union[Sequence, Dict[str, object]], use_initializers: bool = True) -> bool:
        """ComputationalGraph.Execute: user inputs by position (list) or by name (dict),
        as DeviceTensor or numpy arrays (uploaded)."""
        init()
        names, arr, n = self._pack(user_inputs)
        st = L.lib().lx_graph_execute(self._h, n, names, arr, int(use_initializers))
        self.LastError = "" if st == L.OK else L.last_error()
        self.LastStatus = st
        return st == L.OK

    def Capture(self, user_inputs: Union[Sequence, Dict[str, object]], use_initializers: bool = True) -> bool:
        """Execute once, then record an execution into a HIP graph and run it (lx_graph_capture).  The
        record keeps the inputs' device addresses: write new values into the same DeviceTensors and
        call Replay()."""
        init()
        names, arr, n = self._pack(user_inputs)
        self._captured = self._borrowed  # the record reads these buffers on every replay
        st = L.lib().lx_graph_capture(self._h, n, names, arr, int(use_initializers))
        self.LastError = "" if st == L.OK else L.last_error()
        self.LastStatus = st
        return st == L.OK

    def Replay(self) -> bool:
        """Runs the captured execution again with one launch (lx_graph_replay)."""
        st = L.lib().lx_graph_replay(self._h)
        self.LastError = "" if st == L.OK else L.last_error()
        self.LastStatus = st
        return st == L.OK

    def ReleaseCapture(self):
        L.lib().lx_graph_release_capture(self._h)
        self._captured = []

    def ExecuteNode(self, user_inputs, node_label: str, use_initializers: bool = True) -> bool:
        """ComputationalGraph.ExecuteNode (ComputationalGraph.cs:274-334)."""
        init()
        names, arr, n = self._pack(user_inputs)
        st = L.lib().lx_graph_execute_node(self._h, _b(node_label), n, names, arr, int(use_initializers))
        self.LastError = "" if st == L.OK else L.last_error()
        self.LastStatus = st
        return st == L.OK

    def Output(self, name: str) -> DeviceTensor:
        h = L.LxTensor()
        _check(L.lib().lx_graph_output(self._h, _b(name), ctypes.byref(h)), "lx_graph_output")
        return DeviceTensor(h, keepalive=self)  # a view; valid until Reset / next execution

    @property
    def Outputs(self) -> Dict[str, DeviceTensor]:
        res = {}
        for nm in self.OutputNames:
            h = L.LxTensor()
            if L.lib().lx_graph_output(self._h, _b(nm), ctypes.byref(h)) == L.OK:
                res[nm] = DeviceTensor(h, keepalive=self)
        return res

    def Reset(self):
        """ComputationalGraph.Reset: intermediate and output storage returns to the pool."""
        L.lib().lx_graph_reset(self._h)
        self._borrowed = []

    def close(self):
        if self._h:
            L.lib().lx_graph_free(self._h)
            self._h = ctypes.c_void_p()

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass


class Model:
    """Model.Parse / Model.Load (Model.cs:14-78)."""

    @staticmethod
    def Load(source: Union[str, bytes, bytearray]) -> ComputationalGraph:
        data = open(source, "rb").read() if isinstance(source, str) else bytes(source)
        h = ctypes.c_void_p()
        buf = ctypes.create_string_buffer(data, len(data))
        _check(L.lib().lx_graph_load_onnx(buf, len(data), ctypes.byref(h)), "lx_graph_load_onnx")
        return ComputationalGraph(_handle=h)
