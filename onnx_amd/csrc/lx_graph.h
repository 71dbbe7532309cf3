// lx_graph.h -- graph runtime structures shared by the executor (lx_graph.cpp)
// and the ONNX model loader (lx_onnx.cpp).
#pragma once

#include <map>
#include <memory>
#include <string>
#include <vector>

#include <hip/hip_runtime.h>

#include "../../include/lonnx.h"
#include "lx_internal.h"

namespace lx {

// A tensor held in host memory: initializers before upload, attribute
// tensors, and the host copy of small integer tensors (shapes, axes).
struct HostTensor {
    int32_t dtype = 0;
    int32_t rank = 0;
    int64_t dims[LX_MAX_RANK] = {0};
    std::vector<uint8_t> bytes;  // row-major
    int64_t numel() const {
        int64_t n = 1;
        for (int i = 0; i < rank; i++) n *= dims[i];
        return n;
    }
};

enum AttrKind { kAttrInt, kAttrInts, kAttrFloat, kAttrFloats, kAttrString, kAttrTensor };

// AttributeProto.Value (NodeUtil.cs:9-22): Int -> long, Ints -> long[],
// Float -> float, Floats -> float[], String -> string, Tensor -> ITensor.
struct Attr {
    AttrKind kind = kAttrInt;
    int64_t i = 0;
    std::vector<int64_t> ints;
    float f = 0.0f;
    std::vector<float> floats;
    std::string s;
    std::shared_ptr<HostTensor> t;
};

// Device storage shared by a tensor and its Reshape / Unsqueeze aliases.
struct Storage {
    void *ptr = nullptr;
    ~Storage();
};

// One named tensor of an execution.
struct Value {
    lx_tensor t{};                      // device view
    std::shared_ptr<Storage> store;     // null for borrowed caller tensors
    std::shared_ptr<HostTensor> host;   // host copy when known
};

struct GNode {
    std::string name, op;
    std::vector<std::string> in, out;
    std::map<std::string, Attr> attrs;
    std::vector<GNode> fused_from;  // the original nodes of a fused subgraph
    int index = -1;                 // position in the node list as built (before fusion)
};

struct GInput {
    std::string name;
    int32_t dtype = 0;
    int32_t rank = 0;
    int64_t dims[LX_MAX_RANK] = {0};
};

// One execution recorded into a HIP graph (lx_graph_capture): the instantiated
// graph, the pool blocks its kernels use (held until release), references to
// every pre-existing device tensor it reads, and the outputs it writes.
struct GraphCapture {
    hipGraph_t graph = nullptr;
    hipGraphExec_t exec = nullptr;
    std::vector<void *> held;                   // pool blocks allocated while recording
    std::map<std::string, Value> values;        // node outputs of the recorded execution
    std::map<std::string, Value> input_vals;    // the caller's inputs it was recorded with
    std::vector<Value> pinned;                  // initializers, cached constants, check records
    std::vector<DeferredCheck> recs;            // the device checks recorded per node
    ~GraphCapture();
};

// One executed node (Profiler.NodeProfile, Profiler.cs:22): the node, its device time between HIP events
// recorded at node boundaries on the library stream (OpStage.Math) and the host time of its dispatch.
struct NodeProf {
    int64_t node_id = 0;     // position in the graph as built (fused nodes: their last original node)
    int32_t node_index = 0;  // position in the current node list
    std::string op;
    double math_ms = 0.0;
    double host_ms = 0.0;
    double start_ms = 0.0;   // device time from the execution's first boundary event to this node's start
};

// HIP events reused by profiled executions (destroyed with the graph).
struct EventPool {
    std::vector<hipEvent_t> ev;
    ~EventPool();
};

}  // namespace lx

struct lx_graph {
    int64_t opset = 13;
    std::string name;
    std::vector<lx::GNode> nodes;
    std::vector<lx::GInput> inputs;
    std::vector<std::string> outputs;
    std::vector<std::pair<std::string, std::shared_ptr<lx::HostTensor>>> initializers;
    // constants made by fusion (stacked projection weights): served like initializers, not listed as them
    std::vector<std::pair<std::string, std::shared_ptr<lx::HostTensor>>> fused_consts;
    int64_t fused_names = 0;                    // counter behind the fused constants' names
    std::map<std::string, lx::Value> init_dev;  // initializers resident in HBM
    std::map<std::string, lx::Value> input_vals;  // graph.Inputs of the current execution
    std::map<std::string, lx::Value> values;    // node outputs of the current execution
    lx::Value check_slots;                      // per node: device error record of its deferred checks
    std::map<std::string, lx::Value> host_cache;  // uploaded Constant / Shape outputs, reused while unchanged
    std::unique_ptr<lx::GraphCapture> capture;    // lx_graph_capture's record, if any
    std::vector<std::string> node_outputs;      // every name a node produces (IntermediateOutputs + Outputs)
    bool profiling = false;                     // Profiler.Enabled, per graph
    std::vector<lx::NodeProf> profile;          // Profiler.Profile: every node executed while enabled
    lx::EventPool prof_events;
};
