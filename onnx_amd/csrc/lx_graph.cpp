// lx_graph.cpp -- ComputationalGraph.Execute / Node.Execute on the device.
//
// Follows src/Lokad.Onnx.Backend/ComputationalGraph.cs:199-272 (input
// resolution, node loop, stop at the first failure, output assignment) and
// Node.cs:80-181 (the op switch and its attribute conventions), with every
// tensor resident in HBM: user inputs are borrowed device tensors, initializers
// are uploaded once, intermediates live in pooled device blocks that return to
// the pool right after their last consumer ran, and Reshape / Unsqueeze are
// views.  The only host round trips are those an op needs by definition: the
// values of shape / axes tensors that were computed on the device, and the
// error record of integer Div and checked Cast.
#include <hip/hip_runtime.h>

#include <algorithm>
#include <cmath>
#include <cstdarg>
#include <cstring>
#include <chrono>
#include <set>
#include <string>
#include <vector>

#include "../../include/lonnx.h"
#include "lx_graph.h"
#include "lx_internal.h"
#include "lx_kernels.h"
#include "lx_pool.h"

namespace lx {
Storage::~Storage() {
    if (ptr) (void)pool_release(ptr);
}

GraphCapture::~GraphCapture() {
    if (api_initialized()) (void)hipStreamSynchronize(api_stream());  // no replay may still run
    if (exec) (void)hipGraphExecDestroy(exec);
    if (graph) (void)hipGraphDestroy(graph);
    values.clear();
    pool_unhold(held);
}
}  // namespace lx

using namespace lx;

namespace {

std::string fmt(const char *f, ...) {
    char buf[2048];
    va_list ap;
    va_start(ap, f);
    vsnprintf(buf, sizeof buf, f, ap);
    va_end(ap);
    return buf;
}

int fail(int code, const std::string &m) { return api_set_error(code, m); }

std::string lower(std::string s) {
    for (auto &c : s) c = (char)tolower(c);
    return s;
}

// Tensor.PrintShape (Tensor.cs:1724)
std::string print_shape(const lx_tensor &t) {
    std::string s = "[";
    for (int i = 0; i < t.rank; i++) s += (i ? "," : "") + std::to_string(t.dims[i]);
    return s + "]";
}

int64_t numel(const lx_tensor &t) {
    int64_t n = 1;
    for (int i = 0; i < t.rank; i++) n *= t.dims[i];
    return n;
}

// ---- OpResult factories (OpResult.cs:34-60) ---------------------------------
int missing_input(const char *name) {
    return fail(LX_ERR_MISSING_INPUT, fmt("The required input parameter %s is missing or null.", name));
}
int not_supported(const std::string &op) {
    return fail(LX_ERR_NOT_SUPPORTED, fmt("The operation %s is not supported by the backend.", op.c_str()));
}
int wrong_input_type(const std::string &tname, const char *param, int want, const lx_tensor &t) {
    return fail(LX_ERR_WRONG_INPUT_TYPE,
                fmt("The input tensor %s for parameter %s has type %s but is required to be %s. ", tname.c_str(), param,
                    api_dtype_name(t.dtype), api_dtype_name(want)));
}
// .NET ArgumentException(message, paramName).Message
int argument_error(const std::string &message, const std::string &param) {
    return fail(LX_ERR_INVALID_ARGUMENT, message + " (Parameter '" + param + "')");
}
int failure(const std::string &message) { return fail(LX_ERR_INVALID_ARGUMENT, message); }

// ---- attributes (Node.cs:21-73) ---------------------------------------------
const Attr *find_attr(const GNode &n, const char *name) {
    auto it = n.attrs.find(name);
    return it == n.attrs.end() ? nullptr : &it->second;
}

// Node.Int: an int attribute, or a long one converted with Convert.ToInt32.
// Returns 0 = absent, 1 = present, negative = conversion failure (error set).
int attr_int(const GNode &n, const char *name, int32_t *v) {
    const Attr *a = find_attr(n, name);
    if (!a || a->kind != kAttrInt) return 0;
    if (a->i < INT32_MIN || a->i > INT32_MAX) {
        failure("Value was either too large or too small for an Int32.");
        return -1;
    }
    *v = (int32_t)a->i;
    return 1;
}

// Node.Ints: int[] or long[] (each converted with Convert.ToInt32).
int attr_ints(const GNode &n, const char *name, std::vector<int64_t> *v) {
    const Attr *a = find_attr(n, name);
    if (!a || a->kind != kAttrInts) return 0;
    for (int64_t x : a->ints)
        if (x < INT32_MIN || x > INT32_MAX) {
            failure("Value was either too large or too small for an Int32.");
            return -1;
        }
    *v = a->ints;
    return 1;
}

// ---- device values ------------------------------------------------------------
Value value_from_output(const lx_tensor &y) {
    Value v;
    v.t = y;
    v.t.owns = 0;  // the Storage releases the block
    v.store = std::make_shared<Storage>();
    v.store->ptr = y.data;
    return v;
}

// set while an execution is being recorded into a HIP graph: no host round trip may happen then
thread_local bool t_capturing = false;

// a device tensor holding a copy of host data (Constant, Shape outputs)
int value_from_host(const std::shared_ptr<HostTensor> &h, Value *out) {
    if (t_capturing)
        return fail(LX_ERR_NOT_SUPPORTED, "A host value would be uploaded during the recording: a graph whose "
                                          "constants or shapes change between executions cannot be captured.");
    lx_tensor t;
    memset(&t, 0, sizeof t);
    int st = lx_tensor_alloc(h->dtype, h->rank, h->dims, &t);
    if (st) return st;
    Value v = value_from_output(t);
    if (!h->bytes.empty()) {
        hipError_t e = hipMemcpyAsync(t.data, h->bytes.data(), h->bytes.size(), hipMemcpyHostToDevice, api_stream());
        if (e == hipSuccess) e = hipStreamSynchronize(api_stream());
        if (e != hipSuccess) return fail(LX_ERR_HIP, fmt("upload: %s", hipGetErrorString(e)));
    }
    v.host = h;
    *out = v;
    return LX_OK;
}

// Integer values of a small tensor (shape / axes): the host copy if there is
// one, else one download (which synchronises the stream).
int host_ints(Value &v, std::vector<int64_t> *out) {
    const int64_t n = numel(v.t);
    if (!v.host && t_capturing)
        return fail(LX_ERR_NOT_SUPPORTED, "A node reads a device-computed shape or axes tensor on the host: a "
                                          "graph with such a node cannot be captured.");
    if (!v.host) {
        auto h = std::make_shared<HostTensor>();
        h->dtype = v.t.dtype;
        h->rank = v.t.rank;
        for (int i = 0; i < v.t.rank; i++) h->dims[i] = v.t.dims[i];
        h->bytes.resize((size_t)(n * api_esize(v.t.dtype)));
        int st = lx_tensor_download(&v.t, h->bytes.data(), (int64_t)h->bytes.size());
        if (st) return st;
        v.host = h;
    }
    out->resize((size_t)n);
    const uint8_t *b = v.host->bytes.data();
    for (int64_t i = 0; i < n; i++) {
        switch (v.t.dtype) {
        case LX_INT64: { int64_t x; memcpy(&x, b + 8 * i, 8); (*out)[i] = x; break; }
        case LX_INT32: { int32_t x; memcpy(&x, b + 4 * i, 4); (*out)[i] = x; break; }
        default: return failure("shape and axes tensors must hold Int32 or Int64 values");
        }
    }
    return LX_OK;
}

// a small integer vector (or scalar) whose values the host holds: the shape arithmetic of exported
// models (Shape -> Gather -> Unsqueeze -> Concat -> Reshape), evaluated on the host so that the Reshape
// reading it needs no download and the graph stays capturable
constexpr int64_t kHostShapeMax = 64;
bool host_int_vector(const Value *v) {
    if (!v || !v->host || (v->t.dtype != LX_INT64 && v->t.dtype != LX_INT32) || v->t.rank > 1) return false;
    const int64_t n = numel(v->t);
    return n <= kHostShapeMax && (int64_t)v->host->bytes.size() == n * api_esize(v->t.dtype);
}

bool same_host_tensor(const HostTensor &a, const HostTensor &b) {
    if (a.dtype != b.dtype || a.rank != b.rank || a.bytes != b.bytes) return false;
    for (int i = 0; i < a.rank; i++)
        if (a.dims[i] != b.dims[i]) return false;
    return true;
}

// the device copy of a node output computed on the host (Constant, Shape): uploaded once and
// reused by later executions while the value is unchanged (no upload, no synchronisation)
int value_from_host_cached(lx_graph *g, const std::string &name, const std::shared_ptr<HostTensor> &h, Value *out) {
    auto it = g->host_cache.find(name);
    if (it != g->host_cache.end() && it->second.host && same_host_tensor(*it->second.host, *h)) {
        *out = it->second;
        return LX_OK;
    }
    int st = value_from_host(h, out);
    if (st) return st;
    g->host_cache[name] = *out;
    return LX_OK;
}

// ---- execution context ------------------------------------------------------
struct Exec {
    lx_graph *g;
    const GNode *failed = nullptr;  // the original node of a fused subgraph that failed
    bool is_node_output(const std::string &name) const {
        return std::find(g->node_outputs.begin(), g->node_outputs.end(), name) != g->node_outputs.end();
    }
    // ComputationalGraph.GetInputTensor (ComputationalGraph.cs:39-41): Inputs, then
    // Initializers, then IntermediateOutputs.
    int lookup(const std::string &name, Value **out) {
        auto it = g->input_vals.find(name);
        if (it != g->input_vals.end()) { *out = &it->second; return LX_OK; }
        auto ii = g->init_dev.find(name);
        if (ii != g->init_dev.end()) { *out = &ii->second; return LX_OK; }
        for (auto &kv : g->initializers) {  // read only by the original nodes of a fused subgraph
            if (kv.first != name) continue;
            Value v;
            int st = value_from_host(kv.second, &v);
            if (st) return st;
            *out = &(g->init_dev[name] = v);
            return LX_OK;
        }
        auto vi = g->values.find(name);
        if (vi != g->values.end()) { *out = &vi->second; return LX_OK; }
        if (is_node_output(name))
            return failure(fmt("The intermediate output tensor %s has not been assigned a value.", name.c_str()));
        return failure(fmt("The given key '%s' was not present in the dictionary.", name.c_str()));
    }
    // Node.InputTensor (Node.cs:75): null past the node's input list
    int input(const GNode &n, size_t k, Value **out) {
        *out = nullptr;
        if (k >= n.in.size()) return LX_OK;
        return lookup(n.in[k], out);
    }
};

// a freshly allocated output from an lx_* operator call
template <typename F>
int run_op(F call, std::vector<Value> &outs) {
    lx_tensor y;
    memset(&y, 0, sizeof y);
    int st = call(&y);
    if (st) {
        lx_tensor_free(&y);
        return st;
    }
    outs.push_back(value_from_output(y));
    return LX_OK;
}

const lx_tensor *T(Value *v) { return v ? &v->t : nullptr; }

// Tensor<T>.Reshape (TensorOps.cs:1256-1310), allowZero = false
int reshape_dims(const lx_tensor &x, const std::vector<int64_t> &shape, int rank_of_shape, std::vector<int64_t> *nd) {
    if (rank_of_shape != 1) return argument_error("shape", "Shape tensors must be of rank 1.");
    for (int64_t v : shape)
        if (v < -1) return argument_error("shape", fmt("A shape dimension cannot be < -1, got %lld.", (long long)v));
    if (std::count(shape.begin(), shape.end(), (int64_t)-1) > 1)
        return argument_error("shape", "At most 1 shape dimension can be -1.");
    int unknown = -1;
    int64_t new_size = 1;
    nd->clear();
    for (size_t i = 0; i < shape.size(); i++) {
        if (shape[i] == -1) {
            unknown = (int)i;
            nd->push_back(-1);
        } else if (shape[i] == 0) {
            if ((int)i >= x.rank) return failure("Index was outside the bounds of the array.");
            nd->push_back(x.dims[i]);
            new_size *= x.dims[i];
        } else {
            if (shape[i] > INT32_MAX) return failure("Value was either too large or too small for an Int32.");
            nd->push_back(shape[i]);
            new_size *= shape[i];
        }
    }
    const int64_t len = numel(x);
    if (unknown != -1) {
        if (new_size == 0) return failure("Attempted to divide by zero.");
        (*nd)[unknown] = len / new_size;
        new_size *= (*nd)[unknown];
    }
    if (new_size != len) {
        // List<int>.Print() as ArrayTensorExtensions.cs:118 writes it (each entry is the list's type name)
        std::string p = "[";
        for (size_t i = 0; i < nd->size(); i++) p += (i ? ", " : "") + std::string("System.Collections.Generic.List`1[System.Int32]");
        p += "]";
        return argument_error("shape", "The input tensor cannot be reshaped to the requested shape. Input shape:" +
                                           print_shape(x) + ", requested shape:" + p);
    }
    if ((int)nd->size() > LX_MAX_RANK) return fail(LX_ERR_NOT_SUPPORTED, fmt("At most %d axes are supported.", LX_MAX_RANK));
    return LX_OK;
}

Value alias(const Value &x, const std::vector<int64_t> &dims) {
    Value v = x;
    v.t.rank = (int32_t)dims.size();
    for (int i = 0; i < LX_MAX_RANK; i++) v.t.dims[i] = i < (int)dims.size() ? dims[i] : 0;
    v.t.owns = 0;
    v.host.reset();
    if (x.host) {  // same bytes, new dims
        auto h = std::make_shared<HostTensor>(*x.host);
        h->rank = v.t.rank;
        for (int i = 0; i < LX_MAX_RANK; i++) h->dims[i] = v.t.dims[i];
        v.host = h;
    }
    return v;
}

bool reshapable_dtype(int dt) {
    switch (dt) {
    case LX_BOOL: case LX_INT8: case LX_UINT8: case LX_INT16: case LX_UINT16: case LX_INT32: case LX_UINT32:
    case LX_INT64: case LX_UINT64: case LX_FLOAT: case LX_DOUBLE: return true;
    default: return false;
    }
}

// ITensor.Unsqueeze (ITensor.cs:185-208)
int unsqueeze_dims(const lx_tensor &x, std::vector<int64_t> axes, std::vector<int64_t> *nd) {
    std::set<int64_t> uniq(axes.begin(), axes.end());
    if (uniq.size() != axes.size()) return argument_error("axes", "axes contains a repeated dimension.");
    const int64_t rank = x.rank, k = (int64_t)axes.size();
    for (auto &a : axes) a = a >= 0 ? a : rank + a;
    for (int64_t a : axes)
        if (a > rank + k - 1) {
            int64_t first = 0;
            for (int64_t b : axes)
                if (b > rank - 1) { first = b; break; }
            return argument_error("axes", fmt("Each specified axis must be less than the rank of the output tensor. Got %lld",
                                              (long long)first));
        }
    std::vector<int64_t> ns((size_t)(rank + k), 0);
    for (int64_t a : axes) {
        if (a < 0) return failure("Index was outside the bounds of the array.");
        ns[(size_t)a] = 1;
    }
    int e = 0;
    for (auto &d : ns)
        if (d == 0) {
            if (e >= rank) return failure("Out of dimensions.");
            d = x.dims[e++];
        }
    if ((int)ns.size() > LX_MAX_RANK) return fail(LX_ERR_NOT_SUPPORTED, fmt("At most %d axes are supported.", LX_MAX_RANK));
    *nd = ns;
    return LX_OK;
}

// axes tensor of ReduceMean / ReduceMax / ReduceSum: rank check (ReduceMean, ReduceMax),
// Int64 -> Int32 (checked), any other type fails the (Tensor<int>) cast
int reduce_axes(Value *a, bool check_rank, const char *op, const std::string &aname, std::vector<int64_t> *axes,
                int *n_axes) {
    if (!a) {
        *n_axes = -1;
        return LX_OK;
    }
    if (check_rank && a->t.rank != 1)
        return fail(LX_ERR_WRONG_INPUT_SHAPE,
                    fmt("The input tensor %s for parameter axes has shape %s but is required to have rank 1.",
                        aname.c_str(), print_shape(a->t).c_str()));
    if (a->t.dtype != LX_INT64 && a->t.dtype != LX_INT32)
        return failure(fmt("Unable to cast object of type 'DenseTensor`1[%s]' to type 'Tensor`1[System.Int32]'.",
                           api_dtype_name(a->t.dtype)));
    int st = host_ints(*a, axes);
    if (st) return st;
    for (int64_t v : *axes)
        if (v < INT32_MIN || v > INT32_MAX) return fail(LX_ERR_OVERFLOW, "Value was either too large or too small for an Int32.");
    *n_axes = (int)axes->size();
    (void)op;
    return LX_OK;
}

int run_node(Exec &X, const GNode &n, std::vector<Value> &outs);

// the original nodes of a fused subgraph, executed one by one
int run_unfused(Exec &X, const GNode &n, std::vector<Value> &outs) {
    std::vector<std::string> made;
    int st = LX_OK;
    for (const GNode &m : n.fused_from) {
        std::vector<Value> o;
        if ((st = run_node(X, m, o))) {
            if (!X.failed) X.failed = &m;
            break;
        }
        for (size_t i = 0; i < m.out.size() && i < o.size(); i++) {
            X.g->values[m.out[i]] = o[i];
            made.push_back(m.out[i]);
        }
    }
    if (!st) {
        for (const std::string &o : n.out) {
            auto it = X.g->values.find(o);
            if (it == X.g->values.end()) { st = failure("fused subgraph produced no " + o); break; }
            outs.push_back(it->second);
        }
    }
    for (const std::string &m : made)  // intermediates of the subgraph
        if (std::find(n.out.begin(), n.out.end(), m) == n.out.end()) X.g->values.erase(m);
    return st;
}

// Node.ExecuteCPU (Node.cs:121-181) with the device operators.
int run_node(Exec &X, const GNode &n, std::vector<Value> &outs) {
    const std::string &op = n.op;
    Value *a = nullptr, *b = nullptr, *c = nullptr;
    int st;
    auto in2 = [&]() -> int {
        int s = X.input(n, 0, &a);
        if (!s) s = X.input(n, 1, &b);
        return s;
    };
    if (op == "Add" || op == "Sub" || op == "Mul" || op == "Div" || op == "Pow") {
        if ((st = in2())) return st;
        auto f = op == "Add" ? lx_Add : op == "Sub" ? lx_Sub : op == "Mul" ? lx_Mul : op == "Div" ? lx_Div : lx_Pow;
        return run_op([&](lx_tensor *y) { return f(T(a), T(b), y); }, outs);
    }
    if (op == "Transpose") {  // CPU.Transpose(InputTensor(0), Ints("perm")) (Node.cs:146)
        if ((st = X.input(n, 0, &a))) return st;
        std::vector<int64_t> perm;
        int r = attr_ints(n, "perm", &perm);
        if (r < 0) return LX_ERR_INVALID_ARGUMENT;
        if (!a) return missing_input("data");
        if (a->t.rank <= 1 && !(r && (int)perm.size() != a->t.rank)) {  // the input tensor itself
            lx_tensor y;
            memset(&y, 0, sizeof y);
            if ((st = lx_Transpose(T(a), r ? perm.data() : nullptr, r ? (int32_t)perm.size() : -1, &y))) return st;
            outs.push_back(*a);
            return LX_OK;
        }
        return run_op([&](lx_tensor *y) {
            return lx_Transpose(T(a), r ? perm.data() : nullptr, r ? (int32_t)perm.size() : -1, y);
        }, outs);
    }
    if (op == "Concat") {  // CPU.Concat(graph.GetInputTensors(Inputs), RequiredInt("axis")) (Node.cs:150)
        std::vector<const lx_tensor *> ins;
        std::vector<Value *> vs;
        for (size_t k = 0; k < n.in.size(); k++) {
            Value *v;
            if ((st = X.input(n, k, &v))) return st;
            ins.push_back(T(v));
            vs.push_back(v);
        }
        int32_t axis;
        int r = attr_int(n, "axis", &axis);
        if (r < 0) return LX_ERR_INVALID_ARGUMENT;
        if (r == 0) return failure("The Int attribute axis is required but was not found.");
        // shape arithmetic: rank-1 integer vectors known on the host, joined on the host
        bool host = !vs.empty() && (axis == 0 || axis == -1);
        int64_t total = 0;
        for (Value *v : vs) {
            host = host && host_int_vector(v) && v->t.rank == 1 && v->t.dtype == vs[0]->t.dtype;
            if (host) total += numel(v->t);
        }
        if (host && total > 0 && total <= kHostShapeMax) {
            auto h = std::make_shared<HostTensor>();
            h->dtype = vs[0]->t.dtype;
            h->rank = 1;
            h->dims[0] = total;
            for (Value *v : vs) h->bytes.insert(h->bytes.end(), v->host->bytes.begin(), v->host->bytes.end());
            Value out;
            if ((st = value_from_host_cached(X.g, n.out.empty() ? n.name : n.out[0], h, &out))) return st;
            outs.push_back(out);
            return LX_OK;
        }
        return run_op([&](lx_tensor *y) { return lx_Concat(ins.data(), (int32_t)ins.size(), axis, 1, y); }, outs);
    }
    if (op == "Gather") {  // CPU.Gather(InputTensor(0), InputTensor(1), Int("axis")) (Node.cs:154)
        if ((st = in2())) return st;
        int32_t axis = 0;
        int r = attr_int(n, "axis", &axis);
        if (r < 0) return LX_ERR_INVALID_ARGUMENT;
        // shape arithmetic: elements of a rank-1 integer vector known on the host, picked on the host
        // when every index lies inside it (after one wrap of a negative index, as the device operator)
        if (a && b && host_int_vector(a) && a->t.rank == 1 && host_int_vector(b) && (axis == 0 || axis == -1)) {
            std::vector<int64_t> idx;
            const int64_t len = a->t.dims[0], es = api_esize(a->t.dtype);
            bool inside = host_ints(*b, &idx) == LX_OK;
            for (auto &i : idx) {
                if (i < 0) i += len;
                inside = inside && i >= 0 && i < len;
            }
            if (inside) {
                auto h = std::make_shared<HostTensor>();
                h->dtype = a->t.dtype;
                h->rank = b->t.rank;
                for (int d = 0; d < b->t.rank; d++) h->dims[d] = b->t.dims[d];
                for (int64_t i : idx)
                    h->bytes.insert(h->bytes.end(), a->host->bytes.begin() + i * es, a->host->bytes.begin() + (i + 1) * es);
                Value out;
                if ((st = value_from_host_cached(X.g, n.out.empty() ? n.name : n.out[0], h, &out))) return st;
                outs.push_back(out);
                return LX_OK;
            }
        }
        return run_op([&](lx_tensor *y) { return lx_Gather(T(a), T(b), axis, r, y); }, outs);
    }
    if (op == "Slice") {  // CPU.Slice(InputTensor(0..4)) (Node.cs:156; CPUExecutionProvider.cs:548-600)
        Value *in[5];
        for (int k = 0; k < 5; k++)
            if ((st = X.input(n, (size_t)k, &in[k]))) return st;
        if (!in[0]) return missing_input("data");
        if (!in[1]) return missing_input("starts");
        if (!in[2]) return missing_input("ends");
        auto shape_err = [&](const char *param, int idx, const char *msg) {
            return fail(LX_ERR_WRONG_INPUT_SHAPE, fmt("The input tensor %s for parameter %s has shape %s. %s.",
                                                      n.in[idx].c_str(), param, print_shape(in[idx]->t).c_str(), msg));
        };
        if (in[0]->t.rank == 0) return shape_err("data", 0, "Cannot slice a tensor of rank 0");
        if (in[1]->t.rank != 1) return shape_err("starts", 1, "The rank of the starts tensor must be 1");
        if (in[2]->t.rank != 1) return shape_err("ends", 2, "The rank of the ends tensor must be 1");
        if (in[3] && in[3]->t.rank != 1)
            return shape_err("axes", 3, "The axes tensor must be a rank 1 tensor with the same length as the start tensor.");
        if (in[4] && in[4]->t.rank != 1)
            return shape_err("steps", 4, "The steps tensor must be a rank 1 tensor with the same length as the start tensor.");
        std::vector<int64_t> v[5];
        for (int k = 1; k < 5; k++) {
            if (in[k] && (st = host_ints(*in[k], &v[k]))) return st;
            v[k].reserve(1);  // a valid pointer for empty lists
        }
        return run_op([&](lx_tensor *y) {
            return lx_Slice(T(in[0]), v[1].data(), (int32_t)v[1].size(), v[2].data(), (int32_t)v[2].size(),
                            in[3] ? v[3].data() : nullptr, (int32_t)v[3].size(), in[4] ? v[4].data() : nullptr,
                            (int32_t)v[4].size(), y);
        }, outs);
    }
    if (op == "MatMul") {
        if ((st = in2())) return st;
        return run_op([&](lx_tensor *y) { return lx_MatMul(T(a), T(b), y); }, outs);
    }
    if (op == "Sqrt" || op == "Erf") {
        if ((st = X.input(n, 0, &a))) return st;
        auto f = op == "Sqrt" ? lx_Sqrt : lx_Erf;
        return run_op([&](lx_tensor *y) { return f(T(a), y); }, outs);
    }
    if (op == "Cast") {
        if ((st = X.input(n, 0, &a))) return st;
        int32_t to;
        int r = attr_int(n, "to", &to);
        if (r < 0) return LX_ERR_INVALID_ARGUMENT;
        if (r == 0) return failure("The Int attribute to is required but was not found.");
        return run_op([&](lx_tensor *y) { return lx_Cast(T(a), to, y); }, outs);
    }
    if (op == "Softmax") {
        if ((st = X.input(n, 0, &a))) return st;
        int32_t axis = -1;
        int r = attr_int(n, "axis", &axis);
        if (r < 0) return LX_ERR_INVALID_ARGUMENT;
        return run_op([&](lx_tensor *y) { return lx_Softmax(T(a), axis, r, y); }, outs);
    }
    if (X.g->opset < 0 && (op == "ReduceMean" || op == "Unsqueeze"))  // graph.OpsetVersion() (ComputationalGraph.cs:37)
        return failure("The domain  does not ezist in the imported opsets.");
    if (op == "ReduceSum" || op == "ReduceMean" || op == "ReduceMax") {
        if ((st = X.input(n, 0, &a))) return st;
        std::vector<int64_t> axes;
        int n_axes = -1;
        const bool attr_axes = op == "ReduceMean" && X.g->opset < 13;
        if (attr_axes) {
            // RequiredInts("axes")?.ToTensor<int>()  (Node.cs:168-176)
            int r = attr_ints(n, "axes", &axes);
            if (r < 0) return LX_ERR_INVALID_ARGUMENT;
            if (r == 0) return failure("The Ints attribute axes is required but was not found.");
            n_axes = (int)axes.size();
        } else {
            if ((st = X.input(n, 1, &b))) return st;
            if (!a) return missing_input("data");
            const std::string bname = n.in.size() > 1 ? n.in[1] : "";
            if ((st = reduce_axes(b, op != "ReduceSum", op.c_str(), bname, &axes, &n_axes))) return st;
        }
        int32_t keep = -1, noop = -1, v;
        int r = attr_int(n, "keepdims", &v);
        if (r < 0) return LX_ERR_INVALID_ARGUMENT;
        if (r) keep = v != 0;
        if (op != "ReduceMax") {
            r = attr_int(n, "noop_with_empty_axes", &v);
            if (r < 0) return LX_ERR_INVALID_ARGUMENT;
            if (r) noop = v != 0;
        }
        const int64_t *ap = axes.empty() ? nullptr : axes.data();
        if (op == "ReduceSum") return run_op([&](lx_tensor *y) { return lx_ReduceSum(T(a), ap, n_axes, keep, noop, y); }, outs);
        if (op == "ReduceMean") return run_op([&](lx_tensor *y) { return lx_ReduceMean(T(a), ap, n_axes, keep, noop, y); }, outs);
        return run_op([&](lx_tensor *y) { return lx_ReduceMax(T(a), ap, n_axes, keep, y); }, outs);
    }
    if (op == "Reshape") {
        // CPUExecutionProvider.Reshape (CPUExecutionProvider.cs:56-80); allow_zero is read as
        // Attr<bool?> and an AttributeProto int never is a bool, so it is always false
        if ((st = in2())) return st;
        if (!a) return missing_input("input");
        if (!b) return missing_input("shape");
        if (b->t.dtype != LX_INT64) return wrong_input_type(n.in[1], "shape", LX_INT64, b->t);
        if (!reshapable_dtype(a->t.dtype)) return not_supported(op);
        std::vector<int64_t> shape, nd;
        if ((st = host_ints(*b, &shape))) return st;
        if ((st = reshape_dims(a->t, shape, b->t.rank, &nd))) return st;
        outs.push_back(alias(*a, nd));
        return LX_OK;
    }
    if (op == "Unsqueeze") {
        // CPUExecutionProvider.Unsqueeze (CPUExecutionProvider.cs:602-621): axes from input 1
        // from opset 13, from the attribute before
        if ((st = X.input(n, 0, &a))) return st;
        std::vector<int64_t> axes;
        if (X.g->opset >= 13) {
            if ((st = X.input(n, 1, &b))) return st;
            if (!a) return missing_input("data");
            if (!b) return missing_input("axes");
            if ((st = host_ints(*b, &axes))) return st;
        } else {
            int r = attr_ints(n, "axes", &axes);
            if (r < 0) return LX_ERR_INVALID_ARGUMENT;
            if (r == 0) return failure("The Ints attribute axes is required but was not found.");
            if (!a) return missing_input("data");
        }
        std::vector<int64_t> nd;
        if ((st = unsqueeze_dims(a->t, axes, &nd))) return st;
        outs.push_back(alias(*a, nd));
        return LX_OK;
    }
    if (op == "Constant") {
        // CPUExecutionProvider.Constant (CPUExecutionProvider.cs:435-449) on
        // Node.OneOfAttr(...) (Node.cs:30-36, 152)
        static const char *names[] = {"sparse_value", "value", "value_float", "value_floats",
                                      "value_int", "value_ints", "value_string", "value_strings"};
        const Attr *v = nullptr;
        for (const char *nm : names)
            if ((v = find_attr(n, nm))) break;
        if (!v) return fail(LX_ERR_MISSING_INPUT, "The required attribute value is missing or null. ");
        auto h = std::make_shared<HostTensor>();
        if (v->kind == kAttrTensor && v->t) {
            *h = *v->t;
        } else if (v->kind == kAttrFloat) {
            h->dtype = LX_FLOAT;
            h->rank = 0;
            h->bytes.resize(4);
            memcpy(h->bytes.data(), &v->f, 4);
        } else if (v->kind == kAttrFloats) {
            h->dtype = LX_FLOAT;
            h->rank = 1;
            h->dims[0] = (int64_t)v->floats.size();
            h->bytes.resize(4 * v->floats.size());
            if (!v->floats.empty()) memcpy(h->bytes.data(), v->floats.data(), h->bytes.size());
        } else {
            return not_supported(op);  // long / long[] / string values match no case of the switch
        }
        Value out;
        if ((st = value_from_host_cached(X.g, n.out.empty() ? n.name : n.out[0], h, &out))) return st;
        outs.push_back(out);
        return LX_OK;
    }
    if (op == "Shape") {
        // CPUExecutionProvider.Shape (CPUExecutionProvider.cs:503-514)
        if ((st = X.input(n, 0, &a))) return st;
        if (!a) return missing_input("data");
        int32_t s0 = 0, e0 = a->t.rank;
        int r1 = attr_int(n, "start", &s0), r2 = attr_int(n, "end", &e0);
        if (r1 < 0 || r2 < 0) return LX_ERR_INVALID_ARGUMENT;
        const int rank = a->t.rank;
        int s = s0 >= 0 ? s0 : rank + s0, e = e0 >= 0 ? e0 : rank + e0;
        s = std::min(std::max(s, 0), rank);
        e = std::min(std::max(e, 0), rank);
        if (s > e) return failure("Specified argument was out of the range of valid values. (Parameter 'length')");
        auto h = std::make_shared<HostTensor>();
        h->dtype = LX_INT64;
        h->rank = 1;
        h->dims[0] = e - s;
        h->bytes.resize(8 * (size_t)(e - s));
        for (int i = s; i < e; i++) memcpy(h->bytes.data() + 8 * (i - s), &a->t.dims[i], 8);
        Value out;
        if ((st = value_from_host_cached(X.g, n.out.empty() ? n.name : n.out[0], h, &out))) return st;
        outs.push_back(out);
        return LX_OK;
    }
    // ---- fused subgraphs (lx_graph_fuse) ----
    if (op == "GeluErf") {
        if ((st = X.input(n, 0, &a))) return st;
        if (!a || a->t.dtype != LX_FLOAT) return run_unfused(X, n, outs);
        return run_op([&](lx_tensor *y) { return lx_GeluErf(T(a), y); }, outs);
    }
    if (op == "LayerNormDecomposed") {
        if ((st = X.input(n, 0, &a)) || (st = X.input(n, 1, &b)) || (st = X.input(n, 2, &c))) return st;
        // the fused kernel applies gamma and beta along the last axis: other shapes run the nodes, which
        // broadcast them as the reference does (or fail with its CannotBroadcast)
        if (!a || !b || !c || a->t.dtype != LX_FLOAT || b->t.dtype != LX_FLOAT || c->t.dtype != LX_FLOAT ||
            a->t.rank < 1 || !api_layernorm_affine_fits(&b->t, &a->t) || !api_layernorm_affine_fits(&c->t, &a->t))
            return run_unfused(X, n, outs);
        const Attr *eps = find_attr(n, "epsilon");
        const float e = eps ? eps->f : 1e-12f;
        return run_op([&](lx_tensor *y) { return lx_LayerNormDecomposed(T(a), T(b), T(c), e, y); }, outs);
    }
    if (op == "AddSoftmax") {
        if ((st = in2())) return st;
        if (!a || !b || a->t.dtype != LX_FLOAT || b->t.dtype != LX_FLOAT) return run_unfused(X, n, outs);
        int32_t axis = -1;
        if (attr_int(n, "axis", &axis) < 0) return LX_ERR_INVALID_ARGUMENT;
        // the larger operand is S; Add is commutative bit for bit
        Value *s = a, *m = b;
        if (numel(a->t) < numel(b->t) || (numel(a->t) == numel(b->t) && a->t.rank < b->t.rank)) std::swap(s, m);
        lx_bcast_plan p;
        if (lx_plan_broadcast(s->t.rank, s->t.dims, m->t.rank, m->t.dims, &p) != LX_OK) return run_unfused(X, n, outs);
        bool same = p.out_rank == s->t.rank;
        for (int i = 0; same && i < p.out_rank; i++) same = p.out_dims[i] == s->t.dims[i];
        if (!same) return run_unfused(X, n, outs);
        return run_op([&](lx_tensor *y) { return lx_AddSoftmax(T(s), T(m), axis, y); }, outs);
    }
    if (op == "MatMulAddLayerNorm") {
        const size_t nin = n.in.size();
        Value *av, *wv, *bv, *rv = nullptr, *gv, *ev;
        if ((st = X.input(n, 0, &av)) || (st = X.input(n, 1, &wv)) || (st = X.input(n, 2, &bv))) return st;
        if (nin == 6 && (st = X.input(n, 3, &rv))) return st;
        if ((st = X.input(n, nin - 2, &gv)) || (st = X.input(n, nin - 1, &ev))) return st;
        auto eps = n.attrs.find("epsilon");
        if (av && wv && bv && gv && ev && eps != n.attrs.end() && eps->second.kind == kAttrFloat) {
            lx_tensor y{};
            if (api_matmul_add_layernorm(&av->t, &wv->t, &bv->t, rv ? &rv->t : nullptr, &gv->t, &ev->t,
                                         eps->second.f, &y) == LX_OK) {
                outs.push_back(value_from_output(y));
                return LX_OK;
            }
            lx_tensor_free(&y);
        }
        return run_unfused(X, n, outs);
    }
    if (op == "MatMulPermuted") {
        Value *av, *bv;
        if ((st = X.input(n, 0, &av)) || (st = X.input(n, 1, &bv))) return st;
        // each permutation as long as its tensor's rank (the output's: the larger operand rank), else the nodes
        int perm[3][LX_MAX_RANK];
        const int *use[3] = {nullptr, nullptr, nullptr};
        static const char *names[3] = {"a_perm", "b_perm", "y_perm"};
        bool fits = av && bv;
        for (int k = 0; fits && k < 3; k++) {
            auto it = n.attrs.find(names[k]);
            if (it == n.attrs.end()) continue;
            const int rank = k == 0 ? av->t.rank : k == 1 ? bv->t.rank : std::max(av->t.rank, bv->t.rank);
            fits = it->second.ints.size() == (size_t)rank;
            for (int d = 0; fits && d < rank; d++) perm[k][d] = (int)it->second.ints[d];
            use[k] = perm[k];
        }
        if (fits) {
            lx_tensor y{};
            if (api_matmul_permuted(&av->t, use[0], &bv->t, use[1], use[2], &y) == LX_OK) {
                outs.push_back(value_from_output(y));
                return LX_OK;
            }
            lx_tensor_free(&y);
        }
        return run_unfused(X, n, outs);
    }
    if (op == "Attention") {
        // inputs Q, K, V, mask[, scale]; the permutations and the Softmax's attributes as attributes
        Value *qv, *kv, *vv, *mv, *cv = nullptr;
        if ((st = X.input(n, 0, &qv)) || (st = X.input(n, 1, &kv)) || (st = X.input(n, 2, &vv)) ||
            (st = X.input(n, 3, &mv)))
            return st;
        if (n.in.size() > 4 && (st = X.input(n, 4, &cv))) return st;
        int perm[4][LX_MAX_RANK];
        const int *use[4] = {nullptr, nullptr, nullptr, nullptr};
        static const char *names[4] = {"q_perm", "k_perm", "v_perm", "y_perm"};
        bool fits = qv && kv && vv && mv && (n.in.size() == 4 || cv);
        for (int k = 0; fits && k < 4; k++) {
            auto it = n.attrs.find(names[k]);
            if (it == n.attrs.end()) continue;
            fits = it->second.ints.size() == (size_t)qv->t.rank;
            for (int d = 0; fits && d < qv->t.rank; d++) perm[k][d] = (int)it->second.ints[d];
            use[k] = perm[k];
        }
        int32_t axis = -1, divide = 1;
        if (attr_int(n, "axis", &axis) < 0 || attr_int(n, "divide", &divide) < 0) return LX_ERR_INVALID_ARGUMENT;
        if (fits) {
            lx_tensor y{};
            if (api_attention(&qv->t, use[0], &kv->t, use[1], cv ? &cv->t : nullptr, divide, &mv->t, axis, &vv->t,
                              use[2], use[3], &y) == LX_OK) {
                outs.push_back(value_from_output(y));
                return LX_OK;
            }
            lx_tensor_free(&y);
        }
        return run_unfused(X, n, outs);  // the three fused nodes
    }
    if (op == "MatMulAddGroup") {
        Value *av, *wv, *bv;
        if ((st = X.input(n, 0, &av)) || (st = X.input(n, 1, &wv)) || (st = X.input(n, 2, &bv))) return st;
        // A [..., M, K] as [1, M', K] (M' the product of A's axes but the last) times W [G, K, N] plus the
        // bias rows [G, 1, N]: the product [G, M', N] in one launch, its G slices the outputs
        const int64_t G = (int64_t)n.out.size();
        bool fits = av && wv && bv && av->t.dtype == LX_FLOAT && av->t.rank >= 2 && wv->t.rank == 3 &&
                    wv->t.dims[0] == G && av->t.dims[av->t.rank - 1] == wv->t.dims[1] && bv->t.rank == 3 &&
                    bv->t.dims[0] == G && bv->t.dims[1] == 1 && bv->t.dims[2] == wv->t.dims[2];
        if (!fits) return run_unfused(X, n, outs);
        const int64_t K = wv->t.dims[1], Nn = wv->t.dims[2], M = numel(av->t) / (K > 0 ? K : 1);
        lx_tensor a3 = av->t;
        a3.owns = 0;
        a3.rank = 3;
        a3.dims[0] = 1;
        a3.dims[1] = M;
        a3.dims[2] = K;
        lx_tensor y{};
        if ((st = api_matmul_add_grouped(&a3, &wv->t, &bv->t, &y))) {
            lx_tensor_free(&y);
            return run_unfused(X, n, outs);
        }
        const Value whole = value_from_output(y);
        for (int64_t gi = 0; gi < G; gi++) {
            Value v = whole;
            v.t.data = (char *)y.data + gi * M * Nn * (int64_t)sizeof(float);
            v.t.capacity = M * Nn * (int64_t)sizeof(float);  // the slice's own bytes, not the whole product's
            v.t.rank = av->t.rank;
            for (int i = 0; i < LX_MAX_RANK; i++) v.t.dims[i] = i < av->t.rank - 1 ? av->t.dims[i] : 0;
            v.t.dims[av->t.rank - 1] = Nn;
            outs.push_back(v);
        }
        return LX_OK;
    }
    if (op == "MatMulAdd") {
        Value *av, *bv, *cv, *rv = nullptr;
        if ((st = X.input(n, 0, &av)) || (st = X.input(n, 1, &bv)) || (st = X.input(n, 2, &cv))) return st;
        if (n.in.size() > 3 && (st = X.input(n, 3, &rv))) return st;
        // the epilogue's shapes (A [..., M, K] x W [K, N] + bias [N] (+ residual [..., M, N])), else the nodes
        bool fits = av && bv && cv && av->t.dtype == LX_FLOAT && bv->t.dtype == LX_FLOAT && cv->t.dtype == LX_FLOAT &&
                    av->t.rank >= 2 && bv->t.rank == 2 && av->t.dims[av->t.rank - 1] == bv->t.dims[0] &&
                    cv->t.rank == 1 && cv->t.dims[0] == bv->t.dims[1];
        if (fits && n.in.size() > 3) {
            fits = rv && rv->t.dtype == LX_FLOAT && rv->t.rank == av->t.rank;
            for (int i = 0; fits && i < av->t.rank - 1; i++) fits = rv->t.dims[i] == av->t.dims[i];
            fits = fits && rv->t.dims[av->t.rank - 1] == bv->t.dims[1];
        }
        if (!fits) return run_unfused(X, n, outs);
        return run_op([&](lx_tensor *y) { return lx_MatMulAdd(T(av), T(bv), T(cv), rv ? T(rv) : nullptr, y); }, outs);
    }
    if (op == "MatMulAddGelu") {
        Value *av, *bv, *cv;
        if ((st = X.input(n, 0, &av)) || (st = X.input(n, 1, &bv)) || (st = X.input(n, 2, &cv))) return st;
        // the epilogue's shapes (A [..., M, K] x W [K, N] + bias [N], Float), else the nodes
        const bool fits = av && bv && cv && av->t.dtype == LX_FLOAT && bv->t.dtype == LX_FLOAT &&
                          cv->t.dtype == LX_FLOAT && av->t.rank >= 2 && bv->t.rank == 2 &&
                          av->t.dims[av->t.rank - 1] == bv->t.dims[0] && cv->t.rank == 1 &&
                          cv->t.dims[0] == bv->t.dims[1];
        if (!fits) return run_unfused(X, n, outs);
        return run_op([&](lx_tensor *y) { return lx_MatMulAddGelu(T(av), T(bv), T(cv), y); }, outs);
    }
    if (op == "ScaleAddSoftmax") {
        Value *sv, *cv, *mv;
        if ((st = X.input(n, 0, &sv)) || (st = X.input(n, 1, &cv)) || (st = X.input(n, 2, &mv))) return st;
        if (!sv || !cv || !mv || (sv->t.dtype != LX_FLOAT && sv->t.dtype != LX_DOUBLE) || cv->t.dtype != sv->t.dtype ||
            mv->t.dtype != sv->t.dtype || numel(cv->t) != 1 || cv->t.rank > sv->t.rank)
            return run_unfused(X, n, outs);
        lx_bcast_plan p;
        if (lx_plan_broadcast(sv->t.rank, sv->t.dims, mv->t.rank, mv->t.dims, &p) != LX_OK) return run_unfused(X, n, outs);
        bool same = p.out_rank == sv->t.rank;
        for (int i = 0; same && i < p.out_rank; i++) same = p.out_dims[i] == sv->t.dims[i];
        if (!same) return run_unfused(X, n, outs);
        int32_t axis = -1, divide = 1;
        if (attr_int(n, "axis", &axis) < 0 || attr_int(n, "divide", &divide) < 0) return LX_ERR_INVALID_ARGUMENT;
        return run_op([&](lx_tensor *y) { return lx_ScaleAddSoftmax(T(sv), T(cv), divide, T(mv), axis, y); }, outs);
    }
    if (op == "ElementwiseChain") {
        std::vector<const lx_tensor *> ts;
        for (size_t k = 0; k < n.in.size(); k++) {
            Value *v;
            if ((st = X.input(n, k, &v))) return st;
            if (!v || v->t.dtype != LX_FLOAT) return run_unfused(X, n, outs);
            ts.push_back(T(v));
        }
        const Attr *ops = find_attr(n, "ops"), *opd = find_attr(n, "operands");
        if (!ops || !opd || ops->kind != kAttrInts || opd->kind != kAttrInts || ops->ints.size() != opd->ints.size())
            return failure("malformed ElementwiseChain node");
        std::vector<int32_t> o(ops->ints.begin(), ops->ints.end()), p(opd->ints.begin(), opd->ints.end());
        // shapes that do not broadcast step by step: the original nodes report it
        int rank = ts[0]->rank;
        int64_t dims[LX_MAX_RANK];
        for (int i = 0; i < rank; i++) dims[i] = ts[0]->dims[i];
        for (size_t k = 0; k < o.size(); k++) {
            if (o[k] >= 16) continue;
            const int j = p[k] < 0 ? -p[k] - 1 : p[k];
            if (j >= (int)ts.size()) return failure("malformed ElementwiseChain node");
            lx_bcast_plan bp;
            if (lx_plan_broadcast(rank, dims, ts[j]->rank, ts[j]->dims, &bp) != LX_OK) return run_unfused(X, n, outs);
            rank = bp.out_rank;
            for (int i = 0; i < rank; i++) dims[i] = bp.out_dims[i];
        }
        return run_op([&](lx_tensor *y) {
            return lx_ElementwiseChain(ts.data(), (int32_t)ts.size(), o.data(), p.data(), (int32_t)o.size(), y);
        }, outs);
    }
    return not_supported(op);
}

// ---- fusion -----------------------------------------------------------------
constexpr int kChainMaxInG = 8, kChainMaxOpsG = 16;  // lx_ElementwiseChain's limits

struct Fuser {
    lx_graph *g;
    std::map<std::string, std::vector<int>> consumers;
    std::set<std::string> graph_outputs, graph_inputs;
    std::map<std::string, std::shared_ptr<HostTensor>> consts;
    std::vector<bool> used;

    void index() {
        consumers.clear();
        for (int i = 0; i < (int)g->nodes.size(); i++)
            for (const auto &nm : g->nodes[i].in) consumers[nm].push_back(i);
        graph_outputs = std::set<std::string>(g->outputs.begin(), g->outputs.end());
        graph_inputs.clear();
        for (auto &in : g->inputs) graph_inputs.insert(in.name);
        consts.clear();
        // initializers a caller cannot replace, and Constant nodes with a tensor / float value
        for (auto &kv : g->initializers)
            if (!graph_inputs.count(kv.first)) consts[kv.first] = kv.second;
        for (auto &n : g->nodes) {
            if (n.op != "Constant" || n.out.empty()) continue;
            auto it = n.attrs.find("value");
            if (it != n.attrs.end() && it->second.kind == kAttrTensor && it->second.t && n.attrs.size() == 1)
                consts[n.out[0]] = it->second.t;
            it = n.attrs.find("value_float");
            if (it != n.attrs.end() && it->second.kind == kAttrFloat && n.attrs.size() == 1) {
                auto h = std::make_shared<HostTensor>();
                h->dtype = LX_FLOAT;
                h->bytes.resize(4);
                memcpy(h->bytes.data(), &it->second.f, 4);
                consts[n.out[0]] = h;
            }
        }
        used.assign(g->nodes.size(), false);
    }
    // the float32 scalar value of a constant (numel 1, rank <= 1)
    bool scalar_f32(const std::string &name, float *v) const {
        auto it = consts.find(name);
        if (it == consts.end()) return false;
        const HostTensor &h = *it->second;
        if (h.dtype != LX_FLOAT || h.numel() != 1 || h.rank > 1 || h.bytes.size() != 4) return false;
        memcpy(v, h.bytes.data(), 4);
        return true;
    }
    bool scalar_bits(const std::string &name, uint32_t bits) const {
        float v;
        if (!scalar_f32(name, &v)) return false;
        uint32_t u;
        memcpy(&u, &v, 4);
        return u == bits;
    }
    bool int_axes_last(const std::string &name) const {  // a constant [-1]
        auto it = consts.find(name);
        if (it == consts.end()) return false;
        const HostTensor &h = *it->second;
        if (h.numel() != 1 || h.rank != 1) return false;
        if (h.dtype == LX_INT64 && h.bytes.size() == 8) { int64_t x; memcpy(&x, h.bytes.data(), 8); return x == -1; }
        if (h.dtype == LX_INT32 && h.bytes.size() == 4) { int32_t x; memcpy(&x, h.bytes.data(), 4); return x == -1; }
        return false;
    }
    // the single consumer of `name` (or -1), provided `name` is no graph output
    int only_consumer(const std::string &name) const {
        if (graph_outputs.count(name)) return -1;
        auto it = consumers.find(name);
        if (it == consumers.end() || it->second.size() != 1) return -1;
        return it->second[0];
    }
    const GNode &N(int i) const { return g->nodes[i]; }
    bool is(int i, const char *op, size_t nin) const {
        return i >= 0 && !used[i] && N(i).op == op && N(i).in.size() == nin && N(i).out.size() == 1;
    }
    // the other input of a two-input node, given one
    bool other(int i, const std::string &one, std::string *o) const {
        const GNode &n = N(i);
        if (n.in[0] == one && n.in[1] != one) { *o = n.in[1]; return true; }
        if (n.in[1] == one && n.in[0] != one) { *o = n.in[0]; return true; }
        return false;
    }
    // ReduceMean over the last axis with keepdims 1
    bool mean_last(int i) const {
        const GNode &n = N(i);
        auto kd = n.attrs.find("keepdims");
        if (kd != n.attrs.end() && !(kd->second.kind == kAttrInt && kd->second.i == 1)) return false;
        if (n.attrs.count("noop_with_empty_axes")) return false;
        if (g->opset < 13) {
            auto ax = n.attrs.find("axes");
            return n.in.size() == 1 && ax != n.attrs.end() && ax->second.kind == kAttrInts && ax->second.ints.size() == 1 &&
                   ax->second.ints[0] == -1;
        }
        return n.in.size() == 2 && int_axes_last(n.in[1]);
    }

    // Div(x, sqrt2) -> Erf -> Add 1 -> Mul x -> Mul 0.5
    bool gelu(int i0, GNode *f, std::vector<int> *nodes) {
        if (!is(i0, "Div", 2) || !scalar_bits(N(i0).in[1], 0x3fb504f3u)) return false;
        const std::string x = N(i0).in[0];
        int i1 = only_consumer(N(i0).out[0]);
        if (!is(i1, "Erf", 1)) return false;
        int i2 = only_consumer(N(i1).out[0]);
        std::string o;
        if (!is(i2, "Add", 2) || !other(i2, N(i1).out[0], &o) || !scalar_bits(o, 0x3f800000u)) return false;
        int i3 = only_consumer(N(i2).out[0]);
        if (!is(i3, "Mul", 2) || !other(i3, N(i2).out[0], &o) || o != x) return false;
        int i4 = only_consumer(N(i3).out[0]);
        if (!is(i4, "Mul", 2) || !other(i4, N(i3).out[0], &o) || !scalar_bits(o, 0x3f000000u)) return false;
        *nodes = {i0, i1, i2, i3, i4};
        f->op = "GeluErf";
        f->in = {x};
        f->out = N(i4).out;
        return true;
    }

    // ReduceMean -> Sub -> Pow 2 -> ReduceMean -> Add eps -> Sqrt -> Div -> Mul gamma -> Add beta
    bool layernorm(int i0, GNode *f, std::vector<int> *nodes) {
        if (!is(i0, "ReduceMean", N(i0).in.size()) || !mean_last(i0)) return false;
        const std::string x = N(i0).in[0], mean = N(i0).out[0];
        int i1 = only_consumer(mean);
        if (!is(i1, "Sub", 2) || N(i1).in[0] != x || N(i1).in[1] != mean) return false;
        const std::string d = N(i1).out[0];
        if (graph_outputs.count(d)) return false;
        auto cd = consumers.find(d);
        if (cd == consumers.end() || cd->second.size() != 2) return false;
        int ipow = -1, idiv = -1;
        for (int k : cd->second) {
            if (is(k, "Pow", 2) && N(k).in[0] == d) ipow = k;
            else if (is(k, "Div", 2) && N(k).in[0] == d) idiv = k;
        }
        if (ipow < 0 || idiv < 0 || !scalar_bits(N(ipow).in[1], 0x40000000u)) return false;
        int i3 = only_consumer(N(ipow).out[0]);
        if (!is(i3, "ReduceMean", N(i3 >= 0 ? i3 : 0).in.size()) || !mean_last(i3) || N(i3).in[0] != N(ipow).out[0])
            return false;
        int i4 = only_consumer(N(i3).out[0]);
        std::string o;
        float eps;
        if (!is(i4, "Add", 2) || !other(i4, N(i3).out[0], &o) || !scalar_f32(o, &eps)) return false;
        int i5 = only_consumer(N(i4).out[0]);
        if (!is(i5, "Sqrt", 1)) return false;
        if (only_consumer(N(i5).out[0]) != idiv || N(idiv).in[1] != N(i5).out[0]) return false;
        int i7 = only_consumer(N(idiv).out[0]);
        std::string gamma, beta;
        if (!is(i7, "Mul", 2) || !other(i7, N(idiv).out[0], &gamma)) return false;
        int i8 = only_consumer(N(i7).out[0]);
        if (!is(i8, "Add", 2) || !other(i8, N(i7).out[0], &beta)) return false;
        *nodes = {i0, i1, ipow, i3, i4, i5, idiv, i7, i8};
        f->op = "LayerNormDecomposed";
        f->in = {x, gamma, beta};
        f->out = N(i8).out;
        Attr a;
        a.kind = kAttrFloat;
        a.f = eps;
        f->attrs["epsilon"] = a;
        return true;
    }

    // MatMul(A, W) -> Add(., b) [-> Add(., r)] for a Float row-vector constant b: the projection with
    // its bias (and residual) in one MatMul epilogue
    bool matmul_add(int i0, GNode *f, std::vector<int> *nodes) {
        if (!is(i0, "MatMul", 2)) return false;
        const std::string &prod = N(i0).out[0];
        const int i1 = only_consumer(prod);
        std::string bias;
        if (!is(i1, "Add", 2) || !other(i1, prod, &bias)) return false;
        auto it = consts.find(bias);
        if (it == consts.end() || it->second->dtype != LX_FLOAT || it->second->rank != 1) return false;
        *nodes = {i0, i1};
        f->op = "MatMulAdd";
        f->in = {N(i0).in[0], N(i0).in[1], bias};
        f->out = N(i1).out;
        const std::string &biased = N(i1).out[0];
        // -> the GELU subgraph on the biased product (a BERT FFN's first projection): its two consumers of
        // the product, the Div and the Mul x, both in the pattern
        auto cb = consumers.find(biased);
        if (!graph_outputs.count(biased) && cb != consumers.end() && cb->second.size() == 2) {
            for (int k : cb->second) {
                GNode fg;
                std::vector<int> gn;
                if (!gelu(k, &fg, &gn) || fg.in[0] != biased) continue;
                bool inside = true;
                for (int c : cb->second) inside = inside && std::find(gn.begin(), gn.end(), c) != gn.end();
                if (!inside) continue;
                nodes->insert(nodes->end(), gn.begin(), gn.end());
                f->op = "MatMulAddGelu";
                f->out = fg.out;
                return true;
            }
        }
        const int i2 = only_consumer(biased);
        std::string res;
        if (is(i2, "Add", 2) && other(i2, biased, &res)) {
            nodes->push_back(i2);
            f->in.push_back(res);
            f->out = N(i2).out;
        }
        return true;
    }

    // a Transpose whose perm keeps the last axis last (or, k_last, puts it second to last: a right operand
    // then read by columns)
    bool keeps_last(int i, bool k_last = false) const {
        if (!is(i, "Transpose", 1)) return false;
        auto it = N(i).attrs.find("perm");
        if (it == N(i).attrs.end() || it->second.kind != kAttrInts) return false;
        const std::vector<int64_t> &pm = it->second.ints;
        const int64_t r = (int64_t)pm.size();
        if (r == 0 || r > LX_MAX_RANK) return false;
        return pm[r - 1] == r - 1 || (k_last && r >= 2 && pm[r - 2] == r - 1);
    }
    // the unfused node that produces `name`, or -1
    int producer(const std::string &name) const {
        for (int k = 0; k < (int)g->nodes.size(); k++)
            if (!used[k] && N(k).out.size() == 1 && N(k).out[0] == name) return k;
        return -1;
    }
    // Transpose -> MatMul input and MatMul -> Transpose, each Transpose keeping the last axis last (the right
    // operand's may also make it K: read by columns) and its tensor read only by the MatMul: the MatMul reads and
    // writes the transposed views through their strides (an attention layer's Q, K, V and context heads)
    bool matmul_permuted(int i0, GNode *f, std::vector<int> *nodes) {
        if (!is(i0, "MatMul", 2)) return false;
        const GNode &m = N(i0);
        std::vector<int> ns = {i0};
        f->in = m.in;
        f->out = m.out;
        static const char *names[2] = {"a_perm", "b_perm"};
        for (int side = 0; side < 2 && m.in[0] != m.in[1]; side++) {
            const int t = producer(m.in[side]);
            if (t < 0 || !keeps_last(t, side == 1) || only_consumer(m.in[side]) != i0) continue;
            f->in[side] = N(t).in[0];
            f->attrs[names[side]] = N(t).attrs.at("perm");
            ns.push_back(t);
        }
        const int c = only_consumer(m.out[0]);
        if (keeps_last(c)) {
            f->out = N(c).out;
            f->attrs["y_perm"] = N(c).attrs.at("perm");
            ns.push_back(c);
        }
        if (ns.size() == 1) return false;
        f->op = "MatMulPermuted";
        *nodes = ns;
        return true;
    }

    // Add(S, mask) -> Softmax, and Div(S, c) / Mul(S, c) -> Add(., mask) -> Softmax for a Float scalar
    // constant c (the scaled attention scores)
    bool add_softmax(int i0, GNode *f, std::vector<int> *nodes) {
        if (!is(i0, "Add", 2)) return false;
        int i1 = only_consumer(N(i0).out[0]);
        if (!is(i1, "Softmax", 1)) return false;
        auto ax = N(i1).attrs.find("axis");
        if (ax != N(i1).attrs.end()) f->attrs["axis"] = ax->second;
        f->out = N(i1).out;
        for (int side = 0; side < 2; side++) {  // the Add operand that a scaling node produces
            const std::string &sv = N(i0).in[side];
            int is_ = -1;
            for (int k = 0; k < i0; k++)
                if (!used[k] && N(k).out.size() == 1 && N(k).out[0] == sv) is_ = k;
            if (is_ < 0 || only_consumer(sv) != i0 || N(i0).in[1 - side] == sv) continue;
            const GNode &sc = N(is_);
            float c;
            std::string src, cname;
            int divide;
            if (is(is_, "Div", 2) && scalar_f32(sc.in[1], &c)) {
                src = sc.in[0], cname = sc.in[1], divide = 1;
            } else if (is(is_, "Mul", 2) && scalar_f32(sc.in[1], &c)) {
                src = sc.in[0], cname = sc.in[1], divide = 0;
            } else if (is(is_, "Mul", 2) && scalar_f32(sc.in[0], &c)) {
                src = sc.in[1], cname = sc.in[0], divide = 0;
            } else {
                continue;
            }
            *nodes = {is_, i0, i1};
            f->op = "ScaleAddSoftmax";
            f->in = {src, cname, N(i0).in[1 - side]};
            Attr a;
            a.kind = kAttrInt;
            a.i = divide;
            f->attrs["divide"] = a;
            return true;
        }
        *nodes = {i0, i1};
        f->op = "AddSoftmax";
        f->in = N(i0).in;
        return true;
    }

    // a linear chain of Float elementwise nodes (Add/Sub/Mul/Div/Pow/Sqrt/Erf), each intermediate
    // consumed only by the next node of the chain: one ElementwiseChain node
    static int chain_op(const GNode &n) {
        static const char *bin[] = {"Add", "Sub", "Mul", "Div", "Pow"};
        if (n.out.size() != 1) return -1;
        for (int k = 0; k < 5; k++)
            if (n.op == bin[k]) return n.in.size() == 2 ? k : -1;
        if (n.op == "Sqrt") return n.in.size() == 1 ? 16 : -1;
        if (n.op == "Erf") return n.in.size() == 1 ? 17 : -1;
        return -1;
    }
    bool chain(int i0, GNode *f, std::vector<int> *nodes) {
        if (used[i0] || chain_op(N(i0)) < 0) return false;
        std::vector<std::string> ins;
        std::vector<int64_t> ops, operands;
        auto input_index = [&](const std::string &nm) {
            for (size_t j = 0; j < ins.size(); j++)
                if (ins[j] == nm) return (int)j;
            ins.push_back(nm);
            return (int)ins.size() - 1;
        };
        const int op0 = chain_op(N(i0));
        input_index(N(i0).in[0]);
        ops.push_back(op0);
        operands.push_back(op0 < 16 ? input_index(N(i0).in[1]) : 0);
        std::vector<int> chain_nodes = {i0};
        int cur = i0;
        while ((int)ops.size() < kChainMaxOpsG) {
            const std::string &v = N(cur).out[0];
            const int c = only_consumer(v);
            if (c < 0 || used[c]) break;
            const int op = chain_op(N(c));
            if (op < 0) break;
            int64_t operand = 0;
            if (op < 16) {
                const bool left = N(c).in[0] == v, right = N(c).in[1] == v;
                if (left == right) break;  // both operands are the chain value, or neither
                const std::string &other = left ? N(c).in[1] : N(c).in[0];
                const size_t before = ins.size();
                const int j = input_index(other);
                if ((int)ins.size() > kChainMaxInG) {
                    ins.resize(before);
                    break;
                }
                operand = left ? j : -(j + 1);
            }
            ops.push_back(op);
            operands.push_back(operand);
            chain_nodes.push_back(c);
            cur = c;
        }
        if (chain_nodes.size() < 2) return false;
        *nodes = chain_nodes;
        f->op = "ElementwiseChain";
        f->in = ins;
        f->out = N(cur).out;
        Attr a;
        a.kind = kAttrInts;
        a.ints = ops;
        f->attrs["ops"] = a;
        a.ints = operands;
        f->attrs["operands"] = a;
        return true;
    }

    int run() {
        index();
        int fused = 0;
        std::vector<std::pair<int, GNode>> placed;  // fused node at the index of its last original
        auto place = [&](GNode &f, std::vector<int> &nodes) {
            std::sort(nodes.begin(), nodes.end());
            for (int k : nodes) {
                used[k] = true;
                f.fused_from.push_back(N(k));
            }
            f.name = N(nodes.back()).name;
            f.index = N(nodes.back()).index;
            placed.push_back({nodes.back(), f});
            fused++;
        };
        // the specific subgraphs first, then elementwise chains among the remaining nodes
        for (int i = 0; i < (int)g->nodes.size(); i++) {
            if (used[i]) continue;
            GNode f;
            std::vector<int> nodes;
            if (layernorm(i, &f, &nodes) || gelu(i, &f, &nodes) || add_softmax(i, &f, &nodes) ||
                matmul_add(i, &f, &nodes) || matmul_permuted(i, &f, &nodes))
                place(f, nodes);
        }
        for (int i = 0; i < (int)g->nodes.size(); i++) {
            GNode f;
            std::vector<int> nodes;
            if (chain(i, &f, &nodes)) place(f, nodes);
        }
        if (!fused) return 0;
        std::vector<GNode> out;
        for (int i = 0; i < (int)g->nodes.size(); i++) {
            for (auto &p : placed)
                if (p.first == i) out.push_back(p.second);
            if (!used[i]) out.push_back(g->nodes[i]);
        }
        g->nodes.swap(out);
        const int grouped = group_projections();
        const int merged = merge_layernorms();
        return fused - grouped - merged - merge_attention();
    }

    // A MatMulAdd whose result only a LayerNormDecomposed reads (x): one MatMulAddLayerNorm node (inputs A, W,
    // bias, [residual,] gamma, beta), which normalises the rows in the split product's ordered sum when the
    // product splits, else runs the two fused kernels.  Placed where the LayerNorm was.  Returns the nodes
    // removed.
    int merge_layernorms() {
        index();
        std::set<int> drop;
        for (int i = 0; i < (int)g->nodes.size(); i++) {
            const GNode &m = g->nodes[i];
            if (m.op != "MatMulAdd" || m.out.size() != 1 || (m.in.size() != 3 && m.in.size() != 4)) continue;
            const int c = only_consumer(m.out[0]);
            if (c < 0 || drop.count(c)) continue;
            const GNode &l = g->nodes[c];
            if (l.op != "LayerNormDecomposed" || l.in.size() != 3 || l.in[0] != m.out[0]) continue;
            GNode f;
            f.op = "MatMulAddLayerNorm";
            f.name = l.name;
            f.index = l.index;
            f.in = m.in;
            f.in.push_back(l.in[1]);
            f.in.push_back(l.in[2]);
            f.out = l.out;
            f.attrs = l.attrs;
            f.fused_from = m.fused_from;
            f.fused_from.insert(f.fused_from.end(), l.fused_from.begin(), l.fused_from.end());
            g->nodes[c] = f;
            drop.insert(i);
        }
        if (drop.empty()) return 0;
        std::vector<GNode> out;
        for (int i = 0; i < (int)g->nodes.size(); i++)
            if (!drop.count(i)) out.push_back(g->nodes[i]);
        g->nodes.swap(out);
        return (int)drop.size();
    }

    // MatMulPermuted (the scores, no output permutation) -> ScaleAddSoftmax / AddSoftmax -> MatMulPermuted (the
    // context, the probabilities its left operand as they are), each intermediate read only by the next: one
    // Attention node (inputs Q, K, V, mask[, scale]) that runs the three in one launch where every head fits
    // and else runs them as they are (its fused_from).  Placed where the context was.  Returns the nodes
    // removed.
    int merge_attention() {
        index();
        std::set<int> drop;
        for (int i = 0; i < (int)g->nodes.size(); i++) {
            const GNode &sn = g->nodes[i];
            if (sn.op != "MatMulPermuted" || sn.in.size() != 2 || sn.out.size() != 1 || sn.attrs.count("y_perm"))
                continue;
            const std::string &scores = sn.out[0];
            const int c = only_consumer(scores);
            if (c < 0 || drop.count(c)) continue;
            const GNode &sm = g->nodes[c];
            std::string mask, scale;
            if (sm.op == "ScaleAddSoftmax" && sm.in.size() == 3 && sm.in[0] == scores && sm.in[2] != scores) {
                scale = sm.in[1];
                mask = sm.in[2];
            } else if (sm.op == "AddSoftmax" && sm.in.size() == 2 && (sm.in[0] == scores) != (sm.in[1] == scores)) {
                mask = sm.in[sm.in[0] == scores ? 1 : 0];
            } else {
                continue;
            }
            if (sm.out.size() != 1) continue;
            const int d = only_consumer(sm.out[0]);
            if (d < 0 || drop.count(d)) continue;
            const GNode &cn = g->nodes[d];
            if (cn.op != "MatMulPermuted" || cn.in.size() != 2 || cn.out.size() != 1 || cn.in[0] != sm.out[0] ||
                cn.in[1] == sm.out[0] || cn.attrs.count("a_perm"))
                continue;
            GNode f;
            f.op = "Attention";
            f.name = cn.name;
            f.index = cn.index;
            f.in = {sn.in[0], sn.in[1], cn.in[1], mask};
            if (!scale.empty()) f.in.push_back(scale);
            f.out = cn.out;
            auto copy = [&](const GNode &from, const char *key, const char *as) {
                auto it = from.attrs.find(key);
                if (it != from.attrs.end()) f.attrs[as] = it->second;
            };
            copy(sn, "a_perm", "q_perm");
            copy(sn, "b_perm", "k_perm");
            copy(cn, "b_perm", "v_perm");
            copy(cn, "y_perm", "y_perm");
            copy(sm, "axis", "axis");
            copy(sm, "divide", "divide");
            f.fused_from = {sn, sm, cn};
            g->nodes[d] = f;
            drop.insert(i);
            drop.insert(c);
        }
        if (drop.empty()) return 0;
        std::vector<GNode> out;
        for (int i = 0; i < (int)g->nodes.size(); i++)
            if (!drop.count(i)) out.push_back(g->nodes[i]);
        g->nodes.swap(out);
        return (int)drop.size();
    }

    // MatMulAdd nodes (no residual) that share their input A, with constant Float weights [K, N] of one
    // shape and constant biases [N]: one MatMulAddGroup node over the stacked weights [G, K, N] and
    // biases [G, 1, N] -- one batched launch instead of G launches that each leave CUs idle (the Q, K, V
    // projections of an attention layer).  Its outputs are the G slices of one [G, M, N] product, each
    // bit-identical to its MatMulAdd.  Placed where the first of them was.  Returns the nodes removed.
    // a tensor name that no initializer, fused constant, graph input or output, or node input or output
    // (the original nodes of fused subgraphs included) uses: nodes may be unnamed, so a name derived from
    // a node's could repeat
    std::string fresh_name(const char *prefix) {
        std::set<std::string> taken(g->outputs.begin(), g->outputs.end());
        for (auto &kv : g->initializers) taken.insert(kv.first);
        for (auto &kv : g->fused_consts) taken.insert(kv.first);
        for (auto &in : g->inputs) taken.insert(in.name);
        std::vector<const GNode *> todo;
        for (auto &n : g->nodes) todo.push_back(&n);
        while (!todo.empty()) {
            const GNode *n = todo.back();
            todo.pop_back();
            taken.insert(n->in.begin(), n->in.end());
            taken.insert(n->out.begin(), n->out.end());
            for (auto &m : n->fused_from) todo.push_back(&m);
        }
        for (;;) {
            std::string s = prefix + std::to_string(g->fused_names++);
            if (!taken.count(s)) return s;
        }
    }

    int group_projections() {
        index();
        std::map<std::pair<std::string, std::pair<int64_t, int64_t>>, std::vector<int>> groups;
        for (int i = 0; i < (int)g->nodes.size(); i++) {
            const GNode &n = g->nodes[i];
            if (n.op != "MatMulAdd" || n.in.size() != 3 || n.out.size() != 1) continue;
            auto w = consts.find(n.in[1]), b = consts.find(n.in[2]);
            if (w == consts.end() || b == consts.end()) continue;
            const HostTensor &W = *w->second, &B = *b->second;
            if (W.dtype != LX_FLOAT || W.rank != 2 || B.dtype != LX_FLOAT || B.rank != 1 || B.dims[0] != W.dims[1] ||
                W.bytes.size() != (size_t)W.numel() * 4 || B.bytes.size() != (size_t)B.numel() * 4)
                continue;
            groups[{n.in[0], {W.dims[0], W.dims[1]}}].push_back(i);
        }
        std::set<int> drop;
        std::map<int, GNode> at;
        for (auto &kv : groups) {
            const std::vector<int> &ms = kv.second;
            if (ms.size() < 2) continue;
            const int64_t K = kv.first.second.first, Nn = kv.first.second.second, G = (int64_t)ms.size();
            GNode f;
            f.op = "MatMulAddGroup";
            f.name = g->nodes[ms[0]].name;
            f.index = g->nodes[ms[0]].index;
            auto w = std::make_shared<HostTensor>(), b = std::make_shared<HostTensor>();
            w->dtype = b->dtype = LX_FLOAT;
            w->rank = b->rank = 3;
            w->dims[0] = b->dims[0] = G;
            w->dims[1] = K;
            w->dims[2] = b->dims[2] = Nn;
            b->dims[1] = 1;
            for (int i : ms) {
                const GNode &n = g->nodes[i];
                const HostTensor &W = *consts[n.in[1]], &B = *consts[n.in[2]];
                w->bytes.insert(w->bytes.end(), W.bytes.begin(), W.bytes.end());
                b->bytes.insert(b->bytes.end(), B.bytes.begin(), B.bytes.end());
                f.out.push_back(n.out[0]);
                for (auto &o : n.fused_from) f.fused_from.push_back(o);
                if (n.fused_from.empty()) f.fused_from.push_back(n);
            }
            const std::string wn = fresh_name("__group_w_"), bn = fresh_name("__group_b_");
            g->fused_consts.push_back({wn, w});
            g->fused_consts.push_back({bn, b});
            f.in = {kv.first.first, wn, bn};
            at[ms[0]] = f;
            for (size_t k = 1; k < ms.size(); k++) drop.insert(ms[k]);
        }
        if (at.empty()) return 0;
        std::vector<GNode> out;
        for (int i = 0; i < (int)g->nodes.size(); i++) {
            if (drop.count(i)) continue;
            auto it = at.find(i);
            out.push_back(it != at.end() ? it->second : g->nodes[i]);
        }
        const int removed = (int)(g->nodes.size() - out.size());
        g->nodes.swap(out);
        return removed;
    }
};

// the names an execution can read from the initializers without a fallback: inputs of the current
// nodes, graph outputs, and graph inputs (which an initializer of the same name may serve)
std::set<std::string> live_names(const lx_graph *g) {
    std::set<std::string> live(g->outputs.begin(), g->outputs.end());
    for (auto &n : g->nodes) live.insert(n.in.begin(), n.in.end());
    for (auto &in : g->inputs) live.insert(in.name);
    return live;
}

// Uploads the initializers an execution reads and the fused constants.  An initializer that only the
// original nodes of a fused subgraph read (the separate Q / K / V weights once they are stacked) stays in
// host memory and is uploaded by the first lookup that needs it, i.e. when a fused node falls back to its
// original nodes.
int upload_initializers(lx_graph *g) {
    const std::set<std::string> live = live_names(g);
    for (auto *list : {&g->initializers, &g->fused_consts}) {
        for (auto &kv : *list) {
            if (g->init_dev.count(kv.first)) continue;
            if (list == &g->initializers && !live.count(kv.first)) continue;
            Value v;
            int st = value_from_host(kv.second, &v);
            if (st) return st;
            g->init_dev[kv.first] = v;
        }
    }
    return LX_OK;
}

bool same_dims(const lx_tensor &t, const GInput &in) {
    if (t.rank != in.rank) return false;
    for (int i = 0; i < t.rank; i++)
        if (t.dims[i] != in.dims[i]) return false;
    return true;
}

// ComputationalGraph.GetRequiredInputs (ComputationalGraph.cs:43-71): graph inputs not
// served by an initializer of the same dims and element type
std::vector<const GInput *> required_inputs(lx_graph *g, bool use_init) {
    std::vector<const GInput *> req;
    for (auto &in : g->inputs) {
        if (use_init) {
            auto it = g->init_dev.find(in.name);
            if (it != g->init_dev.end() && it->second.t.dtype == in.dtype && same_dims(it->second.t, in)) continue;
        }
        req.push_back(&in);
    }
    return req;
}

Value borrowed(const lx_tensor &t) {
    Value v;
    v.t = t;
    v.t.owns = 0;
    return v;
}

std::string desc(const std::string &name, const lx_tensor &t) {
    std::string s = name + ":" + lower(api_dtype_name(t.dtype)) + ":";
    for (int i = 0; i < t.rank; i++) s += (i ? "x" : "") + std::to_string(t.dims[i]);
    return s;
}

// whether a node can run a device-side check: Gather (indices), Div (integer operands), Cast
// (narrowing), or a fused node whose original nodes can
bool may_check(const GNode &n) {
    if (n.op == "Gather" || n.op == "Div" || n.op == "Cast") return true;
    for (const GNode &m : n.fused_from)
        if (may_check(m)) return true;
    return false;
}

// one 16-byte error record per node; a node clears its record when it launches a check, so
// graphs whose checking-capable nodes run on floats (Div) pay nothing
int prepare_check_slots(lx_graph *g) {
    bool any = false;
    for (const GNode &n : g->nodes) any = any || may_check(n);
    if (!any) return LX_OK;
    const int64_t want = 2 * (int64_t)std::max<size_t>(g->nodes.size(), 1);
    if (!g->check_slots.store || g->check_slots.t.dims[0] < want) {
        lx_tensor t;
        memset(&t, 0, sizeof t);
        int st = lx_tensor_alloc(LX_UINT64, 1, &want, &t);
        if (st) return st;
        g->check_slots = value_from_output(t);
    }
    return LX_OK;
}

// the first node before `limit` whose deferred device check failed: its index in *j, the status
// returned (lx_last_error holds the operator's message), 0 when none failed
int first_device_failure(lx_graph *g, const std::vector<DeferredCheck> &recs, int limit, int *j) {
    int last = -1;
    for (int k = 0; k < limit; k++)
        if (recs[k].kind != kCheckNone) last = k;
    if (last < 0) return LX_OK;
    std::vector<ErrFlags> flags(last + 1);
    const int rd = api_read_device(g->check_slots.t.data, flags.size() * sizeof(ErrFlags), flags.data());
    if (rd) {
        *j = last;
        return rd;
    }
    for (int k = 0; k <= last; k++) {
        if (recs[k].kind == kCheckNone) continue;
        const int st = api_check_status(recs[k], flags[k]);
        if (st) {
            *j = k;
            return st;
        }
    }
    return LX_OK;
}

// node j failed on the device: the outputs of j and of every later node are discarded (the reference
// never ran them) and the failure is reported as node j's
int report_device_failure(lx_graph *g, int j, int st) {
    const std::string m = lx_last_error();
    for (int k = j; k < (int)g->nodes.size(); k++)
        for (const std::string &o : g->nodes[k].out) g->values.erase(o);
    const GNode &nd = g->nodes[j];
    const int num = nd.index >= 0 ? nd.index + 1 : j + 1;
    return fail(st, fmt("Execution of node %d %s with op %s failed: %s", num, nd.name.c_str(), nd.op.c_str(), m.c_str()));
}

// ComputationalGraph.Execute (ComputationalGraph.cs:199-272).  recording != null: the execution is
// being captured into a HIP graph -- nothing may wait for the device, so the deferred checks are
// handed to the caller (who reads them after each replay) instead of read back here.
// Per-node timing of one execution for lx_graph_set_profiling: boundary events on the library stream,
// host time per node; finish() (also run by the destructor) waits for the last event and appends records.
// Every executed node appends one record.  If an event cannot be recorded, timing stops there: the nodes
// timed up to that point keep their device times and the later ones are appended with math_ms = 0.
struct NodeProfiler {
    lx_graph *g;
    bool on;
    bool timing = true;  // every node so far has its end event
    int used = 0;        // events recorded: the start event, then one per timed node
    std::vector<NodeProf> pend;
    NodeProfiler(lx_graph *gr, bool enabled) : g(gr), on(enabled) {}
    ~NodeProfiler() { finish(); }
    int event(hipEvent_t *e) {
        auto &ev = g->prof_events.ev;
        if (used == (int)ev.size()) {
            hipEvent_t x;
            hipError_t r = hipEventCreate(&x);
            if (r != hipSuccess) return fail(LX_ERR_HIP, fmt("hipEventCreate: %s", hipGetErrorString(r)));
            ev.push_back(x);
        }
        hipError_t r = hipEventRecord(ev[used], api_stream());
        if (r != hipSuccess) return fail(LX_ERR_HIP, fmt("hipEventRecord: %s", hipGetErrorString(r)));
        *e = ev[used++];
        return LX_OK;
    }
    int start() {
        if (!on) return LX_OK;
        hipEvent_t e;
        return event(&e);
    }
    void node_done(int k, const GNode &node, std::chrono::steady_clock::time_point h0) {
        if (!on) return;
        NodeProf p;
        p.node_id = node.index >= 0 ? node.index : k;
        p.node_index = k;
        p.op = node.op;
        p.host_ms = std::chrono::duration<double, std::milli>(std::chrono::steady_clock::now() - h0).count();
        hipEvent_t e;
        if (timing && event(&e) != LX_OK) timing = false;
        pend.push_back(p);
    }
    void finish() {
        if (!on || pend.empty()) return;
        on = false;
        auto &ev = g->prof_events.ev;
        const int timed = used - 1;  // nodes whose end event was recorded
        const bool ready = timed > 0 && hipEventSynchronize(ev[timed]) == hipSuccess;
        for (size_t i = 0; i < pend.size(); i++) {
            float ms = 0.0f, at = 0.0f;
            if (ready && (int)i < timed && hipEventElapsedTime(&ms, ev[i], ev[i + 1]) == hipSuccess &&
                hipEventElapsedTime(&at, ev[0], ev[i]) == hipSuccess) {
                pend[i].math_ms = ms;
                pend[i].start_ms = at;
            }
            g->profile.push_back(pend[i]);
        }
    }
};

int execute_impl(lx_graph *g, int32_t n, const char *const *names, const lx_tensor *inputs, int32_t use_initializers,
                 std::vector<DeferredCheck> *recording) {
    int st = upload_initializers(g);
    if (st) return st;
    g->values.clear();
    g->input_vals.clear();
    // ResolveInputs (ComputationalGraph.cs:73-130)
    auto req = required_inputs(g, use_initializers != 0);
    if ((size_t)n != req.size())
        return failure(fmt("%d user input(s) required for graph execution but %d specified.", (int)req.size(), n));
    for (size_t i = 0; i < req.size(); i++) {
        const lx_tensor *t = nullptr;
        if (names) {
            for (int k = 0; k < n; k++)
                if (names[k] && req[i]->name == names[k]) t = &inputs[k];
            if (!t) return failure(fmt("User inputs do not contain required input %s.", req[i]->name.c_str()));
        } else {
            t = &inputs[i];
        }
        if (t->rank != req[i]->rank || t->dtype != req[i]->dtype)
            return failure(fmt("Cannot use user input %s for required input %s. Tensor type or rank does not match.",
                               desc("", *t).c_str(), req[i]->name.c_str()));
        g->input_vals[req[i]->name] = borrowed(*t);
    }
    // liveness: the index of each name's last consumer
    std::map<std::string, int> last;
    for (int k = 0; k < (int)g->nodes.size(); k++)
        for (auto &nm : g->nodes[k].in) last[nm] = k;
    std::set<std::string> keep(g->outputs.begin(), g->outputs.end());
    // device checks (Gather indices, integer division, narrowing casts) are deferred: each node records
    // into its own slot and the slots are read back once, after the last node -- or when a node fails
    // on the host, to report an earlier device failure first, as node-by-node execution would
    const int nn = (int)g->nodes.size();
    if ((st = prepare_check_slots(g))) return st;
    std::vector<DeferredCheck> recs(nn);
    ErrFlags *slots = (ErrFlags *)g->check_slots.t.data;
    Exec X{g};
    // Profiler.StartNodeProfile / StopNodeProfile (ComputationalGraph.cs:241-243) on the device: an event at
    // every node boundary (not under capture, where events would become graph nodes), the records appended
    // once the last event has completed, on every way out of the loop
    NodeProfiler prof(g, g->profiling && !recording);
    if ((st = prof.start())) return st;
    for (int k = 0; k < nn; k++) {
        const GNode &node = g->nodes[k];
        std::vector<Value> outs;
        // a node that cannot check gets no slot: a check it did make would be read back at once
        api_defer_checks(slots && may_check(node) ? slots + k : nullptr, &recs[k]);
        const auto h0 = std::chrono::steady_clock::now();
        st = run_node(X, node, outs);
        api_defer_checks(nullptr, nullptr);
        prof.node_done(k, node, h0);
        if (!st && outs.size() != node.out.size())
            st = failure(fmt("The operation returned %d outputs but the graph node has %d outputs.", (int)outs.size(),
                             (int)node.out.size()));
        if (st) {
            std::string m = lx_last_error();
            int j = -1;
            const int dst = recording ? 0 : first_device_failure(g, recs, k, &j);
            if (dst) return report_device_failure(g, j, dst);
            // a fused node that fell back to its original nodes reports the one that failed, numbered
            // as in the graph before fusion, so the message is the unfused graph's
            const GNode &rep = X.failed ? *X.failed : node;
            const int num = rep.index >= 0 ? rep.index + 1 : k + 1;
            return fail(st, fmt("Execution of node %d %s with op %s failed: %s", num, rep.name.c_str(), rep.op.c_str(),
                                m.c_str()));
        }
        for (size_t i = 0; i < outs.size(); i++) g->values[node.out[i]] = outs[i];
        // intermediates whose last consumer has run go back to the pool (aliases keep their block)
        for (auto &nm : node.in)
            if (last[nm] == k && !keep.count(nm)) g->values.erase(nm);
    }
    if (recording) {
        *recording = recs;
        return LX_OK;
    }
    int j = -1;
    const int dst = first_device_failure(g, recs, nn, &j);
    if (dst) return report_device_failure(g, j, dst);
    return LX_OK;
}

}  // namespace

// ===========================================================================
namespace lx {
EventPool::~EventPool() {
    for (hipEvent_t e : ev) (void)hipEventDestroy(e);
}
}  // namespace lx

extern "C" {

int lx_graph_set_profiling(lx_graph *g, int32_t enabled) {
    if (!g) return failure("null graph");
    g->profiling = enabled != 0;
    return LX_OK;
}

int32_t lx_graph_profile_count(const lx_graph *g) { return g ? (int32_t)g->profile.size() : 0; }

static void copy_str(const std::string &s, char *buf, int32_t len);

int lx_graph_profile(const lx_graph *g, int32_t i, lx_node_profile *out) {
    if (!g || !out) return failure("null argument");
    if (i < 0 || i >= (int32_t)g->profile.size()) return failure("invalid profile record index");
    const NodeProf &p = g->profile[i];
    memset(out, 0, sizeof *out);
    out->node_id = p.node_id;
    out->node_index = p.node_index;
    copy_str(p.op, out->op, (int32_t)sizeof out->op);
    out->math_ms = p.math_ms;
    out->host_ms = p.host_ms;
    out->start_ms = p.start_ms;
    return LX_OK;
}

int lx_graph_profile_reset(lx_graph *g) {
    if (!g) return failure("null graph");
    g->profile.clear();
    return LX_OK;
}

int lx_graph_create(int64_t opset, lx_graph **out) {
    if (!out) return failure("out is null");
    *out = new lx_graph();
    (*out)->opset = opset;
    return LX_OK;
}

int lx_graph_free(lx_graph *g) {
    if (!g) return LX_OK;
    if (api_initialized()) (void)hipStreamSynchronize(api_stream());
    delete g;
    return LX_OK;
}

int lx_graph_add_input(lx_graph *g, const char *name, int32_t dtype, int32_t rank, const int64_t *dims) {
    if (!g || !name) return failure("null argument");
    g->capture.reset();
    if (rank < 0 || rank > LX_MAX_RANK) return fail(LX_ERR_NOT_SUPPORTED, fmt("At most %d axes are supported.", LX_MAX_RANK));
    GInput in;
    in.name = name;
    in.dtype = dtype;
    in.rank = rank;
    for (int i = 0; i < rank; i++) in.dims[i] = dims && dims[i] > 0 ? dims[i] : 0;
    g->inputs.push_back(in);
    return LX_OK;
}

int lx_graph_add_output(lx_graph *g, const char *name) {
    if (!g || !name) return failure("null argument");
    g->capture.reset();
    g->outputs.push_back(name);
    return LX_OK;
}

int lx_graph_add_initializer(lx_graph *g, const char *name, int32_t dtype, int32_t rank, const int64_t *dims,
                             const void *host, int64_t nbytes) {
    if (!g || !name) return failure("null argument");
    g->capture.reset();
    if (rank < 0 || rank > LX_MAX_RANK) return fail(LX_ERR_NOT_SUPPORTED, fmt("At most %d axes are supported.", LX_MAX_RANK));
    auto h = std::make_shared<HostTensor>();
    h->dtype = dtype;
    h->rank = rank;
    for (int i = 0; i < rank; i++) h->dims[i] = dims[i];
    const int64_t want = h->numel() * api_esize(dtype);
    if (!api_esize(dtype)) return fail(LX_ERR_NOT_SUPPORTED, fmt("Element type %s is not supported.", api_dtype_name(dtype)));
    if (nbytes != want || (want > 0 && !host))
        return failure(fmt("Initializer %s holds %lld bytes, its shape needs %lld.", name, (long long)nbytes, (long long)want));
    h->bytes.assign((const uint8_t *)host, (const uint8_t *)host + nbytes);
    for (auto *list : {&g->initializers, &g->fused_consts})
        for (auto &kv : *list)
            if (kv.first == name) return failure(fmt("An item with the same key has already been added. Key: %s", name));
    g->initializers.push_back({name, h});
    g->init_dev.erase(name);
    return LX_OK;
}

int lx_graph_add_node(lx_graph *g, const char *name, const char *op_type, int32_t n_in, const char *const *inputs,
                      int32_t n_out, const char *const *outputs, int32_t *index) {
    if (!g || !op_type || n_in < 0 || n_out < 0) return failure("null argument");
    g->capture.reset();
    GNode n;
    n.name = name ? name : "";
    n.op = op_type;
    for (int i = 0; i < n_in; i++) n.in.push_back(inputs[i] ? inputs[i] : "");
    for (int i = 0; i < n_out; i++) {
        n.out.push_back(outputs[i] ? outputs[i] : "");
        g->node_outputs.push_back(n.out.back());
    }
    n.index = (int)g->nodes.size();
    g->nodes.push_back(n);
    if (index) *index = (int32_t)g->nodes.size() - 1;
    return LX_OK;
}

static int node_at(lx_graph *g, int32_t node, const char *attr, GNode **n) {
    if (!g || !attr || node < 0 || node >= (int32_t)g->nodes.size()) return failure("invalid node index or attribute name");
    g->capture.reset();
    *n = &g->nodes[node];
    return LX_OK;
}

int lx_graph_set_attr_int(lx_graph *g, int32_t node, const char *attr, int64_t v) {
    GNode *n;
    int st = node_at(g, node, attr, &n);
    if (st) return st;
    Attr a;
    a.kind = kAttrInt;
    a.i = v;
    n->attrs[attr] = a;
    return LX_OK;
}

int lx_graph_set_attr_ints(lx_graph *g, int32_t node, const char *attr, const int64_t *v, int32_t cnt) {
    GNode *n;
    int st = node_at(g, node, attr, &n);
    if (st) return st;
    Attr a;
    a.kind = kAttrInts;
    a.ints.assign(v, v + (cnt > 0 ? cnt : 0));
    n->attrs[attr] = a;
    return LX_OK;
}

int lx_graph_set_attr_float(lx_graph *g, int32_t node, const char *attr, float v) {
    GNode *n;
    int st = node_at(g, node, attr, &n);
    if (st) return st;
    Attr a;
    a.kind = kAttrFloat;
    a.f = v;
    n->attrs[attr] = a;
    return LX_OK;
}

int lx_graph_set_attr_floats(lx_graph *g, int32_t node, const char *attr, const float *v, int32_t cnt) {
    GNode *n;
    int st = node_at(g, node, attr, &n);
    if (st) return st;
    Attr a;
    a.kind = kAttrFloats;
    a.floats.assign(v, v + (cnt > 0 ? cnt : 0));
    n->attrs[attr] = a;
    return LX_OK;
}

int lx_graph_set_attr_string(lx_graph *g, int32_t node, const char *attr, const char *v) {
    GNode *n;
    int st = node_at(g, node, attr, &n);
    if (st) return st;
    Attr a;
    a.kind = kAttrString;
    a.s = v ? v : "";
    n->attrs[attr] = a;
    return LX_OK;
}

int lx_graph_set_attr_tensor(lx_graph *g, int32_t node, const char *attr, int32_t dtype, int32_t rank,
                             const int64_t *dims, const void *host, int64_t nbytes) {
    GNode *n;
    int st = node_at(g, node, attr, &n);
    if (st) return st;
    if (rank < 0 || rank > LX_MAX_RANK) return fail(LX_ERR_NOT_SUPPORTED, fmt("At most %d axes are supported.", LX_MAX_RANK));
    auto h = std::make_shared<HostTensor>();
    h->dtype = dtype;
    h->rank = rank;
    for (int i = 0; i < rank; i++) h->dims[i] = dims[i];
    if (!api_esize(dtype)) return fail(LX_ERR_NOT_SUPPORTED, fmt("Element type %s is not supported.", api_dtype_name(dtype)));
    if (nbytes != h->numel() * api_esize(dtype) || (nbytes > 0 && !host))
        return failure("attribute tensor bytes do not match its shape");
    h->bytes.assign((const uint8_t *)host, (const uint8_t *)host + nbytes);
    Attr a;
    a.kind = kAttrTensor;
    a.t = h;
    n->attrs[attr] = a;
    return LX_OK;
}

int lx_graph_fuse(lx_graph *g, int32_t *n_fused) {
    if (!g) return failure("null graph");
    g->capture.reset();
    Fuser f;
    f.g = g;
    int k = f.run();
    if (n_fused) *n_fused = k;
    // device copies of initializers that no remaining node reads (uploaded at load) are dropped; a
    // fallback to the original nodes uploads them again on first use
    const std::set<std::string> live = live_names(g);
    for (auto it = g->init_dev.begin(); it != g->init_dev.end();) {
        bool keep = live.count(it->first) > 0;
        for (auto &kv : g->fused_consts) keep = keep || kv.first == it->first;
        it = keep ? std::next(it) : g->init_dev.erase(it);
    }
    return LX_OK;
}

int lx_graph_execute(lx_graph *g, int32_t n, const char *const *names, const lx_tensor *inputs,
                     int32_t use_initializers) {
    OpScope nested(nullptr);  // operators called by the graph are its nodes, not eager calls
    if (!api_initialized()) return fail(LX_ERR_NOT_INITIALIZED, "lx_init has not been called");
    if (!g || n < 0 || (n > 0 && !inputs)) return failure("null argument");
    return execute_impl(g, n, names, inputs, use_initializers, nullptr);
}

int lx_graph_capture(lx_graph *g, int32_t n, const char *const *names, const lx_tensor *inputs,
                     int32_t use_initializers) {
    OpScope nested(nullptr);  // operators called by the graph are its nodes, not eager calls
    if (!api_initialized()) return fail(LX_ERR_NOT_INITIALIZED, "lx_init has not been called");
    if (!g || n < 0 || (n > 0 && !inputs)) return failure("null argument");
    g->capture.reset();
    hipStream_t s = api_stream();
    hipStreamCaptureStatus cs = hipStreamCaptureStatusNone;
    if (hipStreamIsCapturing(s, &cs) != hipSuccess || cs != hipStreamCaptureStatusNone)
        return fail(LX_ERR_NOT_SUPPORTED, "The library stream is already being captured.");
    // one ordinary execution first: it uploads the constants, sizes the reduction workspace and
    // fills the pool's free lists, so the recording needs no upload and (mostly) no new block
    int st = execute_impl(g, n, names, inputs, use_initializers, nullptr);
    if (st) return st;
    hipError_t e = hipStreamSynchronize(s);
    if (e != hipSuccess) return fail(LX_ERR_HIP, fmt("capture: %s", hipGetErrorString(e)));
    g->values.clear();
    auto cap = std::make_unique<GraphCapture>();
    pool_record_begin();
    e = hipStreamBeginCapture(s, hipStreamCaptureModeRelaxed);
    if (e != hipSuccess) {
        pool_record_end();
        return fail(LX_ERR_HIP, fmt("hipStreamBeginCapture: %s", hipGetErrorString(e)));
    }
    t_capturing = true;
    st = execute_impl(g, n, names, inputs, use_initializers, &cap->recs);
    t_capturing = false;
    const std::string msg = st ? std::string(lx_last_error()) : std::string();
    e = hipStreamEndCapture(s, &cap->graph);
    cap->held = pool_record_end();
    if (!st && e != hipSuccess) st = fail(LX_ERR_HIP, fmt("hipStreamEndCapture: %s", hipGetErrorString(e)));
    if (!st) {
        e = hipGraphInstantiate(&cap->exec, cap->graph, nullptr, nullptr, 0);
        if (e != hipSuccess) st = fail(LX_ERR_HIP, fmt("hipGraphInstantiate: %s", hipGetErrorString(e)));
    }
    if (st) {  // nothing of the recording ran: its blocks go back as they were released
        if (!msg.empty()) fail(st, msg);
        g->values.clear();
        cap->held.clear();
        return st;
    }
    // the recording's blocks stay reserved, and every older device tensor it reads stays alive
    pool_hold(cap->held);
    cap->values = g->values;
    cap->input_vals = g->input_vals;
    for (auto &kv : g->init_dev) cap->pinned.push_back(kv.second);
    for (auto &kv : g->host_cache) cap->pinned.push_back(kv.second);
    cap->pinned.push_back(g->check_slots);
    g->capture = std::move(cap);
    return lx_graph_replay(g);
}

int lx_graph_replay(lx_graph *g) {
    OpScope nested(nullptr);  // operators called by the graph are its nodes, not eager calls
    if (!api_initialized()) return fail(LX_ERR_NOT_INITIALIZED, "lx_init has not been called");
    if (!g) return failure("null argument");
    if (!g->capture) return fail(LX_ERR_INVALID_ARGUMENT, "The graph has no captured execution.");
    GraphCapture &c = *g->capture;
    g->values = c.values;
    g->input_vals = c.input_vals;
    hipError_t e = hipGraphLaunch(c.exec, api_stream());
    if (e != hipSuccess) return fail(LX_ERR_HIP, fmt("hipGraphLaunch: %s", hipGetErrorString(e)));
    int j = -1;
    const int st = first_device_failure(g, c.recs, (int)c.recs.size(), &j);
    if (st) return report_device_failure(g, j, st);
    return LX_OK;
}

int lx_graph_release_capture(lx_graph *g) {
    if (!g) return failure("null argument");
    g->capture.reset();
    return LX_OK;
}

int lx_graph_execute_node(lx_graph *g, const char *node, int32_t n, const char *const *names, const lx_tensor *inputs,
                          int32_t use_initializers) {
    OpScope nested(nullptr);  // operators called by the graph are its nodes, not eager calls
    if (!api_initialized()) return fail(LX_ERR_NOT_INITIALIZED, "lx_init has not been called");
    if (!g || !node || n < 0 || (n > 0 && !inputs)) return failure("null argument");
    const GNode *nd = nullptr;
    for (auto &x : g->nodes)
        if (x.name == node) { nd = &x; break; }
    if (!nd) return failure(fmt("Could not find node %s in graph.", node));
    int st = upload_initializers(g);
    if (st) return st;
    g->values.clear();
    g->input_vals.clear();
    // ResolveNodeExecuteInputs (ComputationalGraph.cs:132-197)
    std::vector<std::string> req;
    for (auto &i : nd->in) {
        if (use_initializers && g->init_dev.count(i)) g->input_vals[i] = g->init_dev[i];
        else req.push_back(i);
    }
    if ((size_t)n != req.size())
        return failure(fmt("%d user input(s) required for node execution but %d specified.", (int)req.size(), n));
    for (size_t i = 0; i < req.size(); i++) {
        const lx_tensor *t = nullptr;
        if (names) {
            for (int k = 0; k < n; k++)
                if (names[k] && req[i] == names[k]) t = &inputs[k];
            if (!t) return failure(fmt("User inputs do not contain required input %s.", req[i].c_str()));
        } else {
            t = &inputs[i];
        }
        g->input_vals[req[i]] = borrowed(*t);
    }
    Exec X{g};
    std::vector<Value> outs;
    st = run_node(X, *nd, outs);
    if (!st && outs.size() != nd->out.size()) st = failure("output count mismatch");
    if (st) {
        std::string m = lx_last_error();
        return fail(st, fmt("Execution of node %s with op %s failed: %s.", nd->name.c_str(), nd->op.c_str(), m.c_str()));
    }
    for (size_t i = 0; i < outs.size(); i++) g->values[nd->out[i]] = outs[i];
    return LX_OK;
}

int lx_graph_output(lx_graph *g, const char *name, lx_tensor *out) {
    if (!g || !name || !out) return failure("null argument");
    auto it = g->values.find(name);
    if (it == g->values.end()) return failure(fmt("The graph holds no tensor named %s.", name));
    *out = it->second.t;
    out->owns = 0;
    return LX_OK;
}

int lx_graph_reset(lx_graph *g) {
    if (!g) return LX_OK;
    g->values.clear();
    g->input_vals.clear();
    return LX_OK;
}

int32_t lx_graph_node_count(const lx_graph *g) { return g ? (int32_t)g->nodes.size() : 0; }

static void copy_str(const std::string &s, char *buf, int32_t len) {
    if (!buf || len <= 0) return;
    size_t n = std::min((size_t)len - 1, s.size());
    memcpy(buf, s.data(), n);
    buf[n] = 0;
}

int lx_graph_node_info(const lx_graph *g, int32_t i, char *op_type, int32_t op_len, char *name, int32_t name_len) {
    if (!g || i < 0 || i >= (int32_t)g->nodes.size()) return failure("invalid node index");
    copy_str(g->nodes[i].op, op_type, op_len);
    copy_str(g->nodes[i].name, name, name_len);
    return LX_OK;
}

int32_t lx_graph_input_count(const lx_graph *g) { return g ? (int32_t)g->inputs.size() : 0; }

int lx_graph_input_info(const lx_graph *g, int32_t i, char *name, int32_t name_len, int32_t *dtype, int32_t *rank,
                        int64_t *dims) {
    if (!g || i < 0 || i >= (int32_t)g->inputs.size()) return failure("invalid input index");
    const GInput &in = g->inputs[i];
    copy_str(in.name, name, name_len);
    if (dtype) *dtype = in.dtype;
    if (rank) *rank = in.rank;
    if (dims)
        for (int k = 0; k < in.rank; k++) dims[k] = in.dims[k];
    return LX_OK;
}

int32_t lx_graph_initializer_count(const lx_graph *g) { return g ? (int32_t)g->initializers.size() : 0; }

int lx_graph_initializer_info(const lx_graph *g, int32_t i, char *name, int32_t name_len, int32_t *dtype,
                              int32_t *rank, int64_t *dims) {
    if (!g || i < 0 || i >= (int32_t)g->initializers.size()) return failure("invalid initializer index");
    const auto &kv = g->initializers[i];
    copy_str(kv.first, name, name_len);
    if (dtype) *dtype = kv.second->dtype;
    if (rank) *rank = kv.second->rank;
    if (dims)
        for (int k = 0; k < kv.second->rank; k++) dims[k] = kv.second->dims[k];
    return LX_OK;
}

int32_t lx_graph_output_count(const lx_graph *g) { return g ? (int32_t)g->outputs.size() : 0; }

int lx_graph_output_name(const lx_graph *g, int32_t i, char *name, int32_t name_len) {
    if (!g || i < 0 || i >= (int32_t)g->outputs.size()) return failure("invalid output index");
    copy_str(g->outputs[i], name, name_len);
    return LX_OK;
}

}  // extern "C"
