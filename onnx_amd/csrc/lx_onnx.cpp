// lx_onnx.cpp -- Model.Parse + Model.Load (src/Lokad.Onnx.Backend/Model.cs:14-63)
// for the device graph runtime: decodes an ONNX ModelProto from its protobuf
// wire encoding (field numbers of the public onnx.proto schema) and builds an
// lx_graph.  Initializer data follows TensorExtensions.GetTensorData /
// ToTensor (TensorUtil.cs:14-58): Int32, Int64, Float and Double from their
// typed fields or raw_data; other element types fail as they do there.
// Initializers are uploaded to HBM here when the library is initialised, else
// on the first execution.
#include <cstdarg>
#include <cstring>
#include <string>
#include <vector>

#include "../../include/lonnx.h"
#include "lx_graph.h"
#include "lx_internal.h"

using namespace lx;

namespace {

std::string fmt(const char *f, ...) {
    char buf[1024];
    va_list ap;
    va_start(ap, f);
    vsnprintf(buf, sizeof buf, f, ap);
    va_end(ap);
    return buf;
}

// Well-formed UTF-8 (RFC 3629): no overlong forms, no surrogates, nothing above U+10FFFF.
bool utf8_valid(const std::string &s) {
    const uint8_t *p = (const uint8_t *)s.data(), *e = p + s.size();
    while (p < e) {
        uint8_t c = *p++;
        if (c < 0x80) continue;
        int n;
        uint32_t cp, lo;
        if (c >= 0xc2 && c <= 0xdf) { n = 1; cp = c & 0x1f; lo = 0x80; }
        else if (c >= 0xe0 && c <= 0xef) { n = 2; cp = c & 0x0f; lo = 0x800; }
        else if (c >= 0xf0 && c <= 0xf4) { n = 3; cp = c & 0x07; lo = 0x10000; }
        else return false;
        if (e - p < n) return false;
        for (int i = 0; i < n; i++) {
            if ((p[i] & 0xc0) != 0x80) return false;
            cp = (cp << 6) | (p[i] & 0x3f);
        }
        p += n;
        if (cp < lo || cp > 0x10ffff || (cp >= 0xd800 && cp <= 0xdfff)) return false;
    }
    return true;
}

// ---- protobuf wire format -------------------------------------------------------
enum { kVarint = 0, kFixed64 = 1, kLen = 2, kFixed32 = 5 };

struct Reader {
    const uint8_t *p, *e;
    bool ok = true;
    Reader(const uint8_t *b, size_t n) : p(b), e(b + n) {}
    bool more() const { return ok && p < e; }
    uint64_t varint() {
        uint64_t v = 0;
        for (int s = 0; s < 70; s += 7) {
            if (p >= e) { ok = false; return 0; }
            uint8_t b = *p++;
            v |= (uint64_t)(b & 0x7f) << s;
            if (!(b & 0x80)) return v;
        }
        ok = false;
        return 0;
    }
    bool key(uint32_t *field, uint32_t *wt) {
        uint64_t k = varint();
        if (!ok) return false;
        *field = (uint32_t)(k >> 3);
        *wt = (uint32_t)(k & 7);
        return true;
    }
    Reader sub() {
        uint64_t n = varint();
        if (!ok || n > (uint64_t)(e - p)) { ok = false; return Reader(p, 0); }
        Reader r(p, (size_t)n);
        p += n;
        return r;
    }
    std::string str() {
        Reader r = sub();
        return std::string((const char *)r.p, (size_t)(r.e - r.p));
    }
    // a field of protobuf type string (names, op types, domains) holds UTF-8 text; other bytes
    // make the message malformed
    std::string text() {
        std::string s = str();
        if (!utf8_valid(s)) ok = false;
        return s;
    }
    uint32_t fixed32() {
        if (e - p < 4) { ok = false; return 0; }
        uint32_t v;
        memcpy(&v, p, 4);
        p += 4;
        return v;
    }
    uint64_t fixed64() {
        if (e - p < 8) { ok = false; return 0; }
        uint64_t v;
        memcpy(&v, p, 8);
        p += 8;
        return v;
    }
    void skip(uint32_t wt) {
        switch (wt) {
        case kVarint: varint(); break;
        case kFixed64: if (e - p < 8) ok = false; else p += 8; break;
        case kLen: sub(); break;
        case kFixed32: if (e - p < 4) ok = false; else p += 4; break;
        default: ok = false;
        }
    }
};

// repeated scalar fields arrive packed (one LEN record) or one record per value
void read_varints(Reader &r, uint32_t wt, std::vector<int64_t> *out) {
    if (wt == kLen) {
        Reader s = r.sub();
        while (s.more()) out->push_back((int64_t)s.varint());
        if (!s.ok) r.ok = false;
    } else {
        out->push_back((int64_t)r.varint());
    }
}
void read_fixed32s(Reader &r, uint32_t wt, std::vector<uint32_t> *out) {
    if (wt == kLen) {
        Reader s = r.sub();
        while (s.more()) out->push_back(s.fixed32());
        if (!s.ok) r.ok = false;
    } else {
        out->push_back(r.fixed32());
    }
}
void read_fixed64s(Reader &r, uint32_t wt, std::vector<uint64_t> *out) {
    if (wt == kLen) {
        Reader s = r.sub();
        while (s.more()) out->push_back(s.fixed64());
        if (!s.ok) r.ok = false;
    } else {
        out->push_back(r.fixed64());
    }
}

int bad(const char *what) { return api_set_error(LX_ERR_INVALID_ARGUMENT, fmt("Malformed ONNX model: %s.", what)); }

// TensorProto -> HostTensor (TensorExtensions.ToTensor, TensorUtil.cs:14-58)
int parse_tensor(Reader r, HostTensor *h, std::string *name) {
    std::vector<int64_t> dims, i64;
    std::vector<uint32_t> f32;
    std::vector<uint64_t> f64;
    std::string raw;
    int64_t dt = 0;
    uint32_t f, wt;
    while (r.more() && r.key(&f, &wt)) {
        switch (f) {
        case 1: read_varints(r, wt, &dims); break;
        case 2: dt = (int64_t)r.varint(); break;
        case 4: read_fixed32s(r, wt, &f32); break;   // float_data
        case 5: read_varints(r, wt, &i64); break;    // int32_data
        case 7: read_varints(r, wt, &i64); break;    // int64_data
        case 8: *name = r.text(); break;
        case 9: raw = r.str(); break;                // raw_data
        case 10: read_fixed64s(r, wt, &f64); break;  // double_data
        default: r.skip(wt);
        }
    }
    if (!r.ok) return bad("tensor");
    if (dims.size() > LX_MAX_RANK) return api_set_error(LX_ERR_NOT_SUPPORTED, fmt("At most %d axes are supported.", LX_MAX_RANK));
    h->dtype = (int32_t)dt;
    h->rank = (int32_t)dims.size();
    for (size_t i = 0; i < dims.size(); i++) h->dims[i] = dims[i];
    const int64_t n = h->numel();
    size_t es;
    switch (dt) {
    case LX_INT32: case LX_FLOAT: es = 4; break;
    case LX_INT64: case LX_DOUBLE: es = 8; break;
    case LX_BOOL: case LX_INT8: case LX_UINT8: case LX_INT16: case LX_UINT16: case LX_UINT32: case LX_UINT64:
    case 10: case 14: case 16:
        return api_set_error(LX_ERR_NOT_SUPPORTED,
                             fmt("Cannot get embedded tensor data of tensor element type %lld.", (long long)dt));
    default:
        return api_set_error(LX_ERR_NOT_SUPPORTED, fmt("Cannot convert tensor proto of element type %lld.", (long long)dt));
    }
    std::vector<uint8_t> bytes;
    const bool typed = (dt == LX_FLOAT && !f32.empty()) || ((dt == LX_INT32 || dt == LX_INT64) && !i64.empty()) ||
                       (dt == LX_DOUBLE && !f64.empty());
    if (typed) {
        bytes.resize(es * (dt == LX_FLOAT ? f32.size() : dt == LX_DOUBLE ? f64.size() : i64.size()));
        if (dt == LX_FLOAT) memcpy(bytes.data(), f32.data(), bytes.size());
        else if (dt == LX_DOUBLE) memcpy(bytes.data(), f64.data(), bytes.size());
        else if (dt == LX_INT64) memcpy(bytes.data(), i64.data(), bytes.size());
        else
            for (size_t i = 0; i < i64.size(); i++) {
                int32_t v = (int32_t)i64[i];
                memcpy(bytes.data() + 4 * i, &v, 4);
            }
    } else {
        bytes.assign(raw.begin(), raw.end());
        bytes.resize(bytes.size() / es * es);  // MemoryMarshal.Cast drops a partial element
    }
    if ((int64_t)(bytes.size() / es) != n)
        return api_set_error(LX_ERR_INVALID_ARGUMENT,
                             fmt("Length of memory (%lld) must match product of dimensions (%lld).",
                                 (long long)(bytes.size() / es), (long long)n));
    h->bytes.swap(bytes);
    return LX_OK;
}

// ValueInfoProto -> graph input / output (TensorExtensions.ToTensor(ValueInfoProto))
int parse_value_info(Reader r, GInput *v) {
    uint32_t f, wt;
    bool tensor_type = false;
    while (r.more() && r.key(&f, &wt)) {
        if (f == 1) { v->name = r.text(); continue; }
        if (f != 2) { r.skip(wt); continue; }
        Reader tp = r.sub();  // TypeProto
        uint32_t f2, w2;
        while (tp.more() && tp.key(&f2, &w2)) {
            if (f2 != 1) { tp.skip(w2); continue; }
            tensor_type = true;
            Reader tt = tp.sub();  // TypeProto.Tensor
            uint32_t f3, w3;
            while (tt.more() && tt.key(&f3, &w3)) {
                if (f3 == 1) { v->dtype = (int32_t)tt.varint(); continue; }
                if (f3 != 2) { tt.skip(w3); continue; }
                Reader sh = tt.sub();  // TensorShapeProto
                uint32_t f4, w4;
                while (sh.more() && sh.key(&f4, &w4)) {
                    if (f4 != 1) { sh.skip(w4); continue; }
                    Reader dm = sh.sub();  // Dimension: dim_value, or dim_param (DimValue 0)
                    int64_t dv = 0;
                    uint32_t f5, w5;
                    while (dm.more() && dm.key(&f5, &w5)) {
                        if (f5 == 1) dv = (int64_t)dm.varint();
                        else dm.skip(w5);
                    }
                    if (v->rank >= LX_MAX_RANK) return api_set_error(LX_ERR_NOT_SUPPORTED, "too many axes");
                    v->dims[v->rank++] = dv;
                    if (!dm.ok) sh.ok = false;
                }
                if (!sh.ok) tt.ok = false;
            }
            if (!tt.ok) tp.ok = false;
        }
        if (!tp.ok) r.ok = false;
    }
    if (!r.ok) return bad("value info");
    if (!tensor_type) return api_set_error(LX_ERR_NOT_SUPPORTED, fmt("The value info %s is not a tensor type.", v->name.c_str()));
    if (!api_esize(v->dtype))
        return api_set_error(LX_ERR_NOT_SUPPORTED,
                             fmt("Cannot convert value info proto of element type %d.", (int)v->dtype));
    return LX_OK;
}

// AttributeProto.Value (NodeUtil.cs:9-22)
int parse_attr(Reader r, std::string *name, Attr *a) {
    int64_t type = 0;
    float fv = 0;
    int64_t iv = 0;
    std::string sv;
    std::vector<uint32_t> floats;
    std::vector<int64_t> ints;
    std::shared_ptr<HostTensor> t;
    int tst = LX_OK;
    uint32_t f, wt;
    while (r.more() && r.key(&f, &wt)) {
        switch (f) {
        case 1: *name = r.text(); break;
        case 2: { uint32_t u = r.fixed32(); memcpy(&fv, &u, 4); break; }
        case 3: iv = (int64_t)r.varint(); break;
        case 4: sv = r.str(); break;
        case 5: {
            t = std::make_shared<HostTensor>();
            std::string tn;
            tst = parse_tensor(r.sub(), t.get(), &tn);
            break;
        }
        case 7: read_fixed32s(r, wt, &floats); break;
        case 8: read_varints(r, wt, &ints); break;
        case 20: type = (int64_t)r.varint(); break;
        default: r.skip(wt);
        }
    }
    if (!r.ok) return bad("attribute");
    static const char *tnames[] = {"Undefined", "Float", "Int", "String", "Tensor", "Graph", "Floats", "Ints",
                                   "Strings", "Tensors", "Graphs", "SparseTensor", "SparseTensors", "TypeProto",
                                   "TypeProtos"};
    switch (type) {
    case 1: a->kind = kAttrFloat; a->f = fv; return LX_OK;
    case 2: a->kind = kAttrInt; a->i = iv; return LX_OK;
    case 3: a->kind = kAttrString; a->s = sv; return LX_OK;
    case 4:
        if (tst) return tst;
        if (!t) return bad("tensor attribute without a tensor");
        a->kind = kAttrTensor;
        a->t = t;
        return LX_OK;
    case 6:
        a->kind = kAttrFloats;
        for (uint32_t u : floats) { float x; memcpy(&x, &u, 4); a->floats.push_back(x); }
        return LX_OK;
    case 7: a->kind = kAttrInts; a->ints = ints; return LX_OK;
    default:
        return api_set_error(LX_ERR_NOT_SUPPORTED,
                             fmt("Cannot convert attribute proto value of type %s.",
                                 (type >= 0 && type <= 14) ? tnames[type] : "Unknown"));
    }
}

int parse_node(Reader r, GNode *n) {
    uint32_t f, wt;
    while (r.more() && r.key(&f, &wt)) {
        switch (f) {
        case 1: n->in.push_back(r.text()); break;
        case 2: n->out.push_back(r.text()); break;
        case 3: n->name = r.text(); break;
        case 4: n->op = r.text(); break;
        case 5: {
            std::string an;
            Attr a;
            int st = parse_attr(r.sub(), &an, &a);
            if (st) return st;
            n->attrs[an] = a;
            break;
        }
        default: r.skip(wt);
        }
    }
    return r.ok ? LX_OK : bad("node");
}

int parse_graph(Reader r, lx_graph *g) {
    uint32_t f, wt;
    while (r.more() && r.key(&f, &wt)) {
        int st = LX_OK;
        switch (f) {
        case 1: {
            GNode n;
            st = parse_node(r.sub(), &n);
            if (!st) {
                for (auto &o : n.out) g->node_outputs.push_back(o);
                n.index = (int)g->nodes.size();
                g->nodes.push_back(n);
            }
            break;
        }
        case 2: g->name = r.text(); break;
        case 5: {
            auto h = std::make_shared<HostTensor>();
            std::string name;
            st = parse_tensor(r.sub(), h.get(), &name);
            if (!st) g->initializers.push_back({name, h});
            break;
        }
        case 11:
        case 12: {
            GInput v;
            st = parse_value_info(r.sub(), &v);
            if (!st) {
                if (f == 11) g->inputs.push_back(v);
                else g->outputs.push_back(v.name);
            }
            break;
        }
        default: r.skip(wt);
        }
        if (st) return st;
    }
    return r.ok ? LX_OK : bad("graph");
}

}  // namespace

extern "C" int lx_graph_load_onnx(const void *bytes, int64_t nbytes, lx_graph **out) {
    if (!bytes || nbytes <= 0 || !out) return api_set_error(LX_ERR_INVALID_ARGUMENT, "null or empty model buffer");
    *out = nullptr;
    lx_graph *g = new lx_graph();
    g->opset = -1;  // OpsetVersion("") fails when the default domain is not imported
    Reader r((const uint8_t *)bytes, (size_t)nbytes);
    uint32_t f, wt;
    int st = LX_OK;
    bool have_graph = false;
    while (!st && r.more() && r.key(&f, &wt)) {
        if (f == 7) {
            st = parse_graph(r.sub(), g);
            have_graph = true;
        } else if (f == 8) {  // OperatorSetIdProto
            Reader o = r.sub();
            std::string domain;
            int64_t version = 0;
            uint32_t f2, w2;
            while (o.more() && o.key(&f2, &w2)) {
                if (f2 == 1) domain = o.text();
                else if (f2 == 2) version = (int64_t)o.varint();
                else o.skip(w2);
            }
            if (!o.ok) st = bad("opset import");
            else if (domain.empty()) g->opset = version;
        } else {
            r.skip(wt);
        }
    }
    if (!st && !r.ok) st = bad("model");
    if (!st && !have_graph) st = bad("no graph");
    if (st) {
        delete g;
        return st;
    }
    // weights resident in HBM from load time when a device is available
    if (api_initialized()) {
        for (auto &kv : g->initializers) {
            lx_tensor t;
            memset(&t, 0, sizeof t);
            st = lx_tensor_alloc(kv.second->dtype, kv.second->rank, kv.second->dims, &t);
            if (!st && !kv.second->bytes.empty()) st = lx_tensor_upload(&t, kv.second->bytes.data(), (int64_t)kv.second->bytes.size());
            if (st) {
                lx_tensor_free(&t);
                delete g;
                return st;
            }
            Value v;
            v.t = t;
            v.t.owns = 0;
            v.store = std::make_shared<Storage>();
            v.store->ptr = t.data;
            v.host = kv.second;
            g->init_dev[kv.first] = v;
        }
    }
    *out = g;
    return LX_OK;
}
