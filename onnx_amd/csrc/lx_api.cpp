// lx_api.cpp -- host side of the C ABI declared in include/lonnx.h.
//
// Mirrors CPUExecutionProvider (src/Lokad.Onnx.Backend/CPUExecutionProvider.cs):
// the same validation order, the same dtype tables, the same failure kinds and
// messages (OpResult.cs:34-60, Node.cs:107-118), then hands the planned work to
// the gfx950 kernels.  Broadcasting is planned here once (ITensor.Broadcast,
// ITensor.cs:64-120) and executed by the kernels through stride-0 addressing.
#include <hip/hip_runtime.h>

#include <algorithm>
#include <chrono>
#include <cstdarg>
#include <cstdio>
#include <cstring>
#include <string>
#include <vector>

#include "../../include/lonnx.h"
#include "lx_internal.h"
#include "lx_kernels.h"
#include "lx_pool.h"

using namespace lx;

namespace {

// ---------------------------------------------------------------------------
// state
// ---------------------------------------------------------------------------
struct State {
    bool init = false;
    int device = -1;
    hipStream_t own_stream = nullptr;
    hipStream_t stream = nullptr;
    void *workspace = nullptr;
    int64_t ws_bytes = 0;
    ErrFlags *errs = nullptr;      // device
    bool errs_clean = false;       // errs holds its cleared state: the last eager check's publish reset it
    struct Mailbox *mail = nullptr;      // mapped, coherent pinned host memory
    struct Mailbox *mail_dev = nullptr;  // the same memory as the device addresses it
    uint64_t mail_seq = 0;
    uint64_t scan_seq = 0;               // the divisor and index scans' sequence (Mailbox::scan)
};
// Small device-to-host reads (error records) land here: a one-block kernel copies the words and
// then writes a sequence number, which the host polls.  One mailbox per library: calls are
// single-threaded, as the reference's provider is.
constexpr int64_t kMailWords = 8192;  // 64 KiB: 4096 error records
struct Mailbox {
    alignas(128) uint64_t seq;
    alignas(128) uint64_t words[kMailWords];
    alignas(128) uint64_t scan[kScanSlots];  // one verdict per block of a divisor or index scan
};

State g;
thread_local std::string g_err;

// ---- the allocation-free entry point's device memory ------------------------------------------
// One file-scope device array per GPU, loaded with the library's code object and held until the
// process ends.  Its name is a host-side stand-in: host code uses only the address hipGetSymbolAddress
// returns for the current device (scratch_addr), resolved once per device by lx_init.  Layout: split
// partials first, then two slots for the intermediates of multi-pass reductions.  Every allocation-free
// call on a GPU shares that GPU's array, which keeps the last call's contents (nothing in it needs to
// start at zero: partials and intermediates are written before they are read); calls that overlap on
// one GPU (other streams, other threads) race.
constexpr int64_t kScratchWsBytes = kReducePartialBytes;  // partials: the reduction planner caps them here
constexpr int64_t kScratchTempBytes = 1 << 20;  // per intermediate slot
constexpr int64_t kScratchBytes = kScratchWsBytes + 2 * kScratchTempBytes;
static __device__ __align__(256) unsigned char scratch[kScratchBytes];
constexpr int kMaxDevices = 64;
void *scratch_addr[kMaxDevices] = {nullptr};

struct NoAlloc {
    char *base;  // scratch_addr of the library's device
};

int set_err(int code, const char *fmt, ...) {
    char buf[1024];
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(buf, sizeof buf, fmt, ap);
    va_end(ap);
    g_err = buf;
    return code;
}

int hip_fail(hipError_t e, const char *what) {
    if (e == hipErrorOutOfMemory)
        return set_err(LX_ERR_OUT_OF_MEMORY, "%s: out of device memory", what);
    return set_err(LX_ERR_HIP, "%s: %s", what, hipGetErrorString(e));
}

#define HIPCHECK(call, what)                       \
    do {                                           \
        hipError_t e_ = (call);                    \
        if (e_ != hipSuccess) return hip_fail(e_, what); \
    } while (0)

#define REQUIRE_INIT()                                                                    \
    do {                                                                                  \
        if (!g.init) return set_err(LX_ERR_NOT_INITIALIZED, "lx_init has not been called"); \
    } while (0)

// ---------------------------------------------------------------------------
// dtype helpers (TensorElementType, Tensor.cs:31-50)
// ---------------------------------------------------------------------------
int64_t esize(int dt) {
    switch (dt) {
    case LX_FLOAT: case LX_INT32: case LX_UINT32: return 4;
    case LX_DOUBLE: case LX_INT64: case LX_UINT64: return 8;
    case LX_UINT8: case LX_INT8: case LX_BOOL: return 1;
    case LX_UINT16: case LX_INT16: return 2;
    default: return 0;
    }
}

const char *dtype_name(int dt) {
    switch (dt) {
    case 1: return "Float"; case 2: return "UInt8"; case 3: return "Int8"; case 4: return "UInt16";
    case 5: return "Int16"; case 6: return "Int32"; case 7: return "Int64"; case 8: return "String";
    case 9: return "Bool"; case 10: return "Float16"; case 11: return "Double"; case 12: return "UInt32";
    case 13: return "UInt64"; case 14: return "Complex64"; case 15: return "Complex128"; case 16: return "BFloat16";
    default: return "Unknown";
    }
}

std::string lower(std::string s) {
    for (auto &c : s) c = (char)tolower(c);
    return s;
}

// ITensor.TensorNameDesc (ITensor.cs:158) with an empty tensor name.
std::string name_desc(const lx_tensor *t) {
    std::string s = ":" + lower(dtype_name(t->dtype)) + ":";
    for (int i = 0; i < t->rank; i++) {
        if (i) s += "x";
        s += std::to_string(t->dims[i]);
    }
    return s;
}

// Tensor.PrintShape (Tensor.cs:1724)
std::string print_shape(const lx_tensor *t) {
    std::string s = "[";
    for (int i = 0; i < t->rank; i++) {
        if (i) s += ",";
        s += std::to_string(t->dims[i]);
    }
    return s + "]";
}

int64_t numel_of(int rank, const int64_t *dims) {
    int64_t n = 1;
    for (int i = 0; i < rank; i++) n *= dims[i];
    return n;
}

int64_t numel(const lx_tensor *t) { return numel_of(t->rank, t->dims); }

bool aligned16(const void *p) { return ((uintptr_t)p & 15) == 0; }

// whether the byte ranges [a, a + an) and [b, b + bn) share a byte
static bool overlaps(const void *a, int64_t an, const void *b, int64_t bn) {
    const uintptr_t x = (uintptr_t)a, y = (uintptr_t)b;
    return an > 0 && bn > 0 && x < y + (uintptr_t)bn && y < x + (uintptr_t)an;
}

// [lo, hi] of an integer element type (Bool as 0..1); false for floating types
bool int_range(int t, __int128 *lo, __int128 *hi) {
    switch (t) {
    case LX_BOOL: *lo = 0; *hi = 1; return true;
    case LX_UINT8: *lo = 0; *hi = UINT8_MAX; return true;
    case LX_INT8: *lo = INT8_MIN; *hi = INT8_MAX; return true;
    case LX_UINT16: *lo = 0; *hi = UINT16_MAX; return true;
    case LX_INT16: *lo = INT16_MIN; *hi = INT16_MAX; return true;
    case LX_UINT32: *lo = 0; *hi = UINT32_MAX; return true;
    case LX_INT32: *lo = INT32_MIN; *hi = INT32_MAX; return true;
    case LX_UINT64: *lo = 0; *hi = UINT64_MAX; return true;
    case LX_INT64: *lo = INT64_MIN; *hi = INT64_MAX; return true;
    default: return false;
    }
}

// whether every value of integer type src is a value of integer type dst
bool int_range_contains(int dst, int src) {
    __int128 dl, dh, sl, sh;
    return int_range(dst, &dl, &dh) && int_range(src, &sl, &sh) && dl <= sl && sh <= dh;
}

// Whether the fused LayerNorm kernel, which applies gamma / beta along X's last axis, computes what the
// reference's Mul / Add nodes compute (ITensor.Broadcast, ITensor.cs:92-117): the affine tensor must be
// [1, ..., 1, r] with r X's last dimension and no more axes than X.  Any other shape either broadcasts
// differently (gamma [r, 1] against X [r, r] runs down the columns) or cannot broadcast at all, and takes
// the node-by-node path, which gives the reference's result or its CannotBroadcast.
bool layernorm_affine_fits(const lx_tensor *t, const lx_tensor *X) {
    if (t->rank < 1 || t->rank > X->rank || t->dims[t->rank - 1] != X->dims[X->rank - 1]) return false;
    for (int i = 0; i < t->rank - 1; i++)
        if (t->dims[i] != 1) return false;
    return true;
}

// structural validity of a caller-provided tensor
int check_tensor(const lx_tensor *t, const char *name) {
    if (t->rank < 0 || t->rank > LX_MAX_RANK)
        return set_err(LX_ERR_NOT_SUPPORTED, "Tensor %s has rank %d; at most %d axes are supported.", name, t->rank,
                       LX_MAX_RANK);
    for (int i = 0; i < t->rank; i++)
        if (t->dims[i] < 0) return set_err(LX_ERR_INVALID_ARGUMENT, "Tensor %s has a negative dimension.", name);
    int64_t es = esize(t->dtype);
    int64_t bytes = numel(t) * (es ? es : 1);
    if (bytes > 0 && (t->data == nullptr || t->capacity < bytes))
        return set_err(LX_ERR_INVALID_ARGUMENT, "Tensor %s has no device storage for its %lld bytes.", name,
                       (long long)bytes);
    return LX_OK;
}

// ---- failure messages (OpResult.cs) ------------------------------------------------
int missing_input(const char *op, const char *name) {
    return set_err(LX_ERR_MISSING_INPUT, "The required input parameter %s is missing or null.", name);
}
int wrong_type_same(const char *name) {
    return set_err(LX_ERR_WRONG_INPUT_TYPE,
                   "The input tensor  for parameter %s has the wrong type: Input tensors must be of the same type..",
                   name);
}
int type_not_supported(const char *op, const char *name, const lx_tensor *t) {
    return set_err(LX_ERR_INPUT_TYPE_NOT_SUPPORTED,
                   "The type %s for input parameter %s is not supported for operation %s. ", dtype_name(t->dtype), name,
                   op);
}
int not_supported(const char *op) {
    return set_err(LX_ERR_NOT_SUPPORTED, "The operation %s is not supported by the backend.", op);
}
int cannot_broadcast(const lx_tensor *a, const lx_tensor *b) {
    return set_err(LX_ERR_CANNOT_BROADCAST, "The tensors %s and %s are not compatible for broadcasting.",
                   name_desc(a).c_str(), name_desc(b).c_str());
}
// .NET ArgumentException(message, paramName).Message as the reference raises it
int argument_error(const char *message, const char *param) {
    return set_err(LX_ERR_INVALID_ARGUMENT, "%s (Parameter '%s')", message, param);
}

// ---------------------------------------------------------------------------
// output preparation: allocate (Y->data == NULL) or validate caller storage
// ---------------------------------------------------------------------------
int prepare_output(lx_tensor *Y, int dtype, int rank, const int64_t *dims) {
    if (!Y) return set_err(LX_ERR_INVALID_ARGUMENT, "The output tensor handle is null.");
    int64_t bytes = numel_of(rank, dims) * esize(dtype);
    if (Y->data) {
        if (Y->capacity < bytes)
            return set_err(LX_ERR_BUFFER_TOO_SMALL, "Output storage holds %lld bytes, %lld needed.",
                           (long long)Y->capacity, (long long)bytes);
    } else {
        void *p = nullptr;
        size_t cap = 0;
        HIPCHECK(pool_alloc((size_t)bytes, &p, &cap, g.stream), "device allocation (output)");
        Y->data = p;
        Y->capacity = bytes;  // the tensor's own size, not the pool block's rounded one
        Y->owns = 1;
    }
    Y->dtype = dtype;
    Y->rank = rank;
    for (int i = 0; i < LX_MAX_RANK; i++) Y->dims[i] = i < rank ? dims[i] : 0;
    return LX_OK;
}

// Temporaries of multi-pass work: from the pool, or, while the stream is being
// captured into a HIP graph, stream-ordered allocations that the graph owns
// (a pooled block could be handed to other work while the graph still replays
// into it).
hipError_t alloc_temp(void **p, int64_t bytes, bool capturing) {
    if (capturing) return hipMallocAsync(p, bytes, g.stream);
    return pool_alloc((size_t)bytes, p, nullptr, g.stream);
}

void release_temp(void *p, bool capturing) {
    if (!p) return;
    if (capturing) (void)hipFreeAsync(p, g.stream);
    else (void)pool_release(p);
}

int ensure_workspace(int64_t bytes) {
    if (bytes <= g.ws_bytes) return LX_OK;
    HIPCHECK(hipStreamSynchronize(g.stream), "hipStreamSynchronize");
    if (g.workspace) (void)hipFree(g.workspace);
    g.workspace = nullptr;
    g.ws_bytes = 0;
    int64_t want = std::max<int64_t>(bytes, 1 << 20);
    HIPCHECK(hipMalloc(&g.workspace, want), "hipMalloc(workspace)");
    g.ws_bytes = want;
    return LX_OK;
}

// reads back the device error record (synchronises the stream)
// ---------------------------------------------------------------------------
// device-side checks: immediate (reset, launch, read back) or deferred into a
// caller's slot (api_defer_checks)
// ---------------------------------------------------------------------------
thread_local ErrFlags *t_defer_slot = nullptr;
thread_local DeferredCheck *t_defer_rec = nullptr;

int read_errs(ErrFlags *out);
int read_device(const void *src, size_t bytes, void *dst, bool reset_src = false);

// the error record a checking launch writes, cleared first (one small kernel, never a memset:
// the stream may be under capture): the deferred slot or the library's own record.  The library's
// record needs no clearing after an eager check, whose read-back clears it on the device.  A deferred
// slot is always cleared by a recorded kernel (a replay must not depend on eager history); an eager
// check on a stream under capture is refused before it records anything.
int check_begin(int kind, int dst, ErrFlags **errs) {
    *errs = t_defer_slot ? t_defer_slot : g.errs;
    if (t_defer_slot && t_defer_rec) {
        t_defer_rec->kind = kind;
        t_defer_rec->dst = dst;
    }
    if (!t_defer_slot) {
        // an eager check ends in a host read, which a stream under capture cannot make: refuse before
        // anything is recorded, so no recorded graph ever writes the library's record (a replay would
        // leave it dirty behind the host's back)
        hipStreamCaptureStatus cs = hipStreamCaptureStatusNone;
        HIPCHECK(hipStreamIsCapturing(g.stream, &cs), "hipStreamIsCapturing");
        if (cs != hipStreamCaptureStatusNone)
            return set_err(LX_ERR_NOT_SUPPORTED, "This operator checks its inputs on the device and reads the result "
                                                 "back; it cannot run on a stream under capture.");
        const bool clean = g.errs_clean;
        g.errs_clean = false;
        if (clean) return LX_OK;
    }
    HIPCHECK(launch_reset_errs(*errs, g.stream), "reset error flags");
    return LX_OK;
}

int check_status(int kind, int dst, const ErrFlags &e) {
    switch (kind) {
    case kCheckGather:
        if (e.first_ovf != ~0ull) return set_err(LX_ERR_INVALID_ARGUMENT, "Index was outside the bounds of the array.");
        return LX_OK;
    case kCheckDiv:
        if (e.first_dbz == ~0ull && e.first_ovf == ~0ull) return LX_OK;
        if (e.first_dbz <= e.first_ovf) return set_err(LX_ERR_DIVIDE_BY_ZERO, "Attempted to divide by zero.");
        return set_err(LX_ERR_OVERFLOW, "Arithmetic operation resulted in an overflow.");
    case kCheckCast: {
        if (e.first_ovf == ~0ull) return LX_OK;
        const char *what = "an Int32";
        switch (dst) {
        case LX_UINT8: what = "an unsigned byte"; break;
        case LX_INT8: what = "a signed byte"; break;
        case LX_INT16: what = "an Int16"; break;
        case LX_UINT16: what = "a UInt16"; break;
        case LX_UINT32: what = "a UInt32"; break;
        case LX_INT64: what = "an Int64"; break;
        case LX_UINT64: what = "a UInt64"; break;
        }
        return set_err(LX_ERR_OVERFLOW, "Value was either too large or too small for %s.", what);
    }
    default: return LX_OK;
    }
}

// after the launch: nothing when deferred, else the read-back verdict
int check_end(int kind, int dst) {
    if (t_defer_slot) return LX_OK;
    ErrFlags e;
    int st = read_errs(&e);
    if (st) return st;
    return check_status(kind, dst, e);
}

int read_errs(ErrFlags *out) {
    // the device-side checks end in a host read; a stream under capture cannot wait for it
    hipStreamCaptureStatus cs = hipStreamCaptureStatusNone;
    HIPCHECK(hipStreamIsCapturing(g.stream, &cs), "hipStreamIsCapturing");
    if (cs != hipStreamCaptureStatusNone)
        return set_err(LX_ERR_NOT_SUPPORTED, "This operator checks its inputs on the device and reads the result "
                                             "back; it cannot run on a stream under capture.");
    static_assert(sizeof(ErrFlags) % 8 == 0 && sizeof(ErrFlags) / 8 <= kMailWords, "the record takes the mailbox path");
    const int st = read_device(g.errs, sizeof(ErrFlags), out, true);
    if (st == LX_OK) g.errs_clean = true;
    return st;
}

// The host polls the mailbox's sequence number; every 50 us it asks the stream whether work is still
// pending, so a device fault ends the wait with that fault's error instead of spinning on.
int read_device(const void *src, size_t bytes, void *dst, bool reset_src) {
    if (bytes == 0) return LX_OK;
    if (bytes % 8 || bytes / 8 > (size_t)kMailWords) {
        HIPCHECK(hipMemcpyAsync(dst, src, bytes, hipMemcpyDeviceToHost, g.stream), "hipMemcpyAsync(read back)");
        HIPCHECK(hipStreamSynchronize(g.stream), "hipStreamSynchronize");
        return LX_OK;
    }
    const uint64_t want = ++g.mail_seq;
    HIPCHECK(launch_publish((const uint64_t *)src, (int64_t)(bytes / 8), g.mail_dev->words, &g.mail_dev->seq, want,
                            reset_src ? (uint64_t *)const_cast<void *>(src) : nullptr, g.stream),
             "launch publish");
    auto seen = [] { return __atomic_load_n(&g.mail->seq, __ATOMIC_ACQUIRE) == g.mail_seq; };
    const auto t0 = std::chrono::steady_clock::now();
    auto next_query = std::chrono::microseconds(50);
    for (uint32_t spin = 1; !seen(); spin++) {
        __builtin_ia32_pause();
        if (spin % 256) continue;
        const auto dt = std::chrono::steady_clock::now() - t0;
        if (dt < next_query) continue;
        next_query = std::chrono::duration_cast<std::chrono::microseconds>(dt) + std::chrono::microseconds(50);
        const hipError_t q = hipStreamQuery(g.stream);
        if (q == hipSuccess) {
            if (seen()) break;
            return set_err(LX_ERR_HIP, "reading back device results: the stream finished without publishing them");
        }
        if (q != hipErrorNotReady) return hip_fail(q, "reading back device results");
    }
    std::memcpy(dst, g.mail->words, bytes);
    return LX_OK;
}

// Waits for the `blocks` slots of the divisor or index scan `seq` (the watchdog of read_device: every 50 us it asks
// the stream whether work is pending) and ORs their verdict bits into *bits.
int wait_scan(int blocks, uint64_t seq, uint32_t *bits) {
    int seen = 0;
    uint32_t acc = 0;
    auto advance = [&] {
        while (seen < blocks) {
            const uint64_t v = __atomic_load_n(&g.mail->scan[seen], __ATOMIC_ACQUIRE);
            if ((v >> 2) != seq) return false;
            acc |= (uint32_t)(v & 3);
            seen++;
        }
        return true;
    };
    const auto t0 = std::chrono::steady_clock::now();
    auto next_query = std::chrono::microseconds(50);
    for (uint32_t spin = 1; !advance(); spin++) {
        __builtin_ia32_pause();
        if (spin % 256) continue;
        const auto dt = std::chrono::steady_clock::now() - t0;
        if (dt < next_query) continue;
        next_query = std::chrono::duration_cast<std::chrono::microseconds>(dt) + std::chrono::microseconds(50);
        const hipError_t q = hipStreamQuery(g.stream);
        if (q == hipSuccess) {
            if (advance()) break;
            return set_err(LX_ERR_HIP, "reading back device results: the stream finished without publishing them");
        }
        if (q != hipErrorNotReady) return hip_fail(q, "reading back device results");
    }
    *bits = acc;
    return LX_OK;
}

// ---------------------------------------------------------------------------
// broadcast planner
// ---------------------------------------------------------------------------
int plan(int ra, const int64_t *da, int rb, const int64_t *db, lx_bcast_plan *p) {
    memset(p, 0, sizeof *p);
    if (ra < 0 || rb < 0 || ra > LX_MAX_RANK || rb > LX_MAX_RANK) {
        p->status = LX_ERR_NOT_SUPPORTED;
        return set_err(LX_ERR_NOT_SUPPORTED, "At most %d axes are supported.", LX_MAX_RANK);
    }
    int64_t out[LX_MAX_RANK];
    int r;
    // ITensor.Broadcast shape rule (ITensor.cs:64-120)
    if (ra == 0 && rb != 0) {
        r = rb;
        for (int i = 0; i < r; i++) out[i] = db[i];
    } else if (rb == 0 && ra != 0) {
        r = ra;
        for (int i = 0; i < r; i++) out[i] = da[i];
    } else {
        r = std::max(ra, rb);
        for (int i = 0; i < r; i++) {
            int ia = i - r + ra, ib = i - r + rb;
            if (i < r - ra) out[i] = db[ib];
            else if (i < r - rb) out[i] = da[ia];
            else if (da[ia] == db[ib]) out[i] = da[ia];
            else if (da[ia] == 1) out[i] = db[ib];
            else if (db[ib] == 1) out[i] = da[ia];
            else {
                p->status = LX_ERR_CANNOT_BROADCAST;
                return LX_ERR_CANNOT_BROADCAST;
            }
        }
    }
    p->out_rank = r;
    for (int i = 0; i < r; i++) p->out_dims[i] = out[i];
    p->numel = numel_of(r, out);
    if (p->numel == 0) {
        p->kind = LX_PLAN_EMPTY;
        return LX_OK;
    }
    // per-operand strides in the output frame (0 on broadcast or missing axes)
    int64_t sa[LX_MAX_RANK], sb[LX_MAX_RANK];
    auto fill = [&](int ro, const int64_t *dd, int64_t *s) {
        int64_t st = 1;
        for (int i = r - 1; i >= 0; i--) {
            int k = i - (r - ro);
            if (k < 0) { s[i] = 0; continue; }
            s[i] = (dd[k] == 1 && out[i] != 1) ? 0 : st;
            st *= dd[k];
        }
    };
    fill(ra, da, sa);
    fill(rb, db, sb);
    // drop size-1 axes, merge adjacent axes that stay contiguous for both operands
    int64_t cd[LX_MAX_RANK], ca[LX_MAX_RANK], cb[LX_MAX_RANK];
    int n = 0;
    for (int i = r - 1; i >= 0; i--) {  // inner to outer
        if (out[i] == 1) continue;
        if (n > 0 && sa[i] == ca[n - 1] * cd[n - 1] && sb[i] == cb[n - 1] * cd[n - 1]) {
            cd[n - 1] *= out[i];
            continue;
        }
        cd[n] = out[i];
        ca[n] = sa[i];
        cb[n] = sb[i];
        n++;
    }
    if (n == 0) {  // single element
        cd[0] = 1;
        ca[0] = 1;
        cb[0] = 1;
        n = 1;
    }
    p->rank = n;
    for (int i = 0; i < n; i++) {  // store outermost first
        p->dims[i] = cd[n - 1 - i];
        p->a_strides[i] = ca[n - 1 - i];
        p->b_strides[i] = cb[n - 1 - i];
    }
    if (n == 1) {
        if (p->a_strides[0] == 1 && p->b_strides[0] == 1) p->kind = LX_PLAN_SAME;
        else if (p->a_strides[0] == 0) p->kind = LX_PLAN_SCALAR_A;
        else p->kind = LX_PLAN_SCALAR_B;
        if (p->dims[0] == 1) p->kind = LX_PLAN_SAME;
    } else {
        p->kind = LX_PLAN_ND;
    }
    p->status = LX_OK;
    return LX_OK;
}

// NdLayout over the outer axes of a plan (innermost outer axis first)
void nd_layout(const lx_bcast_plan &p, int vec, NdLayout &L, BinArgs *big) {
    memset(&L, 0, sizeof L);
    const int R = p.rank;
    L.nouter = R - 1;
    for (int d = 0; d < R - 1; d++) {
        int ax = R - 2 - d;
        L.odiv[d] = make_fastdiv((uint32_t)std::min<int64_t>(p.dims[ax], 0x7fffffff));
        L.a_str[d] = p.a_strides[ax];
        L.b_str[d] = p.b_strides[ax];
        if (big) big->nd_osize[d] = p.dims[ax];
    }
    L.inner = p.dims[R - 1];
    int64_t inner_v = p.dims[R - 1] / vec;
    L.inner_v = make_fastdiv((uint32_t)std::min<int64_t>(inner_v, 0x7fffffff));
    if (big) big->nd_inner_vn = inner_v;
}

// ---------------------------------------------------------------------------
// binary operators (CPUExecutionProvider.cs:82-236)
// ---------------------------------------------------------------------------
bool binary_dtype_ok(int op, int dt) {
    switch (op) {
    case kAdd: case kSub: case kMul: case kDiv:
        return dt == LX_UINT8 || dt == LX_INT32 || dt == LX_INT64 || dt == LX_FLOAT || dt == LX_DOUBLE;
    case kPow: return dt == LX_FLOAT || dt == LX_DOUBLE;
    default: return false;
    }
}

const char *binop_name(int op) {
    switch (op) {
    case kAdd: return "Add"; case kSub: return "Sub"; case kMul: return "Mul"; case kDiv: return "Div";
    case kPow: return "Pow"; default: return "?";
    }
}

int run_binary(int op, const lx_tensor *A, const lx_tensor *B, lx_tensor *Y) {
    REQUIRE_INIT();
    const char *opn = binop_name(op);
    if (!A) return missing_input(opn, "A");
    if (!B) return missing_input(opn, "B");
    if (A->dtype != B->dtype) return wrong_type_same("B");
    int st;
    if ((st = check_tensor(A, "A")) || (st = check_tensor(B, "B"))) return st;
    lx_bcast_plan p;
    st = plan(A->rank, A->dims, B->rank, B->dims, &p);
    if (st == LX_ERR_CANNOT_BROADCAST) return cannot_broadcast(A, B);
    if (st) return st;
    if (!binary_dtype_ok(op, A->dtype)) return type_not_supported(opn, "A", A);
    if ((st = prepare_output(Y, A->dtype, p.out_rank, p.out_dims))) return st;
    if (p.kind == LX_PLAN_EMPTY) return LX_OK;

    BinArgs args;
    memset(&args, 0, sizeof args);
    args.op = op;
    args.dtype = A->dtype;
    args.a = A->data;
    args.b = B->data;
    args.y = Y->data;
    args.n = p.numel;
    const int64_t es = esize(A->dtype);
    const int64_t V = 16 / es;
    const bool al = aligned16(A->data) && aligned16(B->data) && aligned16(Y->data);
    switch (p.kind) {
    case LX_PLAN_SAME: args.layout = kSame; args.vec = al ? (int)V : 1; break;
    case LX_PLAN_SCALAR_A: args.layout = kScalarA; args.vec = aligned16(B->data) && aligned16(Y->data) ? (int)V : 1; break;
    case LX_PLAN_SCALAR_B: args.layout = kScalarB; args.vec = aligned16(A->data) && aligned16(Y->data) ? (int)V : 1; break;
    default: {
        args.layout = kNd;
        const int64_t inner = p.dims[p.rank - 1];
        args.a_inner = p.a_strides[p.rank - 1] != 0;
        args.b_inner = p.b_strides[p.rank - 1] != 0;
        args.a_once = args.b_once = 1;
        for (int i = 0; i < p.rank; i++) {
            if (p.a_strides[i] == 0) args.a_once = 0;
            if (p.b_strides[i] == 0) args.b_once = 0;
        }
        args.vec = (al && inner % V == 0) ? (int)V : 1;
        args.rag = V > 1 && al && inner % V != 0 && p.numel < (1ll << 31);
        nd_layout(p, args.vec, args.nd, &args);
        break;
    }
    }
    const bool int_div = op == kDiv && (A->dtype == LX_INT32 || A->dtype == LX_INT64 || A->dtype == LX_UINT8);
    ErrFlags *errs = g.errs;
    if (int_div && (st = check_begin(kCheckDiv, 0, &errs))) return st;
    // An eager call must know before it returns whether an element divides by zero or overflows
    // (CPUExecutionProvider.cs:177-206 throws from the call).  When the divisor is at most 1/16 of the
    // output, a scan of the divisor alone, queued before the quotient kernel, answers that: with no zero
    // and (signed) no minus one in B no element can fail, and the call returns as soon as the scan's
    // blocks have stored their verdicts, while the quotient kernel runs.  Otherwise the call waits for the
    // quotient kernel's own record, which names the first failing element.
    // (an output that overlaps the divisor could write a quotient over a divisor element the kernel has
    // still to read, after the scan has passed it: such calls wait for the kernel's record)
    const int64_t nb = numel(B);
    const bool prescan = int_div && !t_defer_slot && nb > 0 && nb * 16 <= p.numel &&
                         !overlaps(Y->data, p.numel * es, B->data, nb * es);
    int scan_blocks = 0;
    uint64_t scan_seq = 0;
    if (prescan) {
        scan_blocks = div_scan_blocks(nb, (int)es);
        scan_seq = ++g.scan_seq;
        HIPCHECK(launch_div_scan(A->dtype, B->data, nb, aligned16(B->data) ? 1 : 0, g.mail_dev->scan, scan_seq,
                                 g.stream),
                 "divisor scan");
    }
    HIPCHECK(launch_binary(args, errs, g.stream), opn);
    if (!int_div) return LX_OK;
    if (prescan) {
        uint32_t bits = 0;
        if ((st = wait_scan(scan_blocks, scan_seq, &bits))) return st;
        if (bits == 0) {
            // no element can fail, so the quotient kernel records nothing: the record stays cleared
            g.errs_clean = true;
            return LX_OK;
        }
    }
    return check_end(kCheckDiv, 0);
}

int run_unary(const char *opn, int op, const lx_tensor *X, const char *xname, lx_tensor *Y) {
    REQUIRE_INIT();
    if (!X) return missing_input(opn, xname);
    int st;
    if ((st = check_tensor(X, xname))) return st;
    if (X->dtype != LX_FLOAT && X->dtype != LX_DOUBLE) return type_not_supported(opn, xname, X);
    if ((st = prepare_output(Y, X->dtype, X->rank, X->dims))) return st;
    const int64_t n = numel(X);
    const int vec = aligned16(X->data) && aligned16(Y->data) ? 2 : 1;
    HIPCHECK(launch_unary(op, X->dtype, X->data, Y->data, n, vec, g.stream), opn);
    return LX_OK;
}

// ---------------------------------------------------------------------------
// reductions (CPUExecutionProvider.cs:623-678, TensorOps.cs:1561-1891)
// ---------------------------------------------------------------------------
int run_reduce(const char *opn, int op, const lx_tensor *X, const int64_t *axes, int32_t n_axes, int32_t keepdims,
               lx_tensor *Y, const NoAlloc *na = nullptr) {
    REQUIRE_INIT();
    if (na && (!Y || !Y->data))
        return set_err(LX_ERR_INVALID_ARGUMENT, "%s without allocation writes into the caller's storage: the output "
                                                "tensor must hold a device pointer.", opn);
    if (!X) return missing_input(opn, "data");
    int st;
    if ((st = check_tensor(X, "data"))) return st;
    const int dt = X->dtype;
    bool ok = (op == kMax) ? (dt == LX_FLOAT || dt == LX_DOUBLE)
                           : (dt == LX_FLOAT || dt == LX_DOUBLE || dt == LX_INT32 || dt == LX_INT64);
    if (!ok) return not_supported(opn);
    const int rank = X->rank;
    // axes validation as TensorOps (1566-1571): count, range, repeats, normalisation
    int ax[LX_MAX_RANK];
    int nax = 0;
    if (n_axes > 0) {
        if (!axes) return missing_input(opn, "axes");
        if (n_axes > rank) return argument_error("axes", "The number of axes specified must be less than the tensor rank.");
        for (int i = 0; i < n_axes; i++) {
            if (axes[i] >= rank) return argument_error("axes", "Each axis specified must be less than the rank of the tensor.");
            if (axes[i] < INT32_MIN || axes[i] > INT32_MAX)
                return set_err(LX_ERR_OVERFLOW, "Value was either too large or too small for an Int32.");
            for (int j = 0; j < i; j++)
                if (axes[j] == axes[i]) return argument_error("axes", "axes contains a repeated dimension.");
        }
        for (int i = 0; i < n_axes; i++) {
            int64_t a = axes[i] < 0 ? axes[i] + rank : axes[i];
            if (a < 0) return argument_error("axes", "Each axis specified must be less than the rank of the tensor.");
            for (int j = 0; j < i; j++)
                if (ax[j] == a) return argument_error("axes", "axes contains a repeated dimension.");
            ax[nax++] = (int)a;
        }
    } else {
        for (int i = 0; i < rank; i++) ax[nax++] = i;
    }
    bool red[LX_MAX_RANK] = {false};
    for (int i = 0; i < nax; i++) red[ax[i]] = true;
    const bool keep = keepdims < 0 ? true : keepdims != 0;
    int64_t odims[LX_MAX_RANK];
    int orank = 0;
    int64_t R = 1;
    for (int d = 0; d < rank; d++) {
        if (red[d]) {
            R *= X->dims[d];
            if (keep) odims[orank++] = 1;
        } else {
            odims[orank++] = X->dims[d];
        }
    }
    if ((st = prepare_output(Y, dt, orank, odims))) return st;
    const int64_t nout = numel_of(orank, odims);
    if (nout == 0) return LX_OK;
    const int64_t es = esize(dt);
    if (R == 0) {
        // folds over nothing: 0 (sum, max seed), mean float = 0/0
        uint64_t bits = 0;
        if (op == kMean && dt == LX_FLOAT) {
            float nanv = __builtin_nanf("");
            uint32_t u;
            memcpy(&u, &nanv, 4);
            bits = u;
        }
        HIPCHECK(launch_fill(Y->data, nout, (int)es, bits, g.stream), "fill");
        return LX_OK;
    }
    // collapse into groups of consecutive kept / reduced axes, size-1 axes dropped
    struct Grp { int64_t size; bool red; };
    std::vector<Grp> grps;
    for (int d = 0; d < rank; d++) {
        if (X->dims[d] == 1) continue;
        if (!grps.empty() && grps.back().red == red[d]) grps.back().size *= X->dims[d];
        else grps.push_back({X->dims[d], red[d]});
    }
    int nred = 0;
    for (auto &gp : grps) nred += gp.red;
    if (nred == 0) {  // reduced axes all of size 1: each output folds one element
        grps.clear();
        grps.push_back({1, true});
        grps.push_back({nout, false});
        nred = 1;
    }
    // passes, innermost reduced group first: planned in full before anything is launched
    struct Pass { int64_t outer, r, inner; int vec; int64_t ws, out_bytes; };
    std::vector<Pass> passes;
    bool src_aligned = aligned16(X->data);
    while (nred > 0) {
        int gi = -1;
        for (int i = (int)grps.size() - 1; i >= 0; i--)
            if (grps[i].red) { gi = i; break; }
        Pass ps;
        ps.outer = 1;
        ps.inner = 1;
        for (int i = 0; i < gi; i++) ps.outer *= grps[i].size;
        for (int i = gi + 1; i < (int)grps.size(); i++) ps.inner *= grps[i].size;
        ps.r = grps[gi].size;
        const int64_t V = 16 / es;
        // rows (inner == 1) of any length: an unaligned head and a tail go element by element
        ps.vec = (src_aligned && (ps.inner == 1 || ps.inner % V == 0)) ? (int)V : 1;
        ps.ws = reduce_workspace_bytes(dt, ps.outer, ps.r, ps.inner, ps.vec);
        ps.out_bytes = std::max<int64_t>(ps.outer * ps.inner * es, 16);
        passes.push_back(ps);
        src_aligned = true;  // temporaries are 256-byte aligned
        grps.erase(grps.begin() + gi);
        // merge neighbours that became adjacent kept groups
        std::vector<Grp> m;
        for (auto &gp : grps) {
            if (!m.empty() && m.back().red == gp.red) m.back().size *= gp.size;
            else m.push_back(gp);
        }
        grps.swap(m);
        nred--;
    }
    if (na) {  // every partial and temporary must fit the static scratch array
        for (size_t k = 0; k < passes.size(); k++) {
            if (passes[k].ws > kScratchWsBytes)
                return set_err(LX_ERR_NOT_SUPPORTED, "%s without allocation: the reduction needs %lld bytes of partials, "
                               "the scratch array holds %lld.", opn, (long long)passes[k].ws, (long long)kScratchWsBytes);
            if (k + 1 < passes.size() && passes[k].out_bytes > kScratchTempBytes)
                return set_err(LX_ERR_NOT_SUPPORTED, "%s without allocation: an intermediate of %lld bytes exceeds the "
                               "scratch array's %lld-byte slot.", opn, (long long)passes[k].out_bytes,
                               (long long)kScratchTempBytes);
        }
    }
    const void *src = X->data;
    void *tmp[2] = {nullptr, nullptr};
    hipStreamCaptureStatus cs = hipStreamCaptureStatusNone;
    (void)hipStreamIsCapturing(g.stream, &cs);
    const bool capturing = cs != hipStreamCaptureStatusNone;
    int result = LX_OK;
    for (size_t pass = 0; pass < passes.size(); pass++) {
        const Pass &ps = passes[pass];
        const bool last = pass + 1 == passes.size();
        void *dst;
        const int slot = pass & 1;
        if (last) {
            dst = Y->data;
        } else if (na) {
            dst = na->base + kScratchWsBytes + slot * kScratchTempBytes;
        } else {
            release_temp(tmp[slot], capturing);
            tmp[slot] = nullptr;
            hipError_t e = alloc_temp(&tmp[slot], ps.out_bytes, capturing);
            if (e != hipSuccess) { result = hip_fail(e, "device allocation (temporary)"); break; }
            dst = tmp[slot];
        }
        ReduceArgs ra;
        memset(&ra, 0, sizeof ra);
        ra.op = op;
        ra.dtype = dt;
        ra.x = src;
        ra.y = dst;
        ra.outer = ps.outer;
        ra.r = ps.r;
        ra.inner = ps.inner;
        ra.pre_div = pass == 0;
        ra.post_div = last;
        ra.r_total = R;
        ra.vec = ps.vec;
        if (na) {
            ra.workspace = na->base;
            ra.ws_bytes = kScratchWsBytes;
        } else {
            if ((result = ensure_workspace(ps.ws))) break;
            ra.workspace = g.workspace;
            ra.ws_bytes = g.ws_bytes;
        }
        hipError_t e = launch_reduce(ra, g.stream);
        if (e != hipSuccess) { result = hip_fail(e, opn); break; }
        src = dst;
    }
    for (void *t : tmp) release_temp(t, capturing);
    return result;
}

int run_softmax(const lx_tensor *X, const lx_tensor *mask, int32_t axis, int32_t has_axis, lx_tensor *Y,
                const char *opn, const lx_tensor *scale = nullptr, int scale_div = 1);
bool softmax_mask_layout(int rank, const int64_t *dims, const lx_tensor *mask, SoftmaxArgs &sa);

}  // namespace

// ---------------------------------------------------------------------------
// internal interface for the graph runtime (lx_internal.h)
// ---------------------------------------------------------------------------
namespace lx {
int api_set_error(int code, const std::string &message) {
    g_err = message;
    return code;
}
bool api_initialized() { return g.init; }
hipStream_t api_stream() { return g.stream; }
int64_t api_esize(int dtype) { return esize(dtype); }
const char *api_dtype_name(int dtype) { return dtype_name(dtype); }
void api_defer_checks(ErrFlags *slot, DeferredCheck *rec) {
    t_defer_slot = slot;
    t_defer_rec = rec;
}
int api_check_status(const DeferredCheck &rec, const ErrFlags &flags) { return check_status(rec.kind, rec.dst, flags); }
bool api_layernorm_affine_fits(const lx_tensor *t, const lx_tensor *X) { return layernorm_affine_fits(t, X); }
int api_read_device(const void *src, size_t bytes, void *dst) { return read_device(src, bytes, dst); }

// ---- eager operator profiling (lx_set_op_profiling) ----------------------------------------------------
// The device twin of the OpStage.Math stage the reference's operators open (Profiler.StartOpStage,
// Profiler.cs:71-80; CPUExecutionProvider.cs:92-103): while enabled, every operator call made from outside
// the library appends one record with two HIP events recorded on the library stream, before the call's
// first launch and after its last.  Nothing waits for them: a record's device time is read when the caller
// asks for it, so consecutive calls stay asynchronous and their intervals tile the stream.  Calls made by
// another operator or by a graph execution are not recorded (graphs have their own node profile).
namespace {
struct OpRecord {
    std::string op;
    hipEvent_t e0 = nullptr, e1 = nullptr;  // null: not timed (capture, or an event failed)
    double host_ms = 0.0;
};
struct OpProfiler {
    bool on = false;
    std::vector<OpRecord> recs;
    std::vector<hipEvent_t> spare;
    hipEvent_t take() {
        if (!spare.empty()) {
            hipEvent_t e = spare.back();
            spare.pop_back();
            return e;
        }
        hipEvent_t e = nullptr;
        return hipEventCreate(&e) == hipSuccess ? e : nullptr;
    }
    void give(hipEvent_t e) {
        if (e) spare.push_back(e);
    }
    void clear() {
        for (auto &r : recs) {
            give(r.e0);
            give(r.e1);
        }
        recs.clear();
    }
    void destroy() {
        clear();
        for (hipEvent_t e : spare) (void)hipEventDestroy(e);
        spare.clear();
    }
} g_ops;
thread_local int t_op_depth = 0;
}  // namespace

OpScope::OpScope(const char *op) {
    if (t_op_depth++ != 0 || !op || !g_ops.on || !g.init) return;
    active_ = true;
    op_ = op;
    h0_ = std::chrono::steady_clock::now();
    hipStreamCaptureStatus cs = hipStreamCaptureStatusNone;
    if (hipStreamIsCapturing(g.stream, &cs) != hipSuccess || cs != hipStreamCaptureStatusNone) return;
    e0_ = g_ops.take();
    if (e0_ && hipEventRecord(e0_, g.stream) != hipSuccess) {
        g_ops.give(e0_);
        e0_ = nullptr;
    }
}

OpScope::~OpScope() {
    t_op_depth--;
    if (!active_) return;
    OpRecord r;
    r.op = op_;
    if (e0_) {
        hipEvent_t e1 = g_ops.take();
        if (e1 && hipEventRecord(e1, g.stream) == hipSuccess) {
            r.e0 = e0_;
            r.e1 = e1;
        } else {
            g_ops.give(e0_);
            g_ops.give(e1);
        }
    }
    r.host_ms = std::chrono::duration<double, std::milli>(std::chrono::steady_clock::now() - h0_).count();
    g_ops.recs.push_back(std::move(r));
}
}  // namespace lx

// ===========================================================================
// C ABI
// ===========================================================================
extern "C" {

const char *lx_last_error(void) { return g_err.c_str(); }
const char *lx_version(void) { return "lonnx-mi355x 0.1 (gfx950)"; }
int64_t lx_dtype_size(int32_t dtype) { return esize(dtype); }

int lx_init(int32_t device) {
    if (g.init) {
        if (device == g.device) return LX_OK;
        return set_err(LX_ERR_INVALID_ARGUMENT, "The library is already initialised on device %d.", g.device);
    }
    int count = 0;
    HIPCHECK(hipGetDeviceCount(&count), "hipGetDeviceCount");
    if (device < 0 || device >= count)
        return set_err(LX_ERR_INVALID_ARGUMENT, "Device %d does not exist (%d devices).", device, count);
    if (device >= kMaxDevices)
        return set_err(LX_ERR_NOT_SUPPORTED, "Devices beyond %d are not supported.", kMaxDevices - 1);
    HIPCHECK(hipSetDevice(device), "hipSetDevice");
    // every resource below is released again if a later step fails, so a failed lx_init leaves nothing
    // behind and can be retried
    State s;
    auto undo = [&s](int st) {
        if (s.workspace) (void)hipFree(s.workspace);
        if (s.errs) (void)hipFree(s.errs);
        if (s.mail) (void)hipHostFree(s.mail);
        if (s.own_stream) (void)hipStreamDestroy(s.own_stream);
        return st;
    };
    hipError_t e;
    // a blocking stream: it orders with the legacy default stream, so work a caller
    // enqueues there (torch's default stream, events around library calls) sees ours
    if ((e = hipStreamCreateWithFlags(&s.own_stream, hipStreamDefault)) != hipSuccess)
        return undo(hip_fail(e, "hipStreamCreate"));
    if ((e = hipMalloc(&s.errs, sizeof(ErrFlags))) != hipSuccess) return undo(hip_fail(e, "hipMalloc(errors)"));
    if ((e = hipHostMalloc((void **)&s.mail, sizeof(Mailbox), hipHostMallocMapped | hipHostMallocCoherent)) != hipSuccess)
        return undo(hip_fail(e, "hipHostMalloc(mailbox)"));
    if ((e = hipHostGetDevicePointer((void **)&s.mail_dev, s.mail, 0)) != hipSuccess)
        return undo(hip_fail(e, "hipHostGetDevicePointer(mailbox)"));
    if (!scratch_addr[device]) {  // once per device, with the device current
        void *p = nullptr;
        if ((e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch))) != hipSuccess)
            return undo(hip_fail(e, "hipGetSymbolAddress(scratch)"));
        scratch_addr[device] = p;
    }
    if ((e = hipMalloc(&s.workspace, 1 << 20)) != hipSuccess) return undo(hip_fail(e, "hipMalloc(workspace)"));
    s.ws_bytes = 1 << 20;
    s.mail->seq = 0;
    for (int i = 0; i < kScanSlots; i++) s.mail->scan[i] = 0;
    s.stream = s.own_stream;
    s.device = device;
    s.init = true;
    g = s;
    return LX_OK;
}

int lx_shutdown(void) {
    if (!g.init) return LX_OK;
    (void)hipDeviceSynchronize();
    g_ops.destroy();
    (void)pool_trim(g.stream);
    if (g.workspace) (void)hipFree(g.workspace);
    if (g.errs) (void)hipFree(g.errs);

    if (g.mail) (void)hipHostFree(g.mail);
    if (g.own_stream) (void)hipStreamDestroy(g.own_stream);
    g = State();
    return LX_OK;
}

int lx_set_op_profiling(int32_t enabled) {
    g_ops.on = enabled != 0;
    return LX_OK;
}

int32_t lx_op_profile_count(void) { return (int32_t)g_ops.recs.size(); }

int lx_op_profile(int32_t i, lx_call_profile *out) {
    if (!out) return set_err(LX_ERR_INVALID_ARGUMENT, "null argument");
    if (i < 0 || i >= (int32_t)g_ops.recs.size()) return set_err(LX_ERR_INVALID_ARGUMENT, "invalid profile record index");
    const OpRecord &r = g_ops.recs[i];
    memset(out, 0, sizeof *out);
    snprintf(out->op, sizeof out->op, "%s", r.op.c_str());
    out->host_ms = r.host_ms;
    if (!r.e0) return LX_OK;
    HIPCHECK(hipEventSynchronize(r.e1), "hipEventSynchronize");
    float ms = 0.0f;
    HIPCHECK(hipEventElapsedTime(&ms, r.e0, r.e1), "hipEventElapsedTime");
    out->math_ms = ms;
    // the start offset from the first timed record since the last reset
    for (const OpRecord &f : g_ops.recs) {
        if (!f.e0) continue;
        float at = 0.0f;
        HIPCHECK(hipEventElapsedTime(&at, f.e0, r.e0), "hipEventElapsedTime");
        out->start_ms = at;
        break;
    }
    return LX_OK;
}

int lx_op_profile_reset(void) {
    g_ops.clear();
    return LX_OK;
}

int lx_set_stream(void *s) {
    REQUIRE_INIT();
    hipStream_t ns = s ? (hipStream_t)s : g.own_stream;
    // pooled blocks released by work on the old stream may be reused by work on
    // the new one: the old stream's work completes first
    if (ns != g.stream) {
        hipStreamCaptureStatus cs = hipStreamCaptureStatusNone;
        (void)hipStreamIsCapturing(g.stream, &cs);
        if (cs == hipStreamCaptureStatusNone) HIPCHECK(hipStreamSynchronize(g.stream), "hipStreamSynchronize");
    }
    g.stream = ns;
    return LX_OK;
}

void *lx_get_stream(void) { return (void *)g.stream; }

int lx_synchronize(void) {
    REQUIRE_INIT();
    HIPCHECK(hipStreamSynchronize(g.stream), "hipStreamSynchronize");
    return LX_OK;
}

int lx_tensor_alloc(int32_t dtype, int32_t rank, const int64_t *dims, lx_tensor *out) {
    REQUIRE_INIT();
    if (!out) return set_err(LX_ERR_INVALID_ARGUMENT, "out is null");
    if (!esize(dtype)) return set_err(LX_ERR_NOT_SUPPORTED, "Element type %s is not supported.", dtype_name(dtype));
    if (rank < 0 || rank > LX_MAX_RANK) return set_err(LX_ERR_NOT_SUPPORTED, "At most %d axes are supported.", LX_MAX_RANK);
    if (rank > 0 && !dims) return set_err(LX_ERR_INVALID_ARGUMENT, "dims is null");
    for (int i = 0; i < rank; i++)
        if (dims[i] < 0) return set_err(LX_ERR_INVALID_ARGUMENT, "negative dimension");
    memset(out, 0, sizeof *out);
    return prepare_output(out, dtype, rank, dims);
}

int lx_tensor_wrap(int32_t dtype, int32_t rank, const int64_t *dims, void *ptr, int64_t capacity, lx_tensor *out) {
    if (!out) return set_err(LX_ERR_INVALID_ARGUMENT, "out is null");
    if (!esize(dtype)) return set_err(LX_ERR_NOT_SUPPORTED, "Element type %s is not supported.", dtype_name(dtype));
    if (rank < 0 || rank > LX_MAX_RANK) return set_err(LX_ERR_NOT_SUPPORTED, "At most %d axes are supported.", LX_MAX_RANK);
    memset(out, 0, sizeof *out);
    out->dtype = dtype;
    out->rank = rank;
    for (int i = 0; i < rank; i++) out->dims[i] = dims[i];
    out->data = ptr;
    out->capacity = capacity;
    out->owns = 0;
    return check_tensor(out, "wrapped");
}

int lx_tensor_free(lx_tensor *t) {
    if (!t) return LX_OK;
    if (t->owns && t->data && !pool_release(t->data)) {
        if (g.init) (void)hipStreamSynchronize(g.stream);
        HIPCHECK(hipFree(t->data), "hipFree");
    }
    t->data = nullptr;
    t->capacity = 0;
    t->owns = 0;
    return LX_OK;
}

int lx_tensor_upload(lx_tensor *t, const void *host, int64_t nbytes) {
    REQUIRE_INIT();
    if (!t || (!host && nbytes > 0)) return set_err(LX_ERR_INVALID_ARGUMENT, "null argument");
    if (nbytes > t->capacity) return set_err(LX_ERR_BUFFER_TOO_SMALL, "upload larger than the tensor storage");
    if (nbytes == 0) return LX_OK;
    HIPCHECK(hipMemcpyAsync(t->data, host, nbytes, hipMemcpyHostToDevice, g.stream), "hipMemcpyAsync(H2D)");
    HIPCHECK(hipStreamSynchronize(g.stream), "hipStreamSynchronize");
    return LX_OK;
}

int lx_tensor_download(const lx_tensor *t, void *host, int64_t nbytes) {
    REQUIRE_INIT();
    if (!t || (!host && nbytes > 0)) return set_err(LX_ERR_INVALID_ARGUMENT, "null argument");
    if (nbytes > t->capacity) return set_err(LX_ERR_BUFFER_TOO_SMALL, "download larger than the tensor storage");
    if (nbytes == 0) return LX_OK;
    HIPCHECK(hipMemcpyAsync(host, t->data, nbytes, hipMemcpyDeviceToHost, g.stream), "hipMemcpyAsync(D2H)");
    HIPCHECK(hipStreamSynchronize(g.stream), "hipStreamSynchronize");
    return LX_OK;
}

int lx_tensor_reshape(const lx_tensor *t, int32_t rank, const int64_t *dims, lx_tensor *out) {
    if (!t || !out) return set_err(LX_ERR_INVALID_ARGUMENT, "null argument");
    if (rank < 0 || rank > LX_MAX_RANK) return set_err(LX_ERR_NOT_SUPPORTED, "At most %d axes are supported.", LX_MAX_RANK);
    if (numel_of(rank, dims) != numel(t))
        return set_err(LX_ERR_INVALID_ARGUMENT,
                       "Cannot reshape array due to mismatch in lengths, currently %lld would become %lld. "
                       "(Parameter 'dimensions')",
                       (long long)numel(t), (long long)numel_of(rank, dims));
    lx_tensor o = *t;
    o.rank = rank;
    for (int i = 0; i < LX_MAX_RANK; i++) o.dims[i] = i < rank ? dims[i] : 0;
    o.owns = 0;  // alias: the original keeps ownership
    *out = o;
    return LX_OK;
}

int lx_pool_trim(void) {
    REQUIRE_INIT();
    HIPCHECK(pool_trim(g.stream), "pool trim");
    return LX_OK;
}

int lx_pool_stats(int64_t *live_bytes, int64_t *cached_bytes) {
    pool_stats(live_bytes, cached_bytes);
    return LX_OK;
}

int lx_plan_broadcast(int32_t ra, const int64_t *da, int32_t rb, const int64_t *db, lx_bcast_plan *p) {
    if (!p) return set_err(LX_ERR_INVALID_ARGUMENT, "plan is null");
    int st = plan(ra, da, rb, db, p);
    if (st == LX_ERR_CANNOT_BROADCAST) set_err(st, "The shapes are not compatible for broadcasting.");
    return st;
}

int lx_Add(const lx_tensor *A, const lx_tensor *B, lx_tensor *Y) { OpScope prof("Add"); return run_binary(kAdd, A, B, Y); }
int lx_Sub(const lx_tensor *A, const lx_tensor *B, lx_tensor *Y) { OpScope prof("Sub"); return run_binary(kSub, A, B, Y); }
int lx_Mul(const lx_tensor *A, const lx_tensor *B, lx_tensor *Y) { OpScope prof("Mul"); return run_binary(kMul, A, B, Y); }
int lx_Div(const lx_tensor *A, const lx_tensor *B, lx_tensor *Y) { OpScope prof("Div"); return run_binary(kDiv, A, B, Y); }
int lx_Pow(const lx_tensor *A, const lx_tensor *B, lx_tensor *Y) { OpScope prof("Pow"); return run_binary(kPow, A, B, Y); }
int lx_Sqrt(const lx_tensor *A, lx_tensor *Y) { OpScope prof("Sqrt"); return run_unary("Sqrt", kSqrt, A, "A", Y); }
int lx_Erf(const lx_tensor *X, lx_tensor *Y) { OpScope prof("Erf"); return run_unary("Erf", kErf, X, "X", Y); }

int lx_Cast(const lx_tensor *X, int64_t to, lx_tensor *Y) {
    OpScope prof("Cast");
    REQUIRE_INIT();
    if (!X) return missing_input("Cast", "input");
    int st;
    if ((st = check_tensor(X, "input"))) return st;
    const int dst = (int)to;
    if (to != dst || !esize(dst))  // Float16 / BFloat16 / Complex / String targets (CPUExecutionProvider.cs:470-473)
        return set_err(LX_ERR_ATTRIBUTE_NOT_SUPPORTED,
                       "The attribute to with value %lld is not supported for operation Cast. ", (long long)to);
    if (!esize(X->dtype))
        return set_err(LX_ERR_INPUT_TYPE_NOT_SUPPORTED, "Object must implement IConvertible.");
    if ((st = prepare_output(Y, dst, X->rank, X->dims))) return st;
    const int64_t n = numel(X);
    if (n == 0) return LX_OK;
    const int src = X->dtype;
    // only conversions into an integer type can raise OverflowException, and only when the source's
    // values are not all inside the target's range (widening integer casts cannot)
    const bool can_overflow = dst != LX_FLOAT && dst != LX_DOUBLE && dst != LX_BOOL && src != dst &&
                              !int_range_contains(dst, src);
    const int vec = aligned16(X->data) && aligned16(Y->data) ? 2 : 1;
    ErrFlags *errs = g.errs;
    if (can_overflow && (st = check_begin(kCheckCast, dst, &errs))) return st;
    HIPCHECK(launch_cast(src, dst, X->data, Y->data, n, vec, errs, g.stream), "Cast");
    return can_overflow ? check_end(kCheckCast, dst) : LX_OK;
}

int lx_ReduceSum(const lx_tensor *X, const int64_t *axes, int32_t n_axes, int32_t keepdims, int32_t noop,
                 lx_tensor *Y) {
    OpScope prof("ReduceSum");
    (void)noop;  // read but unused by TensorOps.ReduceSum (TensorOps.cs:1615)
    return run_reduce("ReduceSum", kSum, X, axes, n_axes, keepdims, Y);
}

int lx_ReduceSum_noalloc(const lx_tensor *X, const int64_t *axes, int32_t n_axes, int32_t keepdims, int32_t noop,
                         lx_tensor *Y) {
    (void)noop;
    REQUIRE_INIT();
    NoAlloc na{(char *)scratch_addr[g.device]};
    return run_reduce("ReduceSum", kSum, X, axes, n_axes, keepdims, Y, &na);
}

int lx_ReduceMean(const lx_tensor *X, const int64_t *axes, int32_t n_axes, int32_t keepdims, int32_t noop,
                  lx_tensor *Y) {
    OpScope prof("ReduceMean");
    (void)noop;
    return run_reduce("ReduceMean", kMean, X, axes, n_axes, keepdims, Y);
}

int lx_ReduceMax(const lx_tensor *X, const int64_t *axes, int32_t n_axes, int32_t keepdims, lx_tensor *Y) {
    OpScope prof("ReduceMax");
    return run_reduce("ReduceMax", kMax, X, axes, n_axes, keepdims, Y);
}

int lx_Softmax(const lx_tensor *X, int32_t axis, int32_t has_axis, lx_tensor *Y) {
    OpScope prof("Softmax");
    return run_softmax(X, nullptr, axis, has_axis, Y, "Softmax");
}

int lx_AddSoftmax(const lx_tensor *S, const lx_tensor *mask, int32_t axis, lx_tensor *Y) {
    OpScope prof("AddSoftmax");
    REQUIRE_INIT();
    if (!S) return missing_input("Add", "A");
    if (!mask) return missing_input("Add", "B");
    return run_softmax(S, mask, axis, 1, Y, "Softmax");
}

int lx_ScaleAddSoftmax(const lx_tensor *S, const lx_tensor *scale, int32_t divide, const lx_tensor *mask, int32_t axis,
                       lx_tensor *Y) {
    OpScope prof("ScaleAddSoftmax");
    REQUIRE_INIT();
    if (!S) return missing_input(divide ? "Div" : "Mul", "A");
    if (!scale) return missing_input(divide ? "Div" : "Mul", "B");
    return run_softmax(S, mask, axis, 1, Y, "Softmax", scale, divide ? 1 : 0);
}

int lx_read_probe(const void *src, int64_t bytes, void *out, int64_t out_bytes) {
    REQUIRE_INIT();
    if (!src || !out || bytes < 0 || out_bytes < 4) return set_err(LX_ERR_INVALID_ARGUMENT, "invalid probe arguments");
    if (bytes % 16 || !aligned16(src)) return set_err(LX_ERR_INVALID_ARGUMENT, "the probe reads whole aligned 16-byte vectors");
    if ((uintptr_t)out % 4) return set_err(LX_ERR_INVALID_ARGUMENT, "the probe writes 32-bit words: out must be 4-byte aligned");
    HIPCHECK(launch_read_probe(src, bytes, (uint32_t *)out, out_bytes / 4, g.stream), "read probe");
    return LX_OK;
}

int lx_GeluErf(const lx_tensor *X, lx_tensor *Y) {
    OpScope prof("GeluErf");
    REQUIRE_INIT();
    if (!X) return missing_input("Div", "A");
    int st;
    if ((st = check_tensor(X, "A"))) return st;
    if (X->dtype != LX_FLOAT) {
        // node by node for other element types
        if (X->dtype != LX_DOUBLE) return type_not_supported("Erf", "X", X);
        double c[3] = {1.4142135623730951, 1.0, 0.5};
        lx_tensor k[3], t1{}, t2{}, t3{}, t4{};
        for (int i = 0; i < 3; i++) {
            if ((st = lx_tensor_alloc(LX_DOUBLE, 0, nullptr, &k[i]))) return st;
            if ((st = lx_tensor_upload(&k[i], &c[i], 8))) return st;
        }
        st = lx_Div(X, &k[0], &t1);
        if (!st) st = lx_Erf(&t1, &t2);
        if (!st) st = lx_Add(&t2, &k[1], &t3);
        if (!st) st = lx_Mul(X, &t3, &t4);
        if (!st) st = lx_Mul(&t4, &k[2], Y);
        for (lx_tensor *t : {&k[0], &k[1], &k[2], &t1, &t2, &t3, &t4}) lx_tensor_free(t);
        return st;
    }
    if ((st = prepare_output(Y, LX_FLOAT, X->rank, X->dims))) return st;
    const int vec = aligned16(X->data) && aligned16(Y->data) ? 4 : 1;
    HIPCHECK(launch_gelu_erf((const float *)X->data, (float *)Y->data, numel(X), vec, g.stream), "GeluErf");
    return LX_OK;
}

int lx_ElementwiseChain(const lx_tensor *const *inputs, int32_t n_in, const int32_t *ops, const int32_t *operands,
                        int32_t n_ops, lx_tensor *Y) {
    OpScope prof("ElementwiseChain");
    REQUIRE_INIT();
    if (!inputs || n_in < 1 || n_in > kChainMaxIn)
        return set_err(LX_ERR_INVALID_ARGUMENT, "An elementwise chain takes 1 to %d inputs.", kChainMaxIn);
    if (!ops || n_ops < 1 || n_ops > kChainMaxOps || (!operands && n_ops > 0))
        return set_err(LX_ERR_INVALID_ARGUMENT, "An elementwise chain takes 1 to %d instructions.", kChainMaxOps);
    int st;
    for (int j = 0; j < n_in; j++) {
        if (!inputs[j]) return missing_input("ElementwiseChain", "inputs");
        if ((st = check_tensor(inputs[j], "inputs"))) return st;
        if (inputs[j]->dtype != LX_FLOAT) return type_not_supported("ElementwiseChain", "inputs", inputs[j]);
    }
    // the shape after each instruction: binary steps broadcast as the separate operators do
    int rank = inputs[0]->rank;
    int64_t dims[LX_MAX_RANK];
    for (int i = 0; i < rank; i++) dims[i] = inputs[0]->dims[i];
    bool erf = false;
    for (int k = 0; k < n_ops; k++) {
        const int op = ops[k];
        if (op == kChainUnary + kSqrt || op == kChainUnary + kErf) {
            erf = erf || op == kChainUnary + kErf;
            continue;
        }
        if (op < kAdd || op > kPow) return set_err(LX_ERR_INVALID_ARGUMENT, "Instruction %d has an unknown op %d.", k, op);
        const int j = operands[k] < 0 ? -operands[k] - 1 : operands[k];
        if (j >= n_in) return set_err(LX_ERR_INVALID_ARGUMENT, "Instruction %d reads input %d of %d.", k, j, n_in);
        lx_bcast_plan bp;
        st = plan(rank, dims, inputs[j]->rank, inputs[j]->dims, &bp);
        if (st == LX_ERR_CANNOT_BROADCAST)
            return set_err(st, "Instruction %d: the tensors are not compatible for broadcasting.", k);
        if (st) return st;
        rank = bp.out_rank;
        for (int i = 0; i < rank; i++) dims[i] = bp.out_dims[i];
    }
    if ((st = prepare_output(Y, LX_FLOAT, rank, dims))) return st;
    const int64_t total = numel_of(rank, dims);
    if (total == 0) return LX_OK;
    // strides of every input in the output frame (0 on broadcast or missing axes), then the axes
    // merged from the inside out while every input stays contiguous across them
    int64_t str[kChainMaxIn][LX_MAX_RANK];
    for (int j = 0; j < n_in; j++) {
        const lx_tensor *t = inputs[j];
        int64_t acc = 1;
        for (int i = rank - 1; i >= 0; i--) {
            const int k = i - (rank - t->rank);
            if (k < 0) { str[j][i] = 0; continue; }
            str[j][i] = (t->dims[k] == 1 && dims[i] != 1) ? 0 : acc;
            acc *= t->dims[k];
        }
    }
    int64_t cd[LX_MAX_RANK], cs[kChainMaxIn][LX_MAX_RANK];
    int n = 0;
    for (int i = rank - 1; i >= 0; i--) {
        if (dims[i] == 1) continue;
        bool merge = n > 0;
        for (int j = 0; merge && j < n_in; j++) merge = str[j][i] == cs[j][n - 1] * cd[n - 1];
        if (merge) {
            cd[n - 1] *= dims[i];
            continue;
        }
        cd[n] = dims[i];
        for (int j = 0; j < n_in; j++) cs[j][n] = str[j][i];
        n++;
    }
    if (n == 0) {  // one element
        cd[0] = 1;
        for (int j = 0; j < n_in; j++) cs[j][0] = 0;
        n = 1;
    }
    ChainArgs a;
    memset(&a, 0, sizeof a);
    a.n_in = n_in;
    a.n_ops = n_ops;
    a.uses_erf = erf ? 1 : 0;
    a.nouter = n - 1;
    bool vec = cd[0] % 4 == 0 && aligned16(Y->data);
    for (int j = 0; j < n_in; j++) {
        a.in[j] = (const float *)inputs[j]->data;
        if (cs[j][0] != 0) {
            a.inner_mode |= 1 << j;
            vec = vec && aligned16(inputs[j]->data);
            for (int d = 1; d < n; d++) vec = vec && cs[j][d] % 4 == 0;
        }
        for (int d = 1; d < n; d++) a.str[j][d - 1] = cs[j][d];
    }
    a.vec = vec ? 4 : 1;
    if (total / a.vec >= (1ll << 31)) return set_err(LX_ERR_NOT_SUPPORTED, "Chains over 2^31 vectors are not supported.");
    a.nv = (uint32_t)(total / a.vec);
    a.inner_v = make_fastdiv((uint32_t)(cd[0] / a.vec));
    for (int d = 1; d < n; d++) a.odiv[d - 1] = make_fastdiv((uint32_t)cd[d]);
    a.y = (float *)Y->data;
    for (int k = 0; k < n_ops; k++) {
        a.op[k] = (int8_t)ops[k];
        a.operand[k] = (int8_t)operands[k];
    }
    HIPCHECK(launch_chain(a, g.stream), "ElementwiseChain");
    return LX_OK;
}

int lx_LayerNormDecomposed(const lx_tensor *X, const lx_tensor *gamma, const lx_tensor *beta, float eps,
                           lx_tensor *Y) {
    OpScope prof("LayerNormDecomposed");
    REQUIRE_INIT();
    if (!X) return missing_input("ReduceMean", "data");
    if (!gamma) return missing_input("Mul", "B");
    if (!beta) return missing_input("Add", "B");
    int st;
    if ((st = check_tensor(X, "data")) || (st = check_tensor(gamma, "gamma")) || (st = check_tensor(beta, "beta")))
        return st;
    const int64_t r = X->rank > 0 ? X->dims[X->rank - 1] : 0;
    const bool fused = X->dtype == LX_FLOAT && gamma->dtype == LX_FLOAT && beta->dtype == LX_FLOAT && X->rank >= 1 &&
                       layernorm_affine_fits(gamma, X) && layernorm_affine_fits(beta, X) && layernorm_supported(r) &&
                       numel(X) / r < (1ll << 31) &&  // one block per row
                       aligned16(X->data) && aligned16(gamma->data) && aligned16(beta->data);
    if (fused) {
        if ((st = prepare_output(Y, LX_FLOAT, X->rank, X->dims))) return st;
        if (!aligned16(Y->data)) return set_err(LX_ERR_INVALID_ARGUMENT, "output storage must be 16-byte aligned");
        HIPCHECK(launch_layernorm((const float *)X->data, (const float *)gamma->data, (const float *)beta->data, eps,
                                  (float *)Y->data, numel(X) / (r ? r : 1), r, g.stream),
                 "LayerNorm");
        return LX_OK;
    }
    // node by node (same numbers, more passes)
    if (X->dtype != LX_FLOAT) return type_not_supported("ReduceMean", "data", X);
    const int64_t ax = -1;
    float two = 2.0f;
    lx_tensor mean{}, d{}, p{}, var{}, ve{}, sd{}, nrm{}, m{}, k2{}, ke{};
    if ((st = lx_tensor_alloc(LX_FLOAT, 0, nullptr, &k2)) || (st = lx_tensor_upload(&k2, &two, 4))) return st;
    if ((st = lx_tensor_alloc(LX_FLOAT, 0, nullptr, &ke)) || (st = lx_tensor_upload(&ke, &eps, 4))) return st;
    st = lx_ReduceMean(X, &ax, 1, 1, -1, &mean);
    if (!st) st = lx_Sub(X, &mean, &d);
    if (!st) st = lx_Pow(&d, &k2, &p);
    if (!st) st = lx_ReduceMean(&p, &ax, 1, 1, -1, &var);
    if (!st) st = lx_Add(&var, &ke, &ve);
    if (!st) st = lx_Sqrt(&ve, &sd);
    if (!st) st = lx_Div(&d, &sd, &nrm);
    if (!st) st = lx_Mul(&nrm, gamma, &m);
    if (!st) st = lx_Add(&m, beta, Y);
    for (lx_tensor *t : {&mean, &d, &p, &var, &ve, &sd, &nrm, &m, &k2, &ke}) lx_tensor_free(t);
    return st;
}

}  // extern "C"

namespace {

// Softmax(axis) of X, optionally of (X / scale) or (X * scale) (a one-element tensor) and of that plus a
// mask broadcast against X: the operators the reference runs one by one, each element rounded as they
// round it, in one kernel when the row-per-wave kernel takes the whole operation, else node by node.
// The mask of a last-axis Softmax over scores of shape dims, as the row-per-wave kernel reads it:
// contiguous or broadcast along the row, and the row index decomposed over the collapsed row axes
// (size-1 axes dropped, contiguous ones merged).  False when the kernel cannot take it.
bool softmax_mask_layout(int rank, const int64_t *dims, const lx_tensor *mask, SoftmaxArgs &sa) {
    const int64_t r = dims[rank - 1];
    // mask strides in the scores' frame (no collapsing of the softmax axis)
    int64_t ms[LX_MAX_RANK];
    int64_t stv = 1;
    for (int i = rank - 1; i >= 0; i--) {
        int k = i - (rank - mask->rank);
        if (k < 0) { ms[i] = 0; continue; }
        ms[i] = (mask->dims[k] == 1 && dims[i] != 1) ? 0 : stv;
        stv *= mask->dims[k];
    }
    sa.mask_inner = (r > 1 && ms[rank - 1] != 0) ? 1 : 0;
    // row axes 0..rank-2: collapse (drop size 1, merge contiguous)
    int64_t cd[LX_MAX_RANK], cs[LX_MAX_RANK];
    int n = 0;
    for (int i = rank - 2; i >= 0; i--) {
        if (dims[i] == 1) continue;
        if (n > 0 && ms[i] == cs[n - 1] * cd[n - 1]) {
            cd[n - 1] *= dims[i];
            continue;
        }
        cd[n] = dims[i];
        cs[n] = ms[i];
        n++;
    }
    if (n > kMaxOuter) return false;
    sa.mask = mask->data;
    sa.mask_rows.nouter = n;
    for (int d = 0; d < n; d++) {
        sa.mask_rows.odiv[d] = make_fastdiv((uint32_t)cd[d]);
        sa.mask_rows.a_str[d] = cs[d];
    }
    return true;
}

int run_softmax(const lx_tensor *X, const lx_tensor *mask, int32_t axis, int32_t has_axis, lx_tensor *Y,
                const char *opn, const lx_tensor *scale, int scale_div) {
    REQUIRE_INIT();
    if (!X) return missing_input(opn, "input");
    int st;
    if ((st = check_tensor(X, "input"))) return st;
    if (scale) {
        if ((st = check_tensor(scale, "scale"))) return st;
        if (scale->dtype != X->dtype) return wrong_type_same("B");
    }
    if (mask) {
        if ((st = check_tensor(mask, "mask"))) return st;
        if (mask->dtype != X->dtype) return wrong_type_same("B");
    }
    // a scale or mask that makes the tensor larger than X: the nodes one by one, Softmax's axis being
    // relative to the larger sum, as the Softmax node's is
    auto grows = [&](const lx_tensor *t) {
        lx_bcast_plan bp;
        if (!t || plan(X->rank, X->dims, t->rank, t->dims, &bp) != LX_OK) return false;
        if (bp.out_rank != X->rank) return true;
        for (int i = 0; i < X->rank; i++)
            if (bp.out_dims[i] != X->dims[i]) return true;
        return false;
    };
    if (grows(scale) || grows(mask)) {
        lx_tensor t0{}, t1{};
        const lx_tensor *x = X;
        st = LX_OK;
        if (scale) {
            st = run_binary(scale_div ? kDiv : kMul, X, scale, &t0);
            x = &t0;
        }
        if (!st && mask) {
            st = run_binary(kAdd, x, mask, &t1);
            x = &t1;
        }
        if (!st) st = run_softmax(x, nullptr, axis, has_axis, Y, opn);
        lx_tensor_free(&t0);
        lx_tensor_free(&t1);
        return st;
    }
    const int rank = X->rank;
    int ax = has_axis ? axis : -1;
    if (ax < 0) ax += rank;
    if (ax < 0 || ax >= rank)
        return argument_error("axis", "The specified axis must be less than the rank of the tensor.");
    int64_t outer = 1, inner = 1;
    for (int i = 0; i < ax; i++) outer *= X->dims[i];
    for (int i = ax + 1; i < rank; i++) inner *= X->dims[i];
    const int64_t r = X->dims[ax];
    const int64_t V = X->dtype == LX_FLOAT ? 4 : 2;
    const int vec = aligned16(X->data) ? (int)V : 1;

    SoftmaxArgs sa;
    memset(&sa, 0, sizeof sa);
    sa.dtype = X->dtype;
    sa.outer = outer;
    sa.r = r;
    sa.inner = inner;
    sa.vec = vec;
    bool fusable = true;  // the row-per-wave kernel takes the mask (and the scale)
    if (mask) {
        lx_bcast_plan p;
        st = plan(X->rank, X->dims, mask->rank, mask->dims, &p);
        if (st == LX_ERR_CANNOT_BROADCAST && !scale) return cannot_broadcast(X, mask);
        if (st && st != LX_ERR_CANNOT_BROADCAST) return st;
        if (X->dtype != LX_FLOAT && X->dtype != LX_DOUBLE && !scale) return type_not_supported("Add", "A", X);
        bool same_shape = st == LX_OK && p.out_rank == X->rank;
        for (int i = 0; same_shape && i < X->rank; i++) same_shape = p.out_dims[i] == X->dims[i];
        fusable = same_shape && softmax_mask_fusable(X->dtype, r, inner, outer, vec) &&
                  softmax_mask_layout(rank, X->dims, mask, sa);
    }
    if (scale) {
        // the scale must leave X's shape as it is (one element, rank <= X's) for the kernel to apply it
        bool ok = fusable && numel(scale) == 1 && scale->rank <= X->rank &&
                  softmax_mask_fusable(X->dtype, r, inner, outer, vec) &&
                  (X->dtype == LX_FLOAT || X->dtype == LX_DOUBLE);
        if (!ok) {  // node by node: Div / Mul, then (Add +) Softmax
            lx_tensor t{};
            st = run_binary(scale_div ? kDiv : kMul, X, scale, &t);
            if (!st) st = run_softmax(&t, mask, ax, 1, Y, opn);
            lx_tensor_free(&t);
            return st;
        }
        sa.scale = scale->data;
        sa.scale_div = scale_div;
    }
    if (mask && !fusable) {
        lx_tensor t{};
        st = run_binary(kAdd, X, mask, &t);
        if (!st) st = run_softmax(&t, nullptr, ax, 1, Y, opn);
        lx_tensor_free(&t);
        return st;
    }
    if (X->dtype != LX_FLOAT && X->dtype != LX_DOUBLE) return type_not_supported(opn, "input", X);
    if ((st = prepare_output(Y, X->dtype, X->rank, X->dims))) return st;
    if (vec > 1 && !aligned16(Y->data)) {
        sa.vec = 1;
        if ((sa.mask || sa.scale) && sa.r > 64 * 8)
            return set_err(LX_ERR_INVALID_ARGUMENT, "output storage must be 16-byte aligned");
    }
    sa.x = X->data;
    sa.y = Y->data;
    HIPCHECK(launch_softmax(sa, g.stream), opn);
    return LX_OK;
}

}  // namespace

// ===========================================================================
// MatMul: CPUExecutionProvider.MatMul (CPUExecutionProvider.cs:359-378) over
// Tensor<T>.MatMul (TensorOps.cs:504-806 for Int32, Float, Double): the same
// shape rules, broadcast cases and exception texts.
// ===========================================================================
namespace {

struct MView {  // a tensor as the reference's (possibly broadcast) view: element strides, 0 on broadcast axes
    int rank = 0;
    int64_t dims[LX_MAX_RANK] = {0};
    int64_t str[LX_MAX_RANK] = {0};
    const void *data = nullptr;
    bool bt = false;  // the matrix stored by columns (set by densify for a right operand that allows it)
};

MView dense_view(const lx_tensor *t) {
    MView v;
    v.rank = t->rank;
    int64_t s = 1;
    for (int d = t->rank - 1; d >= 0; d--) {
        v.dims[d] = t->dims[d];
        v.str[d] = s;
        s *= t->dims[d];
    }
    v.data = t->data;
    return v;
}

std::string shape_str(const MView &v) {
    std::string s = "[";
    for (int i = 0; i < v.rank; i++) s += (i ? "," : "") + std::to_string(v.dims[i]);
    return s + "]";
}

// Tensor<T>.Broadcast(x, shape): right-aligned view of x at `dims`
bool broadcast_view(const MView &x, int rank, const int64_t *dims, MView *out) {
    if (rank < x.rank || rank > LX_MAX_RANK) return false;
    MView v;
    v.rank = rank;
    v.data = x.data;
    for (int d = 0; d < rank; d++) {
        const int xd = d - (rank - x.rank);
        v.dims[d] = dims[d];
        if (xd < 0) v.str[d] = 0;
        else if (x.dims[xd] == dims[d]) v.str[d] = x.str[xd];
        else if (x.dims[xd] == 1) v.str[d] = 0;
        else return false;
    }
    *out = v;
    return true;
}

// numpy / ITensor broadcast shape of two shapes
bool broadcast_dims(int ra, const int64_t *da, int rb, const int64_t *db, int *ro, int64_t *dout) {
    const int r = std::max(ra, rb);
    if (r > LX_MAX_RANK) return false;
    for (int d = 0; d < r; d++) {
        const int ia = d - (r - ra), ib = d - (r - rb);
        const int64_t a = ia >= 0 ? da[ia] : 1, b = ib >= 0 ? db[ib] : 1;
        if (a != b && a != 1 && b != 1) return false;
        dout[d] = a == 1 ? b : a;
    }
    *ro = r;
    return true;
}

const char *net_type(int dt) {
    switch (dt) {
    case LX_FLOAT: return "System.Single"; case LX_DOUBLE: return "System.Double"; case LX_INT32: return "System.Int32";
    case LX_INT64: return "System.Int64"; case LX_UINT8: return "System.Byte"; case LX_INT8: return "System.SByte";
    case LX_INT16: return "System.Int16"; case LX_UINT16: return "System.UInt16"; case LX_UINT32: return "System.UInt32";
    case LX_UINT64: return "System.UInt64"; case LX_BOOL: return "System.Boolean"; default: return "System.Object";
    }
}

// the matrix part (last two axes) must be row-major dense for the kernels; otherwise
// the operand is copied to a dense pooled block first
int densify(int dt, MView *v, std::vector<void *> &temps, bool allow_bt = false) {
    const int r = v->rank;
    // unit column stride and rows that do not overlap (dense, or the rows of a transposed view): as they are
    if ((v->dims[r - 1] == 1 || v->str[r - 1] == 1) && (v->dims[r - 2] == 1 || v->str[r - 2] >= v->dims[r - 1]))
        return LX_OK;
    // a right operand stored by columns (unit row stride, columns that do not overlap), where allowed: as it is
    if (allow_bt && v->dims[r - 1] > 1 && v->dims[r - 2] > 1 && v->str[r - 2] == 1 && v->str[r - 1] >= v->dims[r - 2]) {
        v->bt = true;
        return LX_OK;
    }
    int64_t n = 1;
    for (int d = 0; d < r; d++) n *= v->dims[d];
    void *p = nullptr;
    HIPCHECK(pool_alloc((size_t)std::max<int64_t>(n * esize(dt), 16), &p, nullptr, g.stream), "device allocation (temporary)");
    temps.push_back(p);
    HIPCHECK(launch_strided_copy((int)esize(dt), v->data, p, r, v->dims, v->str, g.stream), "MatMul broadcast copy");
    int64_t s = 1;
    for (int d = r - 1; d >= 0; d--) {
        v->str[d] = s;
        s *= v->dims[d];
    }
    v->data = p;
    return LX_OK;
}

// lx_MatMulAdd's Adds, applied in the MatMul's epilogue when the bias is a row vector of the output's
// last axis (or one such row per batch: [batch..., 1, n] for an output [batch..., m, n]) and the
// residual has the output's shape (Float); `applied` tells the caller
struct MatMulEpilogue {
    const lx_tensor *bias = nullptr, *res = nullptr;
    bool gelu = false;  // then the GELU subgraph on each result (lx_MatMulAddGelu)
    bool applied = false;
};
// The LayerNorm that follows the product (and its epilogue), applied by the split product's ordered sum when the
// product splits (api_matmul_add_layernorm); `applied` tells the caller
struct MatMulLayerNorm {
    const lx_tensor *gamma = nullptr, *beta = nullptr;
    float eps = 0.0f;
    bool applied = false;
};

// What a MatMul call asks beyond A x B, passed down explicitly: the epilogue's Adds (and GELU), the LayerNorm
// after them, the split rule counting one matrix's tiles (grouped projections), the product stored transposed
// and a right operand read by columns (the graph's transposed views)
struct MatMulOpts {
    MatMulEpilogue *epi = nullptr;
    MatMulLayerNorm *ln = nullptr;
    bool per_matrix = false;
    const int *yperm = nullptr;
    bool allow_bt = false;
};

// a permutation of 0 .. rank - 1 that keeps the last axis last
bool last_axis_perm(const int *perm, int rank) {
    bool seen[LX_MAX_RANK] = {false};
    for (int i = 0; i < rank; i++) {
        if (perm[i] < 0 || perm[i] >= rank || seen[perm[i]]) return false;
        seen[perm[i]] = true;
    }
    return rank >= 1 && perm[rank - 1] == rank - 1;
}

bool epilogue_fits(const MatMulEpilogue &e, int out_rank, const int64_t *out_dims, int64_t *bias_bstr) {
    if (out_rank < 2) return false;
    const int64_t n = out_dims[out_rank - 1];
    *bias_bstr = 0;
    if (e.bias) {
        const lx_tensor *b = e.bias;
        if (b->dtype != LX_FLOAT || b->rank < 1 || b->rank > out_rank || b->dims[b->rank - 1] != n) return false;
        bool shared = true;  // [1, ..., 1, n]
        for (int i = 0; i < b->rank - 1; i++) shared = shared && b->dims[i] == 1;
        if (!shared) {       // [batch..., 1, n]: a row per batch
            if (b->rank != out_rank || b->dims[out_rank - 2] != 1) return false;
            for (int i = 0; i < out_rank - 2; i++)
                if (b->dims[i] != out_dims[i]) return false;
            *bias_bstr = n;
        }
    }
    if (e.res) {
        const lx_tensor *r = e.res;
        if (r->dtype != LX_FLOAT || r->rank != out_rank) return false;
        for (int i = 0; i < out_rank; i++)
            if (r->dims[i] != out_dims[i]) return false;
    }
    return true;
}

int matmul_run(int dt, MView x, MView y, int out_rank, const int64_t *out_dims, lx_tensor *Y,
               std::vector<void *> &temps, const MatMulOpts &o) {
    MatMulEpilogue *const epi = o.epi;
    MatMulLayerNorm *const ln = o.ln;
    int st;
    if ((st = densify(dt, &x, temps)) || (st = densify(dt, &y, temps, o.allow_bt && dt == LX_FLOAT))) return st;
    // the product's element strides in Y: dense, or Y = transpose(product, o.yperm)
    int64_t pstr[LX_MAX_RANK];
    const int *yp = o.yperm;
    if (yp) {
        if (out_rank < 2 || !last_axis_perm(yp, out_rank)) return LX_ERR_NOT_SUPPORTED;
        int64_t yd[LX_MAX_RANK];
        for (int i = 0; i < out_rank; i++) yd[i] = out_dims[yp[i]];
        if ((st = prepare_output(Y, dt, out_rank, yd))) return st;
        int64_t s = 1;
        for (int i = out_rank - 1; i >= 0; i--) {
            pstr[yp[i]] = s;
            s *= yd[i];
        }
    } else {
        if ((st = prepare_output(Y, dt, out_rank, out_dims))) return st;
        int64_t s = 1;
        for (int i = out_rank - 1; i >= 0; i--) {
            pstr[i] = s;
            s *= out_dims[i];
        }
    }
    MatMulArgs p;
    memset(&p, 0, sizeof p);
    int64_t bias_bstr = 0;
    if (epi && !yp && dt == LX_FLOAT && epilogue_fits(*epi, out_rank, out_dims, &bias_bstr)) {
        p.bias = epi->bias ? (const float *)epi->bias->data : nullptr;
        p.bias_bstr = bias_bstr;
        p.res = epi->res ? (const float *)epi->res->data : nullptr;
        p.gelu = epi->gelu ? 1 : 0;
    }
    p.split_per_matrix = o.per_matrix ? 1 : 0;
    p.m = (int32_t)x.dims[x.rank - 2];
    p.k = (int32_t)x.dims[x.rank - 1];
    p.n = (int32_t)y.dims[y.rank - 1];
    p.nbatch = x.rank - 2;
    p.batch = 1;
    for (int d = 0; d < p.nbatch; d++) {
        p.bdims[d] = x.dims[d];
        p.a_bstr[d] = x.str[d];
        p.b_bstr[d] = y.str[d];
        // a single matrix along an axis: its stride is never used (dense value, so the 16-byte tests agree)
        p.c_bstr[d] = out_dims[d] == 1 ? 0 : pstr[d];
        p.batch *= x.dims[d];
    }
    // row strides; a single row's is never used (the dense value)
    p.lda = x.dims[x.rank - 2] == 1 ? x.dims[x.rank - 1] : x.str[x.rank - 2];
    p.ldb = y.dims[y.rank - 2] == 1 ? y.dims[y.rank - 1] : y.str[y.rank - 2];
    if (y.bt) {  // by columns: the stride between columns
        p.bt = 1;
        p.ldb = y.str[y.rank - 1];
    }
    p.ldc = (out_rank < 2 || p.m == 1) ? p.n : pstr[out_rank - 2];  // out_rank 1: the [1] of two vectors
    if (p.nbatch > kMaxOuter) return set_err(LX_ERR_NOT_SUPPORTED, "At most %d batch axes are supported.", kMaxOuter);
    if (x.dims[x.rank - 2] > INT32_MAX || x.dims[x.rank - 1] > INT32_MAX || y.dims[y.rank - 1] > INT32_MAX)
        return set_err(LX_ERR_NOT_SUPPORTED, "Matrix dimensions beyond 2^31 are not supported.");
    // One right matrix for every batch and the left matrices stored row after row ([B, S, H] x [H, N]): one
    // [batch * m, k] x [k, n] product, the same rows with the same sums, in one grid of row tiles (at most
    // 65535 of the smallest, 64 rows: a larger product keeps its batch in the grid's third dimension)
    bool fold = p.nbatch > 0 && bias_bstr == 0 && !yp && p.lda == p.k;
    int64_t rows = x.dims[x.rank - 2];
    for (int d = p.nbatch - 1; fold && d >= 0; d--) {
        if (p.bdims[d] != 1) fold = p.b_bstr[d] == 0 && p.a_bstr[d] == rows * p.k;
        rows *= p.bdims[d];
    }
    if (fold && rows <= 65535LL * 64) {
        p.m = (int32_t)rows;
        p.nbatch = 0;
        p.batch = 1;
    }
    if (p.k == 0) {  // empty inner dimension: every output is 0 (the Adds, if any, run afterwards)
        int64_t n = numel(Y);
        HIPCHECK(launch_fill(Y->data, n, (int)esize(dt), 0, g.stream), "MatMul");
        return LX_OK;
    }
    // partial products of a split K (stream-ordered pool block, released with the caller's temporaries); a B
    // stored by columns runs only unsplit and without an epilogue (the caller then takes another path)
    const int64_t pb = matmul_part_bytes(dt, x.data, y.data, Y->data, p);
    if (p.bt && (pb || p.bias || p.res || p.gelu)) return LX_ERR_NOT_SUPPORTED;
    if (pb) {
        void *w = nullptr;
        HIPCHECK(pool_alloc((size_t)pb, &w, nullptr, g.stream), "device allocation (temporary)");
        temps.push_back(w);
        p.part = (float *)w;
    }
    // the LayerNorm after the product, in its ordered sum: every requested Add in the epilogue, the rows the
    // row-per-wave LayerNorm kernel takes, gamma and beta rows of the output's last axis
    if (ln && !yp && (!epi || ((!epi->bias || p.bias) && (!epi->res || p.res))) &&
        matmul_ln_fusable(dt, x.data, y.data, Y->data, p) && ln->gamma->dtype == LX_FLOAT &&
        ln->beta->dtype == LX_FLOAT && layernorm_affine_fits(ln->gamma, Y) && layernorm_affine_fits(ln->beta, Y) &&
        aligned16(ln->gamma->data) && aligned16(ln->beta->data)) {
        HIPCHECK(launch_matmul_ln(x.data, y.data, Y->data, p, (const float *)ln->gamma->data,
                                  (const float *)ln->beta->data, ln->eps, g.stream),
                 "MatMul");
        ln->applied = true;
        if (epi && (p.bias || p.res)) epi->applied = true;
        return LX_OK;
    }
    HIPCHECK(launch_matmul(dt, x.data, y.data, Y->data, p, g.stream), "MatMul");
    if (epi && (p.bias || p.res || p.gelu)) epi->applied = true;
    return LX_OK;
}

int cols_rows_error(int64_t cols, int64_t rows) {
    return set_err(LX_ERR_INVALID_ARGUMENT,
                   "The number of columns in the first matrix (%lld) is not equal to the number of rows in the second "
                   "matrix (%lld).",
                   (long long)cols, (long long)rows);
}

// Tensor<T>.MatMul (TensorOps.cs:600-705)
int matmul_views(int dt, const MView &x, const MView &y, lx_tensor *Y, std::vector<void *> &temps,
                 const MatMulOpts &o) {
    if (x.rank == 0 || y.rank == 0)
        return set_err(LX_ERR_INVALID_ARGUMENT, "The rank of each tensor in matrix multiplication must be greater than 1.");
    if (x.rank == 2 && y.rank == 2) {  // MatMul2D (TensorOps.cs:356-407)
        if (x.dims[1] != y.dims[0]) return cols_rows_error(x.dims[1], y.dims[0]);
        int64_t od[2] = {x.dims[0], y.dims[1]};
        return matmul_run(dt, x, y, 2, od, Y, temps, o);
    }
    if (x.rank >= 2 && y.rank >= 2) {
        const int64_t xm = x.dims[x.rank - 2], xk = x.dims[x.rank - 1];
        const int64_t yk = y.dims[y.rank - 2], yn = y.dims[y.rank - 1];
        if (xk != yk) return cols_rows_error(xk, yk);
        int br;
        int64_t bd[LX_MAX_RANK + 2];
        if (!broadcast_dims(x.rank - 2, x.dims, y.rank - 2, y.dims, &br, bd) || br + 2 > LX_MAX_RANK)
            return set_err(LX_ERR_INVALID_ARGUMENT, "The tensor shapes are not compatible for broadcasting.");
        MView bx, by;
        int64_t dx[LX_MAX_RANK], dy[LX_MAX_RANK], od[LX_MAX_RANK];
        for (int d = 0; d < br; d++) dx[d] = dy[d] = od[d] = bd[d];
        dx[br] = xm; dx[br + 1] = xk;
        dy[br] = yk; dy[br + 1] = yn;
        od[br] = xm; od[br + 1] = yn;
        if (!broadcast_view(x, br + 2, dx, &bx) || !broadcast_view(y, br + 2, dy, &by))
            return set_err(LX_ERR_INVALID_ARGUMENT, "The tensor shapes are not compatible for broadcasting.");
        return matmul_run(dt, bx, by, br + 2, od, Y, temps, o);
    }
    if (x.rank >= 2 || y.rank >= 2) {  // one operand of rank 1: element-wise broadcast of both, then MatMul
        int r;
        int64_t bd[LX_MAX_RANK];
        MView bx, by;
        if (!broadcast_dims(x.rank, x.dims, y.rank, y.dims, &r, bd) || !broadcast_view(x, r, bd, &bx) ||
            !broadcast_view(y, r, bd, &by))
            return set_err(LX_ERR_INVALID_ARGUMENT, "The shapes %s and %s are not compatible for broadcasting.",
                           shape_str(x).c_str(), shape_str(y).c_str());
        return matmul_views(dt, bx, by, Y, temps, o);
    }
    // both rank 1: [1,n] x [n,1] -> [1,1], then RemoveDim(0) -> [1]
    MView px, py;
    px.rank = 2; px.dims[0] = 1; px.dims[1] = x.dims[0]; px.str[0] = x.dims[0]; px.str[1] = x.str[0]; px.data = x.data;
    py.rank = 2; py.dims[0] = y.dims[0]; py.dims[1] = 1; py.str[0] = y.str[0]; py.str[1] = 1; py.data = y.data;
    if (px.dims[1] != py.dims[0]) return cols_rows_error(px.dims[1], py.dims[0]);
    int64_t od[1] = {1};
    return matmul_run(dt, px, py, 1, od, Y, temps, o);
}

// lx_MatMul's checks and product, with the options of the caller
int matmul_call(const lx_tensor *A, const lx_tensor *B, lx_tensor *Y, const MatMulOpts &o) {
    REQUIRE_INIT();
    if (!A) return missing_input("MatMul", "A");
    if (!B) return missing_input("MatMul", "B");
    int st;
    if ((st = check_tensor(A, "A")) || (st = check_tensor(B, "B"))) return st;
    if (A->dtype != LX_INT32 && A->dtype != LX_FLOAT && A->dtype != LX_DOUBLE)
        return type_not_supported("MatMul", "A", A);
    if (B->dtype != A->dtype)
        return set_err(LX_ERR_WRONG_INPUT_TYPE, "Unable to cast object of type 'Lokad.Onnx.DenseTensor`1[%s]' to type "
                                                "'Lokad.Onnx.Tensor`1[%s]'.",
                       net_type(B->dtype), net_type(A->dtype));
    std::vector<void *> temps;
    st = matmul_views(A->dtype, dense_view(A), dense_view(B), Y, temps, o);
    for (void *t : temps) (void)pool_release(t);
    return st;
}

}  // namespace

extern "C" int lx_MatMul(const lx_tensor *A, const lx_tensor *B, lx_tensor *Y) {
    OpScope prof("MatMul");
    return matmul_call(A, B, Y, MatMulOpts{});
}

namespace lx {
int api_matmul_permuted(const lx_tensor *A, const int *a_perm, const lx_tensor *B, const int *b_perm,
                        const int *y_perm, lx_tensor *Y) {
    if (!api_initialized() || !A || !B || A->dtype != LX_FLOAT || B->dtype != LX_FLOAT || A->rank < 2 || B->rank < 2 ||
        check_tensor(A, "A") || check_tensor(B, "B"))
        return LX_ERR_NOT_SUPPORTED;
    MView x = dense_view(A), y = dense_view(B);
    // A: its last axis stays last; B: too, or its last axis becomes the product's K (B read by columns)
    auto permute = [](MView &v, const int *perm, bool k_last_ok) {
        if (!perm) return true;
        if (!last_axis_perm(perm, v.rank)) {
            int q[LX_MAX_RANK];  // the same permutation with its last two entries swapped
            for (int i = 0; i < v.rank; i++) q[i] = perm[i];
            std::swap(q[v.rank - 1], q[v.rank - 2]);
            if (!k_last_ok || !last_axis_perm(q, v.rank)) return false;
        }
        const MView o = v;
        for (int i = 0; i < v.rank; i++) {
            v.dims[i] = o.dims[perm[i]];
            v.str[i] = o.str[perm[i]];
        }
        return true;
    };
    if (!permute(x, a_perm, false) || !permute(y, b_perm, true)) return LX_ERR_NOT_SUPPORTED;
    std::vector<void *> temps;
    MatMulOpts o;
    o.yperm = y_perm;
    o.allow_bt = true;
    const int st = matmul_views(LX_FLOAT, x, y, Y, temps, o);
    for (void *t : temps) (void)pool_release(t);
    return st;
}

int api_attention(const lx_tensor *Q, const int *q_perm, const lx_tensor *K, const int *k_perm,
                  const lx_tensor *scale, int scale_div, const lx_tensor *mask, int32_t axis, const lx_tensor *V,
                  const int *v_perm, const int *y_perm, lx_tensor *Y) {
    if (!api_initialized() || !Q || !K || !V || !mask || !Y) return LX_ERR_NOT_SUPPORTED;
    for (const lx_tensor *t : {Q, K, V, mask, scale})
        if (t && (t->dtype != LX_FLOAT || check_tensor(t, "input"))) return LX_ERR_NOT_SUPPORTED;
    const int R = Q->rank;
    if (R < 2 || R - 2 > kMaxOuter || K->rank != R || V->rank != R) return LX_ERR_NOT_SUPPORTED;
    auto is_perm = [R](const int *p) {
        if (!p) return true;
        bool seen[LX_MAX_RANK] = {false};
        for (int i = 0; i < R; i++) {
            if (p[i] < 0 || p[i] >= R || seen[p[i]]) return false;
            seen[p[i]] = true;
        }
        return true;
    };
    if (!is_perm(q_perm) || !is_perm(k_perm) || !is_perm(v_perm) || !is_perm(y_perm)) return LX_ERR_NOT_SUPPORTED;
    // the operand views of the two products (a transposed view reads through its strides, as MatMulPermuted does)
    MView q = dense_view(Q), k = dense_view(K), v = dense_view(V);
    auto permute = [R](MView &m, const int *perm) {
        if (!perm) return;
        const MView o = m;
        for (int i = 0; i < R; i++) {
            m.dims[i] = o.dims[perm[i]];
            m.str[i] = o.str[perm[i]];
        }
    };
    permute(q, q_perm);
    permute(k, k_perm);
    permute(v, v_perm);
    // equal batch axes (no broadcast), heads of at most kAttentionMax: [.., S, D] x [.., D, SK] and [.., S, SK] x
    // [.., SK, DV]; otherwise the nodes run (and report any shape error)
    for (int i = 0; i < R - 2; i++)
        if (k.dims[i] != q.dims[i] || v.dims[i] != q.dims[i]) return LX_ERR_NOT_SUPPORTED;
    const int64_t S = q.dims[R - 2], D = q.dims[R - 1], SK = k.dims[R - 1], DV = v.dims[R - 1];
    if (k.dims[R - 2] != D || v.dims[R - 2] != SK) return LX_ERR_NOT_SUPPORTED;
    for (int64_t e : {S, D, SK, DV})
        if (e < 1 || e > kAttentionMax) return LX_ERR_NOT_SUPPORTED;
    int64_t batch = 1;
    for (int i = 0; i < R - 2; i++) batch *= q.dims[i];
    if (batch < 1 || batch > 0x7fffffff) return LX_ERR_NOT_SUPPORTED;
    // the Softmax over the scores' last axis with the scale and mask in its kernel, as run_softmax takes them
    int64_t sdims[LX_MAX_RANK];
    for (int i = 0; i < R - 2; i++) sdims[i] = q.dims[i];
    sdims[R - 2] = S;
    sdims[R - 1] = SK;
    if ((axis < 0 ? axis + R : axis) != R - 1) return LX_ERR_NOT_SUPPORTED;
    if (scale && (numel(scale) != 1 || scale->rank > R)) return LX_ERR_NOT_SUPPORTED;
    lx_bcast_plan bp;
    if (plan(R, sdims, mask->rank, mask->dims, &bp) != LX_OK || bp.out_rank != R) return LX_ERR_NOT_SUPPORTED;
    for (int i = 0; i < R; i++)
        if (bp.out_dims[i] != sdims[i]) return LX_ERR_NOT_SUPPORTED;
    SoftmaxArgs sa;
    memset(&sa, 0, sizeof sa);
    sa.dtype = LX_FLOAT;
    if (!softmax_mask_fusable(LX_FLOAT, SK, 1, batch * S, 4) || !softmax_mask_layout(R, sdims, mask, sa))
        return LX_ERR_NOT_SUPPORTED;
    // the context [.., S, DV], written through y_perm
    int64_t cdims[LX_MAX_RANK], ydims[LX_MAX_RANK], cstr[LX_MAX_RANK];
    for (int i = 0; i < R - 2; i++) cdims[i] = q.dims[i];
    cdims[R - 2] = S;
    cdims[R - 1] = DV;
    for (int i = 0; i < R; i++) ydims[i] = y_perm ? cdims[y_perm[i]] : cdims[i];
    int st = prepare_output(Y, LX_FLOAT, R, ydims);
    if (st) return st;
    int64_t ys = 1;
    for (int i = R - 1; i >= 0; i--) {
        cstr[y_perm ? y_perm[i] : i] = ys;
        ys *= ydims[i];
    }
    AttentionArgs a;
    memset(&a, 0, sizeof a);
    a.q = (const float *)Q->data;
    a.k = (const float *)K->data;
    a.v = (const float *)V->data;
    a.y = (float *)Y->data;
    a.s = (int)S;
    a.sk = (int)SK;
    a.d = (int)D;
    a.dv = (int)DV;
    a.nbatch = R - 2;
    a.batch = batch;
    for (int i = 0; i < R - 2; i++) {
        a.bdims[i] = q.dims[i];
        a.q_bstr[i] = q.str[i];
        a.k_bstr[i] = k.str[i];
        a.v_bstr[i] = v.str[i];
        a.y_bstr[i] = cstr[i];
    }
    a.q_rs = q.str[R - 2], a.q_cs = q.str[R - 1];
    a.k_rs = k.str[R - 2], a.k_cs = k.str[R - 1];
    a.v_rs = v.str[R - 2], a.v_cs = v.str[R - 1];
    a.y_rs = cstr[R - 2], a.y_cs = cstr[R - 1];
    a.mask = (const float *)mask->data;
    a.mask_inner = sa.mask_inner;
    a.mask_rows = sa.mask_rows;
    a.scale = scale ? (const float *)scale->data : nullptr;
    a.scale_div = scale_div;
    HIPCHECK(launch_attention(a, g.stream), "Attention");
    return LX_OK;
}
}  // namespace lx

// MatMul -> Add bias [-> Add residual] [-> the GELU subgraph]: in the MatMul's epilogue when the shapes fit
// (Float), else the MatMul and then each node's operator, into new tensors (an Add may broadcast to a larger
// shape than the product's)
int matmul_add_run(const lx_tensor *A, const lx_tensor *B, const lx_tensor *bias, const lx_tensor *residual,
                   bool gelu, lx_tensor *Y, MatMulOpts o = MatMulOpts{}) {
    REQUIRE_INIT();
    if (!bias) return missing_input("Add", "B");
    int st;
    if ((st = check_tensor(bias, "B")) || (residual && (st = check_tensor(residual, "B")))) return st;
    if (!Y) return set_err(LX_ERR_INVALID_ARGUMENT, "The output tensor handle is null.");
    const bool caller_storage = Y->data != nullptr;
    MatMulEpilogue epi;
    epi.bias = bias;
    epi.res = residual;
    epi.gelu = gelu;
    o.epi = &epi;
    lx_tensor c = caller_storage ? *Y : lx_tensor{};
    st = matmul_call(A, B, caller_storage ? &c : Y, o);
    if (st) return st;
    if (epi.applied) {
        if (caller_storage) *Y = c;
        return LX_OK;
    }
    lx_tensor *prod = caller_storage ? &c : Y;
    lx_tensor t1{}, t2{}, t3{};
    st = run_binary(kAdd, prod, bias, &t1);
    if (!st && residual) st = run_binary(kAdd, &t1, residual, &t2);
    lx_tensor *out = residual ? &t2 : &t1;
    if (!st && gelu) {
        st = lx_GeluErf(out, &t3);
        out = &t3;
    }
    if (!st) {
        if (caller_storage) {
            if (!(st = prepare_output(Y, out->dtype, out->rank, out->dims)) && numel(out))
                HIPCHECK(hipMemcpyAsync(Y->data, out->data, numel(out) * esize(out->dtype), hipMemcpyDeviceToDevice,
                                        g.stream),
                         gelu ? "MatMulAddGelu" : "MatMulAdd");
        } else {
            lx_tensor_free(Y);
            *Y = *out;
            *out = lx_tensor{};
        }
    }
    lx_tensor_free(&t1);
    lx_tensor_free(&t2);
    lx_tensor_free(&t3);
    return st;
}

extern "C" int lx_MatMulAdd(const lx_tensor *A, const lx_tensor *B, const lx_tensor *bias, const lx_tensor *residual,
                            lx_tensor *Y) {
    OpScope prof("MatMulAdd");
    return matmul_add_run(A, B, bias, residual, false, Y);
}

namespace lx {
int api_matmul_add_layernorm(const lx_tensor *A, const lx_tensor *W, const lx_tensor *bias, const lx_tensor *residual,
                             const lx_tensor *gamma, const lx_tensor *beta, float eps, lx_tensor *Y) {
    if (!api_initialized() || !A || !W || !bias || !gamma || !beta || !Y || Y->data) return LX_ERR_NOT_SUPPORTED;
    MatMulLayerNorm ln;
    ln.gamma = gamma;
    ln.beta = beta;
    ln.eps = eps;
    MatMulOpts o;
    o.ln = &ln;
    lx_tensor h{};
    int st = matmul_add_run(A, W, bias, residual, false, &h, o);
    if (!st && ln.applied) {
        *Y = h;
        return LX_OK;
    }
    if (!st) st = lx_LayerNormDecomposed(&h, gamma, beta, eps, Y);
    lx_tensor_free(&h);
    return st;
}

int api_matmul_add_grouped(const lx_tensor *A, const lx_tensor *W, const lx_tensor *bias, lx_tensor *Y) {
    if (!W || W->rank != 3 || W->dims[0] > kMatMulSplitBatch) return LX_ERR_NOT_SUPPORTED;
    MatMulOpts o;
    o.per_matrix = true;
    return matmul_add_run(A, W, bias, nullptr, false, Y, o);
}
}  // namespace lx

extern "C" int lx_MatMulAddGelu(const lx_tensor *A, const lx_tensor *B, const lx_tensor *bias, lx_tensor *Y) {
    OpScope prof("MatMulAddGelu");
    return matmul_add_run(A, B, bias, nullptr, true, Y);
}

// ===========================================================================
// Data movement: CPUExecutionProvider.Transpose / Concat / Gather / Slice
// (CPUExecutionProvider.cs:411-433, 477-501, 516-546, 548-600) over
// Tensor<T>.Transpose / Gather / Concat / Slice (TensorOps.cs:1358-1532).
// ===========================================================================
namespace {

bool movable_dtype(int dt) { return esize(dt) != 0; }

int64_t row_major_strides(int rank, const int64_t *dims, int64_t *str) {
    int64_t s = 1;
    for (int d = rank - 1; d >= 0; d--) {
        str[d] = s;
        s *= dims[d];
    }
    return s;
}

int view_copy(int dt, const void *src, void *dst, const ViewCopyArgs &a) {
    int64_t total = 1;
    for (int k = 0; k < a.rank; k++) total *= a.dims[k];
    if (total >= (1ll << 31) * (16 / esize(dt)))
        return set_err(LX_ERR_NOT_SUPPORTED, "Copies of more than 2^31 vectors are not supported.");
    HIPCHECK(launch_view_copy((int)esize(dt), src, dst, a, g.stream), "view copy");
    return LX_OK;
}

}  // namespace

extern "C" int lx_Transpose(const lx_tensor *data, const int64_t *perm, int32_t n_perm, lx_tensor *Y) {
    OpScope prof("Transpose");
    REQUIRE_INIT();
    if (!data) return missing_input("Transpose", "data");
    int st;
    if ((st = check_tensor(data, "data"))) return st;
    if (!movable_dtype(data->dtype)) return not_supported("Transpose");
    const int rank = data->rank;
    int64_t p[LX_MAX_RANK];
    if (n_perm >= 0) {
        // validation in the reference's order, the negative entries normalised last
        if (n_perm != rank)
            return argument_error(("The size of the permutation array must be the rank of the tensor: " +
                                   std::to_string(rank) + ".").c_str(), "perm");
        for (int i = 0; i < n_perm; i++)
            if (perm[i] >= rank)
                return argument_error(("The permuted dimension " + std::to_string(perm[i]) +
                                       " exceeds the number of dimensions in the tensor.").c_str(), "perm");
        for (int i = 0; i < n_perm; i++)
            for (int j = 0; j < i; j++)
                if (perm[i] == perm[j]) return argument_error("The permutation array has a repeated dimension.", "perm");
        for (int i = 0; i < n_perm; i++) {
            p[i] = perm[i] >= 0 ? perm[i] : rank + perm[i];
            if (p[i] < 0) return set_err(LX_ERR_INVALID_ARGUMENT, "Index was outside the bounds of the array.");
        }
        // a negative entry equal to a positive one after normalisation would write one
        // output axis twice; the device path refuses it
        for (int i = 0; i < n_perm; i++)
            for (int j = 0; j < i; j++)
                if (p[i] == p[j]) return argument_error("The permutation array has a repeated dimension.", "perm");
    } else {
        for (int i = 0; i < rank; i++) p[i] = rank - 1 - i;
    }
    if (rank <= 1) {  // the reference returns the input tensor itself
        if (Y && Y->data) {
            if ((st = prepare_output(Y, data->dtype, rank, data->dims))) return st;
            const int64_t bytes = numel(data) * esize(data->dtype);
            if (bytes) HIPCHECK(hipMemcpyAsync(Y->data, data->data, bytes, hipMemcpyDeviceToDevice, g.stream), "Transpose");
            return LX_OK;
        }
        if (!Y) return set_err(LX_ERR_INVALID_ARGUMENT, "The output tensor handle is null.");
        *Y = *data;
        Y->owns = 0;
        return LX_OK;
    }
    // the reference's copy loop visits index [0, ..., 0] of the output even when it has no
    // elements (TensorDimensionsIterator yields its first index unconditionally,
    // TensorDimensionsIterator.cs:36-40) and reads element 0 of the empty input
    if (numel(data) == 0) return set_err(LX_ERR_INVALID_ARGUMENT, "Index was outside the bounds of the array.");
    int64_t od[LX_MAX_RANK], in_str[LX_MAX_RANK];
    row_major_strides(rank, data->dims, in_str);
    for (int i = 0; i < rank; i++) od[i] = data->dims[p[i]];
    if ((st = prepare_output(Y, data->dtype, rank, od))) return st;
    ViewCopyArgs a;
    memset(&a, 0, sizeof a);
    a.rank = rank;
    int64_t out_str[LX_MAX_RANK];
    row_major_strides(rank, od, out_str);
    for (int i = 0; i < rank; i++) {
        a.dims[i] = od[i];
        a.src_str[i] = in_str[p[i]];
        a.dst_str[i] = out_str[i];
    }
    return view_copy(data->dtype, data->data, Y->data, a);
}

extern "C" int lx_Concat(const lx_tensor *const *inputs, int32_t n, int32_t axis, int32_t has_axis, lx_tensor *Y) {
    OpScope prof("Concat");
    REQUIRE_INIT();
    if (!inputs || n < 0) return missing_input("Concat", "inputs");
    int st;
    for (int i = 0; i < n; i++) {
        if (!inputs[i]) return missing_input("Concat", "inputs");
        if ((st = check_tensor(inputs[i], "inputs"))) return st;
    }
    if (n > 0) {
        for (int i = 1; i < n; i++)
            if (inputs[i]->dtype != inputs[0]->dtype)  // OpResult.WrongInputType naming inputs[0] (CPUExecutionProvider.cs:481)
                return set_err(LX_ERR_WRONG_INPUT_TYPE,
                               "The input tensor  for parameter inputs has type %s but is required to be %s. All tensors "
                               "in a concat operation must have the same type.",
                               dtype_name(inputs[0]->dtype), dtype_name(inputs[0]->dtype));
        if (!movable_dtype(inputs[0]->dtype)) return type_not_supported("Concat", "inputs", inputs[0]);
    }
    const int ax0 = has_axis ? axis : 0;
    // Tensor<T>.Concat(Tensor<T>[], axis) (TensorOps.cs:1487-1498)
    if (n < 2) return argument_error("At least two tensors must be specified for the concat operation.", "inputs");
    const int rank = inputs[0]->rank;
    for (int i = 1; i < n; i++)
        if (inputs[i]->rank != rank)
            return argument_error("Each input tensor in a concat operation must be of the same rank.", "inputs");
    for (int i = 1; i < n; i++)
        for (int d = 0; d < rank; d++)
            if (d != ax0 && inputs[i]->dims[d] != inputs[0]->dims[d])
                return argument_error("The dimensions of each tensor in a concat operation must be the same, with the "
                                      "exception of the axis dimension.", "inputs");
    const int ax = ax0 >= 0 ? ax0 : rank + ax0;  // the pairwise Concat normalises (TensorOps.cs:1454)
    if (ax < 0 || ax >= rank) return set_err(LX_ERR_INVALID_ARGUMENT, "Index was outside the bounds of the array.");
    // the pairwise concatenation (TensorOps.cs:1446-1480) writes index [0, ..., 0] of its output even
    // when that output is empty (the iterator's first index); so the call fails when the first pair
    // concatenates to nothing
    {
        int64_t first = inputs[0]->dims[ax] + inputs[1]->dims[ax];
        for (int d = 0; d < rank; d++)
            if (d != ax) first *= inputs[0]->dims[d];
        if (first == 0) return set_err(LX_ERR_INVALID_ARGUMENT, "Index was outside the bounds of the array.");
    }
    int64_t od[LX_MAX_RANK];
    for (int d = 0; d < rank; d++) od[d] = inputs[0]->dims[d];
    od[ax] = 0;
    for (int i = 0; i < n; i++) od[ax] += inputs[i]->dims[ax];
    if ((st = prepare_output(Y, inputs[0]->dtype, rank, od))) return st;
    // input i is a [outer, dims_i[ax] * inner] block at column off_i * inner of the [outer, total] output
    int64_t outer = 1, inner = 1;
    for (int d = 0; d < ax; d++) outer *= od[d];
    for (int d = ax + 1; d < rank; d++) inner *= od[d];
    std::vector<ConcatPart> parts;
    int64_t off = 0;
    for (int i = 0; i < n; i++) {
        const int64_t len = inputs[i]->dims[ax] * inner;
        if (outer * len >= (1ll << 31))
            return set_err(LX_ERR_NOT_SUPPORTED, "Concat inputs of 2^31 elements or more are not supported.");
        parts.push_back({inputs[i]->data, len, off});
        off += len;
    }
    if (outer * off == 0) return LX_OK;
    HIPCHECK(launch_concat((int)esize(inputs[0]->dtype), Y->data, outer, off, parts.data(), n, g.stream), "Concat");
    return LX_OK;
}

extern "C" int lx_Gather(const lx_tensor *data, const lx_tensor *indices, int32_t axis, int32_t has_axis,
                         lx_tensor *Y) {
    OpScope prof("Gather");
    REQUIRE_INIT();
    if (!data) return missing_input("Gather", "data");
    if (!indices) return missing_input("Gather", "indices");
    int st;
    if ((st = check_tensor(data, "data")) || (st = check_tensor(indices, "indices"))) return st;
    if (indices->rank > data->rank)
        return set_err(LX_ERR_WRONG_INPUT_SHAPE,
                       "The input tensor  for parameter indices has shape %s but is required to have rank %d.",
                       print_shape(indices).c_str(), data->rank);
    if (indices->dtype != LX_INT32 && indices->dtype != LX_INT64)
        return set_err(LX_ERR_WRONG_INPUT_TYPE, "Unable to cast object of type 'Lokad.Onnx.DenseTensor`1[%s]' to type "
                                                "'Lokad.Onnx.Tensor`1[System.Int32]'.",
                       net_type(indices->dtype));
    if (!movable_dtype(data->dtype)) return not_supported("Gather");
    if (data->rank == 0) return argument_error("Cannot gather from a tensor of rank 0.", "data");
    const int rank = data->rank;
    int ax = has_axis ? (axis >= 0 ? axis : rank + axis) : 0;
    if (ax > rank - 1)
        return argument_error(("The specified axis " + std::to_string(axis) +
                               " exceeds the number of dimensions in the tensor.").c_str(), "axis");
    if (ax < 0) return set_err(LX_ERR_INVALID_ARGUMENT, "Index was outside the bounds of the array.");
    int64_t od[LX_MAX_RANK * 2];
    int orank = 0;
    for (int d = 0; d < ax; d++) od[orank++] = data->dims[d];
    for (int d = 0; d < indices->rank; d++) od[orank++] = indices->dims[d];
    for (int d = ax + 1; d < rank; d++) od[orank++] = data->dims[d];
    if (orank > LX_MAX_RANK) return set_err(LX_ERR_NOT_SUPPORTED, "At most %d axes are supported.", LX_MAX_RANK);
    if ((st = prepare_output(Y, data->dtype, orank, od))) return st;
    int64_t outer = 1, inner = 1;
    for (int d = 0; d < ax; d++) outer *= data->dims[d];
    for (int d = ax + 1; d < rank; d++) inner *= data->dims[d];
    const int64_t nidx = numel(indices);
    // an empty output still has its index [0, ..., 0] visited by the reference's loop, which then
    // reads past the empty indices, data or output (TensorOps.cs:1432-1440)
    if (outer * nidx * inner == 0) return set_err(LX_ERR_INVALID_ARGUMENT, "Index was outside the bounds of the array.");
    if (outer * nidx * inner >= (1ll << 31))
        return set_err(LX_ERR_NOT_SUPPORTED, "Gathers of 2^31 elements or more are not supported.");
    // Int64 indices: ConvertToInt32 (ITensor.cs:172-183) throws on values outside int32; an index
    // that large is outside the axis anyway, so the range check below reports it
    ErrFlags *errs;
    if ((st = check_begin(kCheckGather, 0, &errs))) return st;
    // as integer Div's divisor scan: with at most 1/16 as many indices as output elements, a scan of the
    // indices queued before the gather decides whether the call fails, and a clean call returns while the
    // gather runs; an index out of range takes the gather's own record
    const bool prescan = !t_defer_slot && nidx * 16 <= outer * nidx * inner &&
                         !overlaps(Y->data, outer * nidx * inner * esize(data->dtype), indices->data,
                                   nidx * esize(indices->dtype));
    int scan_blocks = 0;
    uint64_t scan_seq = 0;
    if (prescan) {
        scan_blocks = index_scan_blocks(nidx);
        scan_seq = ++g.scan_seq;
        HIPCHECK(launch_index_scan(indices->dtype, indices->data, nidx, data->dims[ax], g.mail_dev->scan, scan_seq,
                                   g.stream),
                 "index scan");
    }
    HIPCHECK(launch_gather((int)esize(data->dtype), indices->dtype, data->data, indices->data, Y->data, outer, nidx,
                           inner, data->dims[ax], errs, g.stream),
             "Gather");
    if (prescan) {
        uint32_t bits = 0;
        if ((st = wait_scan(scan_blocks, scan_seq, &bits))) return st;
        if (bits == 0) {
            g.errs_clean = true;  // no index can be recorded: the record stays cleared
            return LX_OK;
        }
    }
    return check_end(kCheckGather, 0);
}

extern "C" int lx_Slice(const lx_tensor *data, const int64_t *starts, int32_t n_starts, const int64_t *ends,
                        int32_t n_ends, const int64_t *axes, int32_t n_axes, const int64_t *steps, int32_t n_steps,
                        lx_tensor *Y) {
    OpScope prof("Slice");
    REQUIRE_INIT();
    if (!data) return missing_input("Slice", "data");
    if (!starts || n_starts < 0) return missing_input("Slice", "starts");
    if (!ends || n_ends < 0) return missing_input("Slice", "ends");
    int st;
    if ((st = check_tensor(data, "data"))) return st;
    // CPUExecutionProvider.Slice checks (CPUExecutionProvider.cs:554-560); the rank-1 checks of the
    // starts / ends / axes / steps tensors are made by the caller that holds them as tensors
    auto shape_err = [&](const char *param, const std::string &shape, const char *msg) {
        return set_err(LX_ERR_WRONG_INPUT_SHAPE, "The input tensor  for parameter %s has shape %s. %s.", param,
                       shape.c_str(), msg);
    };
    const std::string sshape = "[" + std::to_string(n_starts) + "]", eshape = "[" + std::to_string(n_ends) + "]";
    if (data->rank == 0) return shape_err("data", print_shape(data), "Cannot slice a tensor of rank 0");
    if (n_starts > data->rank)
        return shape_err("starts", sshape,
                         "The length of the starts tensor must be less-than or equal to the rank of the data tensor.");
    if (n_starts != n_ends) return shape_err("ends", eshape, "The ends tensor must be the same length as the start tensor.");
    if (axes && n_axes != n_starts)
        return shape_err("axes", "[" + std::to_string(n_axes) + "]",
                         "The axes tensor must be a rank 1 tensor with the same length as the start tensor.");
    if (steps && n_steps != n_starts)
        return shape_err("steps", "[" + std::to_string(n_steps) + "]",
                         "The steps tensor must be a rank 1 tensor with the same length as the start tensor.");
    for (int i = 0; i < n_starts; i++) {
        const int64_t vals[4] = {starts[i], ends[i], axes ? axes[i] : 0, steps ? steps[i] : 1};
        for (int64_t v : vals)
            if (v < INT32_MIN || v > INT32_MAX)
                return set_err(LX_ERR_OVERFLOW, "Value was either too large or too small for an Int32.");
    }
    // Tensor<T>.Slice (TensorOps.cs:1500-1531) + SliceIndex.ToSliceDef (SliceIndex.cs:271-324)
    const int rank = data->rank;
    int64_t sstart[LX_MAX_RANK], sstep[LX_MAX_RANK], scount[LX_MAX_RANK];
    for (int d = 0; d < rank; d++) {
        sstart[d] = 0;
        sstep[d] = 1;
        scount[d] = data->dims[d];
    }
    int64_t ax[LX_MAX_RANK];
    for (int i = 0; i < n_starts; i++) {
        ax[i] = axes ? (axes[i] >= 0 ? axes[i] : rank + axes[i]) : i;
        if (ax[i] < 0 || ax[i] >= rank) return set_err(LX_ERR_INVALID_ARGUMENT, "Index was outside the bounds of the array.");
    }
    for (int d = 0; d < rank; d++) {
        int i = -1;  // axes.IndexOf(d): the first occurrence
        for (int k = 0; k < n_starts; k++)
            if (ax[k] == d) { i = k; break; }
        if (i < 0) continue;
        const int64_t dim = data->dims[d];
        auto clampn = [&](int64_t v) {
            v = v >= 0 ? v : dim + v;
            return v < 0 ? 0 : (v > dim ? dim : v);
        };
        int64_t start = clampn(starts[i]), stop = clampn(ends[i]);
        const int64_t step = steps ? steps[i] : 1;
        int64_t count = 0;
        if (step > 0) {
            if (start < dim && start < stop) count = (stop - start + step - 1) / step;
        } else if (step < 0) {
            if (start >= dim) start = dim - 1;
            if (start > stop) count = (start - stop + (-step) - 1) / (-step);
        }
        sstart[d] = count ? start : 0;
        sstep[d] = count ? step : 0;
        scount[d] = count;
    }
    if ((st = prepare_output(Y, data->dtype, rank, scount))) return st;
    ViewCopyArgs a;
    memset(&a, 0, sizeof a);
    a.rank = rank;
    int64_t in_str[LX_MAX_RANK], out_str[LX_MAX_RANK];
    row_major_strides(rank, data->dims, in_str);
    row_major_strides(rank, scount, out_str);
    for (int d = 0; d < rank; d++) {
        a.dims[d] = scount[d];
        a.src_str[d] = in_str[d] * sstep[d];
        a.dst_str[d] = out_str[d];
        a.src_base += sstart[d] * in_str[d];
    }
    return view_copy(data->dtype, data->data, Y->data, a);
}
