// lx_pool.cpp -- see lx_pool.h.
#include "lx_pool.h"

#include <algorithm>
#include <mutex>
#include <unordered_map>
#include <vector>

namespace lx {

namespace {

struct PoolState {
    std::mutex mu;
    std::unordered_map<size_t, std::vector<void *>> free_lists;  // size class -> cached blocks
    std::unordered_map<void *, size_t> live;                     // block -> size class
    int64_t live_bytes = 0, cached_bytes = 0;
    bool recording = false;
    std::vector<void *> recorded;                                // blocks handed out while recording
    std::unordered_map<void *, bool> held;                       // held block -> released by its owner
};

PoolState &pool() {
    static PoolState *p = new PoolState();  // never destroyed: blocks may be released at process exit
    return *p;
}

hipError_t free_cached_locked(PoolState &ps) {
    hipError_t first = hipSuccess;
    for (auto &kv : ps.free_lists) {
        for (void *b : kv.second) {
            hipError_t e = hipFree(b);
            if (e != hipSuccess && first == hipSuccess) first = e;
        }
        kv.second.clear();
    }
    ps.free_lists.clear();
    ps.cached_bytes = 0;
    return first;
}

}  // namespace

// Classes: powers of two up to 1 MiB, then multiples of 2 MiB, so a reused
// block wastes at most half of a small request and under 2 MiB of a large one.
size_t pool_class(size_t bytes) {
    if (bytes <= 256) return 256;
    if (bytes <= (1u << 20)) {
        size_t c = 512;
        while (c < bytes) c <<= 1;
        return c;
    }
    const size_t g = 2u << 20;
    return (bytes + g - 1) / g * g;
}

hipError_t pool_alloc(size_t bytes, void **p, size_t *cap, hipStream_t s) {
    PoolState &ps = pool();
    const size_t c = pool_class(bytes);
    std::lock_guard<std::mutex> lock(ps.mu);
    auto it = ps.free_lists.find(c);
    if (it != ps.free_lists.end() && !it->second.empty()) {
        *p = it->second.back();
        it->second.pop_back();
        ps.cached_bytes -= (int64_t)c;
    } else {
        hipError_t e = hipMalloc(p, c);
        if (e == hipErrorOutOfMemory && ps.cached_bytes > 0) {
            (void)hipGetLastError();
            e = hipStreamSynchronize(s);
            if (e != hipSuccess) return e;
            e = free_cached_locked(ps);
            if (e != hipSuccess) return e;
            e = hipMalloc(p, c);
        }
        if (e != hipSuccess) return e;
    }
    ps.live[*p] = c;
    ps.live_bytes += (int64_t)c;
    if (ps.recording) ps.recorded.push_back(*p);
    if (cap) *cap = c;
    return hipSuccess;
}

bool pool_release(void *p) {
    PoolState &ps = pool();
    std::lock_guard<std::mutex> lock(ps.mu);
    auto it = ps.live.find(p);
    if (it == ps.live.end()) return false;
    auto h = ps.held.find(p);
    if (h != ps.held.end()) {  // reserved for a captured graph: stays live until unheld
        h->second = true;
        return true;
    }
    const size_t c = it->second;
    ps.live.erase(it);
    ps.live_bytes -= (int64_t)c;
    ps.free_lists[c].push_back(p);
    ps.cached_bytes += (int64_t)c;
    return true;
}

hipError_t pool_trim(hipStream_t s) {
    PoolState &ps = pool();
    std::lock_guard<std::mutex> lock(ps.mu);
    hipError_t e = hipStreamSynchronize(s);
    if (e != hipSuccess) return e;
    return free_cached_locked(ps);
}

void pool_record_begin() {
    PoolState &ps = pool();
    std::lock_guard<std::mutex> lock(ps.mu);
    ps.recording = true;
    ps.recorded.clear();
}

std::vector<void *> pool_record_end() {
    PoolState &ps = pool();
    std::lock_guard<std::mutex> lock(ps.mu);
    ps.recording = false;
    std::vector<void *> out;
    out.swap(ps.recorded);
    std::sort(out.begin(), out.end());
    out.erase(std::unique(out.begin(), out.end()), out.end());
    return out;
}

void pool_hold(const std::vector<void *> &blocks) {
    PoolState &ps = pool();
    std::lock_guard<std::mutex> lock(ps.mu);
    for (void *p : blocks) {
        if (ps.held.count(p)) continue;
        if (ps.live.count(p)) {  // still owned
            ps.held[p] = false;
            continue;
        }
        // released into a free list during the recording: take it back out
        for (auto &kv : ps.free_lists) {
            auto f = std::find(kv.second.begin(), kv.second.end(), p);
            if (f == kv.second.end()) continue;
            kv.second.erase(f);
            ps.cached_bytes -= (int64_t)kv.first;
            ps.live[p] = kv.first;
            ps.live_bytes += (int64_t)kv.first;
            ps.held[p] = true;
            break;
        }
    }
}

void pool_unhold(const std::vector<void *> &blocks) {
    PoolState &ps = pool();
    std::lock_guard<std::mutex> lock(ps.mu);
    for (void *p : blocks) {
        auto h = ps.held.find(p);
        if (h == ps.held.end()) continue;
        const bool released = h->second;
        ps.held.erase(h);
        if (!released) continue;  // its owner still holds it and releases it later
        auto it = ps.live.find(p);
        if (it == ps.live.end()) continue;
        const size_t c = it->second;
        ps.live.erase(it);
        ps.live_bytes -= (int64_t)c;
        ps.free_lists[c].push_back(p);
        ps.cached_bytes += (int64_t)c;
    }
}

void pool_stats(int64_t *live, int64_t *cached) {
    PoolState &ps = pool();
    std::lock_guard<std::mutex> lock(ps.mu);
    if (live) *live = ps.live_bytes;
    if (cached) *cached = ps.cached_bytes;
}

}  // namespace lx
