// lx_pool.h -- stream-ordered caching allocator for device tensors.
//
// All library work runs on one stream, so a block released by a tensor can be
// handed to the next allocation at once: every kernel that read the old
// contents was enqueued before any kernel that writes the new ones.  Released
// blocks wait in per-size-class free lists; hipFree only runs in pool_trim
// (after a stream synchronisation) or when a fresh hipMalloc reports
// out-of-memory, so a steady-state graph execution allocates nothing.
#pragma once

#include <hip/hip_runtime.h>
#include <stddef.h>
#include <stdint.h>

#include <vector>

namespace lx {

// Rounded capacity a request of `bytes` occupies (>= bytes, >= 256).
size_t pool_class(size_t bytes);

// Block of at least `bytes` (capacity reported through *cap); blocks come
// from the free list of the request's size class, else from hipMalloc.
hipError_t pool_alloc(size_t bytes, void **p, size_t *cap, hipStream_t s);

// Returns a block obtained from pool_alloc to its free list.  Returns false
// when `p` did not come from the pool (the caller then owns it).
bool pool_release(void *p);

// Synchronises `s` and hipFrees every cached block.
hipError_t pool_trim(hipStream_t s);

// Bytes held by live blocks and by cached (released) blocks.
void pool_stats(int64_t *live, int64_t *cached);

// HIP-graph capture support.  pool_record_begin / pool_record_end return every
// block pool_alloc handed out in between (work captured into a HIP graph uses
// them on every replay).  pool_hold keeps such blocks from being handed out
// again -- a held block released by its owner stays reserved -- until
// pool_unhold, which returns the released ones to the free lists.
void pool_record_begin();
std::vector<void *> pool_record_end();
void pool_hold(const std::vector<void *> &blocks);
void pool_unhold(const std::vector<void *> &blocks);

}  // namespace lx
