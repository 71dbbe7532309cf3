// lx_probe.hip -- bandwidth ceiling of a pure HBM read on gfx950 (diagnostic, no reference
// counterpart).  The operators' kernels are judged against what the part sustains: a read-only
// stream is the ceiling of the reductions (ReduceMean over a whole tensor reads 1 GiB and writes
// four bytes); a copy is the ceiling of the elementwise operators (Cast float -> float is the
// library's copy).
#include <hip/hip_runtime.h>

#include "lx_device.h"
#include "lx_kernels.h"

namespace lx {

namespace {
constexpr int kProbeBlock = 256;
constexpr int kProbeU = 4;  // 16-byte vectors in flight per lane
}  // namespace

// Each block reads U * 256 consecutive 16-byte vectors per grid-stride step with nontemporal loads
// (all issued before any is folded) and writes the XOR of what it read as one word, so no load can be
// dropped by the compiler and the writes are negligible.
__global__ __launch_bounds__(kProbeBlock) void k_read_probe(const u32x4 *__restrict__ src, int64_t nv,
                                                            uint32_t *__restrict__ out) {
    uint32_t acc = 0;
    for (int64_t i0 = (int64_t)blockIdx.x * kProbeBlock * kProbeU + threadIdx.x; i0 < nv;
         i0 += (int64_t)gridDim.x * kProbeBlock * kProbeU) {
        u32x4 v[kProbeU];
#pragma unroll
        for (int u = 0; u < kProbeU; u++)
            v[u] = i0 + u * kProbeBlock < nv ? __builtin_nontemporal_load(src + i0 + u * kProbeBlock) : u32x4{0, 0, 0, 0};
#pragma unroll
        for (int u = 0; u < kProbeU; u++) acc ^= v[u].x ^ v[u].y ^ v[u].z ^ v[u].w;
    }
    acc = wave_reduce(acc, [](uint32_t a, uint32_t b) { return a ^ b; });
    __shared__ uint32_t part[kProbeBlock / 64];
    if ((threadIdx.x & 63) == 0) part[threadIdx.x >> 6] = acc;
    __syncthreads();
    if (threadIdx.x == 0) out[blockIdx.x] = part[0] ^ part[1] ^ part[2] ^ part[3];
}

// blocks: one per U * 256 vectors, at most max_blocks (the words `out` holds)
hipError_t launch_read_probe(const void *src, int64_t bytes, uint32_t *out, int64_t max_blocks, hipStream_t s) {
    const int64_t nv = bytes / 16;
    if (nv <= 0 || max_blocks <= 0) return hipSuccess;
    int64_t g = (nv + kProbeBlock * kProbeU - 1) / (kProbeBlock * kProbeU);
    if (g > max_blocks) g = max_blocks;
    hipLaunchKernelGGL(k_read_probe, dim3((unsigned)g), dim3(kProbeBlock), 0, s, (const u32x4 *)src, nv, out);
    return hipGetLastError();
}

}  // namespace lx
