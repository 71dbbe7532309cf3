// TEST HELPER (device): checks on the GPU that the v_rcp_f32-seeded reciprocal
// used by the Erf / GELU kernels (recip_newton1 in lx_device.h) equals IEEE
// float division 1.0f / d for every float d in [1, 2^126), and measures the
// largest relative error of v_rcp_f32 itself over every float in [1, 2^31]
// (the seeds of the integer division, sdiv32_core).  Built for gfx950 by
// __graft_entry__.build(); called by the GPU tests through ctypes.
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "../../onnx_amd/csrc/lx_device.h"

namespace {

constexpr uint32_t kLo = 0x3f800000u;  // 1.0f
constexpr uint32_t kHi = 0x7e800000u;  // 2^126

// counts[0]: recip_newton1 from the v_rcp_f32 seed != 1/d; counts[1]: seed != 1/d (informational: the
// seeds the Newton step repairs); counts[2]: seed != 1/d where d's significand is all ones
__global__ void k_check(unsigned long long *counts) {
    unsigned long long bad = 0, seed_off = 0, ones_off = 0;
    const uint32_t stride = gridDim.x * blockDim.x;
    for (uint32_t u = kLo + blockIdx.x * blockDim.x + threadIdx.x; u < kHi; u += stride) {
        const float d = __builtin_bit_cast(float, u);
        const float cr = 1.0f / d;
        const float seed = __builtin_amdgcn_rcpf(d);
        const float y = lx::recip_newton1(d, seed);
        bad += __builtin_bit_cast(uint32_t, y) != __builtin_bit_cast(uint32_t, cr);
        const bool off = __builtin_bit_cast(uint32_t, seed) != __builtin_bit_cast(uint32_t, cr);
        seed_off += off;
        ones_off += off && (u & 0x7fffffu) == 0x7fffffu;
    }
    if (bad) atomicAdd(&counts[0], bad);
    if (seed_off) atomicAdd(&counts[1], seed_off);
    if (ones_off) atomicAdd(&counts[2], ones_off);
}

// largest |rcp(d) * d - 1| over the floats d in [1, 2^31], as the bit pattern
// of a non-negative double (which orders like the double); the product of two
// floats is exact in double
constexpr uint32_t kIntHi = 0x4f000000u;  // 2^31
__global__ void k_rcp_error(unsigned long long *max_bits) {
    double worst = 0.0;
    const uint32_t stride = gridDim.x * blockDim.x;
    for (uint32_t u = kLo + blockIdx.x * blockDim.x + threadIdx.x; u <= kIntHi; u += stride) {
        const float d = __builtin_bit_cast(float, u);
        const double err = __builtin_fabs((double)__builtin_amdgcn_rcpf(d) * (double)d - 1.0);
        worst = err > worst ? err : worst;
    }
    worst = lx::wave_reduce(worst, [](double x, double y) { return x > y ? x : y; });
    if ((threadIdx.x & 63) == 0) atomicMax(max_bits, (unsigned long long)__builtin_bit_cast(uint64_t, worst));
}

}  // namespace

extern "C" int lx_test_device_rcp_error(double *out) {
    unsigned long long *d = nullptr;
    hipError_t e = hipMalloc(&d, sizeof(unsigned long long));
    if (e != hipSuccess) return (int)e;
    e = hipMemset(d, 0, sizeof(unsigned long long));
    if (e == hipSuccess) {
        hipLaunchKernelGGL(k_rcp_error, dim3(8192), dim3(256), 0, 0, d);
        e = hipGetLastError();
    }
    unsigned long long bits = 0;
    if (e == hipSuccess) e = hipMemcpy(&bits, d, sizeof(bits), hipMemcpyDeviceToHost);
    (void)hipFree(d);
    *out = __builtin_bit_cast(double, (uint64_t)bits);
    return (int)e;
}

extern "C" int lx_test_device_recip(long long *out) {
    unsigned long long *d = nullptr;
    hipError_t e = hipMalloc(&d, 3 * sizeof(unsigned long long));
    if (e != hipSuccess) return (int)e;
    e = hipMemset(d, 0, 3 * sizeof(unsigned long long));
    if (e == hipSuccess) {
        hipLaunchKernelGGL(k_check, dim3(8192), dim3(256), 0, 0, d);
        e = hipGetLastError();
    }
    if (e == hipSuccess) e = hipMemcpy(out, d, 3 * sizeof(unsigned long long), hipMemcpyDeviceToHost);
    (void)hipFree(d);
    return (int)e;
}

