// lx_device.h -- device-side building blocks shared by the gfx950 kernels.
//
// Compiled with -ffp-contract=off: every float/double operation written here
// rounds separately unless an explicit fma() is written, so the elementwise
// results keep the per-operation IEEE roundings of the C# reference.
#pragma once

#include <hip/hip_runtime.h>

// The exact float reciprocal of Erf / GELU (recip_newton1: one Newton step) and the int32 division seed
// are proven with gfx950's v_rcp_f32 (every seed checked on that device); another architecture's
// reciprocal could land on the significands where one step is not exact.
#if defined(__HIP_DEVICE_COMPILE__) && !defined(__gfx950__)
#error "liblonnx_hip device code is built for gfx950 only"
#endif
#include <stdint.h>

#include <type_traits>

#include "lx_plan.h"

#pragma clang fp contract(off)

namespace lx {

// ---------------------------------------------------------------------------
// 16-byte (or smaller) register vectors used for coalesced global access.
// ---------------------------------------------------------------------------
template <typename T, int N>
struct alignas((sizeof(T) * N) >= 16 ? 16 : (sizeof(T) * N)) Vec {
    T v[N];
};

template <typename T>
struct VecWidth {
    static constexpr int value = 16 / sizeof(T);
};

template <typename T, int N>
__device__ __forceinline__ Vec<T, N> vload(const T *p) {
    return *reinterpret_cast<const Vec<T, N> *>(p);
}

template <typename T, int N>
__device__ __forceinline__ void vstore(T *p, const Vec<T, N> &v) {
    *reinterpret_cast<Vec<T, N> *>(p) = v;
}

// Streaming (nontemporal) access: data read or written once bypasses cache
// retention; measured on MI355X it lifts a 1 GiB copy from 6.26 to 6.68 TB/s
// and a 1 GiB read from 6.5 to 7.2 TB/s.
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));

template <typename T, int N>
__device__ __forceinline__ Vec<T, N> vload_nt(const T *p) {
    constexpr int B = (int)sizeof(T) * N;
    if constexpr (B == 16) {
        return __builtin_bit_cast(Vec<T, N>, __builtin_nontemporal_load(reinterpret_cast<const u32x4 *>(p)));
    } else if constexpr (B == 8) {
        return __builtin_bit_cast(Vec<T, N>, __builtin_nontemporal_load(reinterpret_cast<const u32x2 *>(p)));
    } else if constexpr (B == 4) {
        return __builtin_bit_cast(Vec<T, N>, __builtin_nontemporal_load(reinterpret_cast<const uint32_t *>(p)));
    } else if constexpr (B == 2) {
        return __builtin_bit_cast(Vec<T, N>, __builtin_nontemporal_load(reinterpret_cast<const uint16_t *>(p)));
    } else if constexpr (B == 1) {
        return __builtin_bit_cast(Vec<T, N>, __builtin_nontemporal_load(reinterpret_cast<const uint8_t *>(p)));
    } else {
        static_assert(B % 16 == 0, "multi-chunk vectors are whole 16-byte chunks");
        struct Chunks {
            u32x4 c[B / 16];
        } r;
#pragma unroll
        for (int i = 0; i < B / 16; i++) r.c[i] = __builtin_nontemporal_load(reinterpret_cast<const u32x4 *>(p) + i);
        return __builtin_bit_cast(Vec<T, N>, r);
    }
}

template <typename T, int N>
__device__ __forceinline__ void vstore_nt(T *p, const Vec<T, N> &v) {
    constexpr int B = (int)sizeof(T) * N;
    if constexpr (B == 16) {
        __builtin_nontemporal_store(__builtin_bit_cast(u32x4, v), reinterpret_cast<u32x4 *>(p));
    } else if constexpr (B == 8) {
        __builtin_nontemporal_store(__builtin_bit_cast(u32x2, v), reinterpret_cast<u32x2 *>(p));
    } else if constexpr (B == 4) {
        __builtin_nontemporal_store(__builtin_bit_cast(uint32_t, v), reinterpret_cast<uint32_t *>(p));
    } else if constexpr (B == 2) {
        __builtin_nontemporal_store(__builtin_bit_cast(uint16_t, v), reinterpret_cast<uint16_t *>(p));
    } else if constexpr (B == 1) {
        __builtin_nontemporal_store(__builtin_bit_cast(uint8_t, v), reinterpret_cast<uint8_t *>(p));
    } else {
        static_assert(B % 16 == 0, "multi-chunk vectors are whole 16-byte chunks");
        struct Chunks {
            u32x4 c[B / 16];
        };
        Chunks r = __builtin_bit_cast(Chunks, v);
#pragma unroll
        for (int i = 0; i < B / 16; i++) __builtin_nontemporal_store(r.c[i], reinterpret_cast<u32x4 *>(p) + i);
    }
}

__device__ __forceinline__ uint32_t fdiv(uint32_t n, const FastDiv &f) {
    return (__umulhi(n, f.m) + n) >> f.s;
}

// ---------------------------------------------------------------------------
// Wave64 reductions (butterfly over __shfl_xor; fixed order -> deterministic).
// ---------------------------------------------------------------------------
template <typename T, typename F>
__device__ __forceinline__ T wave_reduce(T v, F f) {
#pragma unroll
    for (int off = 32; off >= 1; off >>= 1) {
        T o = __shfl_xor(v, off, 64);
        v = f(v, o);
    }
    return v;
}

// Wave64 reduction of a float over data-parallel-primitive (DPP) lane moves, which
// issue as ordinary VALU operations, instead of the LDS crossbar that __shfl_xor
// compiles to (ds_bpermute: tens of cycles each, six in a chain).  Within each
// 16-lane row: quad_perm [1,0,3,2] and [2,3,0,1] (pairs, then quads),
// row_half_mirror (lane i with 7 - i: the two quads of each half row) and
// row_mirror (lane i with 15 - i: the two halves); every lane of a row then holds
// the row's value.  The four rows are read from lanes 0, 16, 32, 48 and combined
// as f(f(r0, r1), f(r2, r3)).  A fixed order: deterministic, and the same value in
// every lane.
template <int CTRL>
__device__ __forceinline__ float dpp_move(float v) {
    return __builtin_bit_cast(float, __builtin_amdgcn_mov_dpp(__builtin_bit_cast(int, v), CTRL, 0xf, 0xf, false));
}

template <typename F>
__device__ __forceinline__ float wave_reduce_dpp(float v, F f) {
    v = f(v, dpp_move<0xb1>(v));   // quad_perm [1,0,3,2]
    v = f(v, dpp_move<0x4e>(v));   // quad_perm [2,3,0,1]
    v = f(v, dpp_move<0x141>(v));  // row_half_mirror
    v = f(v, dpp_move<0x140>(v));  // row_mirror
    const int b = __builtin_bit_cast(int, v);
    const float r0 = __builtin_bit_cast(float, __builtin_amdgcn_readlane(b, 0));
    const float r1 = __builtin_bit_cast(float, __builtin_amdgcn_readlane(b, 16));
    const float r2 = __builtin_bit_cast(float, __builtin_amdgcn_readlane(b, 32));
    const float r3 = __builtin_bit_cast(float, __builtin_amdgcn_readlane(b, 48));
    return f(f(r0, r1), f(r2, r3));
}

// Reduction within aligned groups of L lanes (L a power of two, at most 64): every lane of a group ends
// with the group's value.  Float over DPP for the steps inside a 16-lane row -- quad_perm [1,0,3,2] and
// [2,3,0,1], then row_half_mirror and row_mirror, each combining two halves that already hold their own
// values, so with a commutative f every lane gets the same result -- and a shuffle across rows for L = 32;
// other types over the shuffle butterfly; the whole wave as wave_reduce_dpp / wave_reduce.  A fixed order:
// deterministic.
template <int L, typename T, typename F>
__device__ __forceinline__ T group_reduce(T v, F f) {
    static_assert(L >= 1 && L <= 64 && (L & (L - 1)) == 0, "groups of 1 to 64 lanes");
    if constexpr (L == 64) {
        if constexpr (std::is_same<T, float>::value) return wave_reduce_dpp(v, f);
        else return wave_reduce(v, f);
    } else if constexpr (std::is_same<T, float>::value) {
        if constexpr (L >= 2) v = f(v, dpp_move<0xb1>(v));
        if constexpr (L >= 4) v = f(v, dpp_move<0x4e>(v));
        if constexpr (L >= 8) v = f(v, dpp_move<0x141>(v));
        if constexpr (L >= 16) v = f(v, dpp_move<0x140>(v));
        if constexpr (L >= 32) v = f(v, __shfl_xor(v, 16, 64));
    } else {
#pragma unroll
        for (int off = L / 2; off >= 1; off >>= 1) v = f(v, __shfl_xor(v, off, 64));
    }
    return v;
}

// ---------------------------------------------------------------------------
// expf bit-identical to the host glibc expf that .NET's MathF.Exp calls.
//
// Method: ARM Optimized Routines expf (Szabolcs Nagy, 2017; the expf of glibc
// >= 2.27, selected as its FMA variant on x86-64 CPUs with FMA):
//   x*N/ln2 = k + r, N = 32, |r| <= 1/2
//   2^(k/N) from a 32-entry table T[i] = bits(2^(i/32)) - (i << 47)
//   2^(r/N) ~= C0 r^3 + C1 r^2 + C2 r + 1
// evaluated in double with fused multiply-adds, rounded once to float.
// The table entries are the correctly rounded doubles of 2^(i/32); the
// polynomial coefficients are the published ones of that routine.  The host
// evaluation of this same function (tests/native/expf_check.cpp) is
// compared with the host expf over all 2^32 inputs by the test suite.
// ---------------------------------------------------------------------------
#define LX_EXP2F_TABLE                                                                              \
    {0x3ff0000000000000ULL, 0x3fefd9b0d3158574ULL, 0x3fefb5586cf9890fULL, 0x3fef9301d0125b51ULL,    \
     0x3fef72b83c7d517bULL, 0x3fef54873168b9aaULL, 0x3fef387a6e756238ULL, 0x3fef1e9df51fdee1ULL,    \
     0x3fef06fe0a31b715ULL, 0x3feef1a7373aa9cbULL, 0x3feedea64c123422ULL, 0x3feece086061892dULL,    \
     0x3feebfdad5362a27ULL, 0x3feeb42b569d4f82ULL, 0x3feeab07dd485429ULL, 0x3feea47eb03a5585ULL,    \
     0x3feea09e667f3bcdULL, 0x3fee9f75e8ec5f74ULL, 0x3feea11473eb0187ULL, 0x3feea589994cce13ULL,    \
     0x3feeace5422aa0dbULL, 0x3feeb737b0cdc5e5ULL, 0x3feec49182a3f090ULL, 0x3feed503b23e255dULL,    \
     0x3feee89f995ad3adULL, 0x3feeff76f2fb5e47ULL, 0x3fef199bdd85529cULL, 0x3fef3720dcef9069ULL,    \
     0x3fef5818dcfba487ULL, 0x3fef7c97337b9b5fULL, 0x3fefa4afa2a490daULL, 0x3fefd0765b6e4540ULL}

#define LX_EXPF_INVLN2N (0x1.71547652b82fep+0 * 32.0)
#define LX_EXPF_SHIFT 0x1.8p+52
#define LX_EXPF_C0 (0x1.c6af84b912394p-5 / 32.0 / 32.0 / 32.0)
#define LX_EXPF_C1 (0x1.ebfce50fac4f3p-3 / 32.0 / 32.0)
#define LX_EXPF_C2 (0x1.62e42ff0c52d6p-1 / 32.0)

// Table copy held in LDS by every kernel that evaluates expf.
struct ExpTable {
    uint64_t t[32];
};

static __constant__ uint64_t kExp2fTable[32] = LX_EXP2F_TABLE;

// One load and one LDS write per lane for the first 32 lanes; callers place a
// barrier before the first lookup.
__device__ __forceinline__ void exp_table_fill(ExpTable &s) {
    if (threadIdx.x < 32) s.t[threadIdx.x] = kExp2fTable[threadIdx.x];
}

// The same fill into a table that only the calling wave reads (one-wave blocks,
// or one table per wave): lanes 0..31 write one entry each.  A wave's LDS
// operations execute in issue order, so its later lookups see the entries; the
// wavefront-scope fences and the wave barrier keep the compiler from moving a
// lookup above the writes.  No block barrier: a block's first global loads can
// be issued before the fill and are not held up by it.
__device__ __forceinline__ void exp_table_fill_wave(ExpTable &s) {
    const int lane = threadIdx.x & 63;
    if (lane < 32) s.t[lane] = kExp2fTable[lane];
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
}

// Fills a table on the host (host restatement used by the tests).
__host__ inline void exp_table_fill_host(ExpTable &s) {
    constexpr uint64_t tab[32] = LX_EXP2F_TABLE;
    for (int i = 0; i < 32; i++) s.t[i] = tab[i];
}

// 2^(k/32) as a double: the table entry for k mod 32 plus k << 47 added to its
// bit pattern.  The added term has no bits below 47, so only the upper 32-bit
// word changes: one 32-bit shift-add instead of a 64-bit shift and add.
typedef uint32_t u32x2_lx __attribute__((ext_vector_type(2)));
__host__ __device__ __forceinline__ double expf_scale(uint64_t ki, const ExpTable &tab) {
    u32x2_lx t = __builtin_bit_cast(u32x2_lx, tab.t[ki & 31]);
    t.y += (uint32_t)ki << 15;
    return __builtin_bit_cast(double, t);
}

// The glibc expf method (ARM optimized-routines, N = 32 table, degree-3
// polynomial, FMA variant) without its special-case early-outs: equal to the
// host expf for every x in [-104, 88], and +0 like the host's for x in
// [-105.07, -104) (callers bound the argument).  The polynomial
// 1 + C2 r + C1 r^2 + C0 r^3 is evaluated in Horner form (three FMAs) where the
// published routine splits it (C0 r + C1, r^2, C2 r + 1, one FMA joining them)
// for instruction-level parallelism: the two doubles differ in their last bits
// only, and on every float x in [-104, 88] both round to the host expf's float
// (checked by exhaustion on the host), with one instruction less.
__host__ __device__ __forceinline__ float expf_core_lx(float x, const ExpTable &tab) {
    double xd = (double)x;
    double kd = __builtin_fma(LX_EXPF_INVLN2N, xd, LX_EXPF_SHIFT);
    uint64_t ki = __builtin_bit_cast(uint64_t, kd);
    kd -= LX_EXPF_SHIFT;
    double r = __builtin_fma(LX_EXPF_INVLN2N, xd, -kd);
    double s = expf_scale(ki, tab);
    double y = __builtin_fma(LX_EXPF_C0, r, LX_EXPF_C1);
    y = __builtin_fma(y, r, LX_EXPF_C2);
    y = __builtin_fma(y, r, 1.0);
    y = y * s;
    return (float)y;
}

__host__ __device__ __forceinline__ float expf_lx(float x, const ExpTable &tab) {
    uint32_t ux = __builtin_bit_cast(uint32_t, x);
    uint32_t abstop = (ux >> 20) & 0x7ff;
    if (__builtin_expect(abstop >= 0x42b, 0)) {  // top12(88.0f) == 0x42b
        if (ux == 0xff800000u) return 0.0f;          // -inf
        if (abstop >= 0x7f8) return x + x;            // inf or nan
        if (x > 0x1.62e42ep6f) return __builtin_inff();
        if (x < -0x1.9fe368p6f) return 0.0f;
    }
    return expf_core_lx(x, tab);
}

// expf for arguments <= 0 (or NaN), as produced by Erf (-x*x) and Softmax
// (x - max): the early-out branches collapse into one select.  Arguments below
// -104 are raised to -104, whose exponential (6.8e-46) rounds to +0 like every
// argument below the host expf's underflow threshold -0x1.9fe368p6; NaN passes
// through the select unchanged.  Checked against the host expf for every
// non-positive float by the test suite.
__host__ __device__ __forceinline__ float expf_nonpos_lx(float x, const ExpTable &tab) {
    x = x < -104.0f ? -104.0f : x;
    return expf_core_lx(x, tab);
}

// Float quotient x / 1.4142135f (= float32(sqrt 2)) without a division, in two
// float operations: q = fma(x, zh, x * zl) with zh + zl the reciprocal of the
// divisor split into two floats (zh = 1/c rounded to float, zl = the rest
// rounded to float; Brisebarre, Muller and Raina, "Accelerating correctly
// rounded floating-point division when the divisor is known in advance", IEEE
// Trans. Computers 53(8), 2004).  Correctly rounded for every |x| >= 2^-100
// (checked by exhaustion on the host); below that x * zl loses bits to
// underflow and the quotient can be one ulp off, which the GELU element never
// sees (there d = 1 and the exponential is 1 whatever the quotient's last bit:
// its own exhaustive check covers these inputs).
#define LX_INV_SQRT2F_HI 0x1.6a09e6p-1f
#define LX_INV_SQRT2F_LO 0x1.9fcef4p-26f
__host__ __device__ __forceinline__ float div_sqrt2f_lx(float x) {
    return __builtin_fmaf(x, LX_INV_SQRT2F_HI, x * LX_INV_SQRT2F_LO);
}

// Correctly rounded 1/d for d in [1, 2^126) from a float seed by one float Newton step, e = 1 - d*y (one FMA),
// y' = y + e*y (one FMA).  From the correctly rounded seed the result is exact for every such d; from a seed one
// ulp off it is exact except at 33 significands per binade (32 seeds from above, 1 from below): both checked by
// enumeration on the host.  v_rcp_f32 is one ulp off on about a tenth of the floats, but never at those 33
// significands: with its seed the step equals IEEE 1.0f / d for every float d in [1, 2^126), checked on the
// device for every d by the test suite.
__host__ __device__ __forceinline__ float recip_newton1(float d, float seed) {
    const float e = __builtin_fmaf(-d, seed, 1.0f);
    return __builtin_fmaf(e, seed, seed);
}

// Truncated quotient a / b of int32 operands (b != 0, not INT_MIN / -1) in
// double precision, in place of the integer expansion (five quarter-rate
// 32-bit multiplies plus sign fix-ups): y = 1/b from a seed of relative error
// below 2^-21, one Newton step (error e -> e^2 + 2^-53, below 2^-41.9), then
// q = trunc((a + sign(a) * 0.5) * y).
// Exact: (|a| + 0.5)/|b| = |q| + f with f in [0.5/|b|, 1 - 0.5/|b|], and the
// computed product is within ((2^31 + 0.5)/|b|) * 2^-41.8 < 2^-10/|b| of that
// value (the conversions and a +- 0.5 are exact), so truncation lands on q.
// Checked on the host against integer division with seeds perturbed by
// +-2^-21; the device seed is v_rcp_f32 of the float nearest b, whose error
// (rcp within 2^-22 on every float in [1, 2^31], checked on the device, plus
// 2^-24 for rounding b to float) stays below 2^-21.
// The two halves are separate so that a divisor shared by several dividends
// has its reciprocal computed once; sdiv32_core is their composition.
template <typename SeedFn>
__host__ __device__ __forceinline__ double sdiv32_recip(int32_t b, SeedFn seed) {
    const double d = (double)b;
    double y = seed(d);
    const double e = __builtin_fma(-d, y, 1.0);
    return __builtin_fma(e, y, y);
}

__host__ __device__ __forceinline__ int32_t sdiv32_quot(int32_t a, double y) {
    const double n = (double)a;
    return (int32_t)((n + __builtin_copysign(0.5, n)) * y);
}

template <typename SeedFn>
__host__ __device__ __forceinline__ int32_t sdiv32_core(int32_t a, int32_t b, SeedFn seed) {
    return sdiv32_quot(a, sdiv32_recip(b, seed));
}

struct RcpSeedF32 {
    __device__ __forceinline__ double operator()(double d) const { return (double)__builtin_amdgcn_rcpf((float)d); }
};

__device__ __forceinline__ int32_t sdiv32_lx(int32_t a, int32_t b) { return sdiv32_core(a, b, RcpSeedF32()); }
__device__ __forceinline__ double sdiv32_recip_lx(int32_t b) { return sdiv32_recip(b, RcpSeedF32()); }

// ---------------------------------------------------------------------------
// MathOps.Erf(float) (MathOps.cs:988-1010): Abramowitz & Stegun 7.1.26 in
// float32, one rounding per operation, exp = expf_lx.
// ---------------------------------------------------------------------------
__host__ __device__ __forceinline__ float erf_lx(float x, const ExpTable &tab) {
    const float a1 = 0.254829592f;
    const float a2 = -0.284496736f;
    const float a3 = 1.421413741f;
    const float a4 = -1.453152027f;
    const float a5 = 1.061405429f;
    const float p = 0.3275911f;
    float sign = x < 0.0f ? -1.0f : 1.0f;
    x = __builtin_fabsf(x);
    float t = 1.0f / (1.0f + p * x);
    float poly = ((((a5 * t + a4) * t) + a3) * t + a2) * t + a1;
    float e = expf_lx(-x * x, tab);
    float y = 1.0f - poly * t * e;
    return sign * y;
}

// a / s for many a and one s > 0, given rs = 1/s correctly rounded: the
// product is corrected by one FMA residual step (Markstein).  Used where the
// divisor is a row statistic (Softmax sum, LayerNorm deviation), whose value
// already differs from the reference's by summation order.
__device__ __forceinline__ float div_by_row_lx(float a, float s, float rs) {
    float q = a * rs;
    float rem = __builtin_fmaf(-q, s, a);
    return __builtin_fmaf(rem, rs, q);
}

// erf_lx with its division and exponential replaced by exact equivalents.
// d = 1 + p|x| is clamped to 2^125 before the reciprocal: d >= 2^125 means
// |x| > 1.3e38, where expf(-x*x) is exactly 0 and the product poly*t*0 is 0
// for any finite t; NaN also clamps and still yields NaN through expf.  The
// result equals erf_lx bit for bit for all 2^32 inputs (checked on the host
// with the correctly rounded seed; recip_newton1 gives the same reciprocal
// from the device seed, checked on the device for every d).
template <typename SeedFn>
__host__ __device__ __forceinline__ float erf_fast_core(float x, const ExpTable &tab, SeedFn seed) {
    const float a1 = 0.254829592f;
    const float a2 = -0.284496736f;
    const float a3 = 1.421413741f;
    const float a4 = -1.453152027f;
    const float a5 = 1.061405429f;
    const float p = 0.3275911f;
    float sign = x < 0.0f ? -1.0f : 1.0f;
    x = __builtin_fabsf(x);
    float d = 1.0f + p * x;
    d = d < 0x1p125f ? d : 0x1p125f;
    float t = recip_newton1(d, seed(d));
    float poly = ((((a5 * t + a4) * t) + a3) * t + a2) * t + a1;
    float e = expf_nonpos_lx(-x * x, tab);
    float y = 1.0f - poly * t * e;
    return sign * y;
}

struct RcpSeed {
    __device__ __forceinline__ float operator()(float d) const { return __builtin_amdgcn_rcpf(d); }
};

__device__ __forceinline__ float erf_fast_lx(float x, const ExpTable &tab) { return erf_fast_core(x, tab, RcpSeed()); }

// One element of the GELU subgraph Div(x, sqrt 2) -> Erf -> Add 1 -> Mul x ->
// Mul 0.5, every node rounded as the reference rounds it, with two rewrites
// of the Erf node that the chain's output cannot see: the sign of erf is
// copied from its argument (erf(-0) becomes -0, and -0 + 1 == +0 + 1), and
// |a| is clamped to 10.25 before both of its uses.  For |a| >= 10.25 the
// exponential's argument -a*a lies below expf's underflow threshold (-103.97)
// with or without the clamp, so the exponential is +0 and erf is +-1 exactly,
// whatever the reciprocal t; the clamp keeps d = 1 + p|a| within [1, 4.4] and
// the exponential's argument within [-105.07, 0] (no separate clamps of
// either), and sends a NaN |a| to 10.25 (a NaN a comes from a NaN x, which
// reaches the output through x * b either way).  The Div node is
// div_sqrt2f_lx, exact for |x| >= 2^-100; below, its last bit cannot reach the
// output (d rounds to 1 and the exponential to 1 either way).  Equal to the
// unfused chain bit for bit for all 2^32 inputs (NaN for NaN), checked on the
// host with the correctly rounded seed.
template <typename SeedFn>
__host__ __device__ __forceinline__ float gelu_erf_core(float x, const ExpTable &tab, SeedFn seed) {
    const float a1 = 0.254829592f;
    const float a2 = -0.284496736f;
    const float a3 = 1.421413741f;
    const float a4 = -1.453152027f;
    const float a5 = 1.061405429f;
    const float p = 0.3275911f;
    const float a = div_sqrt2f_lx(x);
    const float aa = __builtin_fabsf(a);
    const float ax = aa < 10.25f ? aa : 10.25f;
    const float d = 1.0f + p * ax;
    const float t = recip_newton1(d, seed(d));
    const float poly = ((((a5 * t + a4) * t) + a3) * t + a2) * t + a1;
    const float e = expf_core_lx(-ax * ax, tab);
    const float erf = __builtin_copysignf(1.0f - poly * t * e, a);
    const float b = erf + 1.0f;
    const float c = x * b;
    return c * 0.5f;
}

__device__ __forceinline__ float gelu_erf_lx(float x, const ExpTable &tab) { return gelu_erf_core(x, tab, RcpSeed()); }

// MathOps.Erf(double) (MathOps.cs:1012-1034) with the device double exp.
__device__ __forceinline__ double erf_lx(double x) {
    const double a1 = 0.254829592;
    const double a2 = -0.284496736;
    const double a3 = 1.421413741;
    const double a4 = -1.453152027;
    const double a5 = 1.061405429;
    const double p = 0.3275911;
    double sign = x < 0.0 ? -1.0 : 1.0;
    x = __builtin_fabs(x);
    double t = 1.0 / (1.0 + p * x);
    double poly = ((((a5 * t + a4) * t) + a3) * t + a2) * t + a1;
    double e = ::exp(-x * x);
    double y = 1.0 - poly * t * e;
    return sign * y;
}

// MathF.Pow -> powf; evaluated as a double pow rounded once to float (within
// one float ulp of the host powf).  Exponent 2 is the correctly rounded x*x
// (the host powf(x, 2) equals it except for 1-ulp differences on ~0.04% of
// inputs).
__device__ __forceinline__ float pow_lx(float x, float y) {
    if (y == 2.0f) return x * x;
    return (float)::pow((double)x, (double)y);
}
__device__ __forceinline__ double pow_lx(double x, double y) {
    if (y == 2.0) return x * x;
    return ::pow(x, y);
}

// The decomposed LayerNorm of one row of r floats (r a multiple of 4, at most 256 NV) held by a wave: lane l holds
// the 16-byte vectors c * 64 + l (c < NV), zero past the row's end.  Each ONNX node keeps its float32 rounding:
// mean = sum(x) / (float)r;  d = x - mean;  p = d*d (Pow 2);  var = sum(p) / (float)r;  ve = var + eps;
// sd = sqrtf(ve);  n = d / sd;  m = n * gamma;  y = m + beta, stored to q; the two sums in lane-vector order,
// then across the wave.  Shared by every kernel that normalises rows this way, so their results are identical.
// The per-vector bounds checks stay even when r fills every vector: without them the compiler issues the gamma
// / beta loads with the row's.
// gpre / bpre: gamma's and beta's vectors already loaded by the caller (a latency-bound caller issues them with its
// other loads), else null.
template <int NV>
__device__ __forceinline__ void ln_row_finish(Vec<float, 4> (&v)[NV], int r, int lane, const float *__restrict__ gamma,
                                              const float *__restrict__ beta, float eps, float *__restrict__ q,
                                              const Vec<float, 4> *gpre = nullptr, const Vec<float, 4> *bpre = nullptr) {
    float s = 0.0f;
#pragma unroll
    for (int c = 0; c < NV; c++) {
        const int col = (c * 64 + lane) * 4;
        if (col < r) s = s + ((v[c].v[0] + v[c].v[1]) + (v[c].v[2] + v[c].v[3]));
    }
    s = wave_reduce_dpp(s, [](float a, float b) { return a + b; });
    const float fr = (float)r;
    const float mean = s / fr;
    float s2 = 0.0f;
#pragma unroll
    for (int c = 0; c < NV; c++) {
        const int col = (c * 64 + lane) * 4;
        if (col < r) {
#pragma unroll
            for (int k = 0; k < 4; k++) v[c].v[k] = v[c].v[k] - mean;
            float p0 = v[c].v[0] * v[c].v[0], p1 = v[c].v[1] * v[c].v[1];
            float p2 = v[c].v[2] * v[c].v[2], p3 = v[c].v[3] * v[c].v[3];
            s2 = s2 + ((p0 + p1) + (p2 + p3));
        }
    }
    s2 = wave_reduce_dpp(s2, [](float a, float b) { return a + b; });
    const float var = s2 / fr;
    const float ve = var + eps;
    const float sd = __builtin_sqrtf(ve);
    const float rsd = 1.0f / sd;
#pragma unroll
    for (int c = 0; c < NV; c++) {
        const int col = (c * 64 + lane) * 4;
        if (col < r) {
            Vec<float, 4> g = gpre ? gpre[c] : vload<float, 4>(gamma + col);
            Vec<float, 4> b = bpre ? bpre[c] : vload<float, 4>(beta + col);
            Vec<float, 4> o;
#pragma unroll
            for (int k = 0; k < 4; k++) {
                float nrm = div_by_row_lx(v[c].v[k], sd, rsd);
                float m = nrm * g.v[k];
                o.v[k] = m + b.v[k];
            }
            vstore_nt<float, 4>(q + col, o);
        }
    }
}

}  // namespace lx
