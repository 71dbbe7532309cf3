// TEST HELPER: evaluates the device expf / erf restatements (lx_device.h) on the
// host and compares them with the host libm expf that the oracle calls.
#include <math.h>
#include <stdint.h>
#include <string.h>

#include "../../onnx_amd/csrc/lx_device.h"

extern "C" {

// number of float bit patterns u in [begin, end) (step) where expf_lx != expf
long long lx_test_expf_mismatches(uint64_t begin, uint64_t end, uint64_t step) {
    lx::ExpTable tab;
    lx::exp_table_fill_host(tab);
    long long bad = 0;
    for (uint64_t u = begin; u < end; u += step) {
        uint32_t b = (uint32_t)u;
        float x;
        memcpy(&x, &b, 4);
        float a = expf(x);
        float c = lx::expf_lx(x, tab);
        uint32_t ua, uc;
        memcpy(&ua, &a, 4);
        memcpy(&uc, &c, 4);
        if (ua != uc && !(a != a && c != c)) bad++;
    }
    return bad;
}

float lx_test_expf(float x) {
    lx::ExpTable tab;
    lx::exp_table_fill_host(tab);
    return lx::expf_lx(x, tab);
}

float lx_test_erf(float x) {
    lx::ExpTable tab;
    lx::exp_table_fill_host(tab);
    return lx::erf_lx(x, tab);
}

uint32_t lx_test_fastdiv(uint32_t n, uint32_t d) { return lx::fastdiv_host(n, lx::make_fastdiv(d)); }

static inline uint32_t bits(float f) {
    uint32_t u;
    memcpy(&u, &f, 4);
    return u;
}
static inline float fbits(uint32_t u) {
    float f;
    memcpy(&f, &u, 4);
    return f;
}
static inline bool same(float a, float b) { return bits(a) == bits(b) || (a != a && b != b); }

// all 2^32 x: div_sqrt2f_lx(x) == x / 1.4142135f
long long lx_test_div_sqrt2_mismatches(void) {
    const volatile float c = 1.41421353816986083984375f;
    long long bad = 0;
#pragma omp parallel for reduction(+ : bad) schedule(static)
    for (long long u = 0; u < (1ll << 32); u++) {
        float x = fbits((uint32_t)u);
        if (!same(lx::div_sqrt2f_lx(x), x / c)) bad++;
    }
    return bad;
}

// every d in [1, 2^126) with every seed within 1 ulp of 1/d: number of
// (d, seed) pairs where recip_newton2 differs from 1/d, split into d with an
// all-ones significand (out[1]) and every other d (out[0])
void lx_test_recip_mismatches(long long *out) {
    long long bad = 0, ones = 0;
    const uint32_t lo = bits(1.0f), hi = bits(0x1p126f);
#pragma omp parallel for reduction(+ : bad, ones) schedule(static)
    for (long long u = lo; u < (long long)hi; u++) {
        float d = fbits((uint32_t)u);
        float cr = 1.0f / d;
        for (int k = -1; k <= 1; k++) {
            float seed = fbits(bits(cr) + k);
            if (!same(lx::recip_newton2(d, seed), cr)) {
                if ((u & 0x7fffff) == 0x7fffff) ones++;
                else bad++;
            }
        }
        // the correctly rounded seed itself is always a fixed point
        if (!same(lx::recip_newton2(d, cr), cr)) bad++;
    }
    out[0] = bad;
    out[1] = ones;
}

// every x <= 0 (sign bit set), +0 and NaN: expf_nonpos_lx(x) == expf(x)
long long lx_test_expf_nonpos_mismatches(void) {
    lx::ExpTable tab;
    lx::exp_table_fill_host(tab);
    long long bad = 0;
#pragma omp parallel for reduction(+ : bad) schedule(static)
    for (long long u = 0x80000000ll; u < (1ll << 32); u++) {
        float x = fbits((uint32_t)u);
        if (!same(lx::expf_nonpos_lx(x, tab), expf(x))) bad++;
    }
    if (!same(lx::expf_nonpos_lx(0.0f, tab), expf(0.0f))) bad++;
    if (!same(lx::expf_nonpos_lx(__builtin_nanf(""), tab), expf(__builtin_nanf("")))) bad++;
    return bad;
}
}

namespace {
struct ExactSeed {
    float operator()(float d) const { return 1.0f / d; }
};
}  // namespace

extern "C" {
// all 2^32 x: the branch-free device erf core == erf_lx (A&S formula with the host-equal expf)
long long lx_test_erf_fast_mismatches(void) {
    lx::ExpTable tab;
    lx::exp_table_fill_host(tab);
    long long bad = 0;
#pragma omp parallel for reduction(+ : bad) schedule(static)
    for (long long u = 0; u < (1ll << 32); u++) {
        float x = fbits((uint32_t)u);
        if (!same(lx::erf_fast_core(x, tab, ExactSeed()), lx::erf_lx(x, tab))) bad++;
    }
    return bad;
}
}

extern "C" {
// all 2^32 x: the fused device GELU element == the unfused chain
// Div(x, 1.4142135f) -> Erf (erf_lx) -> Add 1 -> Mul x -> Mul 0.5 in IEEE float
long long lx_test_gelu_mismatches(void) {
    lx::ExpTable tab;
    lx::exp_table_fill_host(tab);
    const volatile float c = 1.41421353816986083984375f;
    long long bad = 0;
#pragma omp parallel for reduction(+ : bad) schedule(static)
    for (long long u = 0; u < (1ll << 32); u++) {
        float x = fbits((uint32_t)u);
        float a = x / c;
        float e = lx::erf_lx(a, tab);
        float b = e + 1.0f;
        float cc = x * b;
        float ref = cc * 0.5f;
        if (!same(lx::gelu_erf_core(x, tab, ExactSeed()), ref)) bad++;
    }
    return bad;
}
}
