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

// all 2^32 x: div_sqrt2f_lx(x) against x / 1.4142135f.  out[0] = mismatches with |x| >= 2^-100 (none
// allowed), out[1] = mismatches below (results near the denormal range, where x * zl underflows)
void lx_test_div_sqrt2_mismatches(long long *out) {
    const volatile float c = 1.41421353816986083984375f;
    long long big = 0, tiny = 0;
#pragma omp parallel for reduction(+ : big, tiny) schedule(static)
    for (long long u = 0; u < (1ll << 32); u++) {
        float x = fbits((uint32_t)u);
        if (!same(lx::div_sqrt2f_lx(x), x / c)) {
            if (__builtin_fabsf(x) >= 0x1p-100f) big++;
            else tiny++;
        }
    }
    out[0] = big;
    out[1] = tiny;
}

// every float x in [lo, hi] (lo <= hi, both finite): expf_core_lx(x) == expf(x)
long long lx_test_expf_core_range_mismatches(float lo, float hi) {
    lx::ExpTable tab;
    lx::exp_table_fill_host(tab);
    long long bad = 0;
#pragma omp parallel for reduction(+ : bad) schedule(static)
    for (long long u = 0; u < (1ll << 32); u++) {
        float x = fbits((uint32_t)u);
        if (!(x >= lo && x <= hi)) continue;
        if (!same(lx::expf_core_lx(x, tab), expf(x))) bad++;
    }
    return bad;
}

// every d in [1, 2^126): out[0] = d where one Newton step from the correctly rounded seed differs from 1/d,
// out[1] = (d, seed) pairs with a seed one ulp off where it does
void lx_test_recip_mismatches(long long *out) {
    long long bad = 0, off = 0;
    const uint32_t lo = bits(1.0f), hi = bits(0x1p126f);
#pragma omp parallel for reduction(+ : bad, off) schedule(static)
    for (long long u = lo; u < (long long)hi; u++) {
        float d = fbits((uint32_t)u);
        float cr = 1.0f / d;
        if (!same(lx::recip_newton1(d, cr), cr)) bad++;
        for (int k = -1; k <= 1; k += 2)
            if (!same(lx::recip_newton1(d, fbits(bits(cr) + k)), cr)) off++;
    }
    out[0] = bad;
    out[1] = off;
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

namespace {
// 1/d perturbed by a relative factor (1 + rel): a stand-in for a hardware
// reciprocal seed of that accuracy
struct ScaledSeed {
    double rel;
    double operator()(double d) const { return (1.0 / d) * (1.0 + rel); }
};

inline uint64_t splitmix(uint64_t &s) {
    uint64_t z = (s += 0x9e3779b97f4a7c15ull);
    z = (z ^ (z >> 30)) * 0xbf58476d1ce4e5b9ull;
    z = (z ^ (z >> 27)) * 0x94d049bb133111ebull;
    return z ^ (z >> 31);
}

// quotients around multiples of the divisor magnitude ub: |a| = k*ub - 1, k*ub,
// k*ub + ub - 1 for the smallest and largest k and random k in between (|a| and
// ub up to 2^31), each with every sign of a and b that int32 represents
inline long long sdiv_one(int64_t a, int64_t b, const ScaledSeed &seed) {
    if (a < INT32_MIN || a > INT32_MAX || b < INT32_MIN || b > INT32_MAX || b == 0) return 0;
    if (a == INT32_MIN && b == -1) return 0;  // an error case, never divided
    const int64_t q = a / b;                   // C truncation, as the reference
    return lx::sdiv32_core((int32_t)a, (int32_t)b, seed) != (int32_t)q ? 1 : 0;
}

long long sdiv_cases(uint32_t ub, uint64_t &rng, const ScaledSeed &seed) {
    long long bad = 0;
    const uint64_t kmax = 0x80000000ull / ub;
    uint64_t ks[24] = {0, 1, 2, 3, kmax, kmax - 1};
    for (int i = 6; i < 24; i++) ks[i] = splitmix(rng) % (kmax + 1);
    for (uint64_t k : ks) {
        const int64_t base = (int64_t)(k * ub);
        const int64_t cand[3] = {base - 1, base, base + ub - 1};
        for (int64_t a : cand) {
            if (a < 0) continue;
            bad += sdiv_one(a, ub, seed) + sdiv_one(-a, ub, seed) + sdiv_one(a, -(int64_t)ub, seed) +
                   sdiv_one(-a, -(int64_t)ub, seed);
        }
    }
    return bad;
}
}  // namespace

extern "C" {
// sdiv32_core against C integer division, with the seed 1/d scaled by
// (1 + rel): every divisor magnitude up to 2^20 and 2^22 random larger ones up
// to 2^31, each at multiples of the divisor; all a, b in [-2^10, 2^10); and
// the extreme values.  Returns the mismatch count.
long long lx_test_sdiv32_mismatches(double rel) {
    const ScaledSeed seed{rel};
    long long bad = 0;
#pragma omp parallel for reduction(+ : bad) schedule(dynamic, 4096)
    for (long long ub = 1; ub <= (1ll << 20); ub++) {
        uint64_t rng = (uint64_t)ub * 7919u;
        bad += sdiv_cases((uint32_t)ub, rng, seed);
    }
#pragma omp parallel for reduction(+ : bad) schedule(dynamic, 4096)
    for (long long i = 0; i < (1ll << 22); i++) {
        uint64_t rng = (uint64_t)i ^ 0x5851f42d4c957f2dull;
        uint32_t ub = (uint32_t)(splitmix(rng) >> 33) + 1;  // [1, 2^31]
        if (ub <= (1u << 20)) ub |= 1u << 20;
        bad += sdiv_cases(ub, rng, seed);
    }
#pragma omp parallel for reduction(+ : bad) schedule(static)
    for (long long a = -1024; a < 1024; a++)
        for (long long b = -1024; b < 1024; b++) bad += sdiv_one(a, b, seed);
    const int64_t ext[] = {0, 1, -1, 2, -2, 3, INT32_MAX, INT32_MAX - 1, INT32_MIN, INT32_MIN + 1, 1 << 30, -(1 << 30)};
    for (int64_t a : ext)
        for (int64_t b : ext) bad += sdiv_one(a, b, seed);
    return bad;
}
}
