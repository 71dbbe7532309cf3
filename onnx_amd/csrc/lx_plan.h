// lx_plan.h -- plain structs shared by the host planner and the kernels.
#pragma once

#include <stdint.h>

namespace lx {

// Division by a run-time constant d (1 <= d <= 2^31) of numerators n < 2^31:
//   q = (umulhi(n, m) + n) >> s,  s = ceil(log2 d),  m = floor(2^32 (2^s - d) / d) + 1
// (Granlund & Montgomery, "Division by invariant integers using
// multiplication", PLDI 1994, round-up variant).
struct FastDiv {
    uint32_t d, m, s, pad;
};

inline FastDiv make_fastdiv(uint32_t d) {
    FastDiv f;
    uint32_t s = 0;
    while ((1ull << s) < d) s++;
    f.d = d;
    f.s = s;
    f.m = (uint32_t)(((1ull << 32) * ((1ull << s) - d)) / d + 1);
    f.pad = 0;
    return f;
}

inline uint32_t fastdiv_host(uint32_t n, const FastDiv &f) {
    uint32_t hi = (uint32_t)(((uint64_t)n * f.m) >> 32);
    return (hi + n) >> f.s;
}

constexpr int kMaxOuter = 7;

// Kernel view of a broadcast for operands whose innermost collapsed axis is
// either contiguous (stride 1) or broadcast (stride 0):
//   element (row, col) of the output, row = outer linear index,
//   a offset = sum_d idx_d(row) * a_str[d] + col * a_inner
struct NdLayout {
    int32_t nouter;          // number of outer axes (innermost outer axis first)
    int32_t pad0;
    FastDiv odiv[kMaxOuter]; // outer axis sizes
    int64_t a_str[kMaxOuter];
    int64_t b_str[kMaxOuter];
    FastDiv inner_v;         // inner axis length in vector units
    int64_t inner;           // inner axis length in elements
};

}  // namespace lx
