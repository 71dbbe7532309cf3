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
}
