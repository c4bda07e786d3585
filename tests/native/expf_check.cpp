// expf_check.cpp - exhaustive check of expf_ref (the device routing's exp)
// against the host libm's expf over every float bit pattern.  Prints the
// number of inputs compared and of results whose bits differ (NaN payloads
// compared as "both NaN").  Test infrastructure, built by tests/test_expf_ref.py.
#include <math.h>
#include <stdint.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

#include "expf_ref.h"

// A plausible mistake, for the test's own check: the reduction with a
// separate multiply and add (no fused multiply-add), as a build without
// contraction would compute it.
static float expf_unfused_reduction(float x) {
    double r;
    uint64_t ki;
    float sp;
    if (eahmmf::expf_ref_reduce(x, &r, &ki, &sp)) return sp;
    const double inv_ln2_n = 0x1.71547652b82fep+0 * 32, shift = 0x1.8p+52;
    volatile double zv = inv_ln2_n * (double)x;  // volatile: the product is rounded on its own
    const double z = zv;
    volatile double kv = z + shift;
    double kd = kv;
    ki = eahmmf::f64_bits(kd);
    kd -= shift;
    r = z - kd;
    return eahmmf::expf_ref_finish(r, ki, eahmmf::exp2_tab((uint32_t)ki));
}

int main(int argc, char** argv) {
    const uint64_t step = argc > 1 ? (uint64_t)atoll(argv[1]) : 1;
    const bool planted = argc > 2 && strcmp(argv[2], "unfused") == 0;
    long long bad = 0, n = 0;
#pragma omp parallel for reduction(+ : bad, n) schedule(static, 1 << 20)
    for (int64_t i = 0; i < (int64_t)(1ull << 32); i += (int64_t)step) {
        const uint32_t u = (uint32_t)i;
        float x;
        memcpy(&x, &u, 4);
        const float want = expf(x), got = planted ? expf_unfused_reduction(x) : eahmmf::expf_ref(x);
        n++;
        if (isnan(want) && isnan(got)) continue;
        if (eahmmf::f32_bits(want) != eahmmf::f32_bits(got)) {
            if (bad < 8) {
#pragma omp critical
                fprintf(stderr, "x=%a (0x%08x): libm %a, expf_ref %a\n", x, u, want, got);
            }
            bad++;
        }
    }
    printf("%lld %lld\n", n, bad);
    return bad ? 1 : 0;
}
