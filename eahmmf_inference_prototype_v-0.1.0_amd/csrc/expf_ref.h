// expf_ref.h - single-precision exp whose result equals glibc's expf (the
// x86-64 build the reference's host links, which contracts the reduction into
// fused multiply-adds) for every float input.
//
// The routing ranks experts by e_i = expf(l_i - max) with the lower id first
// on equal e (qwen3moe.cpp:1011-1016).  Logits close to each other (or to the
// maximum) often round to the same e, so the device must form e exactly as
// the reference's libm does, or the tie-break picks other experts.
//
// Method (published: Szabolcs Nagy's expf, ARM optimized-routines 2017, the
// expf of glibc >= 2.27): with N = 32,
//   z  = x * N/ln2,   k = round(z) (to nearest, via adding 1.5 * 2^52),
//   r  = z - k                                   (|r| <= 1/2)
//   2^(k/N) = 2^(k>>5) * T[k & 31],  T[i] = 2^(i/N) rounded to double,
//   exp(x) ~= 2^(k/N) * (C0 r^3 + C1 r^2 + C2 r + 1)   in double,
// rounded once to float.  C0..C2 are the method's minimax coefficients for
// 2^(r/N).  The table is stored, as in the method, as the bits of T[i] less
// i << 47, so that adding k << 47 to the entry yields 2^(k/N)'s bits.
// The order of operations and the fused multiply-adds below are what makes
// the result bit-identical; the test that pins it runs every float input
// against the host's expf.
#pragma once
#include <stdint.h>

#if defined(__HIPCC__)
#define EAHMMF_HD __host__ __device__
#else
#define EAHMMF_HD
#include <math.h>
#endif

namespace eahmmf {

// bits(2^(i/32) rounded to nearest double) - (i << 47), i = 0..31
#define EAHMMF_EXP2_TAB                                                                             \
    {0x3ff0000000000000ull, 0x3fefd9b0d3158574ull, 0x3fefb5586cf9890full, 0x3fef9301d0125b51ull,   \
     0x3fef72b83c7d517bull, 0x3fef54873168b9aaull, 0x3fef387a6e756238ull, 0x3fef1e9df51fdee1ull,   \
     0x3fef06fe0a31b715ull, 0x3feef1a7373aa9cbull, 0x3feedea64c123422ull, 0x3feece086061892dull,   \
     0x3feebfdad5362a27ull, 0x3feeb42b569d4f82ull, 0x3feeab07dd485429ull, 0x3feea47eb03a5585ull,   \
     0x3feea09e667f3bcdull, 0x3fee9f75e8ec5f74ull, 0x3feea11473eb0187ull, 0x3feea589994cce13ull,   \
     0x3feeace5422aa0dbull, 0x3feeb737b0cdc5e5ull, 0x3feec49182a3f090ull, 0x3feed503b23e255dull,   \
     0x3feee89f995ad3adull, 0x3feeff76f2fb5e47ull, 0x3fef199bdd85529cull, 0x3fef3720dcef9069ull,   \
     0x3fef5818dcfba487ull, 0x3fef7c97337b9b5full, 0x3fefa4afa2a490daull, 0x3fefd0765b6e4540ull}

EAHMMF_HD inline uint64_t exp2_tab(uint32_t i) {
    constexpr uint64_t t[32] = EAHMMF_EXP2_TAB;
    return t[i & 31u];
}

EAHMMF_HD inline uint32_t f32_bits(float f) { return __builtin_bit_cast(uint32_t, f); }
EAHMMF_HD inline double f64_of(uint64_t u) { return __builtin_bit_cast(double, u); }
EAHMMF_HD inline uint64_t f64_bits(double d) { return __builtin_bit_cast(uint64_t, d); }
EAHMMF_HD inline double fma64(double a, double b, double c) {
#if defined(__HIPCC__)
    return __builtin_fma(a, b, c);
#else
    return fma(a, b, c);
#endif
}

// First half: the special cases (returns true and sets *special), or the
// reduced argument r and the integer k.
EAHMMF_HD inline bool expf_ref_reduce(float x, double* r, uint64_t* ki, float* special) {
    const uint32_t u = f32_bits(x), abstop = (u >> 20) & 0x7ffu;
    if (abstop >= 0x42bu) {  // |x| >= 88, or x is Inf/NaN
        if (u == 0xff800000u) return *special = 0.0f, true;           // -Inf
        if (abstop >= 0x7f8u) return *special = x + x, true;          // +Inf, NaN
        if (x > 0x1.62e42ep6f) return *special = x * 0x1p127f * 0x1p127f, true;  // overflow: +Inf
        if (x < -0x1.9fe368p6f) return *special = 0.0f, true;         // underflow
    }
    const double inv_ln2_n = 0x1.71547652b82fep+0 * 32, shift = 0x1.8p+52;
    const double xd = (double)x;
    double kd = fma64(inv_ln2_n, xd, shift);  // k + 1.5 * 2^52, k = round(x N / ln2)
    *ki = f64_bits(kd);
    kd -= shift;
    *r = fma64(inv_ln2_n, xd, -kd);
    return false;
}

// Second half: 2^(k/N) from the table entry of k & 31, times the cubic.
EAHMMF_HD inline float expf_ref_finish(double r, uint64_t ki, uint64_t tab_entry) {
    const double c0 = 0x1.c6af84b912394p-5 / 32 / 32 / 32, c1 = 0x1.ebfce50fac4f3p-3 / 32 / 32,
                 c2 = 0x1.62e42ff0c52d6p-1 / 32;
    const double s = f64_of(tab_entry + (ki << 47));
    const double z = fma64(c0, r, c1);
    const double r2 = r * r;
    double y = fma64(c2, r, 1.0);
    y = fma64(z, r2, y);
    return (float)(y * s);
}

EAHMMF_HD inline float expf_ref(float x) {
    double r;
    uint64_t ki;
    float sp;
    if (expf_ref_reduce(x, &r, &ki, &sp)) return sp;
    return expf_ref_finish(r, ki, exp2_tab((uint32_t)ki));
}

}  // namespace eahmmf
