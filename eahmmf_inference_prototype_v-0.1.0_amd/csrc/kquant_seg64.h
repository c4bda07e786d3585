// kquant_seg64.h - 64-value row segments for the fused decode kernel.
//
// A segment is 64 consecutive values of one row; every supported format maps
// a segment onto whole bytes of one block:
//   Q4_K  super-block s/4, qs chunk g = s%4 (sub-blocks 2g low / 2g+1 high nibbles)
//   Q5_K  same, plus the 32 qh bytes (bits 2g, 2g+1)
//   Q6_K  super-block s/4, half n = (s%4)/2, nibble half hi = s%2 (quarters 2hi, 2hi+1)
//   Q8_0  blocks 2s and 2s+1
// Each format has a raw-byte holder (loaded straight from HBM, no repacking),
// an integer-dot path against 3-level int8 activations (gate/up), and an fp32
// path against fp32 activations (down projection).
//
// 3-level activations: for each 64-value segment of x, X1..X3 are int8 with
// scales s1 = amax/127, s2 = s1/254, s3 = s2/254, so that
// x ~= s1*X1 + s2*X2 + s3*X3 with |error| <= amax/(127*254*254*2) ~ 6e-8*amax.
// The quantized weight codes are exact small integers, so sum(q*X) is exact in
// int32 (v_dot4 on packed bytes) and the dot is fp32-accurate.
#pragma once
#include "kquant.h"

namespace eahmmf {

constexpr int kLevels = 3;

// Activation levels of one segment held by a lane: 16 dwords per level.
struct XSeg {
    int32_t q[kLevels][16];
    float s[kLevels];
    float sum32[2];  // sum of the original x over values 0..31 and 32..63
};

__device__ __forceinline__ int sdot4(int a, int b, int c) { return __builtin_amdgcn_sdot4(a, b, c, false); }

template <int T> struct RawSeg;

// ---------------------------------------------------------------- Q4_K
template <> struct RawSeg<kQ4_K> {
    uint4 hdr, q0, q1;
    __device__ __forceinline__ void load(const uint8_t* row, int s) {
        const uint8_t* sb = row + (size_t)(s >> 2) * 144;
        const int g = s & 3;
        hdr = ld16(sb);
        q0 = ld16(sb + 16 + 32 * g);
        q1 = ld16(sb + 32 + 32 * g);
    }
    __device__ __forceinline__ void scales(int s, float& d, float& dmin, uint32_t& sc0, uint32_t& m0, uint32_t& sc1,
                                           uint32_t& m1) const {
        d = half_to_float(hdr.x & 0xFFFFu);
        dmin = half_to_float(hdr.x >> 16);
        const int j0 = 2 * (s & 3);
        scale_min_k4(j0, hdr.y, hdr.z, hdr.w, sc0, m0);
        scale_min_k4(j0 + 1, hdr.y, hdr.z, hdr.w, sc1, m1);
    }
    // sum_k w_k x_k over the segment, x given as int8 levels
    __device__ __forceinline__ float dot_q8(int s, const XSeg& x) const {
        float d, dmin;
        uint32_t sc0, m0, sc1, m1;
        scales(s, d, dmin, sc0, m0, sc1, m1);
        const uint32_t q[8] = {q0.x, q0.y, q0.z, q0.w, q1.x, q1.y, q1.z, q1.w};
        float dot = 0.f;
#pragma unroll
        for (int L = 0; L < kLevels; L++) {
            int lo = 0, hi = 0;
#pragma unroll
            for (int i = 0; i < 8; i++) {
                lo = sdot4((int)(q[i] & 0x0F0F0F0Fu), x.q[L][i], lo);
                hi = sdot4((int)((q[i] >> 4) & 0x0F0F0F0Fu), x.q[L][8 + i], hi);
            }
            const int comb = (int)sc0 * lo + (int)sc1 * hi;
            dot = __builtin_fmaf(x.s[L], (float)comb, dot);
        }
        const float mt = __builtin_fmaf((float)m0, x.sum32[0], (float)m1 * x.sum32[1]);
        return __builtin_fmaf(d, dot, -dmin * mt);
    }
    // fp32 activations a[64] (and their 32-value sums)
    __device__ __forceinline__ float dot_f32(int s, const float* a, const float* asum32) const {
        float d, dmin;
        uint32_t sc0, m0, sc1, m1;
        scales(s, d, dmin, sc0, m0, sc1, m1);
        const uint32_t q[8] = {q0.x, q0.y, q0.z, q0.w, q1.x, q1.y, q1.z, q1.w};
        float lo = 0.f, hi = 0.f;
#pragma unroll
        for (int i = 0; i < 32; i++) {
            const uint32_t w = q[i >> 2] >> (8 * (i & 3));
            lo = __builtin_fmaf((float)(w & 15u), a[i], lo);
            hi = __builtin_fmaf((float)((w >> 4) & 15u), a[32 + i], hi);
        }
        const float dot = __builtin_fmaf((float)sc0, lo, (float)sc1 * hi);
        const float mt = __builtin_fmaf((float)m0, asum32[0], (float)m1 * asum32[1]);
        return __builtin_fmaf(d, dot, -dmin * mt);
    }
};

// ---------------------------------------------------------------- Q5_K
template <> struct RawSeg<kQ5_K> {
    uint4 hdr, h0, h1, q0, q1;
    __device__ __forceinline__ void load(const uint8_t* row, int s) {
        const uint8_t* sb = row + (size_t)(s >> 2) * 176;
        const int g = s & 3;
        hdr = ld16(sb);
        h0 = ld16(sb + 16);
        h1 = ld16(sb + 32);
        q0 = ld16(sb + 48 + 32 * g);
        q1 = ld16(sb + 64 + 32 * g);
    }
    __device__ __forceinline__ void codes(int s, uint32_t* lo, uint32_t* hi) const {
        const int j0 = 2 * (s & 3);
        const uint32_t q[8] = {q0.x, q0.y, q0.z, q0.w, q1.x, q1.y, q1.z, q1.w};
        const uint32_t h[8] = {h0.x, h0.y, h0.z, h0.w, h1.x, h1.y, h1.z, h1.w};
#pragma unroll
        for (int i = 0; i < 8; i++) {
            lo[i] = (q[i] & 0x0F0F0F0Fu) | (((h[i] >> j0) & 0x01010101u) << 4);
            hi[i] = ((q[i] >> 4) & 0x0F0F0F0Fu) | (((h[i] >> (j0 + 1)) & 0x01010101u) << 4);
        }
    }
    __device__ __forceinline__ float dot_q8(int s, const XSeg& x) const {
        const float d = half_to_float(hdr.x & 0xFFFFu), dmin = half_to_float(hdr.x >> 16);
        uint32_t sc0, m0, sc1, m1;
        const int j0 = 2 * (s & 3);
        scale_min_k4(j0, hdr.y, hdr.z, hdr.w, sc0, m0);
        scale_min_k4(j0 + 1, hdr.y, hdr.z, hdr.w, sc1, m1);
        uint32_t lo[8], hi[8];
        codes(s, lo, hi);
        float dot = 0.f;
#pragma unroll
        for (int L = 0; L < kLevels; L++) {
            int a = 0, b = 0;
#pragma unroll
            for (int i = 0; i < 8; i++) {
                a = sdot4((int)lo[i], x.q[L][i], a);
                b = sdot4((int)hi[i], x.q[L][8 + i], b);
            }
            dot = __builtin_fmaf(x.s[L], (float)((int)sc0 * a + (int)sc1 * b), dot);
        }
        const float mt = __builtin_fmaf((float)m0, x.sum32[0], (float)m1 * x.sum32[1]);
        return __builtin_fmaf(d, dot, -dmin * mt);
    }
    __device__ __forceinline__ float dot_f32(int s, const float* a, const float* asum32) const {
        const float d = half_to_float(hdr.x & 0xFFFFu), dmin = half_to_float(hdr.x >> 16);
        uint32_t sc0, m0, sc1, m1;
        const int j0 = 2 * (s & 3);
        scale_min_k4(j0, hdr.y, hdr.z, hdr.w, sc0, m0);
        scale_min_k4(j0 + 1, hdr.y, hdr.z, hdr.w, sc1, m1);
        uint32_t lo[8], hi[8];
        codes(s, lo, hi);
        float sl = 0.f, sh = 0.f;
#pragma unroll
        for (int i = 0; i < 32; i++) {
            sl = __builtin_fmaf((float)((lo[i >> 2] >> (8 * (i & 3))) & 0xFFu), a[i], sl);
            sh = __builtin_fmaf((float)((hi[i >> 2] >> (8 * (i & 3))) & 0xFFu), a[32 + i], sh);
        }
        const float dot = __builtin_fmaf((float)sc0, sl, (float)sc1 * sh);
        const float mt = __builtin_fmaf((float)m0, asum32[0], (float)m1 * asum32[1]);
        return __builtin_fmaf(d, dot, -dmin * mt);
    }
};

// ---------------------------------------------------------------- Q6_K
template <> struct RawSeg<kQ6_K> {
    Bytes32A2 l0, l1, qh;
    uint32_t sc;   // four int8 scales of the segment's 16-value groups
    uint32_t dbits;
    __device__ __forceinline__ void load(const uint8_t* row, int s) {
        const uint8_t* sb = row + (size_t)(s >> 2) * 210;
        const int n = (s >> 1) & 1, hi = s & 1;
        l0 = ld32_a2(sb + 64 * n);
        l1 = ld32_a2(sb + 64 * n + 32);
        qh = ld32_a2(sb + 128 + 32 * n);
        sc = (uint32_t)ld_u16(sb + 192 + 8 * n + 4 * hi) | ((uint32_t)ld_u16(sb + 194 + 8 * n + 4 * hi) << 16);
        dbits = ld_u16(sb + 208);
    }
    // 6-bit code bytes (0..63) of quarter u for ql dword i of one 32-byte half
    __device__ __forceinline__ static uint32_t code(uint32_t ql, uint32_t h, int hi, int u) {
        const uint32_t nib = hi ? ((ql >> 4) & 0x0F0F0F0Fu) : (ql & 0x0F0F0F0Fu);
        return nib | (((h >> (2 * u)) & 0x03030303u) << 4);
    }
    __device__ __forceinline__ float dot_q8(int s, const XSeg& x) const {
        const int hi = s & 1;
        const float d = half_to_float(dbits);
        int acc[kLevels][4];
#pragma unroll
        for (int L = 0; L < kLevels; L++)
#pragma unroll
            for (int g = 0; g < 4; g++) acc[L][g] = 0;
#pragma unroll
        for (int i = 0; i < 16; i++) {
            const uint32_t ql = i < 8 ? l0.w[i] : l1.w[i - 8];
            const int u = 2 * hi + (i >> 3);
            // code*4 in the top six bits of each byte, as a signed byte 4*(code-32)
            const uint32_t c = code(ql, qh.w[i & 7], hi, u);
            const int sq = (int)((c << 2) ^ 0x80808080u);
            const int g = i >> 2;  // 16-value group of the segment
#pragma unroll
            for (int L = 0; L < kLevels; L++) acc[L][g] = sdot4(sq, x.q[L][i], acc[L][g]);
        }
        float dot = 0.f;
#pragma unroll
        for (int L = 0; L < kLevels; L++) {
            int comb = 0;
#pragma unroll
            for (int g = 0; g < 4; g++) comb += (int)(int8_t)((sc >> (8 * g)) & 0xFFu) * acc[L][g];
            dot = __builtin_fmaf(x.s[L], (float)comb, dot);
        }
        return 0.25f * d * dot;
    }
    // fp32 activations; asum16[4] = sums of a over each 16-value group
    __device__ __forceinline__ float dot_f32(int s, const float* a, const float* asum16) const {
        const int hi = s & 1;
        const float d = half_to_float(dbits);
        float out = 0.f;
#pragma unroll
        for (int g = 0; g < 4; g++) {
            float p = 0.f;
#pragma unroll
            for (int ii = 0; ii < 4; ii++) {
                const int i = 4 * g + ii;
                const uint32_t ql = i < 8 ? l0.w[i] : l1.w[i - 8];
                const uint32_t c = code(ql, qh.w[i & 7], hi, 2 * hi + (i >> 3));
#pragma unroll
                for (int b = 0; b < 4; b++) p = __builtin_fmaf((float)((c >> (8 * b)) & 0xFFu), a[4 * i + b], p);
            }
            const float scg = (float)(int8_t)((sc >> (8 * g)) & 0xFFu);
            out = __builtin_fmaf(scg, __builtin_fmaf(-32.f, asum16[g], p), out);
        }
        return d * out;
    }
};

// ---------------------------------------------------------------- Q8_0
template <> struct RawSeg<kQ8_0> {
    Bytes32A2 a, b;
    uint32_t d0, d1;
    __device__ __forceinline__ void load(const uint8_t* row, int s) {
        const uint8_t* p = row + (size_t)s * 68;
        d0 = ld_u16(p);
        a = ld32_a2(p + 2);
        d1 = ld_u16(p + 34);
        b = ld32_a2(p + 36);
    }
    __device__ __forceinline__ float dot_q8(int s, const XSeg& x) const {
        float r0 = 0.f, r1 = 0.f;
#pragma unroll
        for (int L = 0; L < kLevels; L++) {
            int i0 = 0, i1 = 0;
#pragma unroll
            for (int i = 0; i < 8; i++) {
                i0 = sdot4((int)a.w[i], x.q[L][i], i0);
                i1 = sdot4((int)b.w[i], x.q[L][8 + i], i1);
            }
            r0 = __builtin_fmaf(x.s[L], (float)i0, r0);
            r1 = __builtin_fmaf(x.s[L], (float)i1, r1);
        }
        return __builtin_fmaf(half_to_float(d0), r0, half_to_float(d1) * r1);
    }
    __device__ __forceinline__ float dot_f32(int s, const float* av, const float*) const {
        float r0 = 0.f, r1 = 0.f;
#pragma unroll
        for (int i = 0; i < 32; i++) {
            r0 = __builtin_fmaf((float)(int8_t)((a.w[i >> 2] >> (8 * (i & 3))) & 0xFFu), av[i], r0);
            r1 = __builtin_fmaf((float)(int8_t)((b.w[i >> 2] >> (8 * (i & 3))) & 0xFFu), av[32 + i], r1);
        }
        return __builtin_fmaf(half_to_float(d0), r0, half_to_float(d1) * r1);
    }
};

// Which sums of the fp32 activations a format's dot_f32 needs: Q6_K four
// 16-value sums, Q4_K/Q5_K two 32-value sums, Q8_0 none.
template <int T> struct SumSpan { static constexpr int n = 0, width = 64; };
template <> struct SumSpan<kQ4_K> { static constexpr int n = 2, width = 32; };
template <> struct SumSpan<kQ5_K> { static constexpr int n = 2, width = 32; };
template <> struct SumSpan<kQ6_K> { static constexpr int n = 4, width = 16; };

}  // namespace eahmmf
