// kquant_seg64.h - 64-value row segments for the fused decode kernel.
//
// A segment is 64 consecutive values of one row; every supported format maps
// a segment onto whole bytes of one block:
//   Q4_K  super-block s/4, qs chunk g = s%4 (sub-blocks 2g low / 2g+1 high nibbles)
//   Q5_K  same, plus the 32 qh bytes (bits 2g, 2g+1)
//   Q6_K  super-block s/4, half n = (s%4)/2, nibble half hi = s%2 (quarters 2hi, 2hi+1)
//   Q8_0  blocks 2s and 2s+1
// RawSeg<T> holds a segment's raw bytes (read from global memory or from an
// LDS copy, no repacking); SegCodes<T> is the same segment decoded for the
// integer dot: sixteen dwords of signed 8-bit codes plus the format's
// integer group scales and float factors.  Decoding and the dot are separate
// so that a segment can be decoded before its activations exist.
//
// 3-level activations: for each 64-value segment of x, X1..X3 are int8 with
// scales s1 = amax/127, s2 = s1/254, s3 = s2/254, so that
// x ~= s1*X1 + s2*X2 + s3*X3 with |error| <= amax/(127*254*254*2) ~ 6e-8*amax.
// The quantized weight codes are exact small integers, so sum(q*X) is exact in
// int32 (v_dot4 on packed bytes) and the dot is fp32-accurate.
#pragma once
#include "dpp.h"
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

// Materialise v in a register here: the compiler may not move the arithmetic
// that produced it past this point (it would otherwise sink a decode done
// ahead of a barrier to the barrier's far side, where the codes are used).
template <class T>
__device__ __forceinline__ void pin(T& v) {
    asm volatile("" : "+v"(v));
}

// Levels of the eight values v of segment seg (eight adjacent lanes share a
// segment, lane part of them holding values 8*part .. 8*part+7); every lane
// of the wave calls it (the segment's amax and sums are exchanged by DPP).
// Level lv of value i lands at q + lv*qstride + seg*64 + i, its scale at
// sc[lv*scstride + seg], the sums of values 0..31 and 32..63 at s32[2*seg],
// s32[2*seg+1].
__device__ __forceinline__ void quantize8(const float (&v)[8], int seg, int part, bool active, int8_t* q, int qstride,
                                          float* sc, int scstride, float* s32) {
    float amax = 0.f, sum = 0.f;
#pragma unroll
    for (int i = 0; i < 8; i++) {
        amax = fmaxf(amax, fabsf(v[i]));
        sum += v[i];
    }
    // over the 8 threads of the segment (DPP quad swaps and row_half_mirror)
    amax = dpp_fmax_step<0xB1, 0xF>(amax, amax);
    amax = dpp_fmax_step<0x4E, 0xF>(amax, amax);
    amax = dpp_fmax_step<0x141, 0xF>(amax, amax);
    sum = dpp_add_step<0xB1>(sum);
    sum = dpp_add_step<0x4E>(sum);  // four threads = 32 values
    if (!active) return;
    // Scales need only be consistent, not exact quotients: each level's
    // residual r - q*s is formed exactly (fma), and an inverse within an ulp
    // (v_rcp) keeps |residual| <= s/2 (1 + 2^-22), inside the next level's
    // +-127 * s/254 range up to its clamp.
    const float s1 = amax * (1.0f / 127.0f);
    const float s2 = s1 * (1.0f / 254.0f), s3 = s2 * (1.0f / 254.0f);
    const float lsc[kLevels] = {s1, s2, s3};
    float r[8];
#pragma unroll
    for (int i = 0; i < 8; i++) r[i] = v[i];
#pragma unroll
    for (int lv = 0; lv < kLevels; lv++) {
        const float inv = lsc[lv] > 0.f ? __builtin_amdgcn_rcpf(lsc[lv]) : 0.f;
        uint32_t packed[2] = {0u, 0u};
#pragma unroll
        for (int i = 0; i < 8; i++) {
            float qf = __builtin_rintf(r[i] * inv);
            qf = fminf(127.f, fmaxf(-127.f, qf));
            r[i] = __builtin_fmaf(-qf, lsc[lv], r[i]);
            packed[i >> 2] |= ((uint32_t)(int)qf & 0xFFu) << (8 * (i & 3));
        }
        *reinterpret_cast<uint2*>(q + lv * qstride + seg * 64 + part * 8) = make_uint2(packed[0], packed[1]);
        if (part == 0) sc[lv * scstride + seg] = lsc[lv];
    }
    if ((part & 3) == 0) s32[seg * 2 + part / 4] = sum;
}

template <int T> struct RawSeg;
template <int T> struct SegCodes;

// fp16 bits -> float by the hardware conversion.  Segment codes only feed dot
// products, where a NaN scale gives a NaN whatever its payload.
__device__ __forceinline__ float h2f(uint32_t h16) { return (float)__builtin_bit_cast(_Float16, (uint16_t)h16); }

// 6-bit scales and mins of sub-blocks j0 and j0 + 1 (j0 even) from the 12
// scale bytes in words s0..s2 (qwen3moe.cpp:133-141): sub-blocks 0-3 keep both
// in the low six bits of bytes j and j+4; sub-blocks 4-7 keep the low four
// bits in the nibbles of byte j+4 and the top two in bits 6-7 of bytes j-4
// and j.  j0 and j0 + 1 share a form, so one set of selects serves both, and
// each field is one or two bit-field extracts (a width of 0 extracts 0).
__device__ __forceinline__ void scale_min_pair(int j0, uint32_t s0, uint32_t s1, uint32_t s2, int& sc0, int& m0,
                                               int& sc1, int& m1) {
    const bool lo = j0 < 4;
    const uint32_t o = 8u * (uint32_t)(j0 & 3);
    const uint32_t A = lo ? s0 : s2, B = lo ? s1 : s2;
    const uint32_t w = lo ? 6u : 4u, wh = lo ? 0u : 2u, om = lo ? 0u : 4u;
    sc0 = (int)(__builtin_amdgcn_ubfe(A, o, w) | (__builtin_amdgcn_ubfe(s0, o + 6u, wh) << 4));
    m0 = (int)(__builtin_amdgcn_ubfe(B, o + om, w) | (__builtin_amdgcn_ubfe(s1, o + 6u, wh) << 4));
    sc1 = (int)(__builtin_amdgcn_ubfe(A, o + 8u, w) | (__builtin_amdgcn_ubfe(s0, o + 14u, wh) << 4));
    m1 = (int)(__builtin_amdgcn_ubfe(B, o + 8u + om, w) | (__builtin_amdgcn_ubfe(s1, o + 14u, wh) << 4));
}

// ---------------------------------------------------------------- Q4_K / Q5_K
// Codes: dwords 0-7 the 32 values of sub-block 2g (values 0..31 of the
// segment), dwords 8-15 those of sub-block 2g+1; value = d*sc*q - dmin*m.
struct SegCodesK {
    int32_t c[16];
    int sc0, sc1;
    float d, dm0, dm1;  // d, dmin*m0, dmin*m1
    __device__ __forceinline__ void pin_all() {
#pragma unroll
        for (int i = 0; i < 16; i++) pin(c[i]);
        pin(sc0); pin(sc1); pin(d); pin(dm0); pin(dm1);
    }
    __device__ __forceinline__ float dot(const XSeg& x) const {
        float dot = 0.f;
#pragma unroll
        for (int L = 0; L < kLevels; L++) {
            int lo = 0, hi = 0;
#pragma unroll
            for (int i = 0; i < 8; i++) {
                lo = sdot4(c[i], x.q[L][i], lo);
                hi = sdot4(c[8 + i], x.q[L][8 + i], hi);
            }
            // |lo|, |hi| <= 32 * 15 * 127 and scales < 64: 24-bit products suffice
            dot = __builtin_fmaf(x.s[L], (float)(__mul24(sc0, lo) + __mul24(sc1, hi)), dot);
        }
        const float mt = __builtin_fmaf(dm0, x.sum32[0], dm1 * x.sum32[1]);
        return __builtin_fmaf(d, dot, -mt);
    }
};
template <> struct SegCodes<kQ4_K> : SegCodesK {};
template <> struct SegCodes<kQ5_K> : SegCodesK {};

template <> struct RawSeg<kQ4_K> {
    uint4 hdr, q0, q1;
    template <class LD = GlobalLd>
    __device__ __forceinline__ void load(const uint8_t* row, int s) {
        const uint8_t* sb = row + (size_t)(s >> 2) * 144;
        const int g = s & 3;
        hdr = LD::b16(sb);
        q0 = LD::b16(sb + 16 + 32 * g);
        q1 = LD::b16(sb + 32 + 32 * g);
    }
    __device__ __forceinline__ SegCodes<kQ4_K> decode(int s) const {
        SegCodes<kQ4_K> k;
        const float dmin = h2f(hdr.x >> 16);
        int m0, m1;
        scale_min_pair(2 * (s & 3), hdr.y, hdr.z, hdr.w, k.sc0, m0, k.sc1, m1);
        const uint32_t q[8] = {q0.x, q0.y, q0.z, q0.w, q1.x, q1.y, q1.z, q1.w};
#pragma unroll
        for (int i = 0; i < 8; i++) {
            k.c[i] = (int)(q[i] & 0x0F0F0F0Fu);
            k.c[8 + i] = (int)((q[i] >> 4) & 0x0F0F0F0Fu);
        }
        k.d = h2f(hdr.x & 0xFFFFu);
        k.dm0 = dmin * (float)m0;
        k.dm1 = dmin * (float)m1;
        return k;
    }
    // sum_k w_k x_k over the segment, x given as int8 levels
    __device__ __forceinline__ float dot_q8(int s, const XSeg& x) const { return decode(s).dot(x); }
};

template <> struct RawSeg<kQ5_K> {
    uint4 hdr, h0, h1, q0, q1;
    template <class LD = GlobalLd>
    __device__ __forceinline__ void load(const uint8_t* row, int s) {
        const uint8_t* sb = row + (size_t)(s >> 2) * 176;
        const int g = s & 3;
        hdr = LD::b16(sb);
        h0 = LD::b16(sb + 16);
        h1 = LD::b16(sb + 32);
        q0 = LD::b16(sb + 48 + 32 * g);
        q1 = LD::b16(sb + 64 + 32 * g);
    }
    __device__ __forceinline__ SegCodes<kQ5_K> decode(int s) const {
        SegCodes<kQ5_K> k;
        const float dmin = h2f(hdr.x >> 16);
        const int j0 = 2 * (s & 3);
        int m0, m1;
        scale_min_pair(j0, hdr.y, hdr.z, hdr.w, k.sc0, m0, k.sc1, m1);
        const uint32_t q[8] = {q0.x, q0.y, q0.z, q0.w, q1.x, q1.y, q1.z, q1.w};
        const uint32_t h[8] = {h0.x, h0.y, h0.z, h0.w, h1.x, h1.y, h1.z, h1.w};
#pragma unroll
        for (int i = 0; i < 8; i++) {
            k.c[i] = (int)((q[i] & 0x0F0F0F0Fu) | (((h[i] >> j0) & 0x01010101u) << 4));
            k.c[8 + i] = (int)(((q[i] >> 4) & 0x0F0F0F0Fu) | (((h[i] >> (j0 + 1)) & 0x01010101u) << 4));
        }
        k.d = h2f(hdr.x & 0xFFFFu);
        k.dm0 = dmin * (float)m0;
        k.dm1 = dmin * (float)m1;
        return k;
    }
    __device__ __forceinline__ float dot_q8(int s, const XSeg& x) const { return decode(s).dot(x); }
};

// ---------------------------------------------------------------- Q6_K
// Codes: 4*(q - 32) as signed bytes (q's six bits in the top of each byte);
// dword i of the segment belongs to 16-value group i/4.
template <> struct SegCodes<kQ6_K> {
    int32_t c[16];
    int sc[4];  // the four signed 8-bit group scales
    float d4;   // d/4
    __device__ __forceinline__ void pin_all() {
#pragma unroll
        for (int i = 0; i < 16; i++) pin(c[i]);
#pragma unroll
        for (int g = 0; g < 4; g++) pin(sc[g]);
        pin(d4);
    }
    __device__ __forceinline__ float dot(const XSeg& x) const {
        float dot = 0.f;
#pragma unroll
        for (int L = 0; L < kLevels; L++) {
            int acc[4] = {0, 0, 0, 0};
#pragma unroll
            for (int i = 0; i < 16; i++) acc[i >> 2] = sdot4(c[i], x.q[L][i], acc[i >> 2]);
            // |acc| <= 16 * 128 * 127 and |sc| <= 128: 24-bit products suffice
            const int comb = __mul24(sc[0], acc[0]) + __mul24(sc[1], acc[1]) + __mul24(sc[2], acc[2]) +
                             __mul24(sc[3], acc[3]);
            dot = __builtin_fmaf(x.s[L], (float)comb, dot);
        }
        return d4 * dot;
    }
};

template <> struct RawSeg<kQ6_K> {
    Bytes32A2 l0, l1, qh;
    uint32_t sc;   // four int8 scales of the segment's 16-value groups
    uint32_t dbits;
    template <class LD = GlobalLd>
    __device__ __forceinline__ void load(const uint8_t* row, int s) {
        const uint8_t* sb = row + (size_t)(s >> 2) * 210;
        const int n = (s >> 1) & 1, hi = s & 1;
        l0 = LD::b32a2(sb + 64 * n);
        l1 = LD::b32a2(sb + 64 * n + 32);
        qh = LD::b32a2(sb + 128 + 32 * n);
        sc = (uint32_t)LD::u16(sb + 192 + 8 * n + 4 * hi) | ((uint32_t)LD::u16(sb + 194 + 8 * n + 4 * hi) << 16);
        dbits = LD::u16(sb + 208);
    }
    __device__ __forceinline__ SegCodes<kQ6_K> decode(int s) const {
        SegCodes<kQ6_K> k;
        const int hi = s & 1;
        // Each byte becomes 4*(code-32) as a signed byte: the code's low nibble
        // (ql, low or high half by hi) in bits 2-5, its two high bits (qh bits
        // 2u, 2u+1 for quarter u = 2 hi + i/8) in bits 6-7, the top bit then
        // flipped.  Both fields are moved with byte-wise-safe rotates (the bits
        // that wrap are masked off).
        const uint32_t rl = hi ? 2u : 30u;  // rotate right: nibble 1 -> bits 2-5, or nibble 0 -> bits 2-5
#pragma unroll
        for (int i = 0; i < 16; i++) {
            const uint32_t ql = i < 8 ? l0.w[i] : l1.w[i - 8];
            const uint32_t u = 2u * (uint32_t)hi + (uint32_t)(i >> 3);
            const uint32_t lo = __builtin_amdgcn_alignbit(ql, ql, rl) & 0x3C3C3C3Cu;
            const uint32_t hb = __builtin_amdgcn_alignbit(qh.w[i & 7], qh.w[i & 7], (2u * u + 26u) & 31u);
            k.c[i] = (int)(((hb & 0xC0C0C0C0u) | lo) ^ 0x80808080u);
        }
#pragma unroll
        for (int g = 0; g < 4; g++) k.sc[g] = (int)(int8_t)((sc >> (8 * g)) & 0xFFu);
        k.d4 = 0.25f * h2f(dbits);
        return k;
    }
    __device__ __forceinline__ float dot_q8(int s, const XSeg& x) const { return decode(s).dot(x); }
};

// ---------------------------------------------------------------- Q8_0
template <> struct SegCodes<kQ8_0> {
    int32_t c[16];  // the two blocks' int8 values
    float d0, d1;
    __device__ __forceinline__ void pin_all() {
#pragma unroll
        for (int i = 0; i < 16; i++) pin(c[i]);
        pin(d0); pin(d1);
    }
    __device__ __forceinline__ float dot(const XSeg& x) const {
        float r0 = 0.f, r1 = 0.f;
#pragma unroll
        for (int L = 0; L < kLevels; L++) {
            int i0 = 0, i1 = 0;
#pragma unroll
            for (int i = 0; i < 8; i++) {
                i0 = sdot4(c[i], x.q[L][i], i0);
                i1 = sdot4(c[8 + i], x.q[L][8 + i], i1);
            }
            r0 = __builtin_fmaf(x.s[L], (float)i0, r0);
            r1 = __builtin_fmaf(x.s[L], (float)i1, r1);
        }
        return __builtin_fmaf(d0, r0, d1 * r1);
    }
};

template <> struct RawSeg<kQ8_0> {
    Bytes32A2 a, b;
    uint32_t d0, d1;
    template <class LD = GlobalLd>
    __device__ __forceinline__ void load(const uint8_t* row, int s) {
        const uint8_t* p = row + (size_t)s * 68;
        d0 = LD::u16(p);
        a = LD::b32a2(p + 2);
        d1 = LD::u16(p + 34);
        b = LD::b32a2(p + 36);
    }
    __device__ __forceinline__ SegCodes<kQ8_0> decode(int) const {
        SegCodes<kQ8_0> k;
#pragma unroll
        for (int i = 0; i < 8; i++) {
            k.c[i] = (int)a.w[i];
            k.c[8 + i] = (int)b.w[i];
        }
        k.d0 = h2f(d0);
        k.d1 = h2f(d1);
        return k;
    }
    __device__ __forceinline__ float dot_q8(int s, const XSeg& x) const { return decode(s).dot(x); }
};

}  // namespace eahmmf
