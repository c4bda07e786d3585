// kquant.h - device-side decoding of the GGML block formats used by MoE
// expert weights on gfx950: Q8_0 (type 8), Q4_K (12), Q5_K (13), Q6_K (14),
// plus F32 (0) for router matrices.
//
// Byte layouts and value formulas follow the reference CPU decoder
// (qwen3moe.cpp:128-202) so that dequantized values are bit-identical:
//   Q8_0  y = d*q                                  (34 B / 32 values)
//   Q4_K  y = fma(d*sc, q, -(dmin*m))              (144 B / 256 values)
//   Q5_K  y = fma(d*sc, q + 16*hbit, -(dmin*m))    (176 B / 256 values)
//   Q6_K  y = (d*sc)*q                             (210 B / 256 values)
// The FMA in Q4_K/Q5_K is the single rounding the reference binary performs
// after GCC contracts `d1 * q - m1` under its -O3 -march=native build.
//
// The unit of work is a 32-value "segment":
//   Q4_K/Q5_K  sub-block j of a super-block (its own 6-bit scale and min)
//   Q6_K       quarter u of half n (two 16-value int8 scales)
//   Q8_0       one block
//   F32        32 consecutive floats
// Super-blocks are read in place with 16-byte loads; Q6_K and Q8_0 blocks sit
// at 2-byte alignment and are read through 2-byte-aligned packed structs (the
// amdhsa target runs in unaligned-access mode, so these stay single vector
// loads).
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

namespace eahmmf {

enum : int { kF32 = 0, kQ8_0 = 8, kQ4_K = 12, kQ5_K = 13, kQ6_K = 14 };

template <int T> struct Fmt;
template <> struct Fmt<kF32>  { static constexpr int blck = 32,  bytes = 128, segs = 1; };
template <> struct Fmt<kQ8_0> { static constexpr int blck = 32,  bytes = 34,  segs = 1; };
template <> struct Fmt<kQ4_K> { static constexpr int blck = 256, bytes = 144, segs = 8; };
template <> struct Fmt<kQ5_K> { static constexpr int blck = 256, bytes = 176, segs = 8; };
template <> struct Fmt<kQ6_K> { static constexpr int blck = 256, bytes = 210, segs = 8; };

__host__ __device__ inline int type_blck(int t) {
    return t == kQ4_K || t == kQ5_K || t == kQ6_K ? 256 : (t == kQ8_0 || t == kF32 ? 32 : 0);
}
__host__ __device__ inline int type_bytes(int t) {
    switch (t) {
        case kF32: return 128;
        case kQ8_0: return 34;
        case kQ4_K: return 144;
        case kQ5_K: return 176;
        case kQ6_K: return 210;
        default: return 0;
    }
}

struct __attribute__((packed, aligned(2))) Bytes16A2 { uint32_t w[4]; };
struct __attribute__((packed, aligned(2))) Bytes32A2 { uint32_t w[8]; };

__device__ __forceinline__ uint4 ld16(const uint8_t* p) {  // 16-byte aligned
    return *reinterpret_cast<const uint4*>(p);
}
__device__ __forceinline__ Bytes32A2 ld32_a2(const uint8_t* p) {  // 2-byte aligned
    return *reinterpret_cast<const Bytes32A2*>(p);
}
__device__ __forceinline__ uint16_t ld_u16(const uint8_t* p) {
    return *reinterpret_cast<const uint16_t*>(p);
}

// 32 bytes at a 2-byte-aligned LDS address: nine aligned dwords realigned
// with v_alignbit, so no LDS access is unaligned.  Reads up to 2 bytes past
// the 32 (the callers' LDS buffers leave room).
__device__ __forceinline__ Bytes32A2 lds_ld32_a2(const uint8_t* p) {
    const uint32_t off = (uint32_t)(uintptr_t)p & 3u;
    const uint32_t* b = reinterpret_cast<const uint32_t*>(p - off);
    uint32_t d[9];
#pragma unroll
    for (int i = 0; i < 9; i++) d[i] = b[i];
    Bytes32A2 r;
#pragma unroll
    for (int i = 0; i < 8; i++) r.w[i] = __builtin_amdgcn_alignbit(d[i + 1], d[i], off * 8u);
    return r;
}

// How a weight row segment is read: straight from global memory, or from an
// LDS copy that keeps the row's global alignment modulo 16 (16-byte loads
// stay aligned; 2-byte-aligned 32-byte groups are realigned in registers).
// GlobalLd reads through global-address-space pointers: a row pointer taken
// from a table in memory is otherwise generic, and generic (flat) loads also
// count against the LDS/scalar counter, so every wait for a scalar or LDS
// operation would wait for the weight loads in flight as well.
typedef uint32_t __attribute__((ext_vector_type(4))) u32x4_t;
typedef uint32_t __attribute__((aligned(2))) u32_a2_t;
__device__ __forceinline__ uint4 gld16(const uint8_t* p) {  // 16-byte aligned
    const u32x4_t v = *(const __attribute__((address_space(1))) u32x4_t*)p;
    return make_uint4(v.x, v.y, v.z, v.w);
}
__device__ __forceinline__ Bytes32A2 gld32_a2(const uint8_t* p) {  // 2-byte aligned
    const __attribute__((address_space(1))) u32_a2_t* q = (const __attribute__((address_space(1))) u32_a2_t*)p;
    Bytes32A2 r;
#pragma unroll
    for (int i = 0; i < 8; i++) r.w[i] = q[i];
    return r;
}
__device__ __forceinline__ uint16_t gld_u16(const uint8_t* p) {
    return *(const __attribute__((address_space(1))) uint16_t*)p;
}
struct GlobalLd {
    static __device__ __forceinline__ uint4 b16(const uint8_t* p) { return gld16(p); }
    static __device__ __forceinline__ Bytes32A2 b32a2(const uint8_t* p) { return gld32_a2(p); }
    static __device__ __forceinline__ uint16_t u16(const uint8_t* p) { return gld_u16(p); }
};
struct LdsLd {
    static __device__ __forceinline__ uint4 b16(const uint8_t* p) { return ld16(p); }
    static __device__ __forceinline__ Bytes32A2 b32a2(const uint8_t* p) { return lds_ld32_a2(p); }
    static __device__ __forceinline__ uint16_t u16(const uint8_t* p) { return ld_u16(p); }
};

// One nontemporal LDS DMA instruction (global_load_lds_dwordx4 ... nt): lane
// i's 16 bytes at gaddr land at LDS address lds + 16*i (lds wave-uniform).
// Written as inline assembly on purpose: the compiler does not see the LDS
// write, so it adds no wait of its own (it would otherwise wait for every DMA
// in flight before any read of the target buffer).  Every read of DMA'd data
// is therefore ordered by an explicit s_waitcnt vmcnt of the issuing wave,
// followed by a barrier where other waves read it.  Counters are retired in
// issue order, so the compiler's own waits for its loads stay correct (they
// can only become longer).
__device__ __forceinline__ void lds_dma16(uintptr_t gaddr, const uint8_t* lds) {
    // wave-uniform by contract; readfirstlane puts it in an SGPR for M0
    const uint32_t base = (uint32_t)__builtin_amdgcn_readfirstlane(
        (int)(uint32_t)(uintptr_t)(__attribute__((address_space(3))) const uint8_t*)lds);
#pragma clang diagnostic push
#pragma clang diagnostic ignored "-Winline-asm"
    asm volatile("s_mov_b32 m0, %1\n\tglobal_load_lds_dwordx4 %0, off nt"
                 :
                 : "v"(gaddr), "s"(base)
                 : "memory", "m0");
#pragma clang diagnostic pop
}

// Copy NI x 1024 bytes from global memory into LDS, one wave, one 16-byte
// chunk per lane per instruction: the n bytes from src (n >= 1) land at
// dst + (src & 15), dst 16-byte aligned.  Exactly NI instructions are issued
// whatever n is (lanes past the end re-read the last chunk into dst's tail),
// so a caller can count them in vmcnt.  Measured on MI355X: a 24.5 MB
// one-pass read this way finishes in about half the time plain loads into
// registers take.
template <int NI>
__device__ __forceinline__ void dma_to_lds(const uint8_t* src, int n, uint8_t* dst, int lane) {
    const uintptr_t a = (uintptr_t)src & ~(uintptr_t)15;
    const int n16 = (int)(((((uintptr_t)src + (uintptr_t)n + 15) & ~(uintptr_t)15) - a) / 16);
#pragma unroll
    for (int i = 0; i < NI; i++) {
        const int c = min(i * 64 + lane, n16 - 1);
        lds_dma16(a + (uintptr_t)c * 16, dst + i * 1024);
    }
}

// s_waitcnt vmcnt(N): at most N of this wave's vector memory operations are
// still outstanding (gfx9 encoding: vmcnt in bits 3:0 and 15:14, expcnt 7,
// lgkmcnt 15).  Compiler fences keep memory accesses on their side of it.
template <int N>
__device__ __forceinline__ void wait_vm_upto() {
    static_assert(N >= 0 && N < 64, "vmcnt range");
    __atomic_signal_fence(__ATOMIC_SEQ_CST);
    __builtin_amdgcn_s_waitcnt((N & 15) | ((N >> 4) << 14) | (7 << 4) | (15 << 8));
    __atomic_signal_fence(__ATOMIC_SEQ_CST);
}

// s_waitcnt vmcnt(n) for a run-time n (0..15).
__device__ __forceinline__ void wait_vm_n(int n) {
    switch (n) {
        case 0: wait_vm_upto<0>(); break;
        case 1: wait_vm_upto<1>(); break;
        case 2: wait_vm_upto<2>(); break;
        case 3: wait_vm_upto<3>(); break;
        case 4: wait_vm_upto<4>(); break;
        case 5: wait_vm_upto<5>(); break;
        case 6: wait_vm_upto<6>(); break;
        case 7: wait_vm_upto<7>(); break;
        case 8: wait_vm_upto<8>(); break;
        case 9: wait_vm_upto<9>(); break;
        case 10: wait_vm_upto<10>(); break;
        case 11: wait_vm_upto<11>(); break;
        case 12: wait_vm_upto<12>(); break;
        case 13: wait_vm_upto<13>(); break;
        case 14: wait_vm_upto<14>(); break;
        default: wait_vm_upto<15>(); break;
    }
}

// Exact half -> float.  Finite values and infinities convert exactly in
// hardware; NaN is canonicalised (sign kept) as the reference's table does
// (qwen3moe.cpp:59).
__device__ __forceinline__ float half_to_float(uint32_t h) {
    const float v = (float)__builtin_bit_cast(_Float16, (uint16_t)h);
    const bool nan = ((h & 0x7C00u) == 0x7C00u) & ((h & 0x3FFu) != 0u);
    return nan ? __builtin_bit_cast(float, 0x7FC00000u | ((h & 0x8000u) << 16)) : v;
}

__device__ __forceinline__ uint32_t byte_of(uint32_t w, int i) { return (w >> (8 * i)) & 0xFFu; }

// 12 scale bytes held in three words -> 6-bit (scale, min) of sub-block j
// (qwen3moe.cpp:133-141).
__device__ __forceinline__ void scale_min_k4(int j, uint32_t s0, uint32_t s1, uint32_t s2, uint32_t& sc, uint32_t& mn) {
    // bytes q[0..3] = s0, q[4..7] = s1, q[8..11] = s2; both forms are formed
    // and one selected, so lanes with different j do not diverge
    const int jj = j & 3;
    const uint32_t b0 = byte_of(s0, jj);  // q[j] (j < 4) or q[j-4]
    const uint32_t b1 = byte_of(s1, jj);  // q[j+4] (j < 4) or q[j]
    const uint32_t b2 = byte_of(s2, jj);  // q[j+4] (j >= 4)
    const bool lo = j < 4;
    sc = lo ? (b0 & 63u) : ((b2 & 15u) | ((b0 >> 6) << 4));
    mn = lo ? (b1 & 63u) : ((b2 >> 4) | ((b1 >> 6) << 4));
}

// ---------------------------------------------------------------------------
// Segment decoders: 32 dequantized values, bit-identical to the reference.
// `blk` points at the block (super-block) start; `j` is the segment in it.

template <class LD = GlobalLd>
__device__ __forceinline__ void decode_seg_q4k(const uint8_t* blk, int j, float* w) {
    const uint4 hdr = LD::b16(blk);
    const float d = half_to_float(hdr.x & 0xFFFFu), dmin = half_to_float(hdr.x >> 16);
    uint32_t sc, mn;
    scale_min_k4(j, hdr.y, hdr.z, hdr.w, sc, mn);
    const float ds = d * (float)sc, dm = dmin * (float)mn;
    const int g = j >> 1, sh = (j & 1) * 4;
    const uint4 a = LD::b16(blk + 16 + 32 * g), b = LD::b16(blk + 32 + 32 * g);
    const uint32_t q[8] = {a.x, a.y, a.z, a.w, b.x, b.y, b.z, b.w};
#pragma unroll
    for (int i = 0; i < 32; i++) {
        const uint32_t v = (q[i >> 2] >> (8 * (i & 3) + sh)) & 15u;
        w[i] = __builtin_fmaf(ds, (float)v, -dm);
    }
}

template <class LD = GlobalLd>
__device__ __forceinline__ void decode_seg_q5k(const uint8_t* blk, int j, float* w) {
    const uint4 hdr = LD::b16(blk);
    const float d = half_to_float(hdr.x & 0xFFFFu), dmin = half_to_float(hdr.x >> 16);
    uint32_t sc, mn;
    scale_min_k4(j, hdr.y, hdr.z, hdr.w, sc, mn);
    const float ds = d * (float)sc, dm = dmin * (float)mn;
    const int g = j >> 1, sh = (j & 1) * 4;
    const uint4 h0 = LD::b16(blk + 16), h1 = LD::b16(blk + 32);
    const uint4 a = LD::b16(blk + 48 + 32 * g), b = LD::b16(blk + 64 + 32 * g);
    const uint32_t q[8] = {a.x, a.y, a.z, a.w, b.x, b.y, b.z, b.w};
    const uint32_t qh[8] = {h0.x, h0.y, h0.z, h0.w, h1.x, h1.y, h1.z, h1.w};
#pragma unroll
    for (int i = 0; i < 32; i++) {
        uint32_t v = (q[i >> 2] >> (8 * (i & 3) + sh)) & 15u;
        v |= ((qh[i >> 2] >> (8 * (i & 3) + j)) & 1u) << 4;
        w[i] = __builtin_fmaf(ds, (float)v, -dm);
    }
}

template <class LD = GlobalLd>
__device__ __forceinline__ void decode_seg_q6k(const uint8_t* blk, int j, float* w) {
    const int n = j >> 2, u = j & 3;
    const float d = half_to_float(LD::u16(blk + 208));
    const Bytes32A2 lo = LD::b32a2(blk + 64 * n + 32 * (u & 1));
    const Bytes32A2 hi = LD::b32a2(blk + 128 + 32 * n);
    const uint16_t scw = LD::u16(blk + 192 + 8 * n + 2 * u);  // scales for l<16 and l>=16
    const float ds0 = d * (float)(int8_t)(scw & 0xFFu);
    const float ds1 = d * (float)(int8_t)(scw >> 8);
    const int shl = (u >> 1) * 4, shh = 2 * u;
#pragma unroll
    for (int i = 0; i < 32; i++) {
        const uint32_t l4 = (lo.w[i >> 2] >> (8 * (i & 3) + shl)) & 15u;
        const uint32_t h2 = (hi.w[i >> 2] >> (8 * (i & 3) + shh)) & 3u;
        const int q = (int)(l4 | (h2 << 4)) - 32;
        w[i] = (i < 16 ? ds0 : ds1) * (float)q;
    }
}

template <class LD = GlobalLd>
__device__ __forceinline__ void decode_seg_q8_0(const uint8_t* blk, float* w) {
    const float d = half_to_float(LD::u16(blk));
    const Bytes32A2 q = LD::b32a2(blk + 2);
#pragma unroll
    for (int i = 0; i < 32; i++) w[i] = d * (float)(int8_t)byte_of(q.w[i >> 2], i & 3);
}

template <class LD = GlobalLd>
__device__ __forceinline__ void decode_seg_f32(const uint8_t* blk, float* w) {
#pragma unroll
    for (int i = 0; i < 8; i++) {
        const uint4 v = LD::b16(blk + 16 * i);
        w[4 * i] = __uint_as_float(v.x); w[4 * i + 1] = __uint_as_float(v.y);
        w[4 * i + 2] = __uint_as_float(v.z); w[4 * i + 3] = __uint_as_float(v.w);
    }
}

// Segment s (0-based, 32 values each) of a row.
template <int T, class LD = GlobalLd>
__device__ __forceinline__ void decode_row_seg(const uint8_t* row, int s, float* w) {
    if constexpr (T == kQ4_K) decode_seg_q4k<LD>(row + (size_t)(s >> 3) * 144, s & 7, w);
    else if constexpr (T == kQ5_K) decode_seg_q5k<LD>(row + (size_t)(s >> 3) * 176, s & 7, w);
    else if constexpr (T == kQ6_K) decode_seg_q6k<LD>(row + (size_t)(s >> 3) * 210, s & 7, w);
    else if constexpr (T == kQ8_0) decode_seg_q8_0<LD>(row + (size_t)s * 34, w);
    else decode_seg_f32<LD>(row + (size_t)s * 128, w);
}

// Wave-wide float sum (wave64); every lane receives the total.
// s_waitcnt vmcnt(0): this wave's memory operations have completed (gfx9
// encoding: vmcnt 0, expcnt 7, lgkmcnt 15).  Compiler fences keep the
// stores before it.
__device__ __forceinline__ void wait_vm() {
    __atomic_signal_fence(__ATOMIC_SEQ_CST);
    __builtin_amdgcn_s_waitcnt(0x0F70);
    __atomic_signal_fence(__ATOMIC_SEQ_CST);
}

__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) v += __shfl_xor(v, off, 64);
    return v;
}

}  // namespace eahmmf
