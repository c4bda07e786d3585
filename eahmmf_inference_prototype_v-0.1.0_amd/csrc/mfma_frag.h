// mfma_frag.h - exact fp16 operands for v_mfma_f32_16x16x32_f16 in the
// grouped expert matmuls (kernels_grouped_mfma.hip, kernels_grouped_wave.hip).
//
// Operand layout (16x16x32): lane l holds A[l%16][8*(l/16) + i],
// B[8*(l/16) + i][l%16] and C[4*(l/16) + i][l%16], i < 8 (C: i < 4).
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

namespace eahmmf {

typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
typedef _Float16 f16x2 __attribute__((ext_vector_type(2)));
typedef float f32x4 __attribute__((ext_vector_type(4)));

constexpr int kPassTok = 64;  // tokens per pass: four 16-token tiles
constexpr float kSumScale = 1.0f / 16.0f;  // sub-block sums (32 values) kept below 2^14

// Weight bytes are read through global-address-space pointers: a row pointer
// taken from the expert table is otherwise generic, and generic (flat) loads
// also count against the LDS counter, so every LDS wait and barrier would
// drain the weight loads in flight.
typedef uint32_t __attribute__((ext_vector_type(2))) mf_u32x2;
typedef uint32_t __attribute__((aligned(2))) mf_u32a2;
__device__ __forceinline__ uint2 ld8_a2(const uint8_t* p) {  // 2-byte aligned
    const __attribute__((address_space(1))) mf_u32a2* q = (const __attribute__((address_space(1))) mf_u32a2*)p;
    return make_uint2(q[0], q[1]);
}
__device__ __forceinline__ uint2 ld8(const uint8_t* p) {  // 8-byte aligned
    const mf_u32x2 v = *(const __attribute__((address_space(1))) mf_u32x2*)p;
    return make_uint2(v.x, v.y);
}
__device__ __forceinline__ int ld_i8(const uint8_t* p) { return (int)*(const __attribute__((address_space(1))) int8_t*)p; }

// Two fp16 values b0, b1 from bytes 2m, 2m+1 of w (each < 256): the byte is
// placed under the exponent of 1024 (0x64XX = 1024 + XX) and 1024 removed.
template <int M>
__device__ __forceinline__ f16x2 byte_pair(uint32_t w) {
    constexpr uint32_t sel = M == 0 ? 0x04010400u : 0x04030402u;
    const f16x2 v = __builtin_bit_cast(f16x2, __builtin_amdgcn_perm(0x64646464u, w, sel));
    return v - (f16x2){(_Float16)1024.0f, (_Float16)1024.0f};
}

// Eight codes (bytes of c) times an integer factor f (|code * f| exact in fp16).
__device__ __forceinline__ f16x8 codes_times(uint2 c, _Float16 f, _Float16 bias) {
    const f16x2 fv = {f, f}, bv = {bias, bias};
    const f16x2 a = (byte_pair<0>(c.x) + bv) * fv, b = (byte_pair<1>(c.x) + bv) * fv;
    const f16x2 d = (byte_pair<0>(c.y) + bv) * fv, e = (byte_pair<1>(c.y) + bv) * fv;
    return (f16x8){a.x, a.y, b.x, b.y, d.x, d.y, e.x, e.y};
}

__device__ __forceinline__ f32x4 mfma(f16x8 a, f16x8 b, f32x4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_f16(a, b, c, 0, 0, 0);
}

// Workgroup barrier for LDS hand-offs only.  __syncthreads() carries a
// workgroup release fence, which on this target waits for every outstanding
// vector-memory operation, loads included (s_waitcnt vmcnt(0)), and so would
// stall on the next chunk's prefetch at every barrier.  This one waits for
// this wave's LDS operations (lgkmcnt 0; vmcnt and expcnt left at their
// maxima), then meets the other waves; global data is consumed only through
// its own registers, so no global ordering is needed here.
__device__ __forceinline__ void lds_barrier() {
    __atomic_signal_fence(__ATOMIC_SEQ_CST);
    __builtin_amdgcn_s_waitcnt(0xC07F);
    __builtin_amdgcn_s_barrier();
    __atomic_signal_fence(__ATOMIC_SEQ_CST);
}

__device__ __forceinline__ float half_at(const uint8_t* p) {  // a weight row's fp16 scale (global)
    return (float)__builtin_bit_cast(_Float16, *(const __attribute__((address_space(1))) uint16_t*)p);
}

}  // namespace eahmmf
