// kernels_basic.hip - dequantization and the general quantized matmul used by
// the drop-in eahmmf_hip_matmul / eahmmf_hip_matmul_pair entry points.
//
//   dequant_kernel<T>   one 32-value segment per thread, bit-identical to the
//                       reference CPU decoder (qwen3moe.cpp:128-202)
//   matmul_kernel<T,TT> out[t*ldo + r] = sum_k W[r,k] x[t*ldx + k], one wave64
//                       per output row, lanes striding over 32-value segments,
//                       TT tokens per launch column (grid.y); fp32 accumulate.
//                       Same contract as the reference's expert matmul
//                       (expert_cuda.cu:128-247, qwen3moe.cpp:397-419).
#include "internal.h"
#include "kquant.h"

namespace eahmmf {

template <int T>
__global__ __launch_bounds__(256) void dequant_kernel(const uint8_t* __restrict__ w, int64_t segs_per_row, int64_t nrows,
                                                      size_t row_bytes, float* __restrict__ out) {
    const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= segs_per_row * nrows) return;
    const int64_t r = i / segs_per_row, s = i % segs_per_row;
    float v[32];
    decode_row_seg<T>(w + (size_t)r * row_bytes, (int)s, v);
    float4* o = reinterpret_cast<float4*>(out + (size_t)r * segs_per_row * 32 + (size_t)s * 32);
#pragma unroll
    for (int q = 0; q < 8; q++) o[q] = make_float4(v[4 * q], v[4 * q + 1], v[4 * q + 2], v[4 * q + 3]);
}

template <int T, int TT>
__global__ __launch_bounds__(256) void matmul_kernel(const uint8_t* __restrict__ w, int ne0, int ne1, size_t row_bytes,
                                                     const float* __restrict__ x, int nb, int ldx,
                                                     float* __restrict__ out, int ldo) {
    const int lane = threadIdx.x & 63;
    const int row = blockIdx.x * 4 + (threadIdx.x >> 6);
    if (row >= ne1) return;  // whole wave leaves together
    const int t0 = blockIdx.y * TT;
    const int nt = min(TT, nb - t0);
    const int nseg = ne0 / 32;
    const uint8_t* wr = w + (size_t)row * row_bytes;
    float acc[TT];
#pragma unroll
    for (int t = 0; t < TT; t++) acc[t] = 0.f;
    for (int s = lane; s < nseg; s += 64) {
        float wv[32];
        decode_row_seg<T>(wr, s, wv);
#pragma unroll
        for (int t = 0; t < TT; t++) {
            if (t < nt) {
                const float* xp = x + (size_t)(t0 + t) * ldx + (size_t)s * 32;
                float p = 0.f;
#pragma unroll
                for (int i = 0; i < 32; i++) p = __builtin_fmaf(wv[i], xp[i], p);
                acc[t] += p;
            }
        }
    }
#pragma unroll
    for (int t = 0; t < TT; t++) {
        if (t < nt) {
            const float v = wave_sum(acc[t]);
            if (lane == 0) out[(size_t)(t0 + t) * ldo + row] = v;
        }
    }
}

hipError_t launch_dequant(int type, const uint8_t* w, int64_t ne0, int64_t nrows, size_t row_bytes, float* out,
                          hipStream_t st) {
    const int64_t segs = ne0 / 32;
    const int64_t total = segs * nrows;
    if (total <= 0) return hipSuccess;
    clear_stale_error();
    const dim3 grid((unsigned)((total + 255) / 256)), block(256);
    switch (type) {
        case kQ4_K: dequant_kernel<kQ4_K><<<grid, block, 0, st>>>(w, segs, nrows, row_bytes, out); break;
        case kQ5_K: dequant_kernel<kQ5_K><<<grid, block, 0, st>>>(w, segs, nrows, row_bytes, out); break;
        case kQ6_K: dequant_kernel<kQ6_K><<<grid, block, 0, st>>>(w, segs, nrows, row_bytes, out); break;
        case kQ8_0: dequant_kernel<kQ8_0><<<grid, block, 0, st>>>(w, segs, nrows, row_bytes, out); break;
        case kF32: dequant_kernel<kF32><<<grid, block, 0, st>>>(w, segs, nrows, row_bytes, out); break;
        default: return hipErrorInvalidValue;
    }
    return hipGetLastError();
}

hipError_t launch_matmul(int type, const uint8_t* w, int ne0, int ne1, size_t row_bytes, const float* x, int nb,
                         int ldx, float* out, int ldo, hipStream_t st) {
    constexpr int TT = 8;
    clear_stale_error();
    const dim3 grid((unsigned)((ne1 + 3) / 4), (unsigned)((nb + TT - 1) / TT)), block(256);
    switch (type) {
        case kQ4_K: matmul_kernel<kQ4_K, TT><<<grid, block, 0, st>>>(w, ne0, ne1, row_bytes, x, nb, ldx, out, ldo); break;
        case kQ5_K: matmul_kernel<kQ5_K, TT><<<grid, block, 0, st>>>(w, ne0, ne1, row_bytes, x, nb, ldx, out, ldo); break;
        case kQ6_K: matmul_kernel<kQ6_K, TT><<<grid, block, 0, st>>>(w, ne0, ne1, row_bytes, x, nb, ldx, out, ldo); break;
        case kQ8_0: matmul_kernel<kQ8_0, TT><<<grid, block, 0, st>>>(w, ne0, ne1, row_bytes, x, nb, ldx, out, ldo); break;
        case kF32: matmul_kernel<kF32, TT><<<grid, block, 0, st>>>(w, ne0, ne1, row_bytes, x, nb, ldx, out, ldo); break;
        default: return hipErrorInvalidValue;
    }
    return hipGetLastError();
}

// Small copies between pinned host staging and device buffers as a kernel
// (the GPU reads and writes pinned host memory directly): for the few KB a
// synchronous entry point moves per call this starts sooner than a copy
// engine transfer.  Two regions of 4-byte words per launch.
__global__ __launch_bounds__(256) void copy_words_kernel(uint32_t* d0, const uint32_t* s0, size_t n0, uint32_t* d1,
                                                         const uint32_t* s1, size_t n1) {
    const size_t stride = (size_t)gridDim.x * blockDim.x;
    for (size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x; i < n0 + n1; i += stride) {
        if (i < n0)
            d0[i] = s0[i];
        else
            d1[i - n0] = s1[i - n0];
    }
}

hipError_t launch_copy_words(void* d0, const void* s0, size_t bytes0, void* d1, const void* s1, size_t bytes1,
                             hipStream_t st) {
    if ((bytes0 | bytes1) & 3) return hipErrorInvalidValue;
    const size_t n = (bytes0 + bytes1) / 4;
    if (n == 0) return hipSuccess;
    clear_stale_error();
    const size_t blocks = (n + 255) / 256;
    copy_words_kernel<<<(unsigned)(blocks < 64 ? blocks : 64), 256, 0, st>>>(
        (uint32_t*)d0, (const uint32_t*)s0, bytes0 / 4, (uint32_t*)d1, (const uint32_t*)s1, bytes1 / 4);
    return hipGetLastError();
}

// The same copies by one workgroup, then a completion word for a host that
// waits by polling pinned memory: every thread's stores are done (barrier),
// then one system-scope fence and the word `seq` stored to `flag`, so a host
// that reads seq there finds the copied data in place.
__global__ __launch_bounds__(256) void copy_words_signal_kernel(uint32_t* d0, const uint32_t* s0, size_t n0,
                                                                uint32_t* d1, const uint32_t* s1, size_t n1,
                                                                unsigned* flag, unsigned seq) {
    for (size_t i = threadIdx.x; i < n0 + n1; i += blockDim.x) {
        if (i < n0)
            d0[i] = s0[i];
        else
            d1[i - n0] = s1[i - n0];
    }
    __syncthreads();
    if (threadIdx.x == 0) {
        __threadfence_system();
        __hip_atomic_store(flag, seq, __ATOMIC_RELEASE, __HIP_MEMORY_SCOPE_SYSTEM);
    }
}

hipError_t launch_copy_words_signal(void* d0, const void* s0, size_t bytes0, void* d1, const void* s1, size_t bytes1,
                                    unsigned* flag, unsigned seq, hipStream_t st) {
    if ((bytes0 | bytes1) & 3 || !flag) return hipErrorInvalidValue;
    clear_stale_error();
    copy_words_signal_kernel<<<1, 256, 0, st>>>((uint32_t*)d0, (const uint32_t*)s0, bytes0 / 4, (uint32_t*)d1,
                                                (const uint32_t*)s1, bytes1 / 4, flag, seq);
    return hipGetLastError();
}

}  // namespace eahmmf
