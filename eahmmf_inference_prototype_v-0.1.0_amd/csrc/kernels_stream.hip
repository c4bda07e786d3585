// Streaming read: the achievable HBM read rate of the device, the measured
// ceiling the decode kernels are read against beside the nominal 8 TB/s.
//
// Workgroup g of G reads the contiguous chunk [g per, (g+1) per) of the buffer
// (16-byte units) with nontemporal 16-byte loads, eight per thread in flight,
// and XORs every 32-bit word it reads into one value, stored to sink[g]; the
// other words of the kStreamMaxGroups-word sink are set to 0, so the XOR of
// the whole sink is the XOR of the buffer and no load can be dropped.
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "internal.h"

namespace eahmmf {

constexpr int kStreamThreads = 512;
constexpr int kStreamBatch = 8;          // loads in flight per thread
constexpr int kStreamMaxGroups = 4096;   // 16 per CU

typedef uint32_t v4u __attribute__((ext_vector_type(4)));

__global__ __launch_bounds__(kStreamThreads) void stream_read_kernel(const v4u* buf, size_t n16, size_t per,
                                                                    uint32_t* sink) {
    const size_t b = (size_t)blockIdx.x * per;
    const size_t e = b + per < n16 ? b + per : n16;
    uint32_t acc = 0;
    // every batch issues all eight loads (those past the chunk are masked
    // off), so a partial batch costs one round trip, not one per load
    for (size_t i = b + threadIdx.x; i < e; i += kStreamBatch * kStreamThreads) {
        v4u v[kStreamBatch];
#pragma unroll
        for (int u = 0; u < kStreamBatch; u++) {
            const size_t j = i + (size_t)u * kStreamThreads;
            v[u] = j < e ? __builtin_nontemporal_load(buf + j) : v4u{0u, 0u, 0u, 0u};
        }
#pragma unroll
        for (int u = 0; u < kStreamBatch; u++) acc ^= (v[u].x ^ v[u].y) ^ (v[u].z ^ v[u].w);
    }
    for (int off = 32; off > 0; off >>= 1) acc ^= (uint32_t)__shfl_xor((int)acc, off, 64);
    __shared__ uint32_t wv[kStreamThreads / 64];
    if (threadIdx.x % 64 == 0) wv[threadIdx.x / 64] = acc;
    __syncthreads();
    if (threadIdx.x == 0) {
        uint32_t t = 0;
        for (int w = 0; w < kStreamThreads / 64; w++) t ^= wv[w];
        sink[blockIdx.x] = t;
    }
    // the sink words past the grid read as 0 (plain stores: no atomics on
    // one address, which would serialise across the XCDs)
    for (unsigned w = blockIdx.x + gridDim.x * (threadIdx.x + 1u); w < (unsigned)kStreamMaxGroups;
         w += gridDim.x * kStreamThreads)
        sink[w] = 0u;
}

// Workgroups: one full batch per thread at least, rounded up to a multiple of
// 256 (one per CU) so that every CU reads the same share; small reads use
// fewer.
int stream_groups(size_t bytes) {
    const size_t n16 = bytes / 16;
    size_t g = (n16 + (size_t)kStreamThreads * kStreamBatch - 1) / ((size_t)kStreamThreads * kStreamBatch);
    if (g > 256) g = (g + 255) / 256 * 256;
    if (g < 1) g = 1;
    if (g > (size_t)kStreamMaxGroups) g = kStreamMaxGroups;
    return (int)g;
}

hipError_t launch_stream_read(const void* buf, size_t bytes, uint32_t* sink, hipStream_t st) {
    if (bytes == 0) return hipSuccess;
    if (!buf || !sink || bytes % 16 || (uintptr_t)buf % 16 || (uintptr_t)sink % 4) return hipErrorInvalidValue;
    const size_t n16 = bytes / 16;
    const int g = stream_groups(bytes);
    const size_t per = (n16 + (size_t)g - 1) / (size_t)g;
    hipLaunchKernelGGL(stream_read_kernel, dim3(g), dim3(kStreamThreads), 0, st, static_cast<const v4u*>(buf), n16,
                       per, sink);
    return hipGetLastError();
}

}  // namespace eahmmf
