// kernels_gemv.hip - single-token matrix-vector products of the dense decode
// path, with the steps around them fused in.
//
// One launch computes out = W x for up to three weight matrices of one type
// and row length (Q, K and V projections in one go), where the input may be
// formed on the fly: x + x_add (the residual stream after the previous expert
// block) and then RMSNorm with a weight vector (qwen3moe.cpp:527-532), exactly
// as a separate rmsnorm would.  Every block forms the input itself (D floats
// from L2), so no launch is spent on the norm or the residual add; block 0
// also stores the summed and/or normalized input where the next steps need
// them.  An output may add a residual (out[r] = resid[r] + (W x)[r]), and the
// launch may track the first largest output (the greedy argmax of the output
// head, std::max_element order) in a 64-bit key.
//
// Memory layout: a wave takes `rpw` rows at a time (a unit) and copies their
// bytes into its own LDS slots with 16-byte DMA loads (coalesced whatever the
// format's block size; the next unit's copy is in flight while the current
// one is decoded, the first one while the input is formed), then decodes
// 32-value segments from LDS
// (bit-identical dequantization, kquant.h) against the input held in LDS in a
// segment-transposed layout (lane s reads segment s's values without bank
// conflicts).
#include "dpp.h"
#include "internal.h"
#include "kquant.h"

namespace eahmmf {

constexpr int kGemvWaves = 4;      // waves per block when streaming
constexpr int kGemvMaxWaves = 4;   // at most, in a single-shot launch (measured: 8 and 16 start later)
constexpr int kCUs = 256;  // MI355X compute units

// Orderable key of (value, index): larger value wins, then smaller index.
__device__ __forceinline__ unsigned long long argmax_key(float v, unsigned idx) {
    const unsigned u = __builtin_bit_cast(unsigned, v);
    const unsigned o = (u & 0x80000000u) ? ~u : (u | 0x80000000u);
    return ((unsigned long long)o << 32) | (unsigned long long)(0xFFFFFFFFu - idx);
}

// The launch's row segments in registers (no reference to the kernel
// argument block: taking its address would copy it to scratch memory, and a
// scratch load's wait would also wait for the DMA in flight).
struct Segs {
    const uint8_t *w0, *w1, *w2;
    float *o0, *o1, *o2;
    const float *r0, *r1, *r2;
    int rows0, rows1, nseg, rb, ni, rpw, total;

    // global row -> (segment, row in it)
    __device__ __forceinline__ int seg_of(int& row) const {
        const int sg = (nseg > 1 && row >= rows0) ? ((nseg > 2 && row >= rows0 + rows1) ? 2 : 1) : 0;
        row -= sg == 0 ? 0 : (sg == 1 ? rows0 : rows0 + rows1);
        return sg;
    }
    // pointer of segment sg by integer arithmetic (a select chain over
    // pointers is lowered to a lookup in a scratch copy)
    template <class P>
    static __device__ __forceinline__ P pick(int sg, P a, P b, P c) {
        const uint64_t ia = (uint64_t)a, ib = (uint64_t)b, ic = (uint64_t)c;
        return (P)(ia + (sg >= 1 ? ib - ia : 0ull) + (sg >= 2 ? ic - ib : 0ull));
    }
    __device__ __forceinline__ const uint8_t* w(int sg) const { return pick(sg, w0, w1, w2); }
    __device__ __forceinline__ float* out(int sg) const { return pick(sg, o0, o1, o2); }
    __device__ __forceinline__ const float* resid(int sg) const { return pick(sg, r0, r1, r2); }
};

// A float read through the scalar cache (a wave-uniform address; the data is
// not written during the launch).
__device__ __forceinline__ float scalar_ld(const float* p) {
    return *(const __attribute__((address_space(4))) float*)p;
}

// Issues the DMA of unit u's rows into `buf` (rpw slots of ni KiB): always
// rpw * ni instructions (rows past the end repeat the last row), so the
// number in flight is known to the waits.
__device__ __forceinline__ void issue_unit(const Segs& g, int u, uint8_t* buf, int lane) {
    for (int r = 0; r < g.rpw; r++) {
        int row = min(u * g.rpw + r, g.total - 1);
        const int sg = g.seg_of(row);
        const uintptr_t src = (uintptr_t)(g.w(sg) + (size_t)row * g.rb);
        const uintptr_t base = src & ~(uintptr_t)15;
        const int nc = (int)((src + g.rb + 15 - base) / 16);
        uint8_t* dst = buf + (size_t)r * g.ni * 1024;
        for (int i = 0; i < g.ni; i++) lds_dma16(base + (uintptr_t)min(i * 64 + lane, nc - 1) * 16, dst + i * 1024);
    }
}

// IN: four-value input groups per thread (ne0 <= IN * 4 * 256)
template <int T, int IN>
__global__ __launch_bounds__(kGemvMaxWaves * 64) void gemv_kernel(GemvArgs a) {
    extern __shared__ __align__(16) uint8_t smem[];
    __shared__ float red[kGemvMaxWaves];
    __shared__ unsigned long long bkey[kGemvMaxWaves];
    const int tid = threadIdx.x, w = __builtin_amdgcn_readfirstlane(tid / 64), lane = tid % 64;
    const int waves = blockDim.x / 64;
    const int nseg = a.ne0 / 32;
    const Segs g{a.seg[0].w, a.seg[1].w, a.seg[2].w, a.seg[0].out, a.seg[1].out, a.seg[2].out,
                 a.seg[0].resid, a.seg[1].resid, a.seg[2].resid, a.seg[0].rows, a.seg[1].rows,
                 a.nseg, a.rb, a.ni, a.rpw, a.total_rows};
    float4* xt = reinterpret_cast<float4*>(smem);  // [8][nseg]: values 4*i4 .. 4*i4+3 of segment s
    const size_t unit_bytes = (size_t)a.rpw * a.ni * 1024;
    uint8_t* bufs = smem + (size_t)a.ne0 * 4 + (size_t)w * a.nbuf * unit_bytes;  // nbuf units per wave
    const int n_units = (a.total_rows + a.rpw - 1) / a.rpw;
    const int stride = gridDim.x * waves;
    int u = blockIdx.x * waves + w;
    // the first unit's rows are on their way while the input is formed
    // (ni == 0: rows too long to stage, read straight from memory)
    if (a.ni && u < n_units) issue_unit(g, u, bufs, lane);
    // ---- input: x (+ x_add), optionally RMS-normalized; each thread keeps
    // its IN four-value groups in registers, and every load (x, x_add, the
    // norm weights) is issued in one round
    float4 xv[IN], nv[IN];
    float ss = 0.f;
#pragma unroll
    for (int k = 0; k < IN; k++) {
        const int i = (tid + k * waves * 64) * 4;
        if (i < a.ne0) {
            xv[k] = *reinterpret_cast<const float4*>(a.x + i);
            if (a.norm_w) nv[k] = *reinterpret_cast<const float4*>(a.norm_w + i);
            if (a.x_add) {
                const float4 q = *reinterpret_cast<const float4*>(a.x_add + i);
                xv[k].x += q.x; xv[k].y += q.y; xv[k].z += q.z; xv[k].w += q.w;
                if (a.x_sum_out && blockIdx.x == 0) *reinterpret_cast<float4*>(a.x_sum_out + i) = xv[k];
            }
            ss += xv[k].x * xv[k].x + xv[k].y * xv[k].y + xv[k].z * xv[k].z + xv[k].w * xv[k].w;
        }
    }
    float sc = 1.f;
    if (a.norm_w) {
        ss = group_sum_all<64>(ss);
        if (lane == 0) red[w] = ss;
        __syncthreads();
        float tot = 0.f;
        for (int i = 0; i < waves; i++) tot += red[i];
        sc = 1.0f / sqrtf(tot / (float)a.ne0 + a.eps);
    }
#pragma unroll
    for (int k = 0; k < IN; k++) {
        const int i = (tid + k * waves * 64) * 4;
        if (i < a.ne0) {
            float4 v = xv[k];
            if (a.norm_w) {
                v.x = v.x * sc * nv[k].x; v.y = v.y * sc * nv[k].y; v.z = v.z * sc * nv[k].z; v.w = v.w * sc * nv[k].w;
                if (a.xn_out && blockIdx.x == 0) *reinterpret_cast<float4*>(a.xn_out + i) = v;
            }
            xt[((i % 32) / 4) * nseg + i / 32] = v;
        }
    }
    __syncthreads();
    // ---- rows: each wave walks its units, the next unit's DMA in flight
    // while the current one is decoded
    float best = -INFINITY;
    unsigned best_i = 0xFFFFFFFFu;
    const int per_unit = a.rpw * a.ni;  // DMA instructions per unit
    for (int k = 0; u < n_units; u += stride, k++) {
        uint8_t* cur = bufs + (a.nbuf == 2 ? (k & 1) * unit_bytes : 0);
        if (a.ni && a.nbuf == 2 && u + stride < n_units) {
            issue_unit(g, u + stride, bufs + ((k + 1) & 1) * unit_bytes, lane);
            wait_vm_n(per_unit);
        } else if (a.ni) {
            wait_vm();
        }
        const int r0 = u * a.rpw, nr = min(a.rpw, a.total_rows - r0);
        for (int r = 0; r < nr; r++) {
            int row = r0 + r;
            const int sg = g.seg_of(row);
            const uint8_t* rg = g.w(sg) + (size_t)row * a.rb;
            const uint8_t* rl = cur + (size_t)r * a.ni * 1024 + ((uintptr_t)rg & 15);
            const float* resid = g.resid(sg);
            const float rv = resid ? scalar_ld(resid + row) : 0.f;
            float acc = 0.f;
            for (int s = lane; s < nseg; s += 64) {
                float wv[32];
                if (a.ni)
                    decode_row_seg<T, LdsLd>(rl, s, wv);
                else
                    decode_row_seg<T, GlobalLd>(rg, s, wv);
                float p = 0.f;
#pragma unroll
                for (int i4 = 0; i4 < 8; i4++) {
                    const float4 xv = xt[i4 * nseg + s];
                    p = __builtin_fmaf(wv[4 * i4], xv.x, p);
                    p = __builtin_fmaf(wv[4 * i4 + 1], xv.y, p);
                    p = __builtin_fmaf(wv[4 * i4 + 2], xv.z, p);
                    p = __builtin_fmaf(wv[4 * i4 + 3], xv.w, p);
                }
                acc += p;
            }
            acc = group_sum<64>(acc);  // the total is in lane 63
            if (lane == 63) {
                const float v = resid ? rv + acc : acc;
                *(__attribute__((address_space(1))) float*)(g.out(sg) + row) = v;  // (a global store, not flat)
                if (v > best || best_i == 0xFFFFFFFFu) {
                    best = v;
                    best_i = (unsigned)(r0 + r);
                }
            }
        }
        // one slot: the next unit's copy starts once this one is decoded
        if (a.ni && a.nbuf == 1 && u + stride < n_units) issue_unit(g, u + stride, bufs, lane);
    }
    if (a.amax) {  // one atomic per block, and only when it can raise the key
        if (lane == 63) bkey[w] = best_i == 0xFFFFFFFFu ? 0ull : argmax_key(best, best_i);
        __syncthreads();
        if (tid == 0) {
            unsigned long long kmax = bkey[0];
            for (int i = 1; i < waves; i++) kmax = bkey[i] > kmax ? bkey[i] : kmax;
            if (kmax > __hip_atomic_load(a.amax, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT)) atomicMax(a.amax, kmax);
        }
    }
}

template <int IN>
static bool launch_in(int type, int blocks, int th, size_t lds, const GemvArgs& a, hipStream_t st) {
    switch (type) {
        case kF32: gemv_kernel<kF32, IN><<<blocks, th, lds, st>>>(a); return true;
        case kQ8_0: gemv_kernel<kQ8_0, IN><<<blocks, th, lds, st>>>(a); return true;
        case kQ4_K: gemv_kernel<kQ4_K, IN><<<blocks, th, lds, st>>>(a); return true;
        case kQ5_K: gemv_kernel<kQ5_K, IN><<<blocks, th, lds, st>>>(a); return true;
        case kQ6_K: gemv_kernel<kQ6_K, IN><<<blocks, th, lds, st>>>(a); return true;
        default: return false;
    }
}

static bool launch_typed(int type, int in, int blocks, int th, size_t lds, const GemvArgs& a, hipStream_t st) {
    return in == 2 ? launch_in<2>(type, blocks, th, lds, a, st)
                   : (in == 4 ? launch_in<4>(type, blocks, th, lds, a, st) : launch_in<8>(type, blocks, th, lds, a, st));
}

size_t gemv_lds_bytes(const GemvArgs& a, int waves) {
    return (size_t)a.ne0 * 4 + (size_t)waves * a.nbuf * a.rpw * a.ni * 1024;
}

bool gemv_supported(int type, int ne0, size_t rb) {
    if (type != kF32 && !type_supported(type)) return false;
    if (ne0 <= 0 || ne0 % 32 || ne0 % type_blck(type) || ne0 > 8192) return false;  // 8192 = 8 x 4 x 256
    // rows of 16-byte loads (F32, Q4_K, Q5_K) 16-byte aligned for the direct reads
    const bool a16 = type == kF32 || type == kQ4_K || type == kQ5_K;
    return rb >= (size_t)(ne0 / type_blck(type)) * type_bytes(type) && (!a16 || rb % 16 == 0);
}

hipError_t launch_gemv(int type, GemvArgs a, hipStream_t st) {
    if (a.nseg < 1 || a.nseg > 3 || !a.x || !gemv_supported(type, a.ne0, (size_t)a.rb)) return hipErrorInvalidValue;
    a.total_rows = 0;
    for (int i = 0; i < a.nseg; i++) {
        if (!a.seg[i].w || !a.seg[i].out || a.seg[i].rows <= 0) return hipErrorInvalidValue;
        a.total_rows += a.seg[i].rows;
    }
    // a row's LDS slot: 1 KiB DMA groups holding its bytes at any 16-byte phase
    // (up to 15 bytes of lead) plus the 4 bytes the realigning reads may touch;
    // rows whose slots do not fit next to the input (at most 15 DMA
    // instructions a row, 64 KiB of LDS) are read straight from memory
    a.ni = (a.rb + 19 + 1023) / 1024;
    if (a.ni > 15 || a.ne0 * 4 + kGemvWaves * a.ni * 1024 > 64 * 1024) {
        a.ni = 0;
        a.nbuf = 1;
        a.rpw = 1;
        const int want = (a.total_rows + kGemvWaves - 1) / kGemvWaves;
        const int blocks = want < 2048 ? want : 2048;
        clear_stale_error();
        if (!launch_typed(type, a.ne0 <= 2048 ? 2 : (a.ne0 <= 4096 ? 4 : 8), blocks, kGemvWaves * 64,
                          (size_t)a.ne0 * 4, a, st))
            return hipErrorInvalidValue;
        return hipGetLastError();
    }
    // Single shot when one row per wave for every row fits on the chip at
    // once (blocks resident together, by LDS and by waves per CU): every
    // row's DMA is in flight from the start.  Otherwise stream: two units of
    // rpw rows per wave in LDS (one if two do not fit), at most 15 DMA
    // instructions a unit, the next unit in flight while one is decoded.
    // (single shot: the most waves per block whose LDS stays within 64 KiB,
    // so that fewer, larger blocks form the input fewer times)
    int waves = kGemvWaves, blocks = 0;
    for (int wv = kGemvMaxWaves; wv >= kGemvWaves; wv /= 2) {
        const int lds1 = a.ne0 * 4 + wv * a.ni * 1024;
        if (lds1 > 64 * 1024) continue;
        const int per_cu = min(32 / wv, (160 * 1024) / lds1);
        const int blocks1 = (a.total_rows + wv - 1) / wv;
        if (blocks1 <= kCUs * per_cu) {
            waves = wv;
            blocks = blocks1;
            break;
        }
    }
    if (blocks) {
        a.nbuf = 1;
        a.rpw = 1;
    } else {
        const int avail_kb = (64 * 1024 - a.ne0 * 4) / 1024;
        a.nbuf = avail_kb >= kGemvWaves * 2 * a.ni ? 2 : 1;
        a.rpw = avail_kb / (kGemvWaves * a.nbuf * a.ni);
        if (a.rpw > 2) a.rpw = 2;
        if (a.rpw * a.ni > 15) a.rpw = 15 / a.ni;
        if (a.rpw < 1) return hipErrorInvalidValue;
        const int n_units = (a.total_rows + a.rpw - 1) / a.rpw;
        const int want = (n_units + kGemvWaves - 1) / kGemvWaves;
        blocks = want < 2048 ? want : 2048;
    }
    const size_t lds = gemv_lds_bytes(a, waves);
    if (lds > 64 * 1024) return hipErrorInvalidValue;
    clear_stale_error();
    const int th = waves * 64;
    const int in = a.ne0 <= 2048 ? 2 : (a.ne0 <= 4096 ? 4 : 8);
    if (!launch_typed(type, in, blocks, th, lds, a, st)) return hipErrorInvalidValue;
    return hipGetLastError();
}

}  // namespace eahmmf
