// kernels_moe.hip - fused single-token MoE expert FFN (decode) and routing.
//
// The reference runs this block as host code around per-expert GPU matmuls
// (qwen3moe.cpp:1024-1067: gate/up pair, SiLU*up on the CPU, down, weighted
// scatter-add on the CPU).  Here the whole block for one token is two
// launches on one stream:
//   phase A  moe_gate_up_kernel<GT,UT>: h[j][f] = silu(gate_j[f].x) * (up_j[f].x)
//            for all k routed experts j; x is staged once per workgroup in LDS.
//   phase B  moe_down_kernel<DT>: y[r] = sum_j w_j * (down_j[r].h_j); h staged in
//            LDS; the k experts of one output row are reduced inside one wave,
//            so no atomics and the result is deterministic.
// route_topk_kernel does softmax -> top-k -> renormalise (qwen3moe.cpp:1011-1023).
#include "dpp.h"
#include "expf_ref.h"
#include "internal.h"
#include "kquant.h"

namespace eahmmf {

struct SlotSource {
    DecodeSlots direct;        // used when table == nullptr
    const ExpertEntry* table;  // device table indexed by expert id
    const int* ids;            // device [k]
    const float* w;            // device [k]
    int n_expert;
};

__device__ __forceinline__ bool resolve_slot(const SlotSource& src, int j, const uint8_t*& g, const uint8_t*& u,
                                             const uint8_t*& d, float& w) {
    if (!src.table) {
        g = src.direct.gate[j];
        u = src.direct.up[j];
        d = src.direct.down[j];
        w = src.direct.w[j];
        return true;
    }
    const int id = src.ids[j];
    if (id < 0 || id >= src.n_expert) return false;  // malformed routing contributes nothing
    const ExpertEntry e = src.table[id];
    g = e.gate;
    u = e.up;
    d = e.down;
    w = src.w[j];
    return g && u && d;
}

__device__ __forceinline__ float silu_mul(float g, float u) { return g / (1.0f + expf(-g)) * u; }

template <int GT, int UT>
__global__ __launch_bounds__(256) void moe_gate_up_kernel(MoeShape s, SlotSource src, int k,
                                                          const float* __restrict__ x, float* __restrict__ h) {
    extern __shared__ float xs[];
    for (int i = threadIdx.x; i < s.D; i += blockDim.x) xs[i] = x[i];
    __syncthreads();
    const int lane = threadIdx.x & 63;
    const int item = blockIdx.x * 4 + (threadIdx.x >> 6);  // (expert slot, row) pair
    if (item >= k * s.FF) return;
    const int j = item / s.FF, f = item % s.FF;
    const uint8_t *gp, *up, *dp;
    float wj;
    float gs = 0.f, us = 0.f;
    if (resolve_slot(src, j, gp, up, dp, wj)) {
        const uint8_t* grow = gp + (size_t)f * s.gate_rb;
        const uint8_t* urow = up + (size_t)f * s.up_rb;
        const int nseg = s.D / 32;
        for (int sg = lane; sg < nseg; sg += 64) {
            float wv[32];
            const float* xp = xs + sg * 32;
            decode_row_seg<GT>(grow, sg, wv);
            float pg = 0.f;
#pragma unroll
            for (int i = 0; i < 32; i++) pg = __builtin_fmaf(wv[i], xp[i], pg);
            decode_row_seg<UT>(urow, sg, wv);
            float pu = 0.f;
#pragma unroll
            for (int i = 0; i < 32; i++) pu = __builtin_fmaf(wv[i], xp[i], pu);
            gs += pg;
            us += pu;
        }
    }
    gs = wave_sum(gs);
    us = wave_sum(us);
    if (lane == 0) h[item] = silu_mul(gs, us);
}

template <int DT>
__global__ __launch_bounds__(256) void moe_down_kernel(MoeShape s, SlotSource src, int k,
                                                       const float* __restrict__ h, float* __restrict__ y) {
    extern __shared__ float hs[];
    const int n = k * s.FF;
    for (int i = threadIdx.x; i < n; i += blockDim.x) hs[i] = h[i];
    __syncthreads();
    const int lane = threadIdx.x & 63;
    const int r = blockIdx.x * 4 + (threadIdx.x >> 6);
    if (r >= s.D) return;
    const int segs = s.FF / 32;
    float acc = 0.f;
    for (int q = lane; q < k * segs; q += 64) {
        const int j = q / segs, sg = q % segs;
        const uint8_t *gp, *up, *dp;
        float wj;
        if (!resolve_slot(src, j, gp, up, dp, wj)) continue;
        float wv[32];
        decode_row_seg<DT>(dp + (size_t)r * s.down_rb, sg, wv);
        const float* hp = hs + j * s.FF + sg * 32;
        float p = 0.f;
#pragma unroll
        for (int i = 0; i < 32; i++) p = __builtin_fmaf(wv[i], hp[i], p);
        acc = __builtin_fmaf(wj, p, acc);
    }
    acc = wave_sum(acc);
    if (lane == 0) y[r] = acc;
}

// ---------------------------------------------------------------------------
// Routing: one wave per token.  Ranking uses the same key as the reference,
// e_i = expf(l_i - max) (desc, bit for bit as the reference's libm forms it:
// expf_ref.h) with the lower index winning ties; the chosen e are summed in
// rank order and divided (qwen3moe.cpp:1011-1023).  Each candidate is a word
// bits(e_i) + 1 in registers (0 for a NaN e_i and past n_expert); a round
// picks the largest word left by a DPP wave maximum and the lowest id holding
// it by ballots over the per-lane chunks (no LDS round trip; a shuffle-based
// argmax cost about 1 us a round).  Slots past the last valid candidate (NaN
// logits) get id -1 and weight 0, as the fused kernel's routing gives them.
__global__ __launch_bounds__(256) void route_topk_kernel(const float* __restrict__ logits, int nb, int n_expert, int k,
                                                         int* __restrict__ ids, float* __restrict__ w) {
    const int lane = threadIdx.x & 63;
    const int t = blockIdx.x * 4 + (threadIdx.x >> 6);
    if (t >= nb) return;  // wave-uniform
    constexpr int kMaxPerLane = 8;  // n_expert <= 512
    const float* l = logits + (size_t)t * n_expert;
    float lv[kMaxPerLane];
#pragma unroll
    for (int i = 0; i < kMaxPerLane; i++) {
        const int id = lane + 64 * i;
        lv[i] = id < n_expert ? l[id] : -INFINITY;
    }
    float mx = lv[0];
#pragma unroll
    for (int i = 1; i < kMaxPerLane; i++) mx = fmaxf(mx, lv[i]);
    mx = dpp_max(mx);
    uint32_t hi[kMaxPerLane];
#pragma unroll
    for (int i = 0; i < kMaxPerLane; i++) {
        const int id = lane + 64 * i;
        const float e = id < n_expert ? expf_ref(lv[i] - mx) : -1.0f;
        hi[i] = (id < n_expert && e == e) ? __builtin_bit_cast(uint32_t, e) + 1u : 0u;
    }
    uint32_t my_hi = 0u;  // lane r: slot r's word
    int my_id = -1;
    for (int r = 0; r < k; r++) {
        uint32_t m = hi[0];
#pragma unroll
        for (int i = 1; i < kMaxPerLane; i++) m = max(m, hi[i]);
        m = dpp_max_u32(m);
        if (m == 0u) break;  // only NaN candidates left
        int id = -1;
#pragma unroll
        for (int i = kMaxPerLane - 1; i >= 0; i--) {
            const uint64_t b = __ballot(hi[i] == m);
            if (b) id = 64 * i + __builtin_ctzll(b);
        }
        if (lane == r) {
            my_hi = m;
            my_id = id;
        }
        const bool mine = lane == (id & 63);
#pragma unroll
        for (int i = 0; i < kMaxPerLane; i++)
            if (mine && (id >> 6) == i) hi[i] = 0u;
    }
    const float my_e = my_hi ? __builtin_bit_cast(float, my_hi - 1u) : 0.f;
    float tot = 0.f;
    for (int r = 0; r < k; r++) tot += __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, my_e), r));
    if (lane < k) {
        ids[(size_t)t * k + lane] = my_id;
        w[(size_t)t * k + lane] = my_hi ? my_e / tot : 0.f;
    }
}

// The routing's exp on its own (glibc's expf, bit for bit): y[i] = e^x[i].
__global__ __launch_bounds__(256) void expf_ref_kernel(const float* __restrict__ x, float* __restrict__ y, int64_t n) {
    for (int64_t i = blockIdx.x * (int64_t)blockDim.x + threadIdx.x; i < n; i += (int64_t)gridDim.x * blockDim.x)
        y[i] = expf_ref(x[i]);
}

hipError_t launch_expf_ref(const float* x, float* y, int64_t n, hipStream_t st) {
    if (n < 0 || (n > 0 && (!x || !y))) return hipErrorInvalidValue;
    if (n == 0) return hipSuccess;
    const int64_t blocks = (n + 255) / 256;
    clear_stale_error();
    hipLaunchKernelGGL(expf_ref_kernel, dim3((unsigned)(blocks < 4096 ? blocks : 4096)), dim3(256), 0, st, x, y, n);
    return hipGetLastError();
}

// ---------------------------------------------------------------------------

bool type_supported(int t) { return t == kQ4_K || t == kQ5_K || t == kQ6_K || t == kQ8_0; }

bool moe_shape_ok(const MoeShape& s) {
    if (!type_supported(s.gate_type) || !type_supported(s.up_type) || !type_supported(s.down_type)) return false;
    if (s.D <= 0 || s.FF <= 0) return false;
    if (s.D % type_blck(s.gate_type) || s.D % type_blck(s.up_type) || s.FF % type_blck(s.down_type)) return false;
    if (s.gate_rb != (size_t)(s.D / type_blck(s.gate_type)) * type_bytes(s.gate_type)) return false;
    if (s.up_rb != (size_t)(s.D / type_blck(s.up_type)) * type_bytes(s.up_type)) return false;
    if (s.down_rb != (size_t)(s.FF / type_blck(s.down_type)) * type_bytes(s.down_type)) return false;
    return true;
}

template <int GT, int UT>
static void launch_phase_a(const MoeShape& s, const SlotSource& src, int k, const float* x, float* h, hipStream_t st) {
    const dim3 grid((unsigned)((k * s.FF + 3) / 4)), block(256);
    moe_gate_up_kernel<GT, UT><<<grid, block, (size_t)s.D * sizeof(float), st>>>(s, src, k, x, h);
}

template <int GT>
static hipError_t dispatch_phase_a_up(const MoeShape& s, const SlotSource& src, int k, const float* x, float* h,
                                      hipStream_t st) {
    switch (s.up_type) {
        case kQ4_K: launch_phase_a<GT, kQ4_K>(s, src, k, x, h, st); break;
        case kQ5_K: launch_phase_a<GT, kQ5_K>(s, src, k, x, h, st); break;
        case kQ6_K: launch_phase_a<GT, kQ6_K>(s, src, k, x, h, st); break;
        case kQ8_0: launch_phase_a<GT, kQ8_0>(s, src, k, x, h, st); break;
        default: return hipErrorInvalidValue;
    }
    return hipSuccess;
}

static hipError_t run_decode(const MoeShape& s, const SlotSource& src, int k, const float* x, float* h, float* y,
                             hipStream_t st) {
    if (!moe_shape_ok(s) || k <= 0 || k > kMaxSlots) return hipErrorInvalidValue;
    if ((size_t)k * s.FF * sizeof(float) > 64 * 1024 || (size_t)s.D * sizeof(float) > 64 * 1024)
        return hipErrorInvalidValue;
    clear_stale_error();
    hipError_t e;
    switch (s.gate_type) {
        case kQ4_K: e = dispatch_phase_a_up<kQ4_K>(s, src, k, x, h, st); break;
        case kQ5_K: e = dispatch_phase_a_up<kQ5_K>(s, src, k, x, h, st); break;
        case kQ6_K: e = dispatch_phase_a_up<kQ6_K>(s, src, k, x, h, st); break;
        case kQ8_0: e = dispatch_phase_a_up<kQ8_0>(s, src, k, x, h, st); break;
        default: return hipErrorInvalidValue;
    }
    if (e != hipSuccess) return e;
    if ((e = hipGetLastError()) != hipSuccess) return e;
    const dim3 grid((unsigned)((s.D + 3) / 4)), block(256);
    const size_t lds = (size_t)k * s.FF * sizeof(float);
    switch (s.down_type) {
        case kQ4_K: moe_down_kernel<kQ4_K><<<grid, block, lds, st>>>(s, src, k, h, y); break;
        case kQ5_K: moe_down_kernel<kQ5_K><<<grid, block, lds, st>>>(s, src, k, h, y); break;
        case kQ6_K: moe_down_kernel<kQ6_K><<<grid, block, lds, st>>>(s, src, k, h, y); break;
        case kQ8_0: moe_down_kernel<kQ8_0><<<grid, block, lds, st>>>(s, src, k, h, y); break;
        default: return hipErrorInvalidValue;
    }
    return hipGetLastError();
}

hipError_t launch_moe_decode(const MoeShape& s, const DecodeSlots& slots, const float* x, float* h, float* y,
                             hipStream_t st) {
    SlotSource src{};
    src.direct = slots;
    src.table = nullptr;
    return run_decode(s, src, slots.k, x, h, y, st);
}

hipError_t launch_moe_decode_routed(const MoeShape& s, const ExpertEntry* table, int n_expert, const int* ids,
                                    const float* w, int k, const float* x, float* h, float* y, hipStream_t st) {
    if (!table || !ids || !w || n_expert <= 0) return hipErrorInvalidValue;
    SlotSource src{};
    src.table = table;
    src.ids = ids;
    src.w = w;
    src.n_expert = n_expert;
    return run_decode(s, src, k, x, h, y, st);
}

hipError_t launch_route_topk(const float* logits, int nb, int n_expert, int k, int* ids, float* w, hipStream_t st) {
    if (nb <= 0 || n_expert <= 0 || n_expert > 512 || k <= 0 || k > kMaxSlots || k > n_expert)
        return hipErrorInvalidValue;
    clear_stale_error();
    const dim3 grid((unsigned)((nb + 3) / 4)), block(256);
    route_topk_kernel<<<grid, block, 0, st>>>(logits, nb, n_expert, k, ids, w);
    return hipGetLastError();
}

}  // namespace eahmmf
