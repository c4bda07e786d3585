// kernels_fused.hip - one persistent launch per token for the whole MoE
// expert block: routing -> gate/up + SiLU -> down + router-weighted sum.
//
// This replaces, for one decode token, the reference's host loop
// (qwen3moe.cpp:1011-1067): softmax/top-k/renormalise, per expert a
// gate/up pair and a down matmul on the GPU with SiLU and the weighted
// scatter-add on the CPU, 16 synchronous round trips per layer.
//
// The grid is sized to what the device holds at once (occupancy x CUs), so
// every workgroup is resident and they may wait on each other:
//   1. wave 0 routes (expf(l - max), top-k with the lower id winning ties,
//      renormalise in rank order); waves 1-2 quantize x into 3 int8 levels
//      per 64-value segment (in LDS);
//   2. phase A: lane groups of min(64, D/64) lanes own one 64-value segment
//      of x each and walk (expert, row) tasks; each task loads the gate and
//      up row segments straight from HBM, takes exact int8 dots (v_dot4)
//      against the activation levels, reduces across the group and stores
//      h = silu(g) * u;
//   3. the down-projection row segments each thread will need are issued as
//      loads before waiting, so they stream from HBM during phase A;
//   4. h is written with device-coherent stores; a counter incremented once
//      per workgroup (after its stores completed) releases everyone when the
//      last workgroup finishes phase A;
//   5. phase B: threads own (expert, 64-value segment of FF) units, hold that
//      slice of h in registers (fp32), and produce w_j * down_j[r].h_j per
//      row; partials are summed in LDS in a fixed order (deterministic) and
//      y[r] is written once;
//   6. the last workgroup to finish resets the counters for the next launch.
// The wait is bounded: if it ever runs out, an error flag is raised and the
// kernel still exits.
#include <mutex>

#include "internal.h"
#include "kquant_seg64.h"

namespace eahmmf {

constexpr int kFusedThreads = 192;
constexpr int kMaxD = 4096;
constexpr int kMaxRowsB = 16;
constexpr int kPrefetchB = 2;
constexpr unsigned kSpinLimit = 1u << 22;

struct FusedArgs {
    MoeShape s;
    int k, n_expert, mode;  // mode 0: direct slots, 1: logits + table, 2: ids/w + table
    DecodeSlots direct;
    const ExpertEntry* table;
    const float* logits;
    const int* ids_in;
    const float* w_in;
    int* ids_out;
    float* w_out;
    const float* x;
    float* y;
    float* h;
    unsigned* sync;  // [0] phase-A done, [1] finished, [2] error flag
};

template <int CTRL, int ROWS>
__device__ __forceinline__ float dpp_fmax_step(float a, float fill) {
    return fmaxf(a, __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(__builtin_bit_cast(int, fill),
                                                                          __builtin_bit_cast(int, a), CTRL, ROWS, 0xF,
                                                                          false)));
}

template <int CTRL, int ROWS>
__device__ __forceinline__ int dpp_imin_step(int a, int fill) {
    return min(a, __builtin_amdgcn_update_dpp(fill, a, CTRL, ROWS, 0xF, false));
}

// wave64 reductions with DPP row operations; lane 63 collects the total,
// which is then broadcast.  Controls: 0xB1/0x4E quad permutes, 0x141
// row_half_mirror, 0x140 row_mirror, 0x142 row_bcast:15 (rows 1,3),
// 0x143 row_bcast:31 (rows 2,3).
__device__ __forceinline__ float dpp_max(float v) {
    v = dpp_fmax_step<0xB1, 0xF>(v, v);
    v = dpp_fmax_step<0x4E, 0xF>(v, v);
    v = dpp_fmax_step<0x141, 0xF>(v, -INFINITY);
    v = dpp_fmax_step<0x140, 0xF>(v, -INFINITY);
    v = dpp_fmax_step<0x142, 0xA>(v, -INFINITY);
    v = dpp_fmax_step<0x143, 0xC>(v, -INFINITY);
    return __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), 63));
}

__device__ __forceinline__ int dpp_min_int(int v) {
    v = dpp_imin_step<0xB1, 0xF>(v, v);
    v = dpp_imin_step<0x4E, 0xF>(v, v);
    v = dpp_imin_step<0x141, 0xF>(v, 0x7fffffff);
    v = dpp_imin_step<0x140, 0xF>(v, 0x7fffffff);
    v = dpp_imin_step<0x142, 0xA>(v, 0x7fffffff);
    v = dpp_imin_step<0x143, 0xC>(v, 0x7fffffff);
    return __builtin_amdgcn_readlane(v, 63);
}

// Device-coherent (sc1) store: written through past the XCD's L2, so no
// whole-cache writeback is needed before other XCDs may read it.
__device__ __forceinline__ void store_coherent(float* p, float v) {
    __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
// s_waitcnt vmcnt(0): this wave's stores have completed (gfx9 encoding:
// vmcnt 0, expcnt 7, lgkmcnt 15).  Compiler fences keep the stores before it.
__device__ __forceinline__ void wait_stores() {
    __atomic_signal_fence(__ATOMIC_SEQ_CST);
    __builtin_amdgcn_s_waitcnt(0x0F70);
    __atomic_signal_fence(__ATOMIC_SEQ_CST);
}

template <int W>
__device__ __forceinline__ float group_sum(float v) {
#pragma unroll
    for (int off = W / 2; off > 0; off >>= 1) v += __shfl_xor(v, off, 64);
    return v;
}

constexpr int kMaxH = 16384;  // k * FF floats held in LDS during phase B

struct alignas(16) FusedLds {
    union {
        struct {  // phase A: activation levels
            int8_t xq[kLevels][kMaxD];
            float xsc[kLevels][kMaxD / 64];
            float xs32[kMaxD / 32];
        } a;
        struct {  // phase B: h and the row partials
            float h[kMaxH];
            float part[kFusedThreads * kMaxRowsB];
        } b;
    };
    const uint8_t* gate[kMaxSlots];
    const uint8_t* up[kMaxSlots];
    const uint8_t* down[kMaxSlots];
    float w[kMaxSlots];
};

// Route one token with wave 0 (n_expert <= 256).  Results into LDS.
__device__ void route_wave(const FusedArgs& a, FusedLds& L) {
    const int lane = threadIdx.x;
    float e[4];
    float mx = -INFINITY;
#pragma unroll
    for (int i = 0; i < 4; i++) {
        const int id = lane + 64 * i;
        e[i] = id < a.n_expert ? a.logits[id] : -INFINITY;
        mx = fmaxf(mx, e[i]);
    }
    mx = dpp_max(mx);
#pragma unroll
    for (int i = 0; i < 4; i++) {
        const int id = lane + 64 * i;
        e[i] = id < a.n_expert ? expf(e[i] - mx) : -1.0f;
    }
    float tot = 0.f;
    float mine = 0.f;  // lane r keeps the r-th chosen e
    for (int r = 0; r < a.k; r++) {
        float be = -2.0f;
        int bi = 0x7fffffff;
#pragma unroll
        for (int i = 0; i < 4; i++)
            if (e[i] > be) { be = e[i]; bi = lane + 64 * i; }  // ascending ids: ties keep the lower
        const float m = dpp_max(be);
        const int id = dpp_min_int(be == m ? bi : 0x7fffffff);
#pragma unroll
        for (int i = 0; i < 4; i++)
            if (lane + 64 * i == id) e[i] = -1.0f;
        if (lane == r) mine = m;
        tot += m;  // rank order, as the reference sums
        if (lane == 0) {
            // NaN logits can leave no candidate: that slot then contributes nothing
            const bool valid = id >= 0 && id < a.n_expert;
            const ExpertEntry ent = valid ? a.table[id] : ExpertEntry{nullptr, nullptr, nullptr};
            L.gate[r] = ent.gate;
            L.up[r] = ent.up;
            L.down[r] = ent.down;
            if (a.ids_out && blockIdx.x == 0) a.ids_out[r] = valid ? id : -1;
        }
    }
    if (lane < a.k) {
        const float wr = mine / tot;
        L.w[lane] = wr;
        if (a.w_out && blockIdx.x == 0) a.w_out[lane] = wr;
    }
}

// x (fp32, D) -> 3 int8 levels per 64-value segment + 32-value sums, into LDS.
// Eight threads per segment, eight values each; threads [t0, t0+nthr).
__device__ void quantize_x(const FusedArgs& a, FusedLds& L, int t, int nthr) {
    const int D = a.s.D;
    const int nseg = D / 64;
    const int per_pass = nthr / 8;
    for (int base = 0; base < nseg; base += per_pass) {
        const int seg = base + t / 8;
        const int part = t % 8;
        const bool active = seg < nseg && t < per_pass * 8;
        float v[8];
        float amax = 0.f, sum = 0.f;
        if (active) {
            const float4* p = reinterpret_cast<const float4*>(a.x + seg * 64 + part * 8);
            const float4 v0 = p[0], v1 = p[1];
            v[0] = v0.x; v[1] = v0.y; v[2] = v0.z; v[3] = v0.w;
            v[4] = v1.x; v[5] = v1.y; v[6] = v1.z; v[7] = v1.w;
#pragma unroll
            for (int i = 0; i < 8; i++) {
                amax = fmaxf(amax, fabsf(v[i]));
                sum += v[i];
            }
        } else {
#pragma unroll
            for (int i = 0; i < 8; i++) v[i] = 0.f;
        }
        // the 8 threads of a segment are adjacent lanes
        amax = fmaxf(amax, __shfl_xor(amax, 1, 64));
        amax = fmaxf(amax, __shfl_xor(amax, 2, 64));
        amax = fmaxf(amax, __shfl_xor(amax, 4, 64));
        sum += __shfl_xor(sum, 1, 64);
        sum += __shfl_xor(sum, 2, 64);  // four threads = 32 values
        if (active) {
            const float s1 = amax / 127.0f;
            const float s2 = s1 / 254.0f, s3 = s2 / 254.0f;
            const float sc[kLevels] = {s1, s2, s3};
            float r[8];
#pragma unroll
            for (int i = 0; i < 8; i++) r[i] = v[i];
#pragma unroll
            for (int lv = 0; lv < kLevels; lv++) {
                const float inv = sc[lv] > 0.f ? 1.0f / sc[lv] : 0.f;
                uint32_t packed[2] = {0u, 0u};
#pragma unroll
                for (int i = 0; i < 8; i++) {
                    float qf = __builtin_rintf(r[i] * inv);
                    qf = fminf(127.f, fmaxf(-127.f, qf));
                    r[i] = __builtin_fmaf(-qf, sc[lv], r[i]);
                    packed[i >> 2] |= ((uint32_t)(int)qf & 0xFFu) << (8 * (i & 3));
                }
                *reinterpret_cast<uint2*>(&L.a.xq[lv][seg * 64 + part * 8]) = make_uint2(packed[0], packed[1]);
                if (part == 0) L.a.xsc[lv][seg] = sc[lv];
            }
            if ((part & 3) == 0) L.a.xs32[seg * 2 + part / 4] = sum;
        }
    }
}

template <int LA, int GT, int UT, int DT>
__device__ void fused_body(const FusedArgs& a, FusedLds& L) {
    const int tid = threadIdx.x;
    const MoeShape& s = a.s;
    const int D = s.D, FF = s.FF, k = a.k;
    const int nwg = gridDim.x;

    // ---- 1. routing / slots and activation levels
    if (a.mode == 1) {
        if (tid < 64) route_wave(a, L);
        else quantize_x(a, L, tid - 64, kFusedThreads - 64);
    } else {
        if (tid < k) {
            if (a.mode == 0) {
                L.gate[tid] = a.direct.gate[tid];
                L.up[tid] = a.direct.up[tid];
                L.down[tid] = a.direct.down[tid];
                L.w[tid] = a.direct.w[tid];
            } else {
                const int id = a.ids_in[tid];
                const bool ok = id >= 0 && id < a.n_expert;
                const ExpertEntry ent = ok ? a.table[id] : ExpertEntry{nullptr, nullptr, nullptr};
                L.gate[tid] = ent.gate;
                L.up[tid] = ent.up;
                L.down[tid] = ent.down;
                L.w[tid] = ok ? a.w_in[tid] : 0.f;
            }
        }
        quantize_x(a, L, tid, kFusedThreads);
    }
    __syncthreads();

    // ---- phase-B assignment and prefetch of the down rows (independent of h)
    const int segB = FF / 64;
    const int U = k * segB;
    const int S = kFusedThreads / U;  // row slots per workgroup
    const bool b_active = tid < S * U;
    const int slot = tid / U, unit = tid % U;
    const int bj = unit / segB, bseg = unit % segB;
    const int NS = nwg * S;
    const int gslot = blockIdx.x * S + slot;
    const int RB = (D + NS - 1) / NS;
    const uint8_t* bdown = b_active ? L.down[bj] : nullptr;
    RawSeg<DT> pre[kPrefetchB];
#pragma unroll
    for (int i = 0; i < kPrefetchB; i++) {
        const int r = gslot + i * NS;
        if (b_active && bdown && i < RB && r < D) pre[i].load(bdown + (size_t)r * s.down_rb, bseg);
    }

    // ---- 2. phase A
    constexpr int GA = kFusedThreads / LA;
    const int grp = tid / LA, li = tid % LA;
    XSeg xs;
#pragma unroll
    for (int lv = 0; lv < kLevels; lv++) {
        const uint4* p = reinterpret_cast<const uint4*>(&L.a.xq[lv][li * 64]);
#pragma unroll
        for (int q = 0; q < 4; q++) {
            const uint4 v = p[q];
            xs.q[lv][4 * q] = (int)v.x; xs.q[lv][4 * q + 1] = (int)v.y;
            xs.q[lv][4 * q + 2] = (int)v.z; xs.q[lv][4 * q + 3] = (int)v.w;
        }
        xs.s[lv] = L.a.xsc[lv][li];
    }
    xs.sum32[0] = L.a.xs32[2 * li];
    xs.sum32[1] = L.a.xs32[2 * li + 1];
    const int P = k * FF;
    const int NG = nwg * GA;
    for (int t0 = blockIdx.x * GA + grp; t0 < P; t0 += 2 * NG) {
        const int t1 = t0 + NG;
        const bool has1 = t1 < P;
        RawSeg<GT> g0, g1;
        RawSeg<UT> u0, u1;
        const int j0 = t0 / FF, f0 = t0 % FF;
        const int j1 = has1 ? t1 / FF : j0, f1 = has1 ? t1 % FF : f0;
        const bool ok0 = L.gate[j0] && L.up[j0];
        const bool ok1 = has1 && L.gate[j1] && L.up[j1];
        if (ok0) {
            g0.load(L.gate[j0] + (size_t)f0 * s.gate_rb, li);
            u0.load(L.up[j0] + (size_t)f0 * s.up_rb, li);
        }
        if (ok1) {
            g1.load(L.gate[j1] + (size_t)f1 * s.gate_rb, li);
            u1.load(L.up[j1] + (size_t)f1 * s.up_rb, li);
        }
        float dg0 = ok0 ? g0.dot_q8(li, xs) : 0.f;
        float du0 = ok0 ? u0.dot_q8(li, xs) : 0.f;
        float dg1 = ok1 ? g1.dot_q8(li, xs) : 0.f;
        float du1 = ok1 ? u1.dot_q8(li, xs) : 0.f;
        dg0 = group_sum<LA>(dg0);
        du0 = group_sum<LA>(du0);
        dg1 = group_sum<LA>(dg1);
        du1 = group_sum<LA>(du1);
        if (li == 0) {
            store_coherent(&a.h[t0], dg0 / (1.0f + expf(-dg0)) * du0);
            if (has1) store_coherent(&a.h[t1], dg1 / (1.0f + expf(-dg1)) * du1);
        }
    }

    // ---- 4. grid-wide hand-off from phase A to phase B.  h went out with
    // device-coherent stores; each wave waits for its stores to complete,
    // then one counter increment per workgroup; polling uses device-coherent
    // loads (no cache maintenance inside the loop).
    wait_stores();
    __syncthreads();
    if (tid == 0) {
        __hip_atomic_fetch_add(&a.sync[0], 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        unsigned spins = 0;
        while (__hip_atomic_load(&a.sync[0], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) < (unsigned)nwg) {
            __builtin_amdgcn_s_sleep(4);
            if (++spins == kSpinLimit) {
                __hip_atomic_store(&a.sync[2], 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                break;
            }
        }
    }
    // one L2/L1 invalidate per workgroup, then h is read with ordinary cached
    // loads: the first workgroup of each XCD brings it into that XCD's L2
    if (tid == 0) __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "agent");
    __syncthreads();
    {
        const int nh4 = k * FF / 4;
        const float4* src = reinterpret_cast<const float4*>(a.h);
        float4* dst = reinterpret_cast<float4*>(L.b.h);
        for (int i = tid; i < nh4; i += kFusedThreads) dst[i] = src[i];
    }
    __syncthreads();

    // ---- 5. phase B
    if (b_active) {
        float hv[64];
        const float4* hp = reinterpret_cast<const float4*>(&L.b.h[bj * FF + bseg * 64]);
#pragma unroll
        for (int q = 0; q < 16; q++) {
            const float4 v = hp[q];
            hv[4 * q] = v.x; hv[4 * q + 1] = v.y; hv[4 * q + 2] = v.z; hv[4 * q + 3] = v.w;
        }
        constexpr int NSUM = SumSpan<DT>::n > 0 ? SumSpan<DT>::n : 1;
        float hsum[NSUM];
#pragma unroll
        for (int g = 0; g < NSUM; g++) {
            float acc = 0.f;
            if (SumSpan<DT>::n > 0) {
#pragma unroll
                for (int i = 0; i < SumSpan<DT>::width; i++) acc += hv[g * SumSpan<DT>::width + i];
            }
            hsum[g] = acc;
        }
        const float wj = L.w[bj];
        for (int i = 0; i < RB && i < kMaxRowsB; i++) {
            const int r = gslot + i * NS;
            float part = 0.f;
            if (r < D && bdown) {
                RawSeg<DT> raw;
                if (i < kPrefetchB) raw = pre[i];
                else raw.load(bdown + (size_t)r * s.down_rb, bseg);
                part = wj * raw.dot_f32(bseg, hv, hsum);
            }
            L.b.part[(slot * kMaxRowsB + i) * U + unit] = part;
        }
    }
    __syncthreads();
    // reduce partials: wave w takes (slot, row) pairs w, w+3, ...
    {
        const int wave = tid / 64, lane = tid % 64;
        const int pairs = S * min(RB, kMaxRowsB);
        for (int pi = wave; pi < pairs; pi += kFusedThreads / 64) {
            const int sl = pi / min(RB, kMaxRowsB), i = pi % min(RB, kMaxRowsB);
            const int r = blockIdx.x * S + sl + i * NS;
            const float* pp = &L.b.part[(sl * kMaxRowsB + i) * U];
            float v = 0.f;
            for (int u = lane; u < U; u += 64) v += pp[u];
            v = group_sum<64>(v);
            if (lane == 0 && r < D) a.y[r] = v;
        }
    }

    // ---- 6. the last workgroup out resets the counters for the next launch
    __syncthreads();
    if (tid == 0) {
        const unsigned done = __hip_atomic_fetch_add(&a.sync[1], 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        if (done == (unsigned)nwg - 1) {
            __hip_atomic_store(&a.sync[0], 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            __hip_atomic_store(&a.sync[1], 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        }
    }
}

template <int LA, int GT, int UT, int DT>
__global__ __launch_bounds__(kFusedThreads) void moe_decode_fused(FusedArgs a) {
    __shared__ FusedLds L;
    fused_body<LA, GT, UT, DT>(a, L);
}

// ---------------------------------------------------------------------------
// host side

using FusedFn = void (*)(FusedArgs);

template <int LA, int GT, int UT>
static FusedFn pick_down(int dt) {
    switch (dt) {
        case kQ4_K: return moe_decode_fused<LA, GT, UT, kQ4_K>;
        case kQ5_K: return moe_decode_fused<LA, GT, UT, kQ5_K>;
        case kQ6_K: return moe_decode_fused<LA, GT, UT, kQ6_K>;
        case kQ8_0: return moe_decode_fused<LA, GT, UT, kQ8_0>;
        default: return nullptr;
    }
}

template <int LA, int GT>
static FusedFn pick_up(int ut, int dt) {
    if (ut != GT) return nullptr;  // gate and up of one GGUF layer share a type in every supported config
    return pick_down<LA, GT, GT>(dt);
}

template <int LA>
static FusedFn pick_gate(int gt, int ut, int dt) {
    switch (gt) {
        case kQ4_K: return pick_up<LA, kQ4_K>(ut, dt);
        case kQ5_K: return pick_up<LA, kQ5_K>(ut, dt);
        case kQ6_K: return pick_up<LA, kQ6_K>(ut, dt);
        case kQ8_0: return pick_up<LA, kQ8_0>(ut, dt);
        default: return nullptr;
    }
}

static FusedFn pick_fused(const MoeShape& s) {
    switch (s.D / 64) {
        case 4: return pick_gate<4>(s.gate_type, s.up_type, s.down_type);
        case 8: return pick_gate<8>(s.gate_type, s.up_type, s.down_type);
        case 16: return pick_gate<16>(s.gate_type, s.up_type, s.down_type);
        case 32: return pick_gate<32>(s.gate_type, s.up_type, s.down_type);
        case 64: return pick_gate<64>(s.gate_type, s.up_type, s.down_type);
        default: return nullptr;
    }
}

bool fused_supported(const MoeShape& s, int k, int n_expert_for_routing) {
    if (!moe_shape_ok(s) || k <= 0 || k > kMaxSlots) return false;
    if (s.D % 64 || s.FF % 64 || s.D > kMaxD) return false;
    if (!pick_fused(s)) return false;
    const int U = k * (s.FF / 64);
    if (U > kFusedThreads || k * s.FF > kMaxH) return false;
    if (n_expert_for_routing > 256) return false;
    return true;
}

// Grid size: every workgroup must be resident at once.  The
// occupancy answer is cached per kernel and device.
static int fused_grid(FusedFn fn, int device) {
    struct Entry { FusedFn fn; int device, grid; };
    static Entry cache[64];
    static int n = 0;
    static std::mutex mu;
    std::lock_guard<std::mutex> g(mu);
    for (int i = 0; i < n; i++)
        if (cache[i].fn == fn && cache[i].device == device) return cache[i].grid;
    int cus = 0, occ = 0;
    if (hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, device) != hipSuccess) return 0;
    if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&occ, reinterpret_cast<const void*>(fn), kFusedThreads, 0) !=
        hipSuccess)
        return 0;
    const int grid = (occ < 2 ? occ : 2) * cus;
    if (n < 64) cache[n++] = Entry{fn, device, grid};
    return grid;
}

hipError_t launch_moe_fused(const FusedArgsHost& h, hipStream_t st) {
    FusedArgs a{};
    a.s = h.shape;
    a.k = h.k;
    a.n_expert = h.n_expert;
    a.mode = h.mode;
    a.direct = h.direct;
    a.table = h.table;
    a.logits = h.logits;
    a.ids_in = h.ids_in;
    a.w_in = h.w_in;
    a.ids_out = h.ids_out;
    a.w_out = h.w_out;
    a.x = h.x;
    a.y = h.y;
    a.h = h.h;
    a.sync = h.sync;
    if (!fused_supported(a.s, a.k, a.mode == 1 ? a.n_expert : 0)) return hipErrorInvalidValue;
    FusedFn fn = pick_fused(a.s);
    int dev = 0;
    hipError_t e = hipGetDevice(&dev);
    if (e != hipSuccess) return e;
    const int grid = fused_grid(fn, dev);
    if (grid <= 0) return hipErrorInvalidConfiguration;
    // the phase-B partial buffer holds kMaxRowsB rows per slot
    const int S = kFusedThreads / (a.k * (a.s.FF / 64));
    if ((a.s.D + grid * S - 1) / (grid * S) > kMaxRowsB) return hipErrorInvalidValue;
    clear_stale_error();
    // A plain launch: the grid never exceeds what is resident at once, and the
    // stream runs nothing else concurrently, so every workgroup is live.
    hipLaunchKernelGGL(fn, dim3(grid), dim3(kFusedThreads), 0, st, a);
    return hipGetLastError();
}

}  // namespace eahmmf
