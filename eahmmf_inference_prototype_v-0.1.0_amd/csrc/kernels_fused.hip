// kernels_fused.hip - one launch per token for the whole MoE expert block:
// routing -> gate/up + SiLU -> down -> router-weighted sum.
//
// This replaces, for one decode token, the reference's host loop
// (qwen3moe.cpp:1011-1067): softmax/top-k/renormalise, per expert a gate/up
// pair and a down matmul on the GPU, SiLU and the weighted scatter-add on the
// CPU, 16 synchronous round trips per layer.
//
// Layout of the work.  The routed experts are split into NP partitions (one
// expert each for k <= 8, k/8 each for k = 16); workgroup b is rank q = b / NP
// inside its partition.  With NP = 8 the partition is the XCD the workgroup
// runs on (hardware XCC id): the dispatcher hands consecutive workgroups to
// the eight XCDs in turn, starting wherever the previous launch stopped, so
// workgroups b, b+8, b+16, ... share one XCD (checked once per device) and a
// partition's slice of h is exchanged through that XCD's L2.  Otherwise
// workgroup b belongs to partition b % NP and h travels with device-coherent
// stores and loads.
// Per workgroup (256 threads):
//   1. wave 0 routes: logits and the expert table are read once, e_i =
//      expf(l_i - max), top-k by DPP max/min reductions (the lower id wins
//      ties), renormalised in rank order.  Waves 1-3 turn x into three int8
//      levels per 64-value segment in LDS.
//   2. wave 3 copies the down-projection rows this workgroup will need
//      straight from HBM into LDS (global_load_lds, asynchronous), so they
//      stream during phase A.
//   3. phase A on waves 0-2: lane groups of D/64 lanes each own one 64-value
//      segment of x and walk this workgroup's (expert, row) pairs; gate and up
//      row segments are loaded straight from HBM into registers, dotted
//      exactly in int32 (v_dot4) against the activation levels, reduced in
//      the group, and h = silu(g) * u is stored.
//   4. partition barrier.  XCD-local: each workgroup stores the launch epoch
//      in its own flag word and wave 0 polls the partition's m flags with
//      agent-scope loads (which miss the CU's L1).  Otherwise one atomic
//      counter per partition.
//   5. phase B: the partition's h is read into LDS; threads own (expert,
//      64-value segment of FF) units, compute w_j * down_j[r].h_j for the
//      staged rows in fp32, and sum the units of each row in a fixed order
//      into this partition's partial ypart[p][r].
//   6. per row chunk, one workgroup adds the NP partials in partition order
//      (deterministic) and writes y: partition q % NP once all NP epoch flags
//      of the chunk are set (XCD-local), else the last partition to arrive.
// Counters are reset by the last workgroup through each stage, so every
// launch starts from zero; epoch flags need no reset.  Every wait is bounded; if a bound is ever hit an
// error flag is raised and the kernel still exits.
#include <mutex>

#include "internal.h"
#include "kquant_seg64.h"

namespace eahmmf {

constexpr int kThreads = 256;
constexpr int kAThreads = 192;  // waves 0-2 run phase A
constexpr int kMaxD = 4096;
constexpr int kMaxE = 256;
constexpr int kStageB = 32 * 1024;  // LDS bytes for staged down rows
constexpr int kMaxHP = 4096;        // floats of h held per partition
constexpr int kMaxPart = 1024;      // (row, unit) partials per round
constexpr unsigned kSpinLimit = 1u << 22;

// sync buffer layout (unsigned words, kSyncWords in all).  Atomic counters
// serve the device-coherent protocol; epoch flags serve the XCD-local one.
constexpr int kSyncArrive = 0, kSyncPass = 8, kSyncChunk = 16, kSyncErr = kSyncFlagWord;
constexpr int kMaxChunks = 512;
constexpr int kMaxM = 128;                             // workgroups per partition (epoch flags, 2 per lane)
constexpr int kFlagArrive = 1024, kFlagChunk = 2048;  // [8][kMaxM] each
static_assert(kSyncChunk + kMaxChunks <= kSyncErr && kFlagChunk + 8 * kMaxM <= kSyncWords, "sync layout");

struct FusedArgs {
    MoeShape s;
    int k, n_expert, mode;  // mode 0: direct slots, 1: logits + table, 2: ids/w + table
    int np, m;              // partitions and workgroups per partition
    int rows_b;             // output rows per workgroup (chunk)
    int round_b;            // rows staged per phase-B round
    int local_l2;           // 1: partition p runs on XCD p, so h is exchanged through that XCD's L2
    unsigned epoch;         // launch number (>= 1): the value this launch's flags carry
    DecodeSlots direct;
    const ExpertEntry* table;
    const float* logits;
    const int* ids_in;
    const float* w_in;
    int* ids_out;
    float* w_out;
    const float* x;
    float* y;
    float* h;      // k * FF
    float* ypart;  // np * D
    unsigned* sync;
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

// Device-coherent (sc1) accesses: visible across the XCDs' separate L2s
// without whole-cache writeback or invalidate.
__device__ __forceinline__ void store_coherent(float* p, float v) {
    __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ float load_coherent(const float* p) {
    return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ unsigned load_counter(const unsigned* p) {
    return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ unsigned bump_counter(unsigned* p) {
    return __hip_atomic_fetch_add(p, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ void reset_counter(unsigned* p) {
    __hip_atomic_store(p, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// Current value of a counter read with an atomic read-modify-write: it is
// served where the increments are performed, never from a stale cached copy.
__device__ __forceinline__ unsigned poll_counter(unsigned* p) {
    return __hip_atomic_fetch_add(p, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// Poll of a flag another CU of the same XCD stores with a plain store.  The
// load must miss the CU's L1: an sc0 (workgroup-scope) load, even after
// "buffer_inv sc0", is served by a stale L1 line until that line is evicted
// (measured: never within 20 ms on an idle CU), while an agent-scope (sc1)
// load sees the completed store within ~0.2 us.
__device__ __forceinline__ unsigned load_flag(const unsigned* p) {
    return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// XCD (XCC) the calling wave runs on: hardware register HW_REG_XCC_ID (20),
// bits [3:0].
__device__ __forceinline__ int xcc_id() { return (int)(__builtin_amdgcn_s_getreg(20 | (0 << 6) | (3 << 11)) & 0xF); }

template <int W>
__device__ __forceinline__ float group_sum(float v) {
#pragma unroll
    for (int off = W / 2; off > 0; off >>= 1) v += __shfl_xor(v, off, 64);
    return v;
}

struct alignas(16) FusedLds {
    uint8_t bstage[kStageB];  // first member: 16-byte aligned
    union {
        struct {  // steps 1-3: activation levels
            int8_t xq[kLevels][kMaxD];
            float xsc[kLevels][kMaxD / 64];
            float xs32[kMaxD / 32];
        } a;
        struct {  // step 5: the partition's h as int8 levels, and (row, unit) partials
            int8_t hq[kLevels][kMaxHP];
            float hsc[kLevels][kMaxHP / 64];
            float hs32[kMaxHP / 32];
            float part[kMaxPart];
        } b;
    };
    ExpertEntry table[kMaxE];
    const uint8_t* gate[kMaxSlots];
    const uint8_t* up[kMaxSlots];
    const uint8_t* down[kMaxSlots];
    float w[kMaxSlots];
    int flag;
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
        if (id < a.n_expert) L.table[id] = a.table[id];
        mx = fmaxf(mx, e[i]);
    }
    mx = dpp_max(mx);
#pragma unroll
    for (int i = 0; i < 4; i++) {
        const int id = lane + 64 * i;
        e[i] = id < a.n_expert ? expf(e[i] - mx) : -1.0f;
    }
    float tot = 0.f, mine = 0.f;  // lane r keeps the r-th chosen e and id
    int myid = -1;
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
        if (lane == r) {
            mine = m;
            myid = id;
        }
        tot += m;  // rank order, as the reference sums
    }
    if (lane < a.k) {
        // NaN logits can leave a slot without a candidate: it then contributes nothing
        const bool valid = myid >= 0 && myid < a.n_expert;
        const ExpertEntry ent = valid ? L.table[myid] : ExpertEntry{nullptr, nullptr, nullptr};
        L.gate[lane] = ent.gate;
        L.up[lane] = ent.up;
        L.down[lane] = ent.down;
        const float wr = valid ? mine / tot : 0.f;
        L.w[lane] = wr;
        if (blockIdx.x == 0) {
            if (a.ids_out) a.ids_out[lane] = valid ? myid : -1;
            if (a.w_out) a.w_out[lane] = wr;
        }
    }
}

// Activation levels.  n fp32 values (n % 64 == 0) become 3 int8 levels per
// 64-value segment plus 32-value sums, in LDS: level lv of value i at
// q + lv*qstride + i, scale of segment g at sc + lv*scstride + g, sum of
// values [32c, 32c+32) at s32[c].  Eight adjacent threads share a segment,
// eight values each.

// This thread's eight values of segment seg (zeros when inactive).
template <bool COHERENT>
__device__ __forceinline__ void load8(const float* src, int seg, int part, bool active, float (&v)[8]) {
    if (active) {
        const float* sp = src + seg * 64 + part * 8;
        if (COHERENT) {
#pragma unroll
            for (int i = 0; i < 8; i++) v[i] = __hip_atomic_load(sp + i, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        } else {
            const float4 v0 = reinterpret_cast<const float4*>(sp)[0], v1 = reinterpret_cast<const float4*>(sp)[1];
            v[0] = v0.x; v[1] = v0.y; v[2] = v0.z; v[3] = v0.w;
            v[4] = v1.x; v[5] = v1.y; v[6] = v1.z; v[7] = v1.w;
        }
    } else {
#pragma unroll
        for (int i = 0; i < 8; i++) v[i] = 0.f;
    }
}

// Levels of the eight values v of segment seg; every lane of the wave calls it
// (the segment's amax and sums are exchanged by shuffles).
__device__ __forceinline__ void quantize8(const float (&v)[8], int seg, int part, bool active, int8_t* q, int qstride,
                                          float* sc, int scstride, float* s32) {
    float amax = 0.f, sum = 0.f;
#pragma unroll
    for (int i = 0; i < 8; i++) {
        amax = fmaxf(amax, fabsf(v[i]));
        sum += v[i];
    }
    amax = fmaxf(amax, __shfl_xor(amax, 1, 64));
    amax = fmaxf(amax, __shfl_xor(amax, 2, 64));
    amax = fmaxf(amax, __shfl_xor(amax, 4, 64));
    sum += __shfl_xor(sum, 1, 64);
    sum += __shfl_xor(sum, 2, 64);  // four threads = 32 values
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

// All n values by threads t in [0, nthr) (nthr a multiple of 64).
template <bool COHERENT>
__device__ void quantize_levels(const float* src, int n, int8_t* q, int qstride, float* sc, int scstride, float* s32,
                                int t, int nthr) {
    const int nseg = n / 64;
    for (int base = 0; base < nseg; base += nthr / 8) {
        const int seg = base + t / 8, part = t % 8;
        float v[8];
        load8<COHERENT>(src, seg, part, seg < nseg, v);
        quantize8(v, seg, part, seg < nseg, q, qstride, sc, scstride, s32);
    }
}

// The activation levels of segment g (64 values) held by one lane.
__device__ __forceinline__ void load_xseg(XSeg& xs, const int8_t* q, int qstride, const float* sc, int scstride,
                                          const float* s32, int g) {
#pragma unroll
    for (int lv = 0; lv < kLevels; lv++) {
        const uint4* xp = reinterpret_cast<const uint4*>(q + lv * qstride + g * 64);
#pragma unroll
        for (int c = 0; c < 4; c++) {
            const uint4 v = xp[c];
            xs.q[lv][4 * c] = (int)v.x; xs.q[lv][4 * c + 1] = (int)v.y;
            xs.q[lv][4 * c + 2] = (int)v.z; xs.q[lv][4 * c + 3] = (int)v.w;
        }
        xs.s[lv] = sc[lv * scstride + g];
    }
    xs.sum32[0] = s32[2 * g];
    xs.sum32[1] = s32[2 * g + 1];
}

// Copy global bytes [src, src_end) into LDS at dst, one wave, 16 bytes per
// lane per instruction.  The copy covers src rounded down to 16 bytes up to
// src_end rounded up, so every access is an aligned 16-byte block inside the
// pages that hold the range.  src's offset inside the copy is src & 15.
__device__ __forceinline__ void stage_range(const uint8_t* src, const uint8_t* src_end, uint8_t* dst, int lane) {
    const uintptr_t a = (uintptr_t)src & ~(uintptr_t)15;
    const uintptr_t z = ((uintptr_t)src_end + 15) & ~(uintptr_t)15;
    const int n16 = (int)((z - a) / 16);
    for (int base = 0; base < n16; base += 64) {
        // the LDS slot of lane i is dst + base*16 + 16*i; lanes past the end stay idle
        if (base + lane < n16)
            __builtin_amdgcn_global_load_lds(reinterpret_cast<const void*>(a + (uintptr_t)(base + lane) * 16),
                                             (__attribute__((address_space(3))) void*)(dst + base * 16), 16, 0, 0);
    }
}

// LDS bytes reserved per expert for one staged round of rows (16-byte
// rounding slack at both ends).
__host__ __device__ inline int stage_stride(int rows, int row_bytes) { return ((rows * row_bytes + 15) / 16 + 1) * 16; }

template <int LA, int GT, int UT, int DT>
__device__ void fused_body(const FusedArgs& a, FusedLds& L) {
    const int tid = threadIdx.x;
    const int wave = tid / 64, lane = tid % 64;
    const MoeShape& s = a.s;
    const int D = s.D, FF = s.FF, k = a.k;
    const int np = a.np, m = a.m;
    const int xcc = a.local_l2 ? xcc_id() : 0;
    const bool xcc_bad = xcc >= np;  // never on a device that passed the host's placement check
    const int p = a.local_l2 ? (xcc_bad ? 0 : xcc) : (int)blockIdx.x % np, q = blockIdx.x / np;
    const int ep = k / np;  // experts per partition
    const int segB = FF / 64;
    const int UP = ep * segB;  // units of the partition
    const int drb = (int)s.down_rb;

    // ---- 1. routing / slots (wave 0) and activation levels (waves 1-3)
    if (wave == 0) {
        if (a.mode == 1) {
            route_wave(a, L);
        } else if (lane < k) {
            if (a.mode == 0) {
                L.gate[lane] = a.direct.gate[lane];
                L.up[lane] = a.direct.up[lane];
                L.down[lane] = a.direct.down[lane];
                L.w[lane] = a.direct.w[lane];
            } else {
                const int id = a.ids_in[lane];
                const bool ok = id >= 0 && id < a.n_expert;
                const ExpertEntry ent = ok ? a.table[id] : ExpertEntry{nullptr, nullptr, nullptr};
                L.gate[lane] = ent.gate;
                L.up[lane] = ent.up;
                L.down[lane] = ent.down;
                L.w[lane] = ok ? a.w_in[lane] : 0.f;
            }
        }
    } else {
        quantize_levels<false>(a.x, D, &L.a.xq[0][0], kMaxD, &L.a.xsc[0][0], kMaxD / 64, L.a.xs32, tid - 64,
                               kThreads - 64);
    }
    __syncthreads();

    // output rows of this workgroup's chunk, staged in rounds of round_b rows
    const int r_begin = q * a.rows_b;
    const int r_end = min(D, r_begin + a.rows_b);
    const int round_rows = a.round_b;
    const int stride_e = stage_stride(round_rows, drb);
    auto issue_stage = [&](int r0) {  // wave 3 only
        const int r1 = min(r_end, r0 + round_rows);
        for (int e = 0; e < ep; e++) {
            const uint8_t* dw = L.down[p * ep + e];
            if (dw && r1 > r0)
                stage_range(dw + (size_t)r0 * drb, dw + (size_t)r1 * drb, L.bstage + e * stride_e, lane);
        }
    };

    // ---- 2. wave 3 stages the first round of down rows into LDS
    if (wave == 3) issue_stage(r_begin);

    // ---- 3. phase A on waves 0-2
    if (wave < 3) {
        constexpr int GA = kAThreads / LA;
        const int grp = tid / LA, li = tid % LA;
        XSeg xs;
        load_xseg(xs, &L.a.xq[0][0], kMaxD, &L.a.xsc[0][0], kMaxD / 64, L.a.xs32, li);
        // this workgroup's rows of the partition: [ra0, ra1) over ep * FF
        const int rows_a = ep * FF;
        const int per_wg = (rows_a + m - 1) / m;
        const int ra0 = q * per_wg, ra1 = min(rows_a, ra0 + per_wg);
        for (int t0 = ra0 + grp; t0 < ra1; t0 += 2 * GA) {
            const int t1 = t0 + GA;
            const bool has1 = t1 < ra1;
            const int j0 = p * ep + t0 / FF, f0 = t0 % FF;
            const int j1 = has1 ? p * ep + t1 / FF : j0, f1 = has1 ? t1 % FF : f0;
            const bool ok0 = L.gate[j0] && L.up[j0];
            const bool ok1 = has1 && L.gate[j1] && L.up[j1];
            RawSeg<GT> g0, g1;
            RawSeg<UT> u0, u1;
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
                const float h0 = dg0 / (1.0f + expf(-dg0)) * du0;
                const float h1 = dg1 / (1.0f + expf(-dg1)) * du1;
                if (a.local_l2) {  // the partition's readers share this XCD's L2
                    a.h[j0 * FF + f0] = h0;
                    if (has1) a.h[j1 * FF + f1] = h1;
                } else {
                    store_coherent(&a.h[j0 * FF + f0], h0);
                    if (has1) store_coherent(&a.h[j1 * FF + f1], h1);
                }
            }
        }
    }

    // ---- 4. partition barrier (h complete for partition p)
    wait_vm();  // h stores of waves 0-2 and the staging copies of wave 3 have completed
    __syncthreads();
    if (a.local_l2) {
        // every workgroup of the partition publishes the launch epoch in its own
        // flag word (a plain store into this XCD's L2); wave 0 watches all m flags
        if (tid == 0) {
            if (xcc_bad)  // the XCD-to-partition mapping this exchange relies on does not hold
                __hip_atomic_store(&a.sync[kSyncErr], 2u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            a.sync[kFlagArrive + p * kMaxM + q] = a.epoch;
        }
        if (wave == 0) {
            unsigned spins = 0;
            for (;;) {
                const unsigned* fl = &a.sync[kFlagArrive + p * kMaxM];
                const bool mine = (lane >= m || load_flag(fl + lane) == a.epoch) &&
                                  (lane + 64 >= m || load_flag(fl + lane + 64) == a.epoch);
                if (__all(mine)) break;
                __builtin_amdgcn_s_sleep(1);
                if (++spins == kSpinLimit) {
                    if (lane == 0) __hip_atomic_store(&a.sync[kSyncErr], 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                    break;
                }
            }
        }
    } else if (tid == 0) {
        bump_counter(&a.sync[kSyncArrive + p]);
        unsigned spins = 0;
        while (poll_counter(&a.sync[kSyncArrive + p]) < (unsigned)m) {
            __builtin_amdgcn_s_sleep(2);
            if (++spins == kSpinLimit) {
                __hip_atomic_store(&a.sync[kSyncErr], 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                break;
            }
        }
        if (bump_counter(&a.sync[kSyncPass + p]) == (unsigned)m - 1) {  // everyone has passed: reset
            reset_counter(&a.sync[kSyncArrive + p]);
            reset_counter(&a.sync[kSyncPass + p]);
        }
    }
    __syncthreads();  // the activation levels are dead from here: the LDS union switches to phase B

    // ---- 5. phase B: the partition's h as int8 levels (read from L2 when the
    // partition shares an XCD, with device-coherent loads otherwise)
    const int hn = ep * FF;
    if (a.local_l2)
        quantize_levels<false>(a.h + p * ep * FF, hn, &L.b.hq[0][0], kMaxHP, &L.b.hsc[0][0], kMaxHP / 64, L.b.hs32,
                               tid, kThreads);
    else
        quantize_levels<true>(a.h + p * ep * FF, hn, &L.b.hq[0][0], kMaxHP, &L.b.hsc[0][0], kMaxHP / 64, L.b.hs32,
                              tid, kThreads);
    __syncthreads();
    const int slots = kThreads / UP;
    const bool b_active = tid < slots * UP;
    const int slot = tid / UP, unit = tid % UP;
    const int be = unit / segB, bseg = unit % segB;  // expert within the partition, segment
    XSeg hs;
    float wj = 0.f;
    const uint8_t* dexp = nullptr;
    if (b_active) {
        load_xseg(hs, &L.b.hq[0][0], kMaxHP, &L.b.hsc[0][0], kMaxHP / 64, L.b.hs32, be * segB + bseg);
        wj = L.w[p * ep + be];
        dexp = L.down[p * ep + be];
    }
    for (int r0 = r_begin; r0 < r_end; r0 += round_rows) {
        const int rr = min(round_rows, r_end - r0);
        if (r0 != r_begin) {  // later rounds: stage now into the single buffer
            __syncthreads();
            if (wave == 3) issue_stage(r0);
            wait_vm();
            __syncthreads();
        }
        if (b_active && dexp) {
            // row r0 of this expert starts (src & 15) bytes into its staged copy
            const uint8_t* rows = L.bstage + be * stride_e + (int)((uintptr_t)(dexp + (size_t)r0 * drb) & 15);
            for (int i = slot; i < rr; i += slots) {
                RawSeg<DT> raw;
                raw.load(rows + i * drb, bseg);
                L.b.part[i * UP + unit] = wj * raw.dot_q8(bseg, hs);
            }
        } else if (b_active) {
            for (int i = slot; i < rr; i += slots) L.b.part[i * UP + unit] = 0.f;
        }
        __syncthreads();
        // fixed-order sum over the partition's units, one thread per row
        for (int i = tid; i < rr; i += kThreads) {
            float v = 0.f;
            for (int u = 0; u < UP; u++) v += L.b.part[i * UP + u];
            store_coherent(&a.ypart[p * D + r0 + i], v);
        }
    }

    // ---- 6. combine the partitions' partials of this row chunk into y
    wait_vm();
    __syncthreads();
    if (a.local_l2) {
        // partition q % 8 reduces chunk q once all eight partials carry this epoch
        if (tid == 0)
            __hip_atomic_store(&a.sync[kFlagChunk + p * kMaxM + q], a.epoch, __ATOMIC_RELAXED,
                               __HIP_MEMORY_SCOPE_AGENT);
        if (p == q % np) {
            if (wave == 0) {
                unsigned spins = 0;
                for (;;) {
                    const bool mine =
                        lane >= np || __hip_atomic_load(&a.sync[kFlagChunk + lane * kMaxM + q], __ATOMIC_RELAXED,
                                                        __HIP_MEMORY_SCOPE_AGENT) == a.epoch;
                    if (__all(mine)) break;
                    __builtin_amdgcn_s_sleep(1);
                    if (++spins == kSpinLimit) {
                        if (lane == 0)
                            __hip_atomic_store(&a.sync[kSyncErr], 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                        break;
                    }
                }
            }
            __syncthreads();
            for (int r = r_begin + tid; r < r_end; r += kThreads) {
                float v = 0.f;
                for (int pp = 0; pp < np; pp++) v += load_coherent(&a.ypart[pp * D + r]);
                a.y[r] = v;
            }
        }
    } else {
        // the last partition to finish this row chunk writes y
        if (tid == 0) {
            const unsigned done = bump_counter(&a.sync[kSyncChunk + q]);  // returns the coherent count
            L.flag = done == (unsigned)np - 1;
            if (L.flag) reset_counter(&a.sync[kSyncChunk + q]);
        }
        __syncthreads();
        if (L.flag) {
            for (int r = r_begin + tid; r < r_end; r += kThreads) {
                float v = 0.f;
                for (int pp = 0; pp < np; pp++) v += load_coherent(&a.ypart[pp * D + r]);
                a.y[r] = v;
            }
        }
    }
}

template <int LA, int GT, int UT, int DT>
__global__ __launch_bounds__(kThreads) void moe_decode_fused(FusedArgs a) {
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

static int partitions_for(int k) { return k <= 8 ? k : (k % 8 == 0 ? 8 : 0); }

bool fused_supported(const MoeShape& s, int k, int n_expert_for_routing) {
    if (!moe_shape_ok(s) || k <= 0 || k > kMaxSlots) return false;
    if (s.D % 64 || s.FF % 64 || s.D > kMaxD) return false;
    if (!pick_fused(s)) return false;
    const int np = partitions_for(k);
    if (!np) return false;
    const int ep = k / np;
    const int UP = ep * (s.FF / 64);
    if (UP > kThreads || ep * s.FF > kMaxHP || UP > kMaxPart) return false;
    if (n_expert_for_routing > kMaxE) return false;
    if (ep * stage_stride(1, (int)s.down_rb) > kStageB) return false;  // one staged row per expert must fit
    return true;
}

struct GridInfo {
    int cus = 0, per_cu = 0;
};

// Workgroups resident at once on the device (occupancy x CUs), cached per
// kernel and device.
static GridInfo fused_capacity(FusedFn fn, int device) {
    struct Entry {
        FusedFn fn;
        int device;
        GridInfo g;
    };
    static Entry cache[128];
    static int n = 0;
    static std::mutex mu;
    std::lock_guard<std::mutex> lk(mu);
    for (int i = 0; i < n; i++)
        if (cache[i].fn == fn && cache[i].device == device) return cache[i].g;
    GridInfo g;
    int occ = 0;
    if (hipDeviceGetAttribute(&g.cus, hipDeviceAttributeMultiprocessorCount, device) != hipSuccess) return GridInfo{};
    if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&occ, reinterpret_cast<const void*>(fn), kThreads, 0) !=
        hipSuccess)
        return GridInfo{};
    g.per_cu = occ < 2 ? occ : 2;
    if (n < 128) cache[n++] = Entry{fn, device, g};
    return g;
}

__global__ void xcc_probe_kernel(int* out) {
    if (threadIdx.x == 0) out[blockIdx.x] = xcc_id();
}

// One-time check per device that a plain launch places workgroup b on XCD
// (b + s) % 8 for one start s (the round-robin dispatch the XCD-local exchange
// relies on; s depends on the launches before).
static bool xcd_round_robin(int device) {
    static int state[64];  // 0 unknown, 1 yes, 2 no
    static std::mutex mu;
    std::lock_guard<std::mutex> lk(mu);
    if (device < 0 || device >= 64) return false;
    if (state[device]) return state[device] == 1;
    state[device] = 2;
    constexpr int kProbe = 1024;
    int* d = nullptr;
    clear_stale_error();  // an earlier, unrelated failure must not read as the probe's
    if (hipMalloc(&d, kProbe * sizeof(int)) != hipSuccess) return false;
    hipLaunchKernelGGL(xcc_probe_kernel, dim3(kProbe), dim3(64), 0, nullptr, d);
    int hbuf[kProbe];
    bool ok = hipGetLastError() == hipSuccess &&
              hipMemcpy(hbuf, d, sizeof hbuf, hipMemcpyDeviceToHost) == hipSuccess;
    (void)hipFree(d);
    const int s = ok ? hbuf[0] : -1;
    ok = ok && s >= 0 && s < 8;
    for (int b = 0; ok && b < kProbe; b++) ok = hbuf[b] == (b + s) % 8;
    if (ok) state[device] = 1;
    return ok;
}

int fused_exchange_mode(int device) { return xcd_round_robin(device) ? 1 : 0; }

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
    a.ypart = h.ypart;
    a.sync = h.sync;
    if (!fused_supported(a.s, a.k, a.mode == 1 ? a.n_expert : 0) || !a.ypart || !a.h || !a.sync)
        return hipErrorInvalidValue;
    FusedFn fn = pick_fused(a.s);
    int dev = 0;
    hipError_t e = hipGetDevice(&dev);
    if (e != hipSuccess) return e;
    const GridInfo g = fused_capacity(fn, dev);
    if (g.per_cu <= 0) return hipErrorInvalidConfiguration;
    a.np = partitions_for(a.k);
    a.local_l2 = (a.np == 8 && xcd_round_robin(dev)) ? 1 : 0;
    a.epoch = h.epoch;
    const int m0 = g.per_cu * g.cus / a.np;  // every workgroup resident at once
    if (m0 <= 0) return hipErrorInvalidConfiguration;
    a.rows_b = (a.s.D + m0 - 1) / m0;
    a.m = (a.s.D + a.rows_b - 1) / a.rows_b;  // no workgroup without output rows
    if (a.m > kMaxChunks || (a.local_l2 && a.m > kMaxM) || a.epoch == 0) return hipErrorInvalidConfiguration;
    const int ep = a.k / a.np;
    const int UP = ep * (a.s.FF / 64);
    const int slots = kThreads / UP;
    int rr = a.rows_b;
    while (rr > 1 && ep * stage_stride(rr, (int)a.s.down_rb) > kStageB) rr--;
    if (rr * UP > kMaxPart) rr = kMaxPart / UP;
    if (rr > slots && rr < a.rows_b) rr -= rr % slots;  // whole passes over the row slots
    if (rr <= 0) return hipErrorInvalidConfiguration;
    a.round_b = rr;
    clear_stale_error();
    // A plain launch: the grid never exceeds what is resident at once, and the
    // stream runs nothing else concurrently, so every workgroup is live.
    hipLaunchKernelGGL(fn, dim3(a.np * a.m), dim3(kThreads), 0, st, a);
    return hipGetLastError();
}

}  // namespace eahmmf
