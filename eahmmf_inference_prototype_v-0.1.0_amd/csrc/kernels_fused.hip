// kernels_fused.hip - one launch per token for the whole MoE expert block:
// routing -> gate/up + SiLU -> down -> router-weighted sum.
//
// This replaces, for one decode token, the reference's host loop
// (qwen3moe.cpp:1011-1067): softmax/top-k/renormalise, per expert a gate/up
// pair and a down matmul on the GPU, SiLU and the weighted scatter-add on the
// CPU, 16 synchronous round trips per layer.
//
// One 512-thread workgroup per CU, all resident.  A decode token streams
// every routed expert's weights once (24.5 MB at the Qwen3-30B-A3B shape), so
// the kernel is built around the fastest way MI355X has to stream bytes it
// reads once: contiguous nontemporal LDS DMA (global_load_lds ... nt, 1 KB
// per wave instruction), issued for every weight byte straight after routing,
// with the arithmetic done from LDS as the bytes land.
//
// Layout of the work.  The routed experts are split into NP partitions (one
// expert each for k <= 8, k/8 each for k = 16); workgroup b is rank q = b / NP
// inside its partition.  With NP = 8 the partition is the XCD the workgroup
// runs on (hardware XCC id): the dispatcher hands consecutive workgroups to
// the eight XCDs in turn, starting wherever the previous launch stopped, so
// workgroups b, b+8, b+16, ... share one XCD (checked once per device) and a
// partition's h is exchanged through that XCD's L2.  Otherwise workgroup b
// belongs to partition b % NP and h travels with device-coherent stores and
// loads.
//
// Per workgroup (waves 0-3 "A", waves 4-7 "B"):
//   1. routing: wave 0 reads the logits and the expert table and forms the
//      keys e_i = expf(l_i - max) while waves 1-7 turn x into three int8
//      levels per 64-value segment in LDS; then every thread ranks
//      candidates by counting (e desc, id asc - the reference's order) and
//      the top k land in LDS slots.
//   2. A waves: lane groups of D/64 lanes own one 64-value segment of x each.
//      A pass of an A wave is GW = 64 / (D/64) consecutive (expert, row)
//      pairs of the workgroup's slice; the wave DMAs the gate and up rows of
//      up to NPA passes into its own LDS ring, waits for each pass with an
//      exact vmcnt, dots the rows exactly in int32 (v_dot4) against the
//      activation levels, reduces in the group and keeps h = silu(g) * u in
//      LDS; the next pass is issued into the slot just consumed.
//      B waves: once the A waves' first passes are issued, DMA this
//      workgroup's down rows of the partition's experts (its output-row
//      chunk) into LDS; wave 4 renormalises the routing weights.
//   3. partition barrier.  Each A wave stores its h values; the last A wave
//      of a workgroup to see its stores complete publishes the workgroup's
//      arrival.  XCD-local: a flag word per workgroup set to the launch epoch,
//      all m of them polled by wave 0 with agent-scope loads (which miss the
//      CU's L1); otherwise one atomic counter per partition.  B waves take no
//      part, so their outstanding DMA never delays the flag.
//   4. all threads turn the partition's h into int8 levels in LDS; all eight
//      waves compute w_j * down_j[r].h_j per (row, 64-value segment) unit
//      from the staged rows, and the units of each row are summed in a fixed
//      order into this partition's partial ypart[p][r].  Chunks with more
//      rows than the stage holds take several rounds.
//   5. per row chunk, one workgroup adds the NP partials in partition order
//      (deterministic) and writes y: partition q % NP once all NP epoch flags
//      of the chunk are set (XCD-local), else the last partition to arrive.
// Counters are reset by the last workgroup through each stage, so every
// launch starts from zero; epoch flags need no reset.  Every wait is bounded;
// if a bound is ever hit an error flag is raised and the kernel still exits.
#include <mutex>

#include "internal.h"
#include "kquant_seg64.h"

namespace eahmmf {

constexpr int kThreads = 512;
constexpr int kWaves = kThreads / 64;
constexpr int kAWaves = 4;  // waves 0-3: gate/up; waves 4-7: down staging
constexpr int kAThreads = 64 * kAWaves;
constexpr int kMaxD = 4096;
constexpr int kMaxE = 256;
constexpr int kMaxHP = 4096;     // floats of h held per partition
constexpr int kMaxPart = 2048;   // (row, segment) partials of one round
constexpr int kMaxHW = 128;      // h values one workgroup computes
constexpr int NPD = 3;           // phase-B tasks each B wave decodes before the barrier
constexpr int kSlotA = 20 * 1024;   // LDS ring of one A wave
constexpr int kStageB = 40 * 1024;  // LDS for one round of down rows
constexpr unsigned kSpinLimit = 1u << 22;

// One A pass: GW rows of gate and GW rows of up, GW * row bytes =
// 4096 * (bytes per value) whatever D is.  NIR DMA instructions per matrix
// cover it plus 32 bytes (up to 15 of alignment slack, and the 2 bytes past a
// row that a realigned 32-byte LDS read touches); NPA passes are in flight.
template <int T>
struct PassA {
    static constexpr int bytes = 4096 * Fmt<T>::bytes / Fmt<T>::blck;
    static constexpr int nir = (bytes + 32 + 1023) / 1024;
    static constexpr int slot = 2 * nir * 1024;
    static constexpr int n = kSlotA / slot < 3 ? kSlotA / slot : 3;
    static_assert(n >= 1, "an A pass must fit the ring");
};

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
    int rows_a;             // (expert, row) pairs of gate/up per workgroup, a multiple of the A lane groups
    int rows_round;         // output rows staged per phase-B round
    int stride_b;           // LDS bytes per expert in the phase-B stage (multiple of 1024)
    int rank_shift, rank_c;  // routing: log2 of the threads per candidate, keys each of them compares
    int local_l2;            // 1: partition p runs on XCD p, so h is exchanged through that XCD's L2
    unsigned epoch;         // launch number (>= 1): the value this launch's flags carry
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
    // last: read only in mode 0, so the fields above share the first few
    // cache lines of the argument block (the kernel rereads them as it goes)
    DecodeSlots direct;
};

template <int CTRL, int ROWS>
__device__ __forceinline__ float dpp_fmax_step(float a, float fill) {
    return fmaxf(a, __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(__builtin_bit_cast(int, fill),
                                                                          __builtin_bit_cast(int, a), CTRL, ROWS, 0xF,
                                                                          false)));
}

// wave64 max with DPP row operations; lane 63 collects the total, which is
// then broadcast.  Controls: 0xB1/0x4E quad permutes, 0x141 row_half_mirror,
// 0x140 row_mirror, 0x142 row_bcast:15 (rows 1,3), 0x143 row_bcast:31 (rows 2,3).
__device__ __forceinline__ float dpp_max(float v) {
    v = dpp_fmax_step<0xB1, 0xF>(v, v);
    v = dpp_fmax_step<0x4E, 0xF>(v, v);
    v = dpp_fmax_step<0x141, 0xF>(v, -INFINITY);
    v = dpp_fmax_step<0x140, 0xF>(v, -INFINITY);
    v = dpp_fmax_step<0x142, 0xA>(v, -INFINITY);
    v = dpp_fmax_step<0x143, 0xC>(v, -INFINITY);
    return __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), 63));
}

// Device-coherent (sc1) accesses: visible across the XCDs' separate L2s
// without whole-cache writeback or invalidate.
__device__ __forceinline__ void store_coherent(float* p, float v) {
    __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ float load_coherent(const float* p) {
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

__device__ __forceinline__ void raise_error(unsigned* sync, unsigned code) {
    __hip_atomic_store(&sync[kSyncErr], code, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// XCD (XCC) the calling wave runs on: hardware register HW_REG_XCC_ID (20),
// bits [3:0].
__device__ __forceinline__ int xcc_id() { return (int)(__builtin_amdgcn_s_getreg(20 | (0 << 6) | (3 << 11)) & 0xF); }

// v + v of the lane DPP control CTRL names, in rows ROWS (others add 0).
template <int CTRL, int ROWS = 0xF>
__device__ __forceinline__ float dpp_add_step(float v) {
    return v + __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), CTRL, ROWS, 0xF,
                                                                     false));
}

// Sum over each aligned group of W lanes (W a power of two <= 64) with DPP
// steps: quad swaps, row_half_mirror, row_mirror, row_bcast:15 and :31.  The
// group's last lane holds the total (for W <= 16 every lane of the group).
template <int W>
__device__ __forceinline__ float group_sum(float v) {
    if (W >= 2) v = dpp_add_step<0xB1>(v);
    if (W >= 4) v = dpp_add_step<0x4E>(v);
    if (W >= 8) v = dpp_add_step<0x141>(v);
    if (W >= 16) v = dpp_add_step<0x140>(v);
    if (W >= 32) v = dpp_add_step<0x142, 0xA>(v);
    if (W >= 64) v = dpp_add_step<0x143, 0xC>(v);
    return v;
}

struct alignas(16) FusedLds {
    uint8_t stage_a[kAWaves][kSlotA];  // first members: 16-byte aligned
    uint8_t stage_b[kStageB];
    union {
        struct {  // steps 1-2: activation levels
            int8_t xq[kLevels][kMaxD];
            float xsc[kLevels][kMaxD / 64];
            float xs32[kMaxD / 32];
        } a;
        struct {  // step 4: the partition's h as int8 levels
            int8_t hq[kLevels][kMaxHP];
            float hsc[kLevels][kMaxHP / 64];
            float hs32[kMaxHP / 32];
        } b;
    };
    alignas(16) float part[kMaxPart];  // (row, segment) partials of one phase-B round
    float hw[kMaxHW];      // h of this workgroup's (expert, row) pairs before they are stored
    ExpertEntry table[kMaxE];
    alignas(16) uint32_t rkey[kMaxE];  // routing order keys
    float slot_key[kMaxSlots];
    int slot_id[kMaxSlots];
    const uint8_t* gate[kMaxSlots];
    const uint8_t* up[kMaxSlots];
    const uint8_t* down[kMaxSlots];
    float w[kMaxSlots];
    unsigned a_issued;  // A waves whose first passes are issued (the down copies go out after them)
    unsigned b_landed;  // B waves whose down copies have landed
    unsigned a_done;    // A waves whose h stores have completed
    int flag;
};

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

// Routing, step 1 (wave 0): the expert table into LDS and every candidate's
// order key: e_i = expf(l_i - max) as the reference forms it, stored as its
// bits + 1 (non-negative floats order as their bits); 0 for a NaN e_i and for
// ids past n_expert up to 256, which then never rank ahead of a real one.
__device__ void route_keys(const FusedArgs& a, FusedLds& L, int lane) {
    const int n = a.n_expert;
    // every global load of this step goes out before the first use
    float l[4];
    ExpertEntry ent[4];
#pragma unroll
    for (int c = 0; c < 4; c++) {
        const int id = lane + 64 * c;
        l[c] = id < n ? a.logits[id] : -INFINITY;
        ent[c] = id < n ? a.table[id] : ExpertEntry{nullptr, nullptr, nullptr};
    }
    float mx = fmaxf(fmaxf(l[0], l[1]), fmaxf(l[2], l[3]));
    mx = dpp_max(mx);
#pragma unroll
    for (int c = 0; c < 4; c++) {
        const int id = lane + 64 * c;
        const float e = expf(l[c] - mx);
        L.rkey[id] = (id < n && e == e) ? __builtin_bit_cast(uint32_t, e) + 1u : 0u;
        if (id < n) L.table[id] = ent[c];
    }
}

// Routing, step 2 (all threads): candidate i's rank in (e desc, id asc), the
// reference's order (qwen3moe.cpp:1016), is the number of candidates ahead of
// it: larger key, or equal key and lower id.  T = 2^rank_shift adjacent
// threads count over C = rank_c consecutive keys each (read four at a time).
// Ranks are distinct, so the top k fill slots 0..k-1 without collisions.
__device__ void route_rank(const FusedArgs& a, FusedLds& L, int tid) {
    const int n = a.n_expert, C = a.rank_c;
    const int i = tid >> a.rank_shift, part = tid & ((1 << a.rank_shift) - 1);
    int ahead = 0;
    uint32_t ki = 0;
    if (i < n) {
        ki = L.rkey[i];
        const int j0 = part * C;
        if (C >= 4) {
            for (int jb = 0; jb < C; jb += 4) {
                const uint4 v = *reinterpret_cast<const uint4*>(&L.rkey[j0 + jb]);
                const uint32_t kv[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
                for (int c = 0; c < 4; c++) ahead += (kv[c] > ki) | ((kv[c] == ki) & (j0 + jb + c < i));
            }
        } else {
            for (int j = j0; j < j0 + C; j++) ahead += (L.rkey[j] > ki) | ((L.rkey[j] == ki) & (j < i));
        }
    }
    for (int off = (1 << a.rank_shift) / 2; off > 0; off >>= 1) ahead += __shfl_xor(ahead, off, 64);
    if (i < n && part == 0 && ahead < a.k) {
        const bool valid = ki != 0u;
        L.slot_key[ahead] = valid ? __builtin_bit_cast(float, ki - 1u) : -1.0f;
        L.slot_id[ahead] = valid ? i : -1;
    }
}

// Routing, step 3 (one wave, lanes < k): renormalise the chosen e in rank
// order, as the reference sums them.
__device__ void route_weights(const FusedArgs& a, FusedLds& L, int lane) {
    const float kv = lane < a.k ? L.slot_key[lane] : -1.0f;
    const bool valid = kv >= 0.f;
    float tot = 0.f;
    for (int r = 0; r < a.k; r++)
        tot += __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, valid ? kv : 0.f), r));
    if (lane < a.k) {
        const float wr = valid ? kv / tot : 0.f;
        L.w[lane] = wr;
        if (blockIdx.x == 0) {
            if (a.ids_out) a.ids_out[lane] = valid ? L.slot_id[lane] : -1;
            if (a.w_out) a.w_out[lane] = wr;
        }
    }
}

// Weight pointers of routed slot j (matrix c: 0 gate, 1 up, 2 down): from
// the table row of the slot's expert id when the kernel routed, else as the
// caller gave them; null for a slot without an expert.
__device__ __forceinline__ const uint8_t* slot_ptr(const FusedArgs& a, const FusedLds& L, int j, int c) {
    if (a.mode == 1) {
        const int id = L.slot_id[j];
        if (id < 0) return nullptr;
        const ExpertEntry& t = L.table[id];
        return c == 0 ? t.gate : (c == 1 ? t.up : t.down);
    }
    return c == 0 ? L.gate[j] : (c == 1 ? L.up[j] : L.down[j]);
}

// ypart[0][r] + ... + ypart[np-1][r] (np <= 8) in partition order, all
// loads issued before the first add.
__device__ __forceinline__ float sum_partials(const float* ypart, int D, int r, int np) {
    float v[8];
#pragma unroll
    for (int pp = 0; pp < 8; pp++) v[pp] = pp < np ? load_coherent(&ypart[pp * D + r]) : 0.f;
    float t = 0.f;
#pragma unroll
    for (int pp = 0; pp < 8; pp++)
        if (pp < np) t += v[pp];
    return t;
}

// vmcnt(n * NI) for a run-time n in [0, 2].
template <int NI>
__device__ __forceinline__ void wait_passes(int n) {
    if (n <= 0) wait_vm_upto<0>();
    else if (n == 1) wait_vm_upto<NI>();
    else wait_vm_upto<2 * NI>();
}

// Geometry of A pass pp of wave w: GW consecutive (expert, row) pairs from
// t0; nr of them are real rows of expert slot j starting at row f0.
struct PassRows {
    int t0, nr, j, f0;
    bool ok;
    const uint8_t* g;
    const uint8_t* u;
};

template <int LA, int GT, int UT, int DT>
__device__ void fused_body(const FusedArgs& a, FusedLds& L) {
    constexpr int GA = kAThreads / LA;  // A lane groups
    constexpr int GW = 64 / LA;         // A lane groups per wave = rows per pass
    using PA = PassA<GT>;
    static_assert(PassA<UT>::nir == PA::nir, "gate and up share a format");
    constexpr int NPA = PA::n;
    const int tid = threadIdx.x;
    const int wave = __builtin_amdgcn_readfirstlane(tid / 64), lane = tid % 64;
    const MoeShape& s = a.s;
    const int D = s.D, FF = s.FF, k = a.k;
    const int np = a.np, m = a.m;
    const int xcc = a.local_l2 ? xcc_id() : 0;
    const bool xcc_bad = xcc >= np;  // never on a device that passed the host's placement check
    const int p = a.local_l2 ? (xcc_bad ? 0 : xcc) : (int)blockIdx.x % np, q = blockIdx.x / np;
    const int ep = k / np;  // experts per partition
    const int segB = FF / 64;
    const int drb = (int)s.down_rb;
    // output rows of this workgroup's chunk (the host gives every workgroup at least one)
    const int r_begin = q * a.rows_b;
    const int r_end = min(D, r_begin + a.rows_b);

    // ---- 1. routing / slots and activation levels (one barrier)
    // this thread's eight values of x (at most one segment part per thread),
    // loaded first so that their latency overlaps the routing's
    static_assert(kMaxD / 64 * 8 <= kThreads, "one x segment part per thread");
    const int xseg = tid / 8, xpart = tid % 8;
    float xv[8];
    load8<false>(a.x, xseg, xpart, xseg < D / 64, xv);
    if (wave == 0) {
        if (lane == 0) {
            L.a_issued = 0;
            L.b_landed = 0;
            L.a_done = 0;
        }
        if (a.mode == 1) {
            // ranks are a permutation of 0..n_expert-1, so the routing
            // writes the slots below n_expert and these defaults the rest
            if (lane >= a.n_expert && lane < k) {
                L.slot_key[lane] = -1.0f;
                L.slot_id[lane] = -1;
            }
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
    }
    // wave 0 forms the routing keys while waves 1-7 turn x into levels
    // (wave 0's own segments follow its keys); all threads then rank
    if (wave == 0 && a.mode == 1) route_keys(a, L, lane);
    quantize8(xv, xseg, xpart, xseg < D / 64, &L.a.xq[0][0], kMaxD, &L.a.xsc[0][0], kMaxD / 64, L.a.xs32);
    __syncthreads();
    if (a.mode == 1) {
        route_rank(a, L, tid);
        __syncthreads();
    }

    // phase-B stage: rows [r0, r0 + rr) of the chunk, expert e of the
    // partition at stage_b + e * stride_b + (its source & 15)
    auto down_src = [&](int e, int r0) -> const uint8_t* {
        const uint8_t* dw = slot_ptr(a, L, p * ep + e, 2);
        return dw ? dw + (size_t)(r_begin + r0) * drb : reinterpret_cast<const uint8_t*>(a.x);
    };
    // B waves copy the round's rows, one 1 KB instruction each in turn
    auto stage_round = [&](int r0, int rr, int wave_b, int nwaves_b) {
        const int ni = a.stride_b / 1024;
        for (int e = 0; e < ep; e++) {
            const uint8_t* src = down_src(e, r0);
            const int n = slot_ptr(a, L, p * ep + e, 2) ? rr * drb : 16;
            const uintptr_t base = (uintptr_t)src & ~(uintptr_t)15;
            const int n16 = (int)(((((uintptr_t)src + (uintptr_t)n + 15) & ~(uintptr_t)15) - base) / 16);
            for (int i = wave_b; i < ni; i += nwaves_b) {
                const int c = min(i * 64 + lane, n16 - 1);
                lds_dma16(base + (uintptr_t)c * 16, L.stage_b + e * a.stride_b + i * 1024);
            }
        }
    };

    // Phase-B tasks of a round: (expert e of the partition, 64-value segment
    // sg, 64-row block); a lane is one row.  The B waves decode the first NPD
    // tasks each of round 0 into registers before the barrier.
    const int rr0 = min(a.rows_round, r_end - r_begin);
    const int nrb0 = (rr0 + 63) / 64;
    const int n_tasks0 = ep * segB * nrb0;
    struct BTask {
        int e, sg, r;
        const uint8_t* row;
    };
    auto btask = [&](int task, int rr, int r0) {
        const int nrb = (rr + 63) / 64;
        BTask t;
        t.e = task / (segB * nrb);
        const int rest = task - t.e * (segB * nrb);
        t.sg = rest / nrb;
        t.r = (rest - t.sg * nrb) * 64 + lane;
        const uint8_t* src = down_src(t.e, r0);  // rows [r0, r0 + rr) of the chunk are staged
        t.row = L.stage_b + t.e * a.stride_b + ((uintptr_t)src & 15) + min(t.r, rr - 1) * drb;
        return t;
    };
    SegCodes<DT> pre[NPD];

    // ---- 2. gate/up passes.  A pass of A wave w is GW consecutive (expert,
    // row) pairs; w DMAs its passes into its own LDS ring and dots them.
    const int gl = lane / LA, li = lane % LA;
    const int rows_a = ep * FF;
    const int ra0 = min(rows_a, q * a.rows_a), ra1 = min(rows_a, ra0 + a.rows_a);
    const int npass = (ra1 - ra0 + GA - 1) / GA;
    auto rows_of = [&](int pp) {
        PassRows r;
        r.t0 = ra0 + pp * GA + wave * GW;
        r.nr = max(0, min(GW, ra1 - r.t0));
        const int tt = min(r.t0, rows_a - 1);
        r.j = p * ep + tt / FF;
        r.f0 = tt - (tt / FF) * FF;
        const uint8_t* gw = slot_ptr(a, L, r.j, 0);
        const uint8_t* uw = slot_ptr(a, L, r.j, 1);
        r.ok = (r.nr > 0) & (gw != nullptr) & (uw != nullptr);
        // a pass without weights copies 16 bytes of x instead; nothing of it is used
        r.g = r.ok ? gw + (size_t)r.f0 * s.gate_rb : reinterpret_cast<const uint8_t*>(a.x);
        r.u = r.ok ? uw + (size_t)r.f0 * s.up_rb : reinterpret_cast<const uint8_t*>(a.x);
        return r;
    };
    auto wait_lds_count = [&](const unsigned* c, unsigned v) {  // bounded: the other waves always progress
        for (unsigned spins = 0; spins < (1u << 20); spins++) {
            if (__hip_atomic_load(c, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP) >= v) break;
            __builtin_amdgcn_s_sleep(1);
        }
    };

    if (wave < kAWaves) {
        // ---- 2A. this wave's passes through its LDS ring
        auto issue = [&](int pp) {
            const PassRows r = rows_of(pp);
            uint8_t* sl = L.stage_a[wave] + (pp % NPA) * PA::slot;
            dma_to_lds<PA::nir>(r.g, r.ok ? r.nr * (int)s.gate_rb : 16, sl, lane);
            dma_to_lds<PA::nir>(r.u, r.ok ? r.nr * (int)s.up_rb : 16, sl + PA::nir * 1024, lane);
        };
        for (int pp = 0; pp < min(NPA, npass); pp++) issue(pp);
        if (lane == 0) atomicAdd(&L.a_issued, 1u);
        XSeg xs;  // read while the first pass is in flight
        load_xseg(xs, &L.a.xq[0][0], kMaxD, &L.a.xsc[0][0], kMaxD / 64, L.a.xs32, li);
        for (int pp = 0; pp < npass; pp++) {
            // passes pp+1 .. are still allowed in flight: 2 * nir instructions each
            wait_passes<2 * PA::nir>(min(npass - 1 - pp, NPA - 1));
            const PassRows r = rows_of(pp);
            const uint8_t* sl = L.stage_a[wave] + (pp % NPA) * PA::slot;
            const uint8_t* grow = sl + ((uintptr_t)r.g & 15) + gl * s.gate_rb;
            const uint8_t* urow = sl + PA::nir * 1024 + ((uintptr_t)r.u & 15) + gl * s.up_rb;
            RawSeg<GT> g;
            RawSeg<UT> u;
            g.template load<LdsLd>(r.ok && gl < r.nr ? grow : sl, li);
            u.template load<LdsLd>(r.ok && gl < r.nr ? urow : sl, li);
            const float dg = group_sum<LA>(g.dot_q8(li, xs));
            const float du = group_sum<LA>(u.dot_q8(li, xs));
            if (li == LA - 1 && gl < r.nr) L.hw[r.t0 + gl - ra0] = dg / (1.0f + expf(-dg)) * du;
            // every lane's reads of this slot have returned (their values are used above)
            if (pp + NPA < npass) issue(pp + NPA);
        }
        // ---- 3. h stores, then the workgroup's arrival
        for (int e = lane; e < npass * GW; e += 64) {
            const int pp = e / GW, g2 = e % GW;
            const PassRows r = rows_of(pp);
            if (r.ok && g2 < r.nr) {
                const float hv = L.hw[r.t0 + g2 - ra0];
                float* dst = &a.h[r.j * FF + r.f0 + g2];
                if (a.local_l2)  // the partition's readers share this XCD's L2
                    *dst = hv;
                else
                    store_coherent(dst, hv);
            }
        }
        wait_vm();
        if (lane == 0) {
            const unsigned before = atomicAdd(&L.a_done, 1u);
            if (before == kAWaves - 1) {
                if (a.local_l2) {
                    if (xcc_bad)  // the XCD-to-partition mapping this exchange relies on does not hold
                        raise_error(a.sync, 2u);
                    a.sync[kFlagArrive + p * kMaxM + q] = a.epoch;
                } else {
                    bump_counter(&a.sync[kSyncArrive + p]);
                }
            }
        }
        if (wave == 0) {
            if (a.local_l2) {
                unsigned spins = 0;
                for (;;) {
                    const unsigned* fl = &a.sync[kFlagArrive + p * kMaxM];
                    const bool mine = (lane >= m || load_flag(fl + lane) == a.epoch) &&
                                      (lane + 64 >= m || load_flag(fl + lane + 64) == a.epoch);
                    if (__all(mine)) break;
                    __builtin_amdgcn_s_sleep(1);
                    if (++spins == kSpinLimit) {
                        if (lane == 0) raise_error(a.sync, 1u);
                        break;
                    }
                }
            } else if (lane == 0) {
                unsigned spins = 0;
                while (poll_counter(&a.sync[kSyncArrive + p]) < (unsigned)m) {
                    __builtin_amdgcn_s_sleep(2);
                    if (++spins == kSpinLimit) {
                        raise_error(a.sync, 1u);
                        break;
                    }
                }
                if (bump_counter(&a.sync[kSyncPass + p]) == (unsigned)m - 1) {  // everyone has passed: reset
                    reset_counter(&a.sync[kSyncArrive + p]);
                    reset_counter(&a.sync[kSyncPass + p]);
                }
            }
        }
    } else {
        // ---- 2B. the first round of down rows into LDS, queued behind the
        // A waves' first passes (the CU serves its copies in issue order, and
        // h, the barrier and everything after it wait on gate/up first); once
        // they land, this wave decodes its first NPD phase-B tasks into
        // registers, so that after the barrier only their dot with h remains
        wait_lds_count(&L.a_issued, (unsigned)kAWaves);
        stage_round(0, rr0, wave - kAWaves, kWaves - kAWaves);
        if (a.mode == 1 && wave == kAWaves) route_weights(a, L, lane);
        wait_vm();
        if (lane == 0) atomicAdd(&L.b_landed, 1u);
        wait_lds_count(&L.b_landed, (unsigned)(kWaves - kAWaves));
#pragma unroll
        for (int i = 0; i < NPD; i++) {
            const int task = (wave - kAWaves) + (kWaves - kAWaves) * i;
            const BTask t = btask(min(task, n_tasks0 - 1), rr0, 0);
            RawSeg<DT> raw;
            raw.template load<LdsLd>(t.row, t.sg);
            pre[i] = raw.decode(t.sg);
        }
    }
    __syncthreads();  // the activation levels are dead from here: the LDS union switches to h

    // ---- 4. the partition's h as int8 levels (from this XCD's L2 when the
    // partition shares an XCD, with device-coherent loads otherwise)
    const int hn = ep * FF;
    if (a.local_l2)
        quantize_levels<false>(a.h + p * ep * FF, hn, &L.b.hq[0][0], kMaxHP, &L.b.hsc[0][0], kMaxHP / 64, L.b.hs32,
                               tid, kThreads);
    else
        quantize_levels<true>(a.h + p * ep * FF, hn, &L.b.hq[0][0], kMaxHP, &L.b.hsc[0][0], kMaxHP / 64, L.b.hs32,
                              tid, kThreads);
    __syncthreads();

    // Phase B rounds: every wave takes (expert, segment, 64-row block) tasks;
    // a lane is one row, so the h levels of the task are read by all lanes at
    // one address.
    for (int r0 = 0; r0 < r_end - r_begin; r0 += a.rows_round) {
        const int rr = min(a.rows_round, r_end - r_begin - r0);
        if (r0 > 0) {
            __syncthreads();  // the previous round's rows and partials are consumed
            stage_round(r0, rr, wave, kWaves);
            wait_vm();
            __syncthreads();
        }
        auto finish = [&](const BTask& t, const SegCodes<DT>& k) {
            XSeg hs;  // the same address in every lane: one LDS broadcast per read
            load_xseg(hs, &L.b.hq[0][0], kMaxHP, &L.b.hsc[0][0], kMaxHP / 64, L.b.hs32, t.e * segB + t.sg);
            const float v = k.dot(hs);
            if (t.r < rr)
                L.part[(t.e * rr + t.r) * segB + t.sg] = slot_ptr(a, L, p * ep + t.e, 2) ? L.w[p * ep + t.e] * v : 0.f;
        };
        int first = 0;
        if (r0 == 0) {
            // the decoded tasks (B waves), then the rest from LDS
            if (wave >= kAWaves) {
#pragma unroll
                for (int i = 0; i < NPD; i++) {
                    const int task = (wave - kAWaves) + (kWaves - kAWaves) * i;
                    if (task < n_tasks0) finish(btask(task, rr, r0), pre[i]);
                }
            }
            first = (kWaves - kAWaves) * NPD;
        }
        for (int task = first + wave; task < ep * segB * ((rr + 63) / 64); task += kWaves) {
            const BTask t = btask(task, rr, r0);
            RawSeg<DT> raw;
            raw.template load<LdsLd>(t.row, t.sg);
            finish(t, raw.decode(t.sg));
        }
        __syncthreads();
        // fixed-order sum over the partition's (expert, segment) units, one
        // thread per row (float4 reads when segB is a multiple of 4)
        for (int r = tid; r < rr; r += kThreads) {
            float v = 0.f;
            for (int e = 0; e < ep; e++) {
                const float* pr = &L.part[(e * rr + r) * segB];
                if (segB % 4 == 0) {
                    for (int u = 0; u < segB; u += 4) {
                        const float4 c = *reinterpret_cast<const float4*>(pr + u);
                        v += c.x;
                        v += c.y;
                        v += c.z;
                        v += c.w;
                    }
                } else {
                    for (int u = 0; u < segB; u++) v += pr[u];
                }
            }
            store_coherent(&a.ypart[p * D + r_begin + r0 + r], v);
        }
    }

    // ---- 5. combine the partitions' partials of this row chunk into y
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
                        if (lane == 0) raise_error(a.sync, 1u);
                        break;
                    }
                }
            }
            __syncthreads();
            for (int r = r_begin + tid; r < r_end; r += kThreads) a.y[r] = sum_partials(a.ypart, D, r, np);
        }
    } else {
        // the last partition to finish this row chunk writes y
        if (tid == 0) {
            const unsigned done = bump_counter(&a.sync[kSyncChunk + q]);  // returns the coherent count
            L.flag = done == (unsigned)np - 1;
            if (L.flag) reset_counter(&a.sync[kSyncChunk + q]);
        }
        __syncthreads();
        if (L.flag)
            for (int r = r_begin + tid; r < r_end; r += kThreads) a.y[r] = sum_partials(a.ypart, D, r, np);
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

// Workgroups resident at once on the device (CUs, one workgroup each), cached
// per kernel and device; 0 when the kernel cannot be made resident.
static int fused_capacity(FusedFn fn, int device) {
    struct Entry {
        FusedFn fn;
        int device;
        int g;
    };
    static Entry cache[128];
    static int n = 0;
    static std::mutex mu;
    std::lock_guard<std::mutex> lk(mu);
    for (int i = 0; i < n; i++)
        if (cache[i].fn == fn && cache[i].device == device) return cache[i].g;
    int cus = 0, occ = 0;
    if (hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, device) != hipSuccess) return 0;
    if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&occ, reinterpret_cast<const void*>(fn), kThreads, 0) !=
        hipSuccess)
        return 0;
    const int g = occ >= 1 ? cus : 0;
    if (n < 128) cache[n++] = Entry{fn, device, g};
    return g;
}

// Workgroup layout of one launch: m workgroups per partition, rows_b output
// rows each (every workgroup gets at least one), rows_a gate/up pairs each
// (a multiple of the A lane groups), and the phase-B stage geometry.
struct FusedGrid {
    int np = 0, m = 0, rows_b = 0, rows_a = 0, rows_round = 0, stride_b = 0;
};
static FusedGrid fused_grid(const MoeShape& s, int k, int capacity) {
    FusedGrid g;
    g.np = partitions_for(k);
    if (!g.np) return FusedGrid{};
    const int m0 = capacity / g.np;  // every workgroup resident at once
    if (m0 <= 0) return FusedGrid{};
    g.rows_b = (s.D + m0 - 1) / m0;
    g.m = (s.D + g.rows_b - 1) / g.rows_b;
    const int ep = k / g.np;
    const int ga = kAThreads / (s.D / 64);
    const int per = (ep * s.FF + g.m - 1) / g.m;
    g.rows_a = (per + ga - 1) / ga * ga;
    // rows per round: every expert's rows plus 32 bytes of slack (alignment,
    // and the 2 bytes past a row a realigned LDS read touches) in whole 1 KB
    // instructions, all experts within the stage
    const int drb = (int)s.down_rb;
    int rr = g.rows_b;
    auto stride = [&](int rows) { return (rows * drb + 32 + 1023) / 1024 * 1024; };
    while (rr > 1 && (ep * stride(rr) > kStageB || ep * rr * (s.FF / 64) > kMaxPart)) rr--;
    g.rows_round = rr;
    g.stride_b = stride(rr);
    return g;
}

// The layout fits the kernel's fixed LDS and flag arrays.
static bool fused_grid_ok(const MoeShape& s, int k, const FusedGrid& g) {
    if (g.m <= 0 || g.m > kMaxChunks || g.m > kMaxM) return false;
    const int ep = k / g.np;
    if (g.rows_a > kMaxHW || g.rows_round <= 0) return false;
    return ep * g.stride_b <= kStageB && ep * g.rows_round * (s.FF / 64) <= kMaxPart;
}

static int current_capacity(const MoeShape& s) {
    FusedFn fn = pick_fused(s);
    int dev = 0;
    if (!fn || hipGetDevice(&dev) != hipSuccess) return 0;
    return fused_capacity(fn, dev);
}

bool fused_supported(const MoeShape& s, int k, int n_expert_for_routing) {
    if (!moe_shape_ok(s) || k <= 0 || k > kMaxSlots) return false;
    if (s.D % 64 || s.FF % 64 || s.D > kMaxD) return false;
    if (!pick_fused(s)) return false;
    const int np = partitions_for(k);
    if (!np) return false;
    const int ep = k / np;
    if (ep * s.FF > kMaxHP) return false;
    if (n_expert_for_routing > kMaxE) return false;
    return fused_grid_ok(s, k, fused_grid(s, k, current_capacity(s)));
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
    if (!fused_supported(a.s, a.k, a.mode == 1 ? a.n_expert : 0) || !a.ypart || !a.h || !a.sync || !a.x)
        return hipErrorInvalidValue;
    if (a.mode == 1 && (a.n_expert <= 0 || !a.logits || !a.table)) return hipErrorInvalidValue;
    FusedFn fn = pick_fused(a.s);
    int dev = 0;
    hipError_t e = hipGetDevice(&dev);
    if (e != hipSuccess) return e;
    const FusedGrid g = fused_grid(a.s, a.k, fused_capacity(fn, dev));
    if (!fused_grid_ok(a.s, a.k, g) || h.epoch == 0) return hipErrorInvalidConfiguration;
    a.np = g.np;
    a.m = g.m;
    a.rows_b = g.rows_b;
    a.rows_a = g.rows_a;
    a.rows_round = g.rows_round;
    a.stride_b = g.stride_b;
    a.local_l2 = (a.np == 8 && xcd_round_robin(dev)) ? 1 : 0;
    a.epoch = h.epoch;
    // routing: n_expert rounded up to a power of two (at most 256) is split
    // into t runs of rank_c keys, t threads per candidate
    int npow = 1;
    while (npow < a.n_expert) npow *= 2;
    int t = kThreads / npow;
    if (t > 64) t = 64;
    if (t > npow) t = npow;
    a.rank_shift = 0;
    while ((1 << a.rank_shift) < t) a.rank_shift++;
    a.rank_c = npow / t;
    clear_stale_error();
    // A plain launch: the grid never exceeds what is resident at once, and the
    // stream runs nothing else concurrently, so every workgroup is live.
    hipLaunchKernelGGL(fn, dim3(a.np * a.m), dim3(kThreads), 0, st, a);
    return hipGetLastError();
}

}  // namespace eahmmf
