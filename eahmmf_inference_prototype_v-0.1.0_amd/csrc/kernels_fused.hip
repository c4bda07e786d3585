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
// expert each for k <= 8, k/8 each for k = 16); each workgroup is rank q
// inside its partition p.  With NP = 8 on a device whose dispatcher hands
// consecutive workgroups to its eight XCDs in turn (checked once per device),
// the partition is the XCD the workgroup runs on (hardware XCC id) and q is
// b / 8, or optionally a ticket (the workgroup's position in its XCD's
// arrival order, one atomic add on a per-XCD counter), so a partition's h is
// exchanged through that XCD's L2.  Otherwise workgroup b is rank b / NP of
// partition b % NP and h travels with device-coherent stores and loads.
//
// Per workgroup (waves 0-3 "A", waves 4-7 "B"):
//   1. routing: wave 0 reads the logits and the expert table and forms the
//      keys e_i = expf(l_i - max) while waves 1-7 turn x into three int8
//      levels per 64-value segment in LDS; then every thread ranks
//      candidates by counting larger keys (e desc, id asc - the reference's
//      order) and the top k land in LDS slots.  In mode 3 (routing from the
//      residual stream) the logits are formed in the launch first: every
//      workgroup RMS-normalizes x, computes one (logit, slice) unit of the
//      F32 router matmul and stores it as an exchange word; wave 0 of every
//      workgroup then reads all units and goes on as above.
//   2. A waves: lane groups of D/64 lanes own one 64-value segment of x each.
//      A pass of an A wave is GW = 64 / (D/64) consecutive (expert, row)
//      pairs of the workgroup's slice; the wave DMAs the gate and up rows of
//      up to NPA passes into its own LDS ring, waits for each pass with an
//      exact vmcnt, dots the rows exactly in int32 (v_dot4) against the
//      activation levels, reduces in the group and stores h = silu(g) * u
//      with the launch epoch in one 64-bit word; the next pass is issued into
//      the slot just consumed.  B waves: once the A waves' first passes are
//      issued, DMA this workgroup's down rows (its output-row chunk of the
//      partition's experts) into LDS; wave 4 renormalises the routing
//      weights.
//   3. once the down rows have landed the B waves decode their first NPD
//      phase-B tasks each into registers, while the A waves compute; the A
//      waves, done with their passes, read the partition's h - polling until
//      every word carries this launch's epoch - and turn it into int8 levels
//      in LDS.
//   4. every wave computes w_j * down_j[r].h_j per (row, 64-value segment)
//      unit (the B waves from their decoded codes, the rest decoded from the
//      staged rows), and the units of each row are summed in a fixed order
//      into this partition's partial ypart[p][r] (value and epoch again).
//      Chunks with more rows than the stage holds take several rounds.
//   5. workgroup q of partition q % NP polls the NP partials of each row of
//      chunk q until all carry this epoch and adds them in partition order
//      (deterministic) into y.
// Nothing is reset between launches: a word is current exactly when it
// carries this launch's epoch (launches are numbered from 1 and the exchange
// buffers are zeroed when allocated).
//
// Failure is loud.  Every wait is bounded (spin_limit polls) and also ends as
// soon as the launch's error word holds this launch's epoch.  A workgroup
// whose wait gave up stores NaN in place of everything that depended on the
// missing words (its partials; y rows whose partials never came), and the
// error word records the epoch, so the host's synchronous entry points
// return false and the caller falls back (the reference's contract for a
// failed GPU call).  The kernel still exits normally.
#include <stdlib.h>

#include <mutex>

#include "dpp.h"
#include "expf_ref.h"
#include "internal.h"
#include "kquant_seg64.h"

namespace eahmmf {

constexpr int kThreads = 512;
constexpr int kWaves = kThreads / 64;
constexpr int kAWaves = 4;  // waves 0-3: gate/up passes; waves 4-7: down staging
constexpr int kAThreads = 64 * kAWaves;
constexpr int kMaxD = 4096;
constexpr int kMaxE = 256;
constexpr int kMaxHP = 4096;     // values of h held per partition
constexpr int kMaxPart = 2048;   // (row, segment) partials of one round
constexpr int kMaxHW = 128;      // (expert, row) pairs one workgroup computes
constexpr int NPD = 2;           // phase-B tasks each B wave decodes before the barrier
constexpr int kSlotA = 20 * 1024;   // LDS ring of one A wave
constexpr int kStageB = 40 * 1024;  // LDS for one round of down rows
constexpr int kDmaB = kStageB / 1024 / (kWaves - kAWaves);  // round-0 down copies per B wave

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

constexpr int kSyncErr = kSyncFlagWord;  // error word: epoch of the last launch whose wait gave up

// Kernel arguments.  The kernel rereads fields from the argument block where
// it uses them, so the fields every launch uses are packed into the first
// three 64-byte lines: the shape as ints, the knobs in one flags word.
struct FusedArgs {
    int D, FF, grb, urb, drb;  // shape: model width, expert FF, gate/up/down row bytes
    int k, n_expert, mode;     // mode 0: direct slots, 1: logits + table, 2: ids/w + table, 3: router + table
    int np, m;                 // partitions and workgroups per partition
    int rows_b;                // output rows per workgroup (chunk)
    int rows_a;                // (expert, row) pairs of gate/up per workgroup, a multiple of the A lane groups
    int rows_round;            // output rows staged per phase-B round
    int stride_b;              // LDS bytes per expert in the phase-B stage (multiple of 1024)
    int rank_shift, rank_c;    // routing: log2 of the threads per candidate, keys each of them compares
    int local_l2;              // 1: partition p runs on XCD p, so h is exchanged through that XCD's L2
    // bits 0-3: 1 + the partition whose h words are never stored (test knob, 0: none); bit 4: rank by
    // ticket (else by b / np); bit 5: h words device-coherent also within an XCD; bits 8-31: polls
    // before a wait gives up (0: kDefaultSpinLimit)
    unsigned flags;
    unsigned epoch;        // launch number (>= 1): the high word of this launch's exchange words
    unsigned ticket_base;  // local_l2: tickets every XCD's counter handed out before this launch
    const ExpertEntry* table;
    const float* logits;
    const int* ids_in;
    const float* w_in;
    int* ids_out;
    float* w_out;
    const float* x;
    float* y;
    uint64_t* hx;     // k * FF words: h value bits | epoch << 32
    uint64_t* ypart;  // np * D words: partial value bits | epoch << 32
    unsigned* sync;
    // mode 3 (routing from the residual stream): F32 router rows [n_expert][D],
    // the input's RMSNorm weights (null: the input is used as it is) and eps,
    // optional outputs of block 0 (the normalized input, the logits), and the
    // router dot's slices per logit
    const float* router;
    const float* norm_w;
    float eps;
    int rslices;
    float* xn_out;
    float* logits_out;
    // last: read only in mode 0
    DecodeSlots direct;
};
// Exchange words of mode 3's router partials (value | epoch << 32), in the
// launch's sync area from word kLogitWord (64-bit aligned), one per (logit,
// slice): at most kMaxLogitWords.
constexpr int kLogitWord = 2048;
constexpr int kMaxLogitWords = 512;
static_assert(kLogitWord + 2 * kMaxLogitWords <= kSyncWords, "router exchange inside the sync area");
constexpr unsigned kDefaultSpinLimit = 1u << 18;  // polls: a wait gives up after about 0.1-0.3 s
constexpr unsigned kFlagTicket = 1u << 4, kFlagHAgent = 1u << 5, kFlagTicketL2 = 1u << 6;
__device__ __forceinline__ unsigned spin_limit_of(unsigned flags) {
    const unsigned v = flags >> 8;
    return v ? v : kDefaultSpinLimit;
}

// Exchange words: a float and the launch epoch in one 64-bit word, so that a
// reader polls the data itself.  Stores are single-copy atomic; a reader in
// another XCD needs the device-coherent (sc1) store, a reader in the same XCD
// finds a plain store in the shared L2.  Reads are agent-scope (sc1) loads:
// they miss the CU's L1 and never see a stale line (measured: a completed
// store from another CU of the XCD is seen within ~0.2 us).
__device__ __forceinline__ uint64_t epoch_word(float v, unsigned epoch) {
    return ((uint64_t)epoch << 32) | __builtin_bit_cast(uint32_t, v);
}
__device__ __forceinline__ void store_word(uint64_t* p, uint64_t w, bool device) {
    if (device)
        __hip_atomic_store(p, w, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    else
        __hip_atomic_store(p, w, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
}
__device__ __forceinline__ uint64_t load_word(const uint64_t* p) {
    return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

__device__ __forceinline__ void raise_error(unsigned* sync, unsigned epoch) {
    __hip_atomic_store(&sync[kSyncErr], epoch, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
// The error word is read on every (kErrPoll + 1)-th poll of a wait only: a
// load of it on every poll lengthened each poll (a line nobody else touches,
// read device-coherent), and a launch whose wait gave up still ends within
// kErrPoll + 1 polls of every other wait.
constexpr unsigned kErrPoll = 31;
__device__ __forceinline__ unsigned load_error(const unsigned* sync) {
    return __hip_atomic_load(&sync[kSyncErr], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// XCD (XCC) the calling wave runs on: hardware register HW_REG_XCC_ID (20),
// bits [3:0].
__device__ __forceinline__ int xcc_id() { return (int)(__builtin_amdgcn_s_getreg(20 | (0 << 6) | (3 << 11)) & 0xF); }

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
    ExpertEntry table[kMaxE];
    alignas(16) uint64_t rkey[kMaxE];  // routing order keys
    float slot_key[kMaxSlots];
    int slot_id[kMaxSlots];
    const uint8_t* gate[kMaxSlots];
    const uint8_t* up[kMaxSlots];
    const uint8_t* down[kMaxSlots];
    float w[kMaxSlots];
    unsigned a_issued;  // A waves whose first passes are issued (the down copies go out after them)
    unsigned xs_read;   // A waves that have read their activation levels
    unsigned b_landed;  // B waves whose round-0 down copies have landed
    unsigned ticket;    // local_l2: this workgroup's rank in its XCD's arrival order
    unsigned bad;       // a wait of this workgroup gave up: its results are NaN
    float red[kWaves];  // mode 3: per-wave sums of squares, then router partials
};

// Activation levels.  n fp32 values (n % 64 == 0) become 3 int8 levels per
// 64-value segment plus 32-value sums, in LDS: level lv of value i at
// q + lv*qstride + i, scale of segment g at sc + lv*scstride + g, sum of
// values [32c, 32c+32) at s32[c].  Eight adjacent threads share a segment,
// eight values each.

// This thread's eight values of segment seg (zeros when inactive).
__device__ __forceinline__ void load8(const float* src, int seg, int part, bool active, float (&v)[8]) {
    if (active) {
        const float* sp = src + seg * 64 + part * 8;
        const float4 v0 = reinterpret_cast<const float4*>(sp)[0], v1 = reinterpret_cast<const float4*>(sp)[1];
        v[0] = v0.x; v[1] = v0.y; v[2] = v0.z; v[3] = v0.w;
        v[4] = v1.x; v[5] = v1.y; v[6] = v1.z; v[7] = v1.w;
    } else {
#pragma unroll
        for (int i = 0; i < 8; i++) v[i] = 0.f;
    }
}

// The same from exchange words, polled until all eight carry this launch's
// epoch.  Bounded: after spin_limit polls, or once the error word holds this
// epoch, it gives up (raising the error) and returns false.
__device__ __forceinline__ bool load8_words(const uint64_t* src, int seg, int part, bool active, unsigned epoch,
                                            unsigned* sync, unsigned spin_limit, float (&v)[8]) {
    uint64_t w[8];
#pragma unroll
    for (int i = 0; i < 8; i++) w[i] = 0;
    bool good = true;
    if (active) {
        const uint64_t* sp = src + seg * 64 + part * 8;
        for (unsigned spins = 0;; spins++) {
#pragma unroll
            for (int i = 0; i < 8; i++) w[i] = load_word(sp + i);
            const unsigned err = (spins & kErrPoll) == kErrPoll ? load_error(sync) : 0u;
            bool ok = true;
#pragma unroll
            for (int i = 0; i < 8; i++) ok &= (unsigned)(w[i] >> 32) == epoch;
            if (ok) break;
            if (err == epoch || spins >= spin_limit) {
                raise_error(sync, epoch);
                good = false;
                break;
            }
            __builtin_amdgcn_s_sleep(1);
        }
    }
#pragma unroll
    for (int i = 0; i < 8; i++) v[i] = __builtin_bit_cast(float, (uint32_t)w[i]);
    return good;
}

// Levels of n values held as exchange words, by threads t in [0, nthr) (nthr
// a multiple of 64).  False if a wait gave up.
__device__ bool quantize_words(const uint64_t* src, int n, unsigned epoch, unsigned* sync, unsigned spin_limit,
                               int8_t* q, int qstride, float* sc, int scstride, float* s32, int t, int nthr) {
    const int nseg = n / 64;
    bool good = true;
    for (int base = 0; base < nseg; base += nthr / 8) {
        const int seg = base + t / 8, part = t % 8;
        float v[8];
        good &= load8_words(src, seg, part, seg < nseg, epoch, sync, spin_limit, v);
        quantize8(v, seg, part, seg < nseg, q, qstride, sc, scstride, s32);
    }
    return good;
}

// The activation levels of segment g (64 values) held by one lane.  All
// fifteen LDS reads are in flight together: one asm statement takes every
// loaded register, so the compiler cannot pair each read with its uses (it
// did, waiting for one or two reads at a time, which made a phase-B task
// twelve dependent LDS round trips long).
using u32x4 = unsigned __attribute__((ext_vector_type(4)));
__device__ __forceinline__ void load_xseg(XSeg& xs, const int8_t* q, int qstride, const float* sc, int scstride,
                                          const float* s32, int g) {
    u32x4 v[kLevels][4];
    float f[kLevels + 2];
#pragma unroll
    for (int lv = 0; lv < kLevels; lv++) {
        const u32x4* xp = reinterpret_cast<const u32x4*>(q + lv * qstride + g * 64);
#pragma unroll
        for (int c = 0; c < 4; c++) v[lv][c] = xp[c];
        f[lv] = sc[lv * scstride + g];
    }
    f[kLevels] = s32[2 * g];
    f[kLevels + 1] = s32[2 * g + 1];
    static_assert(kLevels == 3, "one operand per loaded register below");
    asm volatile(""
                 : "+v"(v[0][0]), "+v"(v[0][1]), "+v"(v[0][2]), "+v"(v[0][3]), "+v"(v[1][0]), "+v"(v[1][1]),
                   "+v"(v[1][2]), "+v"(v[1][3]), "+v"(v[2][0]), "+v"(v[2][1]), "+v"(v[2][2]), "+v"(v[2][3]),
                   "+v"(f[0]), "+v"(f[1]), "+v"(f[2]), "+v"(f[3]), "+v"(f[4]));
#pragma unroll
    for (int lv = 0; lv < kLevels; lv++) {
#pragma unroll
        for (int c = 0; c < 4; c++) {
            xs.q[lv][4 * c] = (int)v[lv][c].x;
            xs.q[lv][4 * c + 1] = (int)v[lv][c].y;
            xs.q[lv][4 * c + 2] = (int)v[lv][c].z;
            xs.q[lv][4 * c + 3] = (int)v[lv][c].w;
        }
        xs.s[lv] = f[lv];
    }
    xs.sum32[0] = f[kLevels];
    xs.sum32[1] = f[kLevels + 1];
}

// Routing, step 1 (wave 0): the expert table into LDS and every candidate's
// order key.  e_i = expf(l_i - max) bit for bit as the reference's libm forms
// it (expf_ref.h; the table entry 2^(k/32) comes from the lane holding it);
// the key holds e_i's bits + 1 in the high word (non-negative floats order as
// their bits; 0 for a NaN e_i and for ids past n_expert up to 256) and ~i in
// the low word, so keys are distinct and order exactly as (e desc, id asc).
// Stores the eight values of part `part` (values 8 part .. 8 part + 7).
__device__ __forceinline__ void store8(float* dst, int part, const float (&v)[8]) {
    float4* d = reinterpret_cast<float4*>(dst + part * 8);
    d[0] = make_float4(v[0], v[1], v[2], v[3]);
    d[1] = make_float4(v[4], v[5], v[6], v[7]);
}

// Mode 3 (wave 0): candidate lane + 64 c's logit, the sum in slice order of
// its router units' exchange words, polled until every word carries this
// launch's epoch.  Bounded like every wait: false (logits NaN) when it gives
// up.  S <= kMaxRouterSlices.
constexpr int kMaxRouterSlices = 8;
__device__ bool route_logits(const FusedArgs& a, int lane, float (&l)[4]) {
    const int S = a.rslices, n = a.n_expert;
    const uint64_t* lx = reinterpret_cast<const uint64_t*>(a.sync + kLogitWord);
    const unsigned lim = spin_limit_of(a.flags);
    uint64_t w[4][kMaxRouterSlices];
    bool good = true;
    for (unsigned spins = 0;; spins++) {
        bool ok = true;
#pragma unroll
        for (int c = 0; c < 4; c++) {
            const int id = lane + 64 * c;
#pragma unroll
            for (int u = 0; u < kMaxRouterSlices; u++) {
                w[c][u] = id < n && u < S ? load_word(&lx[id * S + u]) : ((uint64_t)a.epoch << 32);
                ok &= (unsigned)(w[c][u] >> 32) == a.epoch;
            }
        }
        const unsigned err = (spins & kErrPoll) == kErrPoll ? load_error(a.sync) : 0u;
        if (__builtin_amdgcn_ballot_w64(!ok) == 0) break;
        if (err == a.epoch || spins >= lim) {
            if (lane == 0) raise_error(a.sync, a.epoch);
            good = false;
            break;
        }
        __builtin_amdgcn_s_sleep(1);
    }
#pragma unroll
    for (int c = 0; c < 4; c++) {
        const int id = lane + 64 * c;
        float v = 0.f;
#pragma unroll
        for (int u = 0; u < kMaxRouterSlices; u++)
            if (u < S) v += __builtin_bit_cast(float, (uint32_t)w[c][u]);
        l[c] = id >= n ? -INFINITY : (good ? v : __builtin_nanf(""));
    }
    return good;
}

// Candidate i = lane + 64 c's logit and table entry (ids past n_expert up
// to 256: -inf and no expert).
__device__ __forceinline__ void route_load_table(const FusedArgs& a, int lane, ExpertEntry (&ent)[4]) {
#pragma unroll
    for (int c = 0; c < 4; c++) {
        const int id = lane + 64 * c;
        ent[c] = id < a.n_expert ? a.table[id] : ExpertEntry{nullptr, nullptr, nullptr};
    }
}

// Routing, step 1 (wave 0): the expert table into LDS and every candidate's
// order key.  e_i = expf(l_i - max) bit for bit as the reference's libm forms
// it (expf_ref.h; the table entry 2^(k/32) comes from the lane holding it);
// the key holds e_i's bits + 1 in the high word (non-negative floats order as
// their bits; 0 for a NaN e_i and for ids past n_expert up to 256) and ~i in
// the low word, so keys are distinct and order exactly as (e desc, id asc).
__device__ void route_keys_from(const FusedArgs& a, FusedLds& L, int lane, const float (&l)[4],
                                const ExpertEntry (&ent)[4]) {
    const int n = a.n_expert;
    const uint64_t tab = exp2_tab((uint32_t)lane);  // lanes 32-63 repeat lanes 0-31
    float mx = fmaxf(fmaxf(l[0], l[1]), fmaxf(l[2], l[3]));
    mx = dpp_max(mx);
    const int nc = (n + 63) / 64;  // chunks of 64 ids holding candidates (wave-uniform)
#pragma unroll
    for (int c = 0; c < 4; c++) {
        const int id = lane + 64 * c;
        if (c >= nc) {  // no candidate in this chunk: its keys rank last
            L.rkey[id] = (uint64_t)(uint32_t)~id;
            continue;
        }
        double rr;
        uint64_t ki;
        float sp;
        const bool special = expf_ref_reduce(l[c] - mx, &rr, &ki, &sp);
        const int src = (int)(ki & 31u);  // every lane takes part in the exchange
        const uint32_t tlo = (uint32_t)__shfl((int)(uint32_t)tab, src, 64);
        const uint32_t thi = (uint32_t)__shfl((int)(uint32_t)(tab >> 32), src, 64);
        const float e = special ? sp : expf_ref_finish(rr, ki, ((uint64_t)thi << 32) | tlo);
        const uint32_t hi = (id < n && e == e) ? __builtin_bit_cast(uint32_t, e) + 1u : 0u;
        L.rkey[id] = ((uint64_t)hi << 32) | (uint32_t)~id;
        if (id < n) L.table[id] = ent[c];
    }
}

// The same from logits in memory (mode 1): every global load of the step
// goes out before the first use.
template <class After>
__device__ void route_keys(const FusedArgs& a, FusedLds& L, int lane, After after_loads) {
    float l[4];
    ExpertEntry ent[4];
#pragma unroll
    for (int c = 0; c < 4; c++) {
        const int id = lane + 64 * c;
        l[c] = id < a.n_expert ? a.logits[id] : -INFINITY;
        ent[c] = id < a.n_expert ? a.table[id] : ExpertEntry{nullptr, nullptr, nullptr};
    }
    after_loads();
    route_keys_from(a, L, lane, l, ent);
}

// acc + (key (hi, lo) > ki) for 64-bit keys, as the borrow out of ki - key:
// three full-rate VALU instructions (a 64-bit compare is not full rate).  The
// borrow lives in an SGPR pair of its own, so independent accumulators are
// independent chains.
__device__ __forceinline__ int add_if_greater(int acc, uint32_t lo, uint32_t hi, uint64_t ki) {
    int r;
    uint32_t t;
    uint64_t c;
    asm("v_sub_co_u32 %1, %2, %3, %4\n\t"
        "v_subb_co_u32 %1, %2, %5, %6, %2\n\t"
        "v_addc_co_u32 %0, %2, 0, %7, %2"
        : "=v"(r), "=&v"(t), "=&s"(c)
        : "v"((uint32_t)ki), "v"(lo), "v"((uint32_t)(ki >> 32)), "v"(hi), "v"(acc));
    return r;
}

// The number of keys larger than ki among keys[0, T C) seen by thread part
// of T: the pairs at 2 part + 2 T j (C even; N reads in flight, four
// independent chains) or the keys at part + T j (C odd).  The T threads of a
// candidate read adjacent banks and every candidate of a wave reads the same
// words (broadcast).
template <int N>
__device__ __forceinline__ void count_pairs(const uint64_t* kp, int stride, int& j, int P, uint64_t ki,
                                            int (&acc)[4]) {
    for (; j + N <= P; j += N) {
        uint4 v[N];
#pragma unroll
        for (int u = 0; u < N; u++) v[u] = *reinterpret_cast<const uint4*>(kp + stride * (j + u));
#pragma unroll
        for (int u = 0; u < N; u++) {
            acc[(2 * u) & 3] = add_if_greater(acc[(2 * u) & 3], v[u].x, v[u].y, ki);
            acc[(2 * u + 1) & 3] = add_if_greater(acc[(2 * u + 1) & 3], v[u].z, v[u].w, ki);
        }
    }
}

__device__ __forceinline__ int count_greater(const uint64_t* keys, int T, int part, int C, uint64_t ki) {
    if ((C & 1) == 0) {
        int acc[4] = {0, 0, 0, 0};
        int j = 0;
        count_pairs<8>(keys + 2 * part, 2 * T, j, C / 2, ki, acc);
        count_pairs<4>(keys + 2 * part, 2 * T, j, C / 2, ki, acc);
        count_pairs<2>(keys + 2 * part, 2 * T, j, C / 2, ki, acc);
        count_pairs<1>(keys + 2 * part, 2 * T, j, C / 2, ki, acc);
        return (acc[0] + acc[1]) + (acc[2] + acc[3]);
    }
    int ahead = 0;
    for (int j = 0; j < C; j++) {
        const uint64_t kj = keys[part + T * j];
        ahead = add_if_greater(ahead, (uint32_t)kj, (uint32_t)(kj >> 32), ki);
    }
    return ahead;
}

// Slot r of the routing: the candidate's softmax numerator (its key's high
// word less one), id and weight pointers, or an empty slot for a NaN logit
// (high word 0).
__device__ __forceinline__ void put_slot(FusedLds& L, int r, uint64_t key, int id, const ExpertEntry& ent) {
    const bool ok = (uint32_t)(key >> 32) != 0u;
    L.slot_key[r] = ok ? __builtin_bit_cast(float, (uint32_t)(key >> 32) - 1u) : -1.0f;
    L.slot_id[r] = ok ? id : -1;
    L.gate[r] = ok ? ent.gate : nullptr;
    L.up[r] = ok ? ent.up : nullptr;
    L.down[r] = ok ? ent.down : nullptr;
}

// Routing, step 2 (all threads): candidate i's rank in the reference's order
// (qwen3moe.cpp:1016) is the number of larger keys; ranks are distinct, so
// the top k fill slots 0..k-1.  T = 2^rank_shift adjacent threads count over
// C = rank_c keys each, and the group's last thread writes the slot.
__device__ void route_rank(const FusedArgs& a, FusedLds& L, int tid) {
    const int n = a.n_expert;
    const int T = 1 << a.rank_shift;
    const int i = tid >> a.rank_shift, part = tid & (T - 1);
    int ahead = 0;
    uint64_t ki = 0;
    ExpertEntry ent{nullptr, nullptr, nullptr};
    if (i < n) {
        ki = L.rkey[i];
        if (part == T - 1) ent = L.table[i];  // read with the keys, used by the slot's writer
        ahead = count_greater(L.rkey, T, part, a.rank_c, ki);
    }
    ahead = group_sum_i(ahead, T);
    if (i < n && part == T - 1 && ahead < a.k) put_slot(L, ahead, ki, i, ent);
}

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

// Weight pointers of slot j (matrix c: 0 gate, 1 up, 2 down), null for a
// slot without an expert.  Every mode fills them before the routing barrier
// (the routing writes them with the slot), so reading them is one LDS round
// trip for all six.
__device__ __forceinline__ const uint8_t* slot_ptr(const FusedLds& L, int j, int c) {
    return c == 0 ? L.gate[j] : (c == 1 ? L.up[j] : L.down[j]);
}

// ypart[0][r] + ... + ypart[np-1][r] (np <= 8) in partition order, once
// every partial carries this launch's epoch (all loads of a poll in flight
// together).  Bounded like every wait: NaN when it gives up.
__device__ __forceinline__ float reduce_row(const uint64_t* ypart, int D, int r, int np, unsigned epoch,
                                            unsigned* sync, unsigned spin_limit) {
    uint64_t v[8];
    for (unsigned spins = 0;; spins++) {
#pragma unroll
        for (int pp = 0; pp < 8; pp++) v[pp] = pp < np ? load_word(&ypart[pp * D + r]) : ((uint64_t)epoch << 32);
        const unsigned err = (spins & kErrPoll) == kErrPoll ? load_error(sync) : 0u;
        bool ok = true;
#pragma unroll
        for (int pp = 0; pp < 8; pp++) ok &= (unsigned)(v[pp] >> 32) == epoch;
        if (ok) break;
        if (err == epoch || spins >= spin_limit) {
            raise_error(sync, epoch);
            return __builtin_nanf("");
        }
        __builtin_amdgcn_s_sleep(1);
    }
    float t = 0.f;
#pragma unroll
    for (int pp = 0; pp < 8; pp++)
        if (pp < np) t += __builtin_bit_cast(float, (uint32_t)v[pp]);
    return t;
}

// vmcnt(n * NI + EXTRA) for a run-time n in [0, 2].
template <int NI, int EXTRA>
__device__ __forceinline__ void wait_passes(int n) {
    if (n <= 0) wait_vm_upto<EXTRA>();
    else if (n == 1) wait_vm_upto<NI + EXTRA>();
    else wait_vm_upto<2 * NI + EXTRA>();
}

// Geometry of A pass pp of a wave: GW consecutive (expert, row) pairs from
// t0; nr of them are real rows of partition expert e starting at row f0; g
// and u are where the gate and up copies start.
struct PassRows {
    int t0, nr, e, f0;
    bool ok;
    const uint8_t* g;
    const uint8_t* u;
};

// Workgroup barrier that waits for this wave's LDS operations only
// (lgkmcnt 0; vmcnt 63 and expcnt 7 leave copies in flight).
__device__ __forceinline__ void barrier_lds() {
    __atomic_signal_fence(__ATOMIC_SEQ_CST);
    __builtin_amdgcn_s_waitcnt(0xC07F);
    __builtin_amdgcn_s_barrier();
    __atomic_signal_fence(__ATOMIC_SEQ_CST);
}

// LDS flag or counter of the workgroup reaching v (acquire; bounded: the
// waves it waits for always progress).
__device__ __forceinline__ void wait_lds(const unsigned* c, unsigned v) {
    for (unsigned spins = 0; spins < (1u << 20); spins++) {
        if (__hip_atomic_load(c, __ATOMIC_ACQUIRE, __HIP_MEMORY_SCOPE_WORKGROUP) >= v) break;
        __builtin_amdgcn_s_sleep(1);
    }
}

// RT: the kernel runs mode 3 (routing from the residual stream); the other
// modes use RT = false instantiations, whose code carries none of it.
template <int LA, int GT, int UT, int DT, bool RT>
__device__ void fused_body(const FusedArgs& a, FusedLds& L) {
    constexpr int GW = 64 / LA;        // lane groups per wave = rows per pass
    constexpr int GA = kAWaves * GW;   // rows per pass of the four A waves
    static_assert(GT == UT, "gate and up share a format");
    using PA = PassA<GT>;
    constexpr int NPA = PA::n;
    const int tid = threadIdx.x;
    const int wave = __builtin_amdgcn_readfirstlane(tid / 64), lane = tid % 64;
    const int D = a.D, FF = a.FF, k = a.k;
    const int np = a.np;
    const int xcc = a.local_l2 ? xcc_id() : 0;
    const int p = a.local_l2 ? xcc : (int)blockIdx.x % np;
    const int ep = k / np;  // experts per partition (1 or 2)
    const int segB = FF / 64;
    const int drb = a.drb;
    // h words read in other XCDs, or forced coherent
    const bool device_words = !a.local_l2 || (a.flags & kFlagHAgent);
    // the XCD-local rank by ticket: lane 0 of wave 0 takes it after the
    // routing's loads are issued (memory operations complete in order, so a
    // wait for those loads does not wait for it) and publishes it after the
    // rank, keeping its latency off the routing's path
    const bool use_ticket = a.local_l2 && (a.flags & kFlagTicket) && xcc < np;
    unsigned ticket = 0;
    auto take_ticket = [&]() {
        if (use_ticket && tid == 0) {
            if (a.flags & kFlagTicketL2)
                ticket = __hip_atomic_fetch_add(&a.sync[kTicketWord + kTicketStride * xcc], 1u, __ATOMIC_RELAXED,
                                                __HIP_MEMORY_SCOPE_WORKGROUP);
            else
                ticket = __hip_atomic_fetch_add(&a.sync[kTicketWord + kTicketStride * xcc], 1u, __ATOMIC_RELAXED,
                                                __HIP_MEMORY_SCOPE_AGENT);
        }
    };
    const bool routes = RT || a.mode == 1;  // wave 0 routes (and takes the ticket after its loads)
    if (!routes) take_ticket();

    // ---- 1. routing / slots and activation levels
    // x in parts of eight values, loaded first so that their latency overlaps
    // the routing's; with routing, threads 64.. take the parts (two rounds
    // for D > 3584) while wave 0 forms the keys
    static_assert(kMaxD / 8 <= 2 * (kThreads - 64), "two rounds of x parts");
    const int xt0 = routes ? 64 : 0, xnt = kThreads - xt0, nxp = D / 8;
    const int xp = tid - xt0;
    float xv[8];
    load8(a.x, xp / 8, xp % 8, xp >= 0 && xp < nxp, xv);
    if (wave == 0) {
        if (lane == 0) {
            L.a_issued = 0u;
            L.xs_read = 0u;
            L.b_landed = 0u;
            L.bad = 0u;
        }
        if (routes) {
            // ranks are a permutation of 0..n_expert-1, so the routing
            // writes the slots below n_expert and these defaults the rest
            if (lane >= a.n_expert && lane < k) {
                L.slot_key[lane] = -1.0f;
                L.slot_id[lane] = -1;
                L.gate[lane] = L.up[lane] = L.down[lane] = nullptr;
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
    if (wave == 0 && a.mode == 1) route_keys(a, L, lane, take_ticket);
    if (tid == 0 && !routes) L.ticket = ticket - a.ticket_base;
    const int xp2 = xp + xnt;
    const bool round2 = xp >= 0 && wave * 64 - xt0 + xnt < nxp;  // wave-uniform: parts in the second round
    float xv2[8];  // the second round's values (D > 3584 with routing)
    if constexpr (RT) {
        // ---- routing from the residual stream: RMSNorm of x, the router
        // matmul split over every workgroup (one (logit, slice) unit each,
        // published as exchange words), then every workgroup's wave 0 reads
        // all units and routes.  Replaces a router launch ahead of the block.
        ExpertEntry ent[4];
        if (wave == 0) route_load_table(a, lane, ent);
        float nw[8], nw2[8], wr[8], wr2[8];
        const int S = a.rslices, span = D / S;
        const int unit = (int)blockIdx.x, ue = unit / S, us = unit % S;
        const bool has_unit = unit < a.n_expert * S;
        const float* wrow = a.router + (size_t)(has_unit ? ue : 0) * D;
        auto in_slice = [&](int part) { return has_unit && part < nxp && part * 8 / span == us; };
        load8(a.x, xp2 / 8, xp2 % 8, round2 && xp2 < nxp, xv2);
        load8(a.norm_w ? a.norm_w : a.x, xp / 8, xp % 8, a.norm_w && xp >= 0 && xp < nxp, nw);
        load8(a.norm_w ? a.norm_w : a.x, xp2 / 8, xp2 % 8, a.norm_w && round2 && xp2 < nxp, nw2);
        load8(wrow, xp / 8, xp % 8, xp >= 0 && in_slice(xp), wr);
        load8(wrow, xp2 / 8, xp2 % 8, round2 && in_slice(xp2), wr2);
        float ss = 0.f;
#pragma unroll
        for (int i = 0; i < 8; i++) ss += xv[i] * xv[i] + xv2[i] * xv2[i];
        ss = group_sum_all<64>(ss);
        if (lane == 0) L.red[wave] = ss;
        barrier_lds();
        float tot = 0.f;
#pragma unroll
        for (int w = 0; w < kWaves; w++) tot += L.red[w];
        const float sc = a.norm_w ? 1.0f / sqrtf(tot / (float)D + a.eps) : 1.0f;
        float dot = 0.f;
#pragma unroll
        for (int i = 0; i < 8; i++) {
            if (a.norm_w) {
                xv[i] = xv[i] * sc * nw[i];
                xv2[i] = xv2[i] * sc * nw2[i];
            }
            dot = __builtin_fmaf(xv[i], wr[i], dot);
            dot = __builtin_fmaf(xv2[i], wr2[i], dot);
        }
        if (blockIdx.x == 0 && a.xn_out && xp >= 0) {
            if (xp < nxp) store8(a.xn_out, xp, xv);
            if (round2 && xp2 < nxp) store8(a.xn_out, xp2, xv2);
        }
        dot = group_sum_all<64>(dot);
        barrier_lds();  // every wave has read the sums of squares
        if (lane == 0) L.red[wave] = dot;
        barrier_lds();
        if (wave == 0) {
            if (lane == 0 && has_unit) {
                float part = 0.f;
#pragma unroll
                for (int w = 0; w < kWaves; w++) part += L.red[w];
                uint64_t* lx = reinterpret_cast<uint64_t*>(a.sync + kLogitWord);
                __hip_atomic_store(&lx[unit], epoch_word(part, a.epoch), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            }
            take_ticket();
            float l[4];
            if (!route_logits(a, lane, l) && lane == 0) L.bad = 1u;
            if (blockIdx.x == 0 && a.logits_out) {
#pragma unroll
                for (int c = 0; c < 4; c++)
                    if (lane + 64 * c < a.n_expert) a.logits_out[lane + 64 * c] = l[c];
            }
            route_keys_from(a, L, lane, l, ent);
        }
    }
    if (xp >= 0) {  // wave-uniform
        quantize8(xv, xp / 8, xp % 8, xp < nxp, &L.a.xq[0][0], kMaxD, &L.a.xsc[0][0], kMaxD / 64, L.a.xs32);
        if (round2) {
            if constexpr (!RT) load8(a.x, xp2 / 8, xp2 % 8, xp2 < nxp, xv2);
            quantize8(xv2, xp2 / 8, xp2 % 8, xp2 < nxp, &L.a.xq[0][0], kMaxD, &L.a.xsc[0][0], kMaxD / 64, L.a.xs32);
        }
    }
    if (routes) {
        // LDS only: keys, x levels (__syncthreads would also wait for the ticket)
        barrier_lds();
        route_rank(a, L, tid);
        if (tid == 0) L.ticket = ticket - a.ticket_base;
    }
    __syncthreads();
    // rank inside the partition; a workgroup outside the launch's layout (an
    // XCD that received more than its share, or an XCC id past the
    // partitions) raises the error and leaves: the share it would have
    // computed is missing elsewhere, and those waits give up
    const int q = use_ticket ? (int)__builtin_amdgcn_readfirstlane(L.ticket) : (int)blockIdx.x / np;
    if (p >= np || q >= a.m) {
        if (tid == 0) raise_error(a.sync, a.epoch);
        return;
    }
    // output rows of this workgroup's chunk (the host gives every workgroup at least one)
    const int r_begin = q * a.rows_b;
    const int r_end = min(D, r_begin + a.rows_b);

    // weight pointers of the partition's (at most two) experts
    // (all six read at once: slot p ep + 1 < kMaxSlots exists even when unused)
    const uint8_t* sp[6];
#pragma unroll
    for (int c = 0; c < 6; c++) sp[c] = slot_ptr(L, p * ep + (c & 1), c >> 1);
    const uint8_t* gptr[2] = {sp[0], ep > 1 ? sp[1] : nullptr};
    const uint8_t* uptr[2] = {sp[2], ep > 1 ? sp[3] : nullptr};
    const uint8_t* dptr[2] = {sp[4], ep > 1 ? sp[5] : nullptr};
    // the source of copies whose bytes are never used (x: valid, 16-byte
    // aligned), held in registers rather than reloaded from the arguments
    const uint8_t* xsrc = reinterpret_cast<const uint8_t*>(a.x);
    asm volatile("" : "+s"(xsrc));

    // phase-B stage: rows [r0, r0 + rr) of the chunk, expert e of the
    // partition at stage_b + e * stride_b + (its source & 15)
    auto down_src = [&](int e, int r0) -> const uint8_t* {
        const uint8_t* dw = dptr[e];
        return dw ? dw + (size_t)(r_begin + r0) * drb : xsrc;
    };
    // global source of 1 KB stage instruction ii of expert e (lanes past the
    // end re-read the last 16 bytes)
    auto stage_src = [&](int e, int ii, int r0, int rr) -> uintptr_t {
        const uint8_t* src = down_src(e, r0);
        const int n = dptr[e] ? rr * drb : 16;
        const uintptr_t base = (uintptr_t)src & ~(uintptr_t)15;
        const int n16 = (int)(((((uintptr_t)src + (uintptr_t)n + 15) & ~(uintptr_t)15) - base) / 16);
        return base + (uintptr_t)min(ii * 64 + lane, n16 - 1) * 16;
    };
    // Phase-B rounds alternate between two stages: round i's rows sit in
    // stage_b (i even) or in the A waves' rings (i odd; free once every A
    // wave has passed the barrier after its passes), so the next round's
    // copies run while a round computes.
    auto stage_of = [&](int r0) -> uint8_t* {
        return (r0 / a.rows_round) & 1 ? &L.stage_a[0][0] : L.stage_b;
    };
    // rounds after the first: all waves copy, one 1 KB instruction each in turn
    auto stage_round = [&](int r0, int rr) {
        const int ni = a.stride_b / 1024;
        uint8_t* st = stage_of(r0);
        for (int e = 0; e < ep; e++)
            for (int i = wave; i < ni; i += kWaves) lds_dma16(stage_src(e, i, r0, rr), st + e * a.stride_b + i * 1024);
    };
    // round 0, B wave wb: exactly kDmaB instructions f = wb + 4i over the
    // experts' stage instructions in order (expert e's instruction ii lands at
    // stage_b + f KB); indices past the last real one copy 16 bytes of x into
    // the unused tail of the stage
    const int rr0 = min(a.rows_round, r_end - r_begin);
    auto stage_round0 = [&](int wb) {
        const int ni = a.stride_b / 1024;
        for (int i = 0; i < kDmaB; i++) {
            const int f = wb + (kWaves - kAWaves) * i;
            const int e = f / ni;
            const uintptr_t g = e < ep ? stage_src(e, f - e * ni, 0, rr0) : ((uintptr_t)a.x & ~(uintptr_t)15);
            lds_dma16(g, L.stage_b + f * 1024);
        }
    };

    // Phase-B tasks of a round: (expert e of the partition, 64-value segment
    // sg, 64-row block); a lane is one row.  The B waves decode their first
    // NPD tasks of round 0 into registers before the barrier.
    // When a round holds at most 32 rows (long down rows, e.g. 1260 B at
    // FF=1536), a task is (expert, segment pair, the round's rows) instead:
    // lanes 32..63 take the pair's second segment of the same rows, so no
    // lane idles.  A lane past an odd segment count writes nothing.
    const bool half = a.rows_round <= 32;
    const int nsg = half ? (segB + 1) / 2 : segB;
    auto n_tasks = [&](int rr) { return ep * nsg * (half ? 1 : (rr + 63) / 64); };
    const int n_tasks0 = n_tasks(rr0);
    struct BTask {
        int e, sg, r;
        const uint8_t* row;
    };
    auto btask = [&](int task, int rr, int r0) {
        const int nrb = half ? 1 : (rr + 63) / 64;
        BTask t;
        t.e = task / (nsg * nrb);
        const int rest = task - t.e * (nsg * nrb);
        const int g = rest / nrb;
        if (half) {
            t.sg = 2 * g + (lane >> 5);
            t.r = lane & 31;
            if (t.sg >= segB) {
                t.sg = segB - 1;
                t.r = kThreads;  // beyond every round: no partial is written
            }
        } else {
            t.sg = g;
            t.r = (rest - g * nrb) * 64 + lane;
        }
        const uint8_t* src = down_src(t.e, r0);  // rows [r0, r0 + rr) of the chunk are staged
        t.row = stage_of(r0) + t.e * a.stride_b + ((uintptr_t)src & 15) + min(t.r, rr - 1) * drb;
        return t;
    };

    // ---- 2. passes.  Pass pp of A wave w: GW consecutive (expert, row)
    // pairs from t0 = ra0 + pp * GA + w * GW, gate and up rows both
    const int gl = lane / LA, li = lane % LA;
    const int rows_a = ep * FF;
    const int ra0 = min(rows_a, q * a.rows_a), ra1 = min(rows_a, ra0 + a.rows_a);
    const int npass = (ra1 - ra0 + GA - 1) / GA;
    const int grb = a.grb, urb = a.urb;
    auto rows_of = [&](int pp) {
        PassRows r;
        r.t0 = ra0 + pp * GA + wave * GW;
        r.nr = max(0, min(GW, ra1 - r.t0));
        const int tt = min(r.t0, rows_a - 1);
        r.e = tt >= FF ? 1 : 0;
        r.f0 = tt - r.e * FF;
        const uint8_t* gw = gptr[r.e];
        const uint8_t* uw = uptr[r.e];
        r.ok = (r.nr > 0) & (gw != nullptr) & (uw != nullptr);
        // a pass without weights copies 16 bytes of x instead; nothing of it is used
        r.g = r.ok ? gw + (size_t)r.f0 * grb : xsrc;
        r.u = r.ok ? uw + (size_t)r.f0 * urb : xsrc;
        return r;
    };

    // What phase B and the combine read from the kernel arguments, loaded by
    // each wave before the barrier that starts phase B and held in scalar
    // registers: the compiler otherwise reloads them where they are used,
    // and after the barrier those loads miss and wait (two dependent round
    // trips ahead of the first phase-B task).
    struct Late {
        const FusedArgs& a;
        unsigned epoch, flags;
        int rows_round, stride_b, D, np;
        uint64_t* ypart;
        float* y;
        unsigned* sync;
        __device__ __forceinline__ void load() {
            epoch = a.epoch;
            flags = a.flags;
            rows_round = a.rows_round;
            stride_b = a.stride_b;
            D = a.D;
            np = a.np;
            ypart = a.ypart;
            y = a.y;
            sync = a.sync;
            asm volatile(""
                         : "+s"(epoch), "+s"(flags), "+s"(rows_round), "+s"(stride_b), "+s"(D), "+s"(np), "+s"(ypart),
                           "+s"(y), "+s"(sync));
        }
    } late{a};
    SegCodes<DT> pre[NPD];  // B waves: their first phase-B tasks, decoded
    BTask tb[NPD];          // and where those tasks are
    // A waves: the round-0 tasks after the B waves' (from (8 - 4) NPD + wave)
    const int task_a = (kWaves - kAWaves) * NPD + wave;
    if (wave < kAWaves) {
        // ---- 2A. this wave's passes through its LDS ring.  Every load the
        // compiler issued is retired first: the copies below are invisible to
        // it, and a wait it inserts later for one of its own loads (for
        // instance before reusing the load's register) would also wait for
        // every copy in flight.
        wait_vm();
        auto slot_of = [&](int pp) { return L.stage_a[wave] + (pp % NPA) * PA::slot; };
        auto issue = [&](int pp) {
            const PassRows r = rows_of(pp);
            uint8_t* sl = slot_of(pp);
            dma_to_lds<PA::nir>(r.g, r.ok ? r.nr * grb : 16, sl, lane);
            dma_to_lds<PA::nir>(r.u, r.ok ? r.nr * urb : 16, sl + PA::nir * 1024, lane);
        };
        for (int pp = 0; pp < min(NPA, npass); pp++) issue(pp);
        if (lane == 0) __hip_atomic_fetch_add(&L.a_issued, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
        XSeg xs;  // read while the first pass is in flight
        load_xseg(xs, &L.a.xq[0][0], kMaxD, &L.a.xsc[0][0], kMaxD / 64, L.a.xs32, li);
        if (lane == 0) __hip_atomic_fetch_add(&L.xs_read, 1u, __ATOMIC_RELEASE, __HIP_MEMORY_SCOPE_WORKGROUP);
        const int goff = gl * grb, uoff = PA::nir * 1024 + gl * urb;
        for (int pp = 0; pp < npass; pp++) {
            // passes pp+1 .. are still allowed in flight: 2 * nir instructions each
            wait_passes<2 * PA::nir, 0>(min(npass - 1 - pp, NPA - 1));
            const PassRows r = rows_of(pp);
            const uint8_t* sl = slot_of(pp);
            const bool live = r.ok && gl < r.nr;
            RawSeg<GT> g;
            RawSeg<UT> u;
            g.template load<LdsLd>(live ? sl + ((uintptr_t)r.g & 15) + goff : sl, li);
            u.template load<LdsLd>(live ? sl + ((uintptr_t)r.u & 15) + uoff : sl, li);
            const float dg = group_sum<LA>(g.dot_q8(li, xs));
            const float du = group_sum<LA>(u.dot_q8(li, xs));
            // every pair of the workgroup gets a word, 0 for a slot without an expert
            if (li == LA - 1 && gl < r.nr && p + 1 != (int)(a.flags & 15u)) {
                const float hv = r.ok ? dg / (1.0f + expf(-dg)) * du : 0.f;
                store_word(&a.hx[(p * ep + r.e) * FF + r.f0 + gl], epoch_word(hv, a.epoch), device_words);
            }
            // every lane's reads of this slot have returned (their values are used above)
            if (pp + NPA < npass) issue(pp + NPA);
        }
        late.load();
        // ---- 4A. the partition's h as int8 levels, once every word carries
        // this launch's epoch (it overwrites the activation levels: every A
        // wave has read its own first).  The A waves decode their phase-B
        // tasks after the barrier: h is on the critical path, and a decode
        // ahead of the first poll (or between the poll and the barrier)
        // delayed phase B by the decode's length.
        wait_lds(&L.xs_read, (unsigned)kAWaves);
        if (!quantize_words(a.hx + p * ep * FF, ep * FF, a.epoch, a.sync, spin_limit_of(a.flags), &L.b.hq[0][0], kMaxHP,
                            &L.b.hsc[0][0], kMaxHP / 64, L.b.hs32, tid, kAThreads))
            L.bad = 1u;
    } else {
        // ---- 2B. the round-0 down rows into LDS, queued behind the A waves'
        // first passes (h, the barrier and everything after it wait on
        // gate/up first); once they land, the B waves decode their first NPD
        // phase-B tasks into registers while the A waves compute
        wait_lds(&L.a_issued, (unsigned)kAWaves);
        stage_round0(wave - kAWaves);
        if (routes && wave == kAWaves) route_weights(a, L, lane);
        wait_vm();
        if (lane == 0) __hip_atomic_fetch_add(&L.b_landed, 1u, __ATOMIC_RELEASE, __HIP_MEMORY_SCOPE_WORKGROUP);
        wait_lds(&L.b_landed, (unsigned)(kWaves - kAWaves));
#pragma unroll
        for (int i = 0; i < NPD; i++) {
            tb[i] = btask(min(wave - kAWaves + (kWaves - kAWaves) * i, n_tasks0 - 1), rr0, 0);
            RawSeg<DT> raw;
            raw.template load<LdsLd>(tb[i].row, tb[i].sg);
            pre[i] = raw.decode(tb[i].sg);
            pre[i].pin_all();  // decoded here, not after the barrier
        }
        late.load();
    }
    __syncthreads();  // the h levels and the first phase-B codes are ready

    // the router weight of each partition expert (0 for a slot without one)
    const float wgt[2] = {dptr[0] ? L.w[p * ep] : 0.f, ep > 1 && dptr[1] ? L.w[p * ep + 1] : 0.f};
    // a wait for h gave up: the partials would be computed from stale words
    const bool poisoned = L.bad != 0u;

    // Phase B rounds: every wave takes (expert, segment, 64-row block) tasks;
    // a lane is one row, so the h levels of the task are read by all lanes at
    // one address.
    const int nrows = r_end - r_begin;
    for (int r0 = 0; r0 < nrows; r0 += late.rows_round) {
        const int rr = min(late.rows_round, nrows - r0);
        if (r0 > 0) {
            // this wave's copies of the round (issued a round ago) have
            // landed; after the barrier everyone's have, and the previous
            // round's rows and partials are consumed
            wait_vm();
            __syncthreads();
        }
        {
            // the next round's copies go out now, into the stage the previous
            // round has finished with (the second round's: the A rings)
            const int r1 = r0 + late.rows_round;
            if (r1 < nrows) stage_round(r1, min(late.rows_round, nrows - r1));
        }
        auto finish = [&](const BTask& t, const SegCodes<DT>& k) {
            XSeg hs;  // the same address in every lane: one LDS broadcast per read
            load_xseg(hs, &L.b.hq[0][0], kMaxHP, &L.b.hsc[0][0], kMaxHP / 64, L.b.hs32, t.e * segB + t.sg);
            const float v = k.dot(hs);
            if (t.r < rr) L.part[__mul24(__mul24(t.e, rr) + t.r, segB) + t.sg] = wgt[t.e] * v;
        };
        int first = wave;
        if (r0 == 0) {
            if (wave >= kAWaves) {
#pragma unroll
                for (int i = 0; i < NPD; i++)
                    if (wave - kAWaves + (kWaves - kAWaves) * i < n_tasks0) finish(tb[i], pre[i]);
                first = (kWaves - kAWaves) * NPD + wave;
            } else {
                first = task_a;
            }
        }
        for (int task = first; task < n_tasks(rr); task += kWaves) {
            const BTask t = btask(task, rr, r0);
            RawSeg<DT> raw;
            raw.template load<LdsLd>(t.row, t.sg);
            finish(t, raw.decode(t.sg));
        }
        // the partials are in LDS; an LDS-only barrier leaves the next
        // round's copies in flight (__syncthreads would wait for them)
        barrier_lds();
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
            store_word(&late.ypart[p * late.D + r_begin + r0 + r], epoch_word(poisoned ? __builtin_nanf("") : v, late.epoch),
                       true);
        }
    }

    // ---- 5. workgroup q of partition q % np adds chunk q's partials into y
    if (p == q % late.np)
        for (int r = r_begin + tid; r < r_end; r += kThreads)
            late.y[r] = reduce_row(late.ypart, late.D, r, late.np, late.epoch, late.sync, spin_limit_of(late.flags));
}

template <int LA, int GT, int UT, int DT, bool RT = false>
__global__ __launch_bounds__(kThreads) void moe_decode_fused(FusedArgs a) {
    __shared__ FusedLds L;
    fused_body<LA, GT, UT, DT, RT>(a, L);
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

// Mode 3 kernels, instantiated for the expert formats of the models this
// library serves whole (Q4_K gate/up with Q6_K or Q4_K down, all-Q5_K,
// all-Q8_0); another mix routes through a router launch first.
template <int LA>
static FusedFn pick_rt_la(int gt, int ut, int dt) {
    if (gt != ut) return nullptr;
    if (gt == kQ4_K && dt == kQ6_K) return moe_decode_fused<LA, kQ4_K, kQ4_K, kQ6_K, true>;
    if (gt == kQ4_K && dt == kQ4_K) return moe_decode_fused<LA, kQ4_K, kQ4_K, kQ4_K, true>;
    if (gt == kQ5_K && dt == kQ5_K) return moe_decode_fused<LA, kQ5_K, kQ5_K, kQ5_K, true>;
    if (gt == kQ8_0 && dt == kQ8_0) return moe_decode_fused<LA, kQ8_0, kQ8_0, kQ8_0, true>;
    return nullptr;
}

static FusedFn pick_fused_rt(const MoeShape& s) {
    switch (s.D / 64) {
        case 4: return pick_rt_la<4>(s.gate_type, s.up_type, s.down_type);
        case 8: return pick_rt_la<8>(s.gate_type, s.up_type, s.down_type);
        case 16: return pick_rt_la<16>(s.gate_type, s.up_type, s.down_type);
        case 32: return pick_rt_la<32>(s.gate_type, s.up_type, s.down_type);
        case 64: return pick_rt_la<64>(s.gate_type, s.up_type, s.down_type);
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
    // more than one round: 32-row rounds, where a task's 64 lanes cover two
    // segments of the rows and none idles
    if (rr < g.rows_b && rr > 32) rr = 32;
    g.rows_round = rr;
    g.stride_b = stride(rr);
    return g;
}

// The layout fits the kernel's fixed LDS and flag arrays.
static bool fused_grid_ok(const MoeShape& s, int k, const FusedGrid& g) {
    if (g.m <= 0) return false;
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

constexpr int kXccProbe = 1024;

__global__ void xcc_probe_kernel(int* out) {
    if (threadIdx.x == 0) out[blockIdx.x] = xcc_id();
}

// One-time check per device that a launch is spread round-robin over eight
// XCDs: workgroup b on XCD (b + s) % 8 for one start s.  The XCD-local
// exchange relies only on what follows from it, that every XCD receives an
// equal share of a grid that is a multiple of 8 (the kernel ranks workgroups
// by tickets, not by their index, and raises its error word if a share is
// off).
// probe_buf: kXccProbe ints of device memory to use, or null to allocate them.
static bool xcd_round_robin(int device, int* probe_buf = nullptr) {
    static int state[64];  // 0 unknown, 1 yes, 2 no
    static std::mutex mu;
    std::lock_guard<std::mutex> lk(mu);
    if (device < 0 || device >= 64) return false;
    if (state[device]) return state[device] == 1;
    int* d = probe_buf;
    clear_stale_error();  // an earlier, unrelated failure must not read as the probe's
    if (!d && hipMalloc(&d, kXccProbe * sizeof(int)) != hipSuccess) {
        state[device] = 2;
        return false;
    }
    hipLaunchKernelGGL(xcc_probe_kernel, dim3(kXccProbe), dim3(64), 0, nullptr, d);
    int hbuf[kXccProbe];
    bool ok = hipGetLastError() == hipSuccess &&
              hipMemcpy(hbuf, d, sizeof hbuf, hipMemcpyDeviceToHost) == hipSuccess;
    if (!probe_buf) (void)hipFree(d);
    const int s = ok ? hbuf[0] : -1;
    ok = ok && s >= 0 && s < 8;
    for (int b = 0; ok && b < kXccProbe; b++) ok = hbuf[b] == (b + s) % 8;
    state[device] = ok ? 1 : 2;
    return ok;
}

int fused_exchange_probe(int device, int* probe_buf) { return xcd_round_robin(device, probe_buf) ? 1 : 0; }

int fused_exchange_mode(int device) { return xcd_round_robin(device) ? 1 : 0; }

// Test knobs (set_fused_fault_injection): 0 / -1 mean the defaults.
static unsigned g_spin_limit = 0;
static int g_drop_part = -1;

void set_fused_fault_injection(unsigned spin_limit, int drop_partition) {
    g_spin_limit = spin_limit;
    g_drop_part = drop_partition < 0 || drop_partition > 7 ? -1 : drop_partition;
}

// Launch options read once from the environment: EAHMMF_HIP_FUSED_COOP=1
// launches cooperatively (the runtime then guarantees that every workgroup is
// resident, at a measured cost of about 19 us per launch on MI355X, more
// than the kernel itself at the Qwen3-30B-A3B shape); EAHMMF_HIP_H_AGENT=1
// stores h device-coherent also within an XCD.
static int env_flag(const char* name, int dflt) {
    const char* e = getenv(name);
    return e && *e ? (*e != '0') : dflt;
}
static bool coop_launch() {
    static const bool v = env_flag("EAHMMF_HIP_FUSED_COOP", 0) != 0;
    return v;
}
// Devices on which a cooperative launch was refused in this process.
static bool g_coop_refused[64];
static bool coop_ok(int dev) { return dev < 0 || dev >= 64 || !__atomic_load_n(&g_coop_refused[dev], __ATOMIC_RELAXED); }
static void coop_refused(int dev) {
    if (dev >= 0 && dev < 64) __atomic_store_n(&g_coop_refused[dev], true, __ATOMIC_RELAXED);
}
// EAHMMF_HIP_TICKET=1 ranks the workgroups of an XCD by an atomic ticket
// (agent scope; 2: workgroup scope, executed in the XCD's L2) instead of by
// b / 8.  Measured at the Qwen3-30B-A3B shape: +0.45 us per launch either
// way (32 workgroups per XCD add to one counter at the same moment), so the
// default ranks by b / 8, which the once-per-device placement check
// validates; a launch placed otherwise shows up as waits that give up.
static int ticket_mode() {
    static const int v = [] {
        const char* e = getenv("EAHMMF_HIP_TICKET");
        return e && *e ? atoi(e) : 0;
    }();
    return v;
}
static int h_agent() {
    static const int v = env_flag("EAHMMF_HIP_H_AGENT", 0);
    return v;
}

__global__ void reset_sync_kernel(unsigned* sync, int clear_error) {
    const int i = threadIdx.x;
    if (i == 0 && clear_error) sync[kSyncFlagWord] = 0u;
    if (i < 8) sync[kTicketWord + kTicketStride * i] = 0u;
}

hipError_t reset_fused_sync(FusedState& fs, hipStream_t st, bool clear_error) {
    if (!fs.sync) return hipErrorInvalidValue;
    clear_stale_error();
    hipLaunchKernelGGL(reset_sync_kernel, dim3(1), dim3(64), 0, st, fs.sync, clear_error ? 1 : 0);
    const hipError_t e = hipGetLastError();
    if (e == hipSuccess) fs.ticket_base = 0;
    return e;
}

hipError_t launch_moe_fused(const FusedArgsHost& h, FusedState& fs, hipStream_t st) {
    const MoeShape& sh = h.shape;
    const bool routes = h.mode == 1 || h.mode == 3;
    if (!fused_supported(sh, h.k, routes ? h.n_expert : 0) || !fs.ypart || !fs.hx || !fs.sync || !h.x)
        return hipErrorInvalidValue;
    if (fs.hx_words < (size_t)h.k * sh.FF || fs.ypart_words < (size_t)8 * sh.D) return hipErrorInvalidValue;
    if (h.mode == 1 && (h.n_expert <= 0 || !h.logits || !h.table)) return hipErrorInvalidValue;
    if (h.mode == 3 && (h.n_expert <= 0 || !h.router || !h.table)) return hipErrorInvalidValue;
    FusedArgs a{};
    a.D = sh.D;
    a.FF = sh.FF;
    a.grb = (int)sh.gate_rb;
    a.urb = (int)sh.up_rb;
    a.drb = (int)sh.down_rb;
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
    a.hx = fs.hx;
    a.ypart = fs.ypart;
    a.sync = fs.sync;
    a.router = h.router;
    a.norm_w = h.norm_w;
    a.eps = h.eps;
    a.xn_out = h.xn_out;
    a.logits_out = h.logits_out;
    FusedFn fn = h.mode == 3 ? pick_fused_rt(sh) : pick_fused(sh);
    if (!fn) return h.mode == 3 ? hipErrorNotSupported : hipErrorInvalidValue;
    int dev = 0;
    hipError_t e = hipGetDevice(&dev);
    if (e != hipSuccess) return e;
    const FusedGrid g = fused_grid(sh, a.k, fused_capacity(fn, dev));
    if (!fused_grid_ok(sh, a.k, g)) return hipErrorInvalidConfiguration;
    a.np = g.np;
    a.m = g.m;
    if (h.mode == 3) {
        // one (logit, slice) unit per workgroup: as many slices as the
        // workgroups allow (a slice a whole number of eight-value parts)
        const int G = a.np * a.m;
        if (G < h.n_expert) return hipErrorNotSupported;
        int S = G / h.n_expert;
        if (S > kMaxRouterSlices) S = kMaxRouterSlices;
        while (S > 1 && sh.D % (8 * S)) S--;
        if (h.n_expert * S > kMaxLogitWords) return hipErrorNotSupported;
        a.rslices = S;
    }
    a.rows_b = g.rows_b;
    a.rows_a = g.rows_a;
    a.rows_round = g.rows_round;
    a.stride_b = g.stride_b;
    a.local_l2 = (a.np == 8 && xcd_round_robin(dev)) ? 1 : 0;
    a.epoch = fs.epoch + 1 == 0 ? 1 : fs.epoch + 1;
    a.ticket_base = fs.ticket_base;
    const unsigned lim = g_spin_limit > 0xFFFFFFu ? 0xFFFFFFu : g_spin_limit;
    a.flags = (unsigned)(g_drop_part + 1) | (ticket_mode() ? kFlagTicket : 0u) | (h_agent() ? kFlagHAgent : 0u) |
              (ticket_mode() == 2 ? kFlagTicketL2 : 0u) | (lim << 8);
    // routing: n_expert rounded up to a power of two (at most 256) is split
    // into t runs of rank_c keys, t threads per candidate (t <= 16)
    int npow = 1;
    while (npow < a.n_expert) npow *= 2;
    int t = kThreads / npow;
    if (t > 16) t = 16;
    if (t > npow) t = npow;
    a.rank_shift = 0;
    while ((1 << a.rank_shift) < t) a.rank_shift++;
    a.rank_c = npow / t;
    clear_stale_error();
    // Workgroups wait for each other, so all of them must be resident at
    // once.  The grid is at most one workgroup per CU, which the occupancy
    // check above admits, and a plain launch of it on an idle device makes
    // every workgroup resident.  When something else holds CUs, a workgroup
    // that is not resident in time shows up as waits that give up: NaN in y
    // and the error word, never a silent result.  A cooperative launch
    // (EAHMMF_HIP_FUSED_COOP=1) guarantees residency instead, at the cost
    // above.  The runtime can refuse it while another process on the GPU
    // holds the device's cooperative-launch resource; the launch is then a
    // plain one, and this process keeps to plain launches on the device.
    if (coop_launch() && coop_ok(dev)) {
        void* args[] = {&a};
        e = hipLaunchCooperativeKernel(reinterpret_cast<const void*>(fn), dim3(a.np * a.m), dim3(kThreads), args, 0,
                                       st);
        if (e != hipSuccess) {
            coop_refused(dev);
            clear_stale_error();
        }
    }
    if (!(coop_launch() && coop_ok(dev))) {
        hipLaunchKernelGGL(fn, dim3(a.np * a.m), dim3(kThreads), 0, st, a);
        e = hipGetLastError();
    }
    if (e == hipSuccess) {
        fs.epoch = a.epoch;
        if (a.local_l2 && (a.flags & kFlagTicket)) fs.ticket_base += (unsigned)a.m;
    }
    return e;
}

}  // namespace eahmmf
