// kernels_grouped_dot.hip - the ragged grouped expert block's matmuls for
// experts holding few tokens: integer dots on int8 activation levels.
//
// A decode batch routes each token to k of E experts, so most routed experts
// hold one or two of the batch's tokens (16 sequences x top-8 over 128
// experts: 82 distinct experts, 1.56 tokens each on average).  A matrix-core
// tile of 16 tokens would be almost empty, and every weight would still be
// decoded into an fp16 fragment.  Here each weight row is streamed once per
// workgroup and dotted exactly in int32 (v_dot4) against three int8 levels
// of each token's activations, the scheme of the single-token decode kernel
// (kquant_seg64.h): x ~= s1*X1 + s2*X2 + s3*X3 per 64-value segment, the
// codes are exact small integers, so the only rounding is in the fp32 scale
// products.
//
//   levels   levels_rows_kernel: each token's x as int8 levels, once.
//   gate/up  one wave per (expert, 16 FF rows, pair of the expert's tokens):
//            the pair's levels in registers, a lane holding one 64-value
//            segment of each; a row is G = D/64 lanes, 64/G rows per step,
//            gate and up rows of the same rows in alternate steps; every
//            decoded segment is dotted against both tokens.  h = silu(g) * u
//            is stored in fp32, then turned into levels (levels_rows_kernel).
//   down     one wave per (expert, 64 D rows, pair of tokens) from h's
//            levels, a row is G' = the power of two >= FF/64 lanes.
// The launches' grids are (row blocks, item slots): the grouping kernel lists
// the (expert, token pair) items, so no workgroup is spent on an expert the
// batch does not route to or on a pair past an expert's group.
// Work items this small keep the launch balanced: a wave streams about
// 4 GB/s when the whole chip streams, so an item's time is set by its bytes,
// and the last items to start end soon after the rest.
// Weight bytes: a step's rows (64 segments' worth, contiguous in memory) are
// copied by the wave with LDS DMA (16-byte global_load_lds, coalesced) into
// the next of its kDotSlots LDS slots, kDotSlots - 1 steps ahead of their
// dot; each wait is an explicit vmcnt over the wave's own copies, so nothing
// the compiler schedules drains the copies in flight.  A row read by several
// tokens' waves of a workgroup is served from the CU's cache after the first.
#include "internal.h"
#include "kquant_seg64.h"

namespace eahmmf {

constexpr int kDotRows = 64;      // down rows per workgroup
constexpr int kGuRowsDot = 16;    // gate/up rows per workgroup
constexpr int kDotSlots = 4;      // LDS slots per gate/up wave: kDotSlots - 1 steps' bytes in flight
constexpr int kDownSlots = 4;     // the same for a down wave
constexpr int kDotMaxNI = 5;      // 1 KB DMA instructions per step (a step holds at most 4352 bytes)
constexpr int kDotMaxTok = 32;    // tokens an expert may hold on this path

// Stored levels of one 64-value segment (rows of n values: level lv at
// q + lv*n, scales sc[lv*(n/64) + seg], sums s32[2*seg], s32[2*seg+1]).
__device__ __forceinline__ void load_levels(const int8_t* q, const float* sc, const float* s32, int n, int seg,
                                            XSeg& xs) {
#pragma unroll
    for (int lv = 0; lv < kLevels; lv++) {
        const uint4* p = reinterpret_cast<const uint4*>(q + (size_t)lv * n + seg * 64);
#pragma unroll
        for (int c = 0; c < 4; c++) {
            const uint4 v = p[c];
            xs.q[lv][4 * c] = (int32_t)v.x;
            xs.q[lv][4 * c + 1] = (int32_t)v.y;
            xs.q[lv][4 * c + 2] = (int32_t)v.z;
            xs.q[lv][4 * c + 3] = (int32_t)v.w;
        }
        xs.s[lv] = sc[lv * (n / 64) + seg];
    }
    xs.sum32[0] = s32[2 * seg];
    xs.sum32[1] = s32[2 * seg + 1];
}

// The workgroup's item (blockIdx.y of the list): false past the list's end.
__device__ __forceinline__ bool dot_item(const DotItems& g, int& e, int& p0, int& n, int& t0) {
    const int i = (int)blockIdx.y;
    const int total = *g.n;
    const int2 v = g.items[i];  // in bounds: the grid has cap rows, the list cap slots
    if (i >= total) return false;
    e = v.x & 0xFFFF;
    t0 = 2 * ((v.x >> 16) & 0xFF);
    n = (int)((unsigned)v.x >> 24);
    p0 = v.y;
    return true;
}

// The units of a workgroup: n tokens x parts, parts = 4 / n for n <= 4.
__device__ __forceinline__ int dot_parts(int n) { return n >= 4 ? 1 : (n == 3 ? 1 : 4 / n); }

// Levels of nb rows of n values (n % 64 == 0): row r of src (stride ld)
// -> q [nb][3][n], sc [nb][3][n/64], s32 [nb][n/32].  One workgroup per row,
// eight threads per 64-value segment.
__global__ __launch_bounds__(256) void levels_rows_kernel(const float* __restrict__ src, int ld, int n,
                                                          int8_t* __restrict__ q, float* __restrict__ sc,
                                                          float* __restrict__ s32) {
    const int r = blockIdx.x, nseg = n / 64;
    const float* row = src + (size_t)r * ld;
    for (int base = 0; base < nseg; base += 32) {
        const int seg = base + (int)threadIdx.x / 8, part = threadIdx.x % 8;
        const bool act = seg < nseg;
        float v[8];
        if (act) {
            const float4 a = *reinterpret_cast<const float4*>(row + seg * 64 + part * 8);
            const float4 c = *reinterpret_cast<const float4*>(row + seg * 64 + part * 8 + 4);
            v[0] = a.x; v[1] = a.y; v[2] = a.z; v[3] = a.w; v[4] = c.x; v[5] = c.y; v[6] = c.z; v[7] = c.w;
        } else {
#pragma unroll
            for (int i = 0; i < 8; i++) v[i] = 0.f;
        }
        quantize8(v, seg, part, act, q + (size_t)r * 3 * n, n, sc + (size_t)r * 3 * nseg, nseg, s32 + (size_t)r * (n / 32));
    }
}

// The levels just loaded stay put: complete their loads here rather than at
// their first use in a step loop (where the compiler's wait would recur every
// step and drain the copies in flight).
__device__ __forceinline__ void pin_levels(XSeg& xs) {
#pragma unroll
    for (int lv = 0; lv < kLevels; lv++) {
#pragma unroll
        for (int i = 0; i < 16; i++) pin(xs.q[lv][i]);
        pin(xs.s[lv]);
    }
    pin(xs.sum32[0]);
    pin(xs.sum32[1]);
}

// DMA of one step's bytes [src, src + bytes) into an LDS slot: NI
// instructions of 64 lanes x 16 bytes from src rounded down to 16 (the slot
// holds the bytes at offset src & 15; chunks past the end repeat the last).
template <int NI>
__device__ __forceinline__ void issue_step(const uint8_t* src, int bytes, uint8_t* slot, int lane) {
    const uintptr_t a = (uintptr_t)src, base = a & ~(uintptr_t)15;
    const int nc = (int)((a + (uintptr_t)bytes + 15 - base) / 16);
#pragma unroll
    for (int i = 0; i < NI; i++) lds_dma16(base + (uintptr_t)min(i * 64 + lane, nc - 1) * 16, slot + i * 1024);
}

// Wait for step j's copies: S - 1 later steps are in flight except
// at the end of a unit (run-time count there).
template <int NI, int S>
__device__ __forceinline__ void wait_step(int j, int nsteps) {
    if (j + S - 1 < nsteps)
        wait_vm_upto<NI * (S - 1)>();
    else
        wait_vm_n(NI * (nsteps - 1 - j));
}

// A wave's tokens are taken two at a time (a pass): the two tokens' levels
// sit in registers and every decoded segment is dotted against both.
struct XPair {
    XSeg a, b;
};

__device__ __forceinline__ void load_pair(const int8_t* q, const float* sc, const float* s32, size_t ra, size_t rb,
                                          int n, int seg, bool two, XPair& x) {
    load_levels(q + ra * 3 * n, sc + ra * 3 * (n / 64), s32 + ra * (n / 32), n, seg, x.a);
    if (two) load_levels(q + rb * 3 * n, sc + rb * 3 * (n / 64), s32 + rb * (n / 32), n, seg, x.b);
    pin_levels(x.a);
    pin_levels(x.b);
}

// gate/up of item blockIdx.y (expert e, pair j of its group: tokens 2j and
// 2j + 1; groups of tmin..tmax tokens; workgroups past the item list leave
// at once), FF rows [kGuRowsDot*blockIdx.x, +kGuRowsDot), from the tokens'
// activation levels (xq/xsc/xs32, levels_rows_kernel over x): h [P][FF]
// fp32.  One wave; dynamic LDS: kDotSlots slots of NI KB.
template <int T, int G, int NI>
__global__ __launch_bounds__(64) void gate_up_dot_kernel(MoeShape s, const ExpertEntry* __restrict__ table,
                                                         DotItems gr, const int* __restrict__ tok,
                                                         const int8_t* __restrict__ xq, const float* __restrict__ xsc,
                                                         const float* __restrict__ xs32, float* __restrict__ h,
                                                         int tmin, int tmax) {
    constexpr int RPS = 64 / G;  // rows per step
    constexpr int SLOT = NI * 1024;
    constexpr int NSTEPS = 2 * kGuRowsDot / RPS;  // gate and up steps of the rows: a multiple of 4
    extern __shared__ __align__(16) uint8_t ring[];
    __shared__ float hb[2][kGuRowsDot];
    int e, p0, n, t0;
    if (!dot_item(gr, e, p0, n, t0) || n < tmin || n > tmax) return;
    const bool two = t0 + 1 < n;  // wave-uniform
    const int l = threadIdx.x;
    const int seg = l % G, sub = l / G;
    const int D = s.D, FF = s.FF, c0 = blockIdx.x * kGuRowsDot;
    const ExpertEntry ent = table[e];
    const int rb = s.gate_rb, bytes = RPS * rb;  // gate and up share type and shape
    // the matrix of a step by integer arithmetic: a select between the two
    // pointers is lowered to an indexed load from a scratch copy of the
    // entry, and its wait would drain the copies in flight
    const uintptr_t gate = (uintptr_t)ent.gate, up_minus_gate = (uintptr_t)ent.up - gate;
    // step j: rows c0 + (j >> 1) * RPS .. + RPS - 1 of gate (j even) or up (j odd)
    auto stepsrc = [&](int j) -> const uint8_t* {
        return (const uint8_t*)(gate + ((j & 1) ? up_minus_gate : (uintptr_t)0) +
                                (uintptr_t)(c0 + (j >> 1) * RPS) * (uintptr_t)rb);
    };
#pragma unroll
    for (int j = 0; j < kDotSlots - 1; j++) issue_step<NI>(stepsrc(j), bytes, ring + j * SLOT, l);
    XPair x;
    load_pair(xq, xsc, xs32, (size_t)tok[p0 + t0], (size_t)tok[p0 + (two ? t0 + 1 : t0)], D, seg, two, x);
    float ga = 0.f, gb = 0.f;
    for (int j0 = 0; j0 < NSTEPS; j0 += kDotSlots) {
#pragma unroll
        for (int v = 0; v < kDotSlots; v++) {
            const int j = j0 + v;
            if (j + kDotSlots - 1 < NSTEPS)
                issue_step<NI>(stepsrc(j + kDotSlots - 1), bytes, ring + ((v + kDotSlots - 1) % kDotSlots) * SLOT, l);
            wait_step<NI, kDotSlots>(j, NSTEPS);
            RawSeg<T> raw;
            raw.template load<LdsLd>(ring + v * SLOT + ((uintptr_t)stepsrc(j) & 15) + sub * rb, seg);
            const SegCodes<T> c = raw.decode(seg);
            const float da = group_sum<G>(c.dot(x.a));
            const float db = two ? group_sum<G>(c.dot(x.b)) : 0.f;
            const int row = (j >> 1) * RPS + sub;
            if (v & 1) {
                if (seg == G - 1) {
                    hb[0][row] = ga / (1.0f + expf(-ga)) * da;
                    hb[1][row] = gb / (1.0f + expf(-gb)) * db;
                }
            } else {
                ga = da;
                gb = db;
            }
        }
    }
    if (l < kGuRowsDot) {
        h[(size_t)(p0 + t0) * FF + c0 + l] = hb[0][l];
        if (two) h[(size_t)(p0 + t0 + 1) * FF + c0 + l] = hb[1][l];
    }
}

// down of item blockIdx.y (expert e, tokens 2j and 2j + 1 of its group), D
// rows [64*blockIdx.x, +64): yp[p][r] = down_r . h[p]
// from h's levels.  One wave.  The outputs are gathered in LDS and stored at
// the end (a global store inside the step loop would count against the
// copies' vmcnt).
template <int T, int G, int NI>
__global__ __launch_bounds__(64) void down_dot_kernel(MoeShape s, const ExpertEntry* __restrict__ table,
                                                      DotItems gr, const int8_t* __restrict__ hq,
                                                      const float* __restrict__ hsc, const float* __restrict__ hs32,
                                                      float* __restrict__ yp, int tmin, int tmax) {
    constexpr int RPS = 64 / G;
    constexpr int SLOT = NI * 1024;
    constexpr int NSTEPS = kDotRows / RPS;
    extern __shared__ __align__(16) uint8_t ring[];
    __shared__ float yb[2][kDotRows];
    int e, p0, n, t0;
    if (!dot_item(gr, e, p0, n, t0) || n < tmin || n > tmax) return;
    const bool two = t0 + 1 < n;
    const int l = threadIdx.x;
    const int FF = s.FF, nseg = FF / 64;
    const int seg = l % G, sub = l / G;
    const bool on = seg < nseg;
    const int lseg = on ? seg : 0;  // lanes past the row's segments read segment 0 and contribute 0
    const int c0 = blockIdx.x * kDotRows;
    const uint8_t* dbase = table[e].down;
    const int rb = s.down_rb, bytes = RPS * rb;
    auto stepsrc = [&](int j) -> const uint8_t* { return dbase + (size_t)(c0 + j * RPS) * rb; };
#pragma unroll
    for (int j = 0; j < kDownSlots - 1 && j < NSTEPS; j++) issue_step<NI>(stepsrc(j), bytes, ring + j * SLOT, l);
    const size_t pa = (size_t)p0 + t0, pb = (size_t)p0 + (two ? t0 + 1 : t0);
    XPair x = {};
    if (on) load_pair(hq, hsc, hs32, pa, pb, FF, seg, two, x);
    pin_levels(x.a);
    pin_levels(x.b);
    for (int j0 = 0; j0 < NSTEPS; j0 += kDownSlots) {
#pragma unroll
        for (int v = 0; v < kDownSlots; v++) {
            const int j = j0 + v;
            if (j >= NSTEPS) break;
            if (j + kDownSlots - 1 < NSTEPS)
                issue_step<NI>(stepsrc(j + kDownSlots - 1), bytes, ring + ((v + kDownSlots - 1) % kDownSlots) * SLOT, l);
            wait_step<NI, kDownSlots>(j, NSTEPS);
            RawSeg<T> raw;
            raw.template load<LdsLd>(ring + v * SLOT + ((uintptr_t)stepsrc(j) & 15) + sub * rb, lseg);
            const SegCodes<T> c = raw.decode(lseg);
            const float da = group_sum<G>(on ? c.dot(x.a) : 0.f);
            const float db = two ? group_sum<G>(on ? c.dot(x.b) : 0.f) : 0.f;
            if (seg == G - 1) {
                yb[0][j * RPS + sub] = da;
                yb[1][j * RPS + sub] = db;
            }
        }
    }
    yp[pa * s.D + c0 + l] = yb[0][l];
    if (two) yp[pb * s.D + c0 + l] = yb[1][l];
}

// ---------------------------------------------------------------------------

static bool pow2_le64(int v) { return v >= 1 && v <= 64 && (v & (v - 1)) == 0; }
static int pow2_at_least(int v) {
    int g = 1;
    while (g < v) g <<= 1;
    return g;
}

bool grouped_dot_gate_up_ok(const MoeShape& s) {
    const bool fmt = s.gate_type == s.up_type &&
                     (s.gate_type == kQ4_K || s.gate_type == kQ5_K || s.gate_type == kQ6_K || s.gate_type == kQ8_0);
    return fmt && s.D % 64 == 0 && s.D >= 1024 && pow2_le64(s.D / 64) && s.FF % kDotRows == 0;
}

bool grouped_dot_down_ok(const MoeShape& s) {
    const bool fmt = s.down_type == kQ4_K || s.down_type == kQ5_K || s.down_type == kQ6_K || s.down_type == kQ8_0;
    return fmt && s.FF % 64 == 0 && s.FF / 64 <= 64 && s.FF / 64 >= 5 && s.D % kDotRows == 0;
}

// 1 KB DMA instructions for a step of `bytes` bytes starting anywhere in a
// 16-byte chunk, plus the 2 bytes a realigned LDS read may touch past them.
static int step_ni(int bytes) { return (15 + bytes + 2 + 1023) / 1024; }

// gate/up: a step is always 64 segments (16 super-blocks or 64 Q8_0 blocks)
template <int T> constexpr int gu_ni() { return T == kQ4_K || T == kQ5_K ? 3 : (T == kQ6_K ? 4 : 5); }

template <int T>
static hipError_t gate_up_dot_g(const MoeShape& s, dim3 g, const ExpertEntry* table, DotItems gr, const int* tok,
                                const int8_t* xq, const float* xsc, const float* xs32, float* h, int tmin, int tmax,
                                hipStream_t st) {
    constexpr int NI = gu_ni<T>();
    const int G = s.D / 64;
    if (step_ni(64 / G * s.gate_rb) > NI) return hipErrorInvalidValue;
    const size_t lds = (size_t)kDotSlots * NI * 1024;
    switch (G) {
        case 16: gate_up_dot_kernel<T, 16, NI><<<g, 64, lds, st>>>(s, table, gr, tok, xq, xsc, xs32, h, tmin, tmax); break;
        case 32: gate_up_dot_kernel<T, 32, NI><<<g, 64, lds, st>>>(s, table, gr, tok, xq, xsc, xs32, h, tmin, tmax); break;
        case 64: gate_up_dot_kernel<T, 64, NI><<<g, 64, lds, st>>>(s, table, gr, tok, xq, xsc, xs32, h, tmin, tmax); break;
        default: return hipErrorInvalidValue;
    }
    return hipGetLastError();
}

// down: a step is RPS rows of FF/64 segments, 3/4 .. 1 of 64 segments' bytes;
// copies sized for 3 KB when that suffices, else the format's 64-segment size
template <int T, int G>
static hipError_t down_dot_gn(const MoeShape& s, dim3 g, const ExpertEntry* table, DotItems gr, const int8_t* hq,
                              const float* hsc, const float* hs32, float* yp, int tmin, int tmax, hipStream_t st) {
    constexpr int NIMAX = gu_ni<T>();
    const int ni = step_ni(64 / G * s.down_rb);
    if (ni > NIMAX) return hipErrorInvalidValue;
    if (ni <= 3) {
        down_dot_kernel<T, G, 3><<<g, 64, (size_t)kDownSlots * 3 * 1024, st>>>(s, table, gr, hq, hsc, hs32, yp, tmin, tmax);
    } else {
        down_dot_kernel<T, G, NIMAX><<<g, 64, (size_t)kDownSlots * NIMAX * 1024, st>>>(s, table, gr, hq, hsc, hs32, yp, tmin, tmax);
    }
    return hipGetLastError();
}

template <int T>
static hipError_t down_dot_g(const MoeShape& s, dim3 g, const ExpertEntry* table, DotItems gr, const int8_t* hq,
                             const float* hsc, const float* hs32, float* yp, int tmin, int tmax, hipStream_t st) {
    switch (pow2_at_least(s.FF / 64)) {
        case 8: return down_dot_gn<T, 8>(s, g, table, gr, hq, hsc, hs32, yp, tmin, tmax, st);
        case 16: return down_dot_gn<T, 16>(s, g, table, gr, hq, hsc, hs32, yp, tmin, tmax, st);
        case 32: return down_dot_gn<T, 32>(s, g, table, gr, hq, hsc, hs32, yp, tmin, tmax, st);
        case 64: return down_dot_gn<T, 64>(s, g, table, gr, hq, hsc, hs32, yp, tmin, tmax, st);
        default: return hipErrorInvalidValue;
    }
}

hipError_t launch_levels_rows(const float* src, int ld, int rows, int n, int8_t* q, float* sc, float* s32,
                              hipStream_t st) {
    if (rows <= 0 || n % 64 || ld % 4) return hipErrorInvalidValue;
    levels_rows_kernel<<<(unsigned)rows, 256, 0, st>>>(src, ld, n, q, sc, s32);
    return hipGetLastError();
}

hipError_t launch_gate_up_dot(const MoeShape& s, const ExpertEntry* table, int E, DotItems gr, const int* tok,
                              const int8_t* xq, const float* xsc, const float* xs32, float* h, int tmin, int tmax,
                              hipStream_t st) {
    if (!grouped_dot_gate_up_ok(s) || tmax > kDotMaxTok || tmax < 1) return hipErrorInvalidValue;
    if (gr.cap < 1) return hipErrorInvalidValue;
    const dim3 g((unsigned)(s.FF / kGuRowsDot), (unsigned)gr.cap);
    switch (s.gate_type) {
        case kQ4_K: return gate_up_dot_g<kQ4_K>(s, g, table, gr, tok, xq, xsc, xs32, h, tmin, tmax, st);
        case kQ5_K: return gate_up_dot_g<kQ5_K>(s, g, table, gr, tok, xq, xsc, xs32, h, tmin, tmax, st);
        case kQ6_K: return gate_up_dot_g<kQ6_K>(s, g, table, gr, tok, xq, xsc, xs32, h, tmin, tmax, st);
        case kQ8_0: return gate_up_dot_g<kQ8_0>(s, g, table, gr, tok, xq, xsc, xs32, h, tmin, tmax, st);
        default: return hipErrorInvalidValue;
    }
}

hipError_t launch_down_dot(const MoeShape& s, const ExpertEntry* table, int E, DotItems gr, const int8_t* hq,
                           const float* hsc, const float* hs32, float* yp, int tmin, int tmax, hipStream_t st) {
    if (!grouped_dot_down_ok(s) || tmax > kDotMaxTok || tmax < 1) return hipErrorInvalidValue;
    if (gr.cap < 1) return hipErrorInvalidValue;
    const dim3 g((unsigned)(s.D / kDotRows), (unsigned)gr.cap);
    switch (s.down_type) {
        case kQ4_K: return down_dot_g<kQ4_K>(s, g, table, gr, hq, hsc, hs32, yp, tmin, tmax, st);
        case kQ5_K: return down_dot_g<kQ5_K>(s, g, table, gr, hq, hsc, hs32, yp, tmin, tmax, st);
        case kQ6_K: return down_dot_g<kQ6_K>(s, g, table, gr, hq, hsc, hs32, yp, tmin, tmax, st);
        case kQ8_0: return down_dot_g<kQ8_0>(s, g, table, gr, hq, hsc, hs32, yp, tmin, tmax, st);
        default: return hipErrorInvalidValue;
    }
}

}  // namespace eahmmf
