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
//   gate/up  one workgroup per (expert, 64 FF rows) and the expert's n
//            tokens: the work is n x 64 rows of gate and up, split into units
//            (token, row part) - 4/n parts per token when n <= 4, else one -
//            and unit u is taken by wave u % 4.  A lane owns one 64-value
//            segment of the unit's token (its levels in registers, formed by
//            the lane itself from x); a row is G = D/64 lanes, 64/G rows per
//            step, gate and up rows of the same row back to back.  The
//            workgroup's 64 values of h = silu(g) * u are one 64-value
//            segment of h per token, turned into levels in the workgroup and
//            stored as such.
//   down     one workgroup per (expert, 64 D rows), the same split; a lane
//            owns one segment of the token's h levels (loaded as stored), a
//            row is G' = the power of two >= FF/64 lanes.
// Weight bytes are loaded straight into registers kDotAhead steps ahead of
// their dot; a row read by several tokens' waves of a workgroup is served
// from the CU's cache after the first.
#include "internal.h"
#include "kquant_seg64.h"

namespace eahmmf {

constexpr int kDotRows = 64;      // output rows per workgroup (one 64-value h segment for gate/up)
constexpr int kDotAhead = 3;      // steps of weight bytes in flight ahead of the dot (ring of 4)
constexpr int kDotMaxTok = 32;    // tokens an expert may hold on this path

// Levels of the 64 values at v (16-byte aligned), formed by one lane alone:
// the same three-level scheme as quantize8.
__device__ __forceinline__ void lane_levels(const float* v, XSeg& xs) {
    float r[64];
#pragma unroll
    for (int i = 0; i < 16; i++) {
        const float4 a = reinterpret_cast<const float4*>(v)[i];
        r[4 * i] = a.x;
        r[4 * i + 1] = a.y;
        r[4 * i + 2] = a.z;
        r[4 * i + 3] = a.w;
    }
    float amax = 0.f, s0 = 0.f, s1 = 0.f;
#pragma unroll
    for (int i = 0; i < 64; i++) {
        amax = fmaxf(amax, fabsf(r[i]));
        if (i < 32) s0 += r[i]; else s1 += r[i];
    }
    xs.sum32[0] = s0;
    xs.sum32[1] = s1;
    const float l1 = amax * (1.0f / 127.0f);
    const float l2 = l1 * (1.0f / 254.0f), l3 = l2 * (1.0f / 254.0f);
    const float lsc[kLevels] = {l1, l2, l3};
#pragma unroll
    for (int lv = 0; lv < kLevels; lv++) {
        const float inv = lsc[lv] > 0.f ? __builtin_amdgcn_rcpf(lsc[lv]) : 0.f;
#pragma unroll
        for (int d = 0; d < 16; d++) {
            uint32_t packed = 0u;
#pragma unroll
            for (int b = 0; b < 4; b++) {
                const int i = 4 * d + b;
                float qf = __builtin_rintf(r[i] * inv);
                qf = fminf(127.f, fmaxf(-127.f, qf));
                r[i] = __builtin_fmaf(-qf, lsc[lv], r[i]);
                packed |= ((uint32_t)(int)qf & 0xFFu) << (8 * b);
            }
            xs.q[lv][d] = (int32_t)packed;
        }
        xs.s[lv] = lsc[lv];
    }
}

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

// The units of a workgroup: n tokens x parts, parts = 4 / n for n <= 4.
__device__ __forceinline__ int dot_parts(int n) { return n >= 4 ? 1 : (n == 3 ? 1 : 4 / n); }

// gate/up of expert blockIdx.y, FF rows [64*blockIdx.x, +64), for the
// expert's tokens (groups of tmin..tmax tokens; others leave at once).  x
// [nb][ldx] fp32 rows, tok[p] the token at group position p.  Output: the
// levels of h segment blockIdx.x of every position p of the group,
// hq [P][3][FF] int8, hsc [P][3][FF/64], hs32 [P][FF/32].
template <int T, int G>
__global__ __launch_bounds__(256) void gate_up_dot_kernel(MoeShape s, const ExpertEntry* __restrict__ table,
                                                          const int* __restrict__ offs, const int* __restrict__ tok,
                                                          const float* __restrict__ x, int ldx,
                                                          int8_t* __restrict__ hq, float* __restrict__ hsc,
                                                          float* __restrict__ hs32, int tmin, int tmax) {
    constexpr int RPS = 64 / G;  // rows per step
    __shared__ float hb[kDotMaxTok][kDotRows];
    const int e = blockIdx.y;
    const int p0 = offs[e], n = offs[e + 1] - p0;
    if (n <= 0 || n < tmin || n > tmax) return;
    const int wave = threadIdx.x >> 6, l = threadIdx.x & 63;
    const int parts = dot_parts(n), units = n * parts, rows_u = kDotRows / parts;
    const int seg = l % G, sub = l / G;
    const int c0 = blockIdx.x * kDotRows;
    const ExpertEntry ent = table[e];
    for (int u = wave; u < units; u += 4) {
        const int t = u / parts, r0 = c0 + (u % parts) * rows_u;
        XSeg xs;
        lane_levels(x + (size_t)tok[p0 + t] * ldx + seg * 64, xs);
        // step j: row r0 + (j >> 1) * RPS + sub of gate (j even) or up (j odd)
        const int nsteps = 2 * rows_u / RPS;  // a multiple of 4 (rows_u >= 16, RPS <= 4)
        auto rowp = [&](int j) -> const uint8_t* {
            const int r = r0 + (j >> 1) * RPS + sub;
            return (j & 1) ? ent.up + (size_t)r * s.up_rb : ent.gate + (size_t)r * s.gate_rb;
        };
        // Every step issues its load (the last steps reload the last row): a
        // load skipped on some path leaves the compiler unable to count the
        // loads issued after a ring slot's, and it then waits for all of them.
        RawSeg<T> ring[kDotAhead + 1];
#pragma unroll
        for (int a = 0; a < kDotAhead; a++) ring[a].load(rowp(a), seg);
        float gv = 0.f;
        for (int j0 = 0; j0 < nsteps; j0 += kDotAhead + 1) {
#pragma unroll
            for (int v = 0; v <= kDotAhead; v++) {
                const int j = j0 + v;
                ring[(v + kDotAhead) % (kDotAhead + 1)].load(rowp(min(j + kDotAhead, nsteps - 1)), seg);
                const float d = group_sum<G>(ring[v].decode(seg).dot(xs));
                if (v & 1) {
                    if (seg == G - 1) hb[t][r0 - c0 + (j >> 1) * RPS + sub] = gv / (1.0f + expf(-gv)) * d;
                } else {
                    gv = d;
                }
            }
        }
    }
    __syncthreads();
    // levels of h segment blockIdx.x for every token: eight lanes per token
    const int FF = s.FF;
    for (int t0 = wave * 8; t0 < n; t0 += 32) {
        const int t = t0 + (l >> 3), part = l & 7;
        const bool act = t < n;
        float v[8];
#pragma unroll
        for (int i = 0; i < 8; i++) v[i] = act ? hb[t][8 * part + i] : 0.f;
        const size_t p = (size_t)p0 + (act ? t : 0);
        quantize8(v, blockIdx.x, part, act, hq + p * 3 * FF, FF, hsc + p * 3 * (FF / 64), FF / 64,
                  hs32 + p * (FF / 32));
    }
}

// down of expert blockIdx.y, D rows [64*blockIdx.x, +64): yp[p][r] =
// down_r . h[p] for the group's positions p, from h's stored levels.
template <int T, int G>
__global__ __launch_bounds__(256) void down_dot_kernel(MoeShape s, const ExpertEntry* __restrict__ table,
                                                       const int* __restrict__ offs, const int8_t* __restrict__ hq,
                                                       const float* __restrict__ hsc, const float* __restrict__ hs32,
                                                       float* __restrict__ yp, int tmin, int tmax) {
    constexpr int RPS = 64 / G;
    const int e = blockIdx.y;
    const int p0 = offs[e], n = offs[e + 1] - p0;
    if (n <= 0 || n < tmin || n > tmax) return;
    const int wave = threadIdx.x >> 6, l = threadIdx.x & 63;
    const int parts = dot_parts(n), units = n * parts, rows_u = kDotRows / parts;
    const int FF = s.FF, nseg = FF / 64;
    const int seg = l % G, sub = l / G;
    const bool on = seg < nseg;
    const int c0 = blockIdx.x * kDotRows;
    const uint8_t* dbase = table[e].down;
    for (int u = wave; u < units; u += 4) {
        const int t = u / parts, r0 = c0 + (u % parts) * rows_u;
        const size_t p = (size_t)p0 + t;
        XSeg xs = {};
        if (on) load_levels(hq + p * 3 * FF, hsc + p * 3 * nseg, hs32 + p * (FF / 32), FF, seg, xs);
        const int nsteps = rows_u / RPS;  // >= 1
        // unconditional loads (see gate_up_dot_kernel); lanes past the row's
        // segments read segment 0 and contribute 0
        const int lseg = on ? seg : 0;
        auto rowp = [&](int j) -> const uint8_t* {
            return dbase + (size_t)(r0 + min(j, nsteps - 1) * RPS + sub) * s.down_rb;
        };
        RawSeg<T> ring[kDotAhead + 1];
#pragma unroll
        for (int a = 0; a < kDotAhead; a++) ring[a].load(rowp(a), lseg);
        for (int j0 = 0; j0 < nsteps; j0 += kDotAhead + 1) {
#pragma unroll
            for (int v = 0; v <= kDotAhead; v++) {
                const int j = j0 + v;
                if (j >= nsteps) break;
                ring[(v + kDotAhead) % (kDotAhead + 1)].load(rowp(j + kDotAhead), lseg);
                const float dd = ring[v].decode(lseg).dot(xs);
                const float d = group_sum<G>(on ? dd : 0.f);
                if (seg == G - 1) yp[p * s.D + r0 + j * RPS + sub] = d;
            }
        }
    }
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
    return fmt && s.FF % 64 == 0 && s.FF / 64 <= 64 && s.FF / 64 >= 4 && s.D % kDotRows == 0;
}

template <int T>
static hipError_t gate_up_dot_g(const MoeShape& s, dim3 g, const ExpertEntry* table, const int* offs, const int* tok,
                                const float* x, int ldx, int8_t* hq, float* hsc, float* hs32, int tmin, int tmax,
                                hipStream_t st) {
    switch (s.D / 64) {
        case 16: gate_up_dot_kernel<T, 16><<<g, 256, 0, st>>>(s, table, offs, tok, x, ldx, hq, hsc, hs32, tmin, tmax); break;
        case 32: gate_up_dot_kernel<T, 32><<<g, 256, 0, st>>>(s, table, offs, tok, x, ldx, hq, hsc, hs32, tmin, tmax); break;
        case 64: gate_up_dot_kernel<T, 64><<<g, 256, 0, st>>>(s, table, offs, tok, x, ldx, hq, hsc, hs32, tmin, tmax); break;
        default: return hipErrorInvalidValue;
    }
    return hipGetLastError();
}

template <int T>
static hipError_t down_dot_g(const MoeShape& s, dim3 g, const ExpertEntry* table, const int* offs, const int8_t* hq,
                             const float* hsc, const float* hs32, float* yp, int tmin, int tmax, hipStream_t st) {
    switch (pow2_at_least(s.FF / 64)) {
        case 4: down_dot_kernel<T, 4><<<g, 256, 0, st>>>(s, table, offs, hq, hsc, hs32, yp, tmin, tmax); break;
        case 8: down_dot_kernel<T, 8><<<g, 256, 0, st>>>(s, table, offs, hq, hsc, hs32, yp, tmin, tmax); break;
        case 16: down_dot_kernel<T, 16><<<g, 256, 0, st>>>(s, table, offs, hq, hsc, hs32, yp, tmin, tmax); break;
        case 32: down_dot_kernel<T, 32><<<g, 256, 0, st>>>(s, table, offs, hq, hsc, hs32, yp, tmin, tmax); break;
        case 64: down_dot_kernel<T, 64><<<g, 256, 0, st>>>(s, table, offs, hq, hsc, hs32, yp, tmin, tmax); break;
        default: return hipErrorInvalidValue;
    }
    return hipGetLastError();
}

hipError_t launch_gate_up_dot(const MoeShape& s, const ExpertEntry* table, int E, const int* offs, const int* tok,
                              const float* x, int ldx, int8_t* hq, float* hsc, float* hs32, int tmin, int tmax,
                              hipStream_t st) {
    if (!grouped_dot_gate_up_ok(s) || tmax > kDotMaxTok || ldx % 4) return hipErrorInvalidValue;
    const dim3 g((unsigned)(s.FF / kDotRows), (unsigned)E);
    switch (s.gate_type) {
        case kQ4_K: return gate_up_dot_g<kQ4_K>(s, g, table, offs, tok, x, ldx, hq, hsc, hs32, tmin, tmax, st);
        case kQ5_K: return gate_up_dot_g<kQ5_K>(s, g, table, offs, tok, x, ldx, hq, hsc, hs32, tmin, tmax, st);
        case kQ6_K: return gate_up_dot_g<kQ6_K>(s, g, table, offs, tok, x, ldx, hq, hsc, hs32, tmin, tmax, st);
        case kQ8_0: return gate_up_dot_g<kQ8_0>(s, g, table, offs, tok, x, ldx, hq, hsc, hs32, tmin, tmax, st);
        default: return hipErrorInvalidValue;
    }
}

hipError_t launch_down_dot(const MoeShape& s, const ExpertEntry* table, int E, const int* offs, const int8_t* hq,
                           const float* hsc, const float* hs32, float* yp, int tmin, int tmax, hipStream_t st) {
    if (!grouped_dot_down_ok(s) || tmax > kDotMaxTok) return hipErrorInvalidValue;
    const dim3 g((unsigned)(s.D / kDotRows), (unsigned)E);
    switch (s.down_type) {
        case kQ4_K: return down_dot_g<kQ4_K>(s, g, table, offs, hq, hsc, hs32, yp, tmin, tmax, st);
        case kQ5_K: return down_dot_g<kQ5_K>(s, g, table, offs, hq, hsc, hs32, yp, tmin, tmax, st);
        case kQ6_K: return down_dot_g<kQ6_K>(s, g, table, offs, hq, hsc, hs32, yp, tmin, tmax, st);
        case kQ8_0: return down_dot_g<kQ8_0>(s, g, table, offs, hq, hsc, hs32, yp, tmin, tmax, st);
        default: return hipErrorInvalidValue;
    }
}

}  // namespace eahmmf
