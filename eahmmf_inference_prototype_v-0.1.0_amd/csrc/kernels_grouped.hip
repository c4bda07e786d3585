// kernels_grouped.hip - the ragged multi-token expert block (prefill and
// batched decode): nb tokens, each routed to k experts, grouped by expert.
//
// This replaces the reference's host loop for a batch (qwen3moe.cpp:1009-1067):
// by_exp[e] collects the (token, w) pairs of expert e in token order, the
// experts are visited in ascending id, each runs gate/up, SiLU and down over its
// gathered tokens as one batched matmul, and every token adds w * y of its
// experts in ascending expert order.
//
// Device steps, all on one stream:
//   1. group_pairs_kernel (one workgroup): a stable counting sort of the
//      (token, slot) pairs by expert id.  Tokens are taken in chunks of 64
//      (one wave each); a chunk's pairs of expert e are the set bits of a
//      64-bit LDS mask, so a pair's rank among the chunk's pairs of e is a
//      popcount and the order is fixed by construction.  Chunk counts are
//      scanned per expert, expert totals across experts, giving
//        offs[e]      first position of expert e's group
//        tok[p], pw[p] token and router weight at position p
//        pos[t*k+r]   position of token t's r-th pair in ascending expert id
//                     (-1 past its valid pairs)
//   2. grouped gate/up: h[p][r] = silu(gate_r . x_tok[p]) * (up_r . x_tok[p]);
//      on the matrix cores for Q4_K/Q5_K (kernels_grouped_mfma.hip), else one
//      wave per (expert, FF row) with the group's tokens in tiles of 8.
//   3. grouped down: yp[p][r] = down_r . h[p]; matrix cores for Q6_K, else one
//      wave per (expert, D row).
//   4. combine: y[t] = sum over the token's pairs in ascending expert id of
//      w * yp[pos] (fma), the reference's accumulation order.
// Expert weights are read once per (expert, row) however many tokens the
// group holds.
#include <mutex>

#include <climits>

#include "internal.h"
#include "kquant.h"

namespace eahmmf {

constexpr int kGroupThreads = 1024;
constexpr int kGroupWaves = kGroupThreads / 64;
constexpr int kGroupMaxE = 256;  // group masks: 16 waves x E x 8 B of LDS
constexpr int kTT = 8;  // tokens per tile in the grouped matmuls

__device__ __forceinline__ void lds_order() { __asm__ volatile("s_waitcnt lgkmcnt(0)" ::: "memory"); }

// Token t's pair positions pj (expert ej, -1: invalid slot) in ascending
// expert id (equal ids in slot order), invalid slots last: the combine's
// summation order.
__device__ __forceinline__ void write_positions(int* __restrict__ pos, int t, int k, const int (&ej)[kMaxSlots],
                                                const int (&pj)[kMaxSlots]) {
    int nvalid = 0;
#pragma unroll
    for (int j = 0; j < kMaxSlots; j++) nvalid += pj[j] >= 0 ? 1 : 0;
#pragma unroll
    for (int j = 0; j < kMaxSlots; j++) {
        if (j >= k) break;
        int r = 0;
#pragma unroll
        for (int i = 0; i < kMaxSlots; i++) {
            if (pj[j] >= 0)
                r += (i != j && pj[i] >= 0 && (ej[i] < ej[j] || (ej[i] == ej[j] && i < j))) ? 1 : 0;
            else
                r += (i < j && i < k && pj[i] < 0) ? 1 : 0;
        }
        pos[(size_t)t * k + (pj[j] >= 0 ? r : nvalid + r)] = pj[j];
    }
}

// The launches' work lists the grouping kernel writes: the integer-dot item
// list ((e, pair j) for every expert holding 1..dmax pairs) and the gate/up
// and down pass lists of the workgroup matrix-core kernels (passes of
// kMfmaGuTok / kMfmaDnTok pairs over every expert holding at least wmin);
// each count at its n pointer.  dmax 0 / a wmin above every group: empty.
struct GroupLists {
    int dmax, wmin, vlo, vhi;  // vlo..vhi: the per-wave kernels' experts (one item each)
    int2* items;
    int* nitems;
    int4* gitems;
    int* ngitems;
    int4* ditems;
    int* nditems;
    int4* vitems;
    int* nvitems;
};

// An exclusive scan over the wave's lanes; total: the sum of all lanes.
__device__ __forceinline__ int wave_excl_scan(int v, int lane, int& total) {
    int incl = v;
#pragma unroll
    for (int off = 1; off < 64; off <<= 1) {
        const int u = __shfl_up(incl, off, 64);
        if (lane >= off) incl += u;
    }
    total = __shfl(incl, 63, 64);
    return incl - v;
}

// Wave 0, with tot[e] = expert e's pair count: the exclusive scan into offs
// (global; tot[e] then holds it too, lane i owning experts [i*per, (i+1)*per))
// and the work lists, in expert order.
__device__ __forceinline__ void scan_offsets(int* tot, int* __restrict__ offs, int E, int lane, const GroupLists& gl) {
    const int per = (E + 63) / 64;
    const int dmax = gl.dmax, wmin = gl.wmin;
    auto n_dot = [&](int te) { return te >= 1 && te <= dmax ? (te + 1) / 2 : 0; };
    auto n_gu = [&](int te) { return te >= wmin ? (te + kMfmaGuTok - 1) / kMfmaGuTok : 0; };
    auto n_dn = [&](int te) { return te >= wmin ? (te + kMfmaDnTok - 1) / kMfmaDnTok : 0; };
    auto n_v = [&](int te) { return te >= 1 && te >= gl.vlo && te <= gl.vhi ? 1 : 0; };
    int local = 0, ld = 0, lg = 0, ln = 0, lv = 0;
    for (int i = 0; i < per; i++) {
        const int e = lane * per + i;
        if (e < E) {
            const int te = tot[e];
            local += te;
            ld += n_dot(te);
            lg += n_gu(te);
            ln += n_dn(te);
            lv += n_v(te);
        }
    }
    int all, nd, ng, nn;
    int run = wave_excl_scan(local, lane, all), rd = wave_excl_scan(ld, lane, nd);
    int rg = wave_excl_scan(lg, lane, ng), rn = wave_excl_scan(ln, lane, nn);
    int nv, rv = wave_excl_scan(lv, lane, nv);
    for (int i = 0; i < per; i++) {
        const int e = lane * per + i;
        if (e < E) {
            const int te = tot[e];
            offs[e] = run;
            tot[e] = run;
            for (int j = 0; j < n_dot(te); j++) gl.items[rd++] = make_int2(e | j << 16 | te << 24, run);
            for (int j = 0; j < n_gu(te); j++) gl.gitems[rg++] = make_int4(e, run + j * kMfmaGuTok, run + te, run);
            for (int j = 0; j < n_dn(te); j++) gl.ditems[rn++] = make_int4(e, run + j * kMfmaDnTok, run + te, run);
            if (n_v(te)) gl.vitems[rv++] = make_int4(e, run, run + te, run);
            run += te;
        }
    }
    if (lane == 63) {
        offs[E] = all;
        *gl.nitems = nd;
        *gl.ngitems = ng;
        *gl.nditems = nn;
        *gl.nvitems = nv;
    }
}

// ids/w [nb][k]; cnt scratch [nchunks][E]; outputs offs [E+1], tok/pw [nb*k],
// pos [nb*k]; gl: the launches' work lists.  Dynamic LDS: kGroupWaves * E uint64 masks + E ints (+ nchunks * E
// ints of per-chunk counts when nchunks <= kGroupWaves).
__global__ __launch_bounds__(kGroupThreads) void group_pairs_kernel(const int* __restrict__ ids,
                                                                    const float* __restrict__ w, int nb, int k, int E,
                                                                    int* __restrict__ cnt, int* __restrict__ offs,
                                                                    int* __restrict__ tok, float* __restrict__ pw,
                                                                    int* __restrict__ pos, GroupLists gl) {
    extern __shared__ unsigned long long g_lds[];
    const int tid = threadIdx.x, wave = tid / 64, lane = tid % 64;
    unsigned long long* mask = g_lds + (size_t)wave * E;
    int* tot = reinterpret_cast<int*>(g_lds + (size_t)kGroupWaves * E);
    const int nchunks = (nb + 63) / 64;
    auto build_mask = [&](int c) {
        for (int e = lane; e < E; e += 64) mask[e] = 0ull;
        lds_order();
        const int t = c * 64 + lane;
        if (t < nb)
            for (int j = 0; j < k; j++) {
                const int e = ids[(size_t)t * k + j];
                if (e >= 0 && e < E) __hip_atomic_fetch_or(&mask[e], 1ull << lane, __ATOMIC_RELAXED,
                                                           __HIP_MEMORY_SCOPE_WORKGROUP);
            }
        lds_order();
    };
    if (nchunks <= kGroupWaves) {
        // One chunk per wave: the wave's ids and weights stay in registers,
        // its mask stays in LDS from the count to the scatter, and the
        // per-chunk counts and the offsets live in LDS.
        int* ccnt = tot + E;  // [nchunks][E]
        const int t = wave * 64 + lane;
        const bool act = wave < nchunks, own = act && t < nb;
        int idr[kMaxSlots];
        float wr[kMaxSlots];
#pragma unroll
        for (int j = 0; j < kMaxSlots; j++) {
            idr[j] = -1;
            wr[j] = 0.f;
            if (own && j < k) {
                idr[j] = ids[(size_t)t * k + j];
                wr[j] = w[(size_t)t * k + j];
            }
        }
        if (act) {
            for (int e = lane; e < E; e += 64) mask[e] = 0ull;
            lds_order();
#pragma unroll
            for (int j = 0; j < kMaxSlots; j++) {
                const int e = idr[j];
                if (j < k && e >= 0 && e < E)
                    __hip_atomic_fetch_or(&mask[e], 1ull << lane, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
            }
            lds_order();
            for (int e = lane; e < E; e += 64) ccnt[wave * E + e] = __popcll(mask[e]);
        }
        __syncthreads();
        for (int e = tid; e < E; e += kGroupThreads) {
            int run = 0;
            for (int c = 0; c < nchunks; c++) {
                const int v = ccnt[c * E + e];
                ccnt[c * E + e] = run;
                run += v;
            }
            tot[e] = run;
        }
        __syncthreads();
        if (wave == 0) scan_offsets(tot, offs, E, lane, gl);
        __syncthreads();
        if (own) {
            const unsigned long long below = (lane == 0) ? 0ull : (~0ull >> (64 - lane));
            int ej[kMaxSlots], pj[kMaxSlots];
#pragma unroll
            for (int j = 0; j < kMaxSlots; j++) {
                ej[j] = 0;
                pj[j] = -1;
                const int e = idr[j];
                if (j < k && e >= 0 && e < E) {
                    const int p = tot[e] + ccnt[wave * E + e] + __popcll(mask[e] & below);
                    tok[p] = t;
                    pw[p] = wr[j];
                    ej[j] = e;
                    pj[j] = p;
                }
            }
            write_positions(pos, t, k, ej, pj);
        }
        return;
    }
    // 1. per-chunk counts
    for (int c = wave; c < nchunks; c += kGroupWaves) {
        build_mask(c);
        for (int e = lane; e < E; e += 64) cnt[(size_t)c * E + e] = __popcll(mask[e]);
    }
    __syncthreads();
    // 2. per expert: chunk bases (exclusive, in place) and the total
    for (int e = tid; e < E; e += kGroupThreads) {
        int run = 0;
        for (int c = 0; c < nchunks; c++) {
            const int v = cnt[(size_t)c * E + e];
            cnt[(size_t)c * E + e] = run;
            run += v;
        }
        tot[e] = run;
    }
    __syncthreads();
    if (wave == 0) scan_offsets(tot, offs, E, lane, gl);
    __syncthreads();
    // 3. scatter every pair to its place
    for (int c = wave; c < nchunks; c += kGroupWaves) {
        build_mask(c);
        const int t = c * 64 + lane;
        if (t < nb) {
            const unsigned long long below = (lane == 0) ? 0ull : (~0ull >> (64 - lane));
            int ej[kMaxSlots], pj[kMaxSlots];
#pragma unroll
            for (int j = 0; j < kMaxSlots; j++) {
                ej[j] = 0;
                pj[j] = -1;
                if (j < k) {
                    const int e = ids[(size_t)t * k + j];
                    if (e >= 0 && e < E) {
                        const int p = offs[e] + cnt[(size_t)c * E + e] + __popcll(mask[e] & below);
                        tok[p] = t;
                        pw[p] = w[(size_t)t * k + j];
                        ej[j] = e;
                        pj[j] = p;
                    }
                }
            }
            write_positions(pos, t, k, ej, pj);
        }
    }
}

// Expert e of the table, rows [blockIdx.x*4 + wave]; the group's tokens in
// tiles of kTT.  x [nb][ldx] fp32.  h [P][FF].
template <int GT, int UT>
__global__ __launch_bounds__(256) void grouped_gate_up_kernel(MoeShape s, const ExpertEntry* __restrict__ table,
                                                              const int* __restrict__ offs,
                                                              const int* __restrict__ tok,
                                                              const float* __restrict__ x, int ldx,
                                                              float* __restrict__ h, int tmin) {
    const int e = blockIdx.y;
    const int p0 = offs[e], p1 = offs[e + 1];
    if (p1 <= p0 || p1 - p0 < tmin) return;  // (smaller groups: the integer-dot kernels)
    const int lane = threadIdx.x & 63;
    const int r = blockIdx.x * 4 + (threadIdx.x >> 6);
    if (r >= s.FF) return;  // whole wave
    const ExpertEntry ent = table[e];
    const uint8_t* gr = ent.gate + (size_t)r * s.gate_rb;
    const uint8_t* ur = ent.up + (size_t)r * s.up_rb;
    const int nseg = s.D / 32;
    for (int t0 = p0; t0 < p1; t0 += kTT) {
        const int nt = min(kTT, p1 - t0);
        const float* xr[kTT];
#pragma unroll
        for (int t = 0; t < kTT; t++) xr[t] = x + (size_t)tok[t < nt ? t0 + t : t0] * ldx;
        float ag[kTT], au[kTT];
#pragma unroll
        for (int t = 0; t < kTT; t++) ag[t] = au[t] = 0.f;
        for (int sg = lane; sg < nseg; sg += 64) {
            float wg[32], wu[32];
            decode_row_seg<GT>(gr, sg, wg);
            decode_row_seg<UT>(ur, sg, wu);
#pragma unroll
            for (int t = 0; t < kTT; t++) {
                if (t < nt) {
                    const float4* xp = reinterpret_cast<const float4*>(xr[t] + (size_t)sg * 32);
                    float pg = 0.f, pu = 0.f;
#pragma unroll
                    for (int i = 0; i < 8; i++) {
                        const float4 v = xp[i];
                        pg = __builtin_fmaf(wg[4 * i], v.x, pg);
                        pg = __builtin_fmaf(wg[4 * i + 1], v.y, pg);
                        pg = __builtin_fmaf(wg[4 * i + 2], v.z, pg);
                        pg = __builtin_fmaf(wg[4 * i + 3], v.w, pg);
                        pu = __builtin_fmaf(wu[4 * i], v.x, pu);
                        pu = __builtin_fmaf(wu[4 * i + 1], v.y, pu);
                        pu = __builtin_fmaf(wu[4 * i + 2], v.z, pu);
                        pu = __builtin_fmaf(wu[4 * i + 3], v.w, pu);
                    }
                    ag[t] += pg;
                    au[t] += pu;
                }
            }
        }
#pragma unroll
        for (int t = 0; t < kTT; t++) {
            if (t < nt) {
                const float g = wave_sum(ag[t]), u = wave_sum(au[t]);
                if (lane == 0) h[(size_t)(t0 + t) * s.FF + r] = g / (1.0f + expf(-g)) * u;
            }
        }
    }
}

// yp [P][D] = down_e . h [P][FF] for the positions of expert e's group.
template <int DT>
__global__ __launch_bounds__(256) void grouped_down_kernel(MoeShape s, const ExpertEntry* __restrict__ table,
                                                           const int* __restrict__ offs, const float* __restrict__ h,
                                                           float* __restrict__ yp, int tmin) {
    const int e = blockIdx.y;
    const int p0 = offs[e], p1 = offs[e + 1];
    if (p1 <= p0 || p1 - p0 < tmin) return;
    const int lane = threadIdx.x & 63;
    const int r = blockIdx.x * 4 + (threadIdx.x >> 6);
    if (r >= s.D) return;
    const uint8_t* dr = table[e].down + (size_t)r * s.down_rb;
    const int nseg = s.FF / 32;
    for (int t0 = p0; t0 < p1; t0 += kTT) {
        const int nt = min(kTT, p1 - t0);
        float acc[kTT];
#pragma unroll
        for (int t = 0; t < kTT; t++) acc[t] = 0.f;
        for (int sg = lane; sg < nseg; sg += 64) {
            float wv[32];
            decode_row_seg<DT>(dr, sg, wv);
#pragma unroll
            for (int t = 0; t < kTT; t++) {
                if (t < nt) {
                    const float4* hp = reinterpret_cast<const float4*>(h + (size_t)(t0 + t) * s.FF + (size_t)sg * 32);
                    float p = 0.f;
#pragma unroll
                    for (int i = 0; i < 8; i++) {
                        const float4 v = hp[i];
                        p = __builtin_fmaf(wv[4 * i], v.x, p);
                        p = __builtin_fmaf(wv[4 * i + 1], v.y, p);
                        p = __builtin_fmaf(wv[4 * i + 2], v.z, p);
                        p = __builtin_fmaf(wv[4 * i + 3], v.w, p);
                    }
                    acc[t] += p;
                }
            }
        }
#pragma unroll
        for (int t = 0; t < kTT; t++) {
            if (t < nt) {
                const float v = wave_sum(acc[t]);
                if (lane == 0) yp[(size_t)(t0 + t) * s.D + r] = v;
            }
        }
    }
}

// y[t][d] = sum over the token's valid pairs, ascending expert id (the order
// of pos), of w * yp[pos][d].  One thread per (token, 4 consecutive d).
__global__ __launch_bounds__(256) void grouped_combine_kernel(const int* __restrict__ pos, const float* __restrict__ pw,
                                                              int nb, int k, int D, const float* __restrict__ yp,
                                                              float* __restrict__ y, int ldy) {
    const int q = blockIdx.x * blockDim.x + threadIdx.x;
    const int per_tok = D / 4;
    if (q >= nb * per_tok) return;
    const int t = q / per_tok, d = (q % per_tok) * 4;
    float4 v[kMaxSlots];
    float wv[kMaxSlots];
    bool ok[kMaxSlots];
#pragma unroll
    for (int r = 0; r < kMaxSlots; r++) {
        const int p = r < k ? pos[(size_t)t * k + r] : -1;
        ok[r] = p >= 0;
        v[r] = ok[r] ? *reinterpret_cast<const float4*>(yp + (size_t)p * D + d) : make_float4(0.f, 0.f, 0.f, 0.f);
        wv[r] = ok[r] ? pw[p] : 0.f;
    }
    float4 acc = make_float4(0.f, 0.f, 0.f, 0.f);
#pragma unroll
    for (int r = 0; r < kMaxSlots; r++) {
        if (!ok[r]) break;  // the valid pairs come first
        acc.x = __builtin_fmaf(wv[r], v[r].x, acc.x);
        acc.y = __builtin_fmaf(wv[r], v[r].y, acc.y);
        acc.z = __builtin_fmaf(wv[r], v[r].z, acc.z);
        acc.w = __builtin_fmaf(wv[r], v[r].w, acc.w);
    }
    *reinterpret_cast<float4*>(y + (size_t)t * ldy + d) = acc;
}

template <int GT>
static hipError_t gate_up_for(int ut, const MoeShape& s, dim3 g, const ExpertEntry* table, const int* offs,
                              const int* tok, const float* x, int ldx, float* h, int tmin, hipStream_t st) {
    switch (ut) {
        case kQ4_K: grouped_gate_up_kernel<GT, kQ4_K><<<g, 256, 0, st>>>(s, table, offs, tok, x, ldx, h, tmin); break;
        case kQ5_K: grouped_gate_up_kernel<GT, kQ5_K><<<g, 256, 0, st>>>(s, table, offs, tok, x, ldx, h, tmin); break;
        case kQ6_K: grouped_gate_up_kernel<GT, kQ6_K><<<g, 256, 0, st>>>(s, table, offs, tok, x, ldx, h, tmin); break;
        case kQ8_0: grouped_gate_up_kernel<GT, kQ8_0><<<g, 256, 0, st>>>(s, table, offs, tok, x, ldx, h, tmin); break;
        default: return hipErrorInvalidValue;
    }
    return hipSuccess;
}

int g_grouped_mfma = 1;  // matrix-core matmuls where the formats allow (see kernels_grouped_mfma.hip)

int set_grouped_mfma(int enable) {
    const int prev = g_grouped_mfma;
    if (enable >= 0) g_grouped_mfma = enable ? 1 : 0;
    return prev;
}

// Experts holding at most this many tokens run on the per-wave matrix-core
// kernels (kernels_grouped_wave.hip), the rest on the workgroup kernels.
int g_wave_max = 32;

int set_grouped_wave_max(int tmax) {
    const int prev = g_wave_max;
    if (tmax >= 0) g_wave_max = tmax > 32 ? 32 : tmax;
    return prev;
}

// The integer-dot kernels (kernels_grouped_dot.hip) take a batch of at most
// kDotWhole tokens whole (every expert then holds at most nb tokens: a
// token's pairs with one expert count once), and in larger batches the
// groups of at most g_dot_max tokens (none by default: there the few small
// groups ran as a long tail of their own).  g_dot_on = 0 turns the path off.
constexpr int kDotWhole = 32;
int g_dot_on = 1;
int g_dot_max = 0;

int set_grouped_dot_max(int tmax) {
    const int prev = !g_dot_on ? 0 : (g_dot_max > 0 ? g_dot_max : kDotWhole + 1);
    if (tmax == 0) {
        g_dot_on = 0;
    } else if (tmax > 0) {
        g_dot_on = 1;
        g_dot_max = tmax > kDotWhole ? 0 : tmax;
    }
    return prev;
}

size_t grouped_scratch_bytes(const MoeShape& s, int nb, int k, int n_expert) {
    const size_t P = (size_t)nb * k, nchunks = ((size_t)nb + 63) / 64;
    auto al = [](size_t b) { return (b + 255) & ~(size_t)255; };
    const size_t base = al(nchunks * n_expert * 4) + al(((size_t)n_expert + 1) * 4) + 3 * al(P * 4) +
                        al(P * s.FF * 4) + al(P * s.D * 4);
    // fp16 hi/lo activations and sub-block sums for the matrix-core path
    const size_t mf = 2 * al(P * s.D * 2) + 2 * al(P * (s.D / 32) * 2) + al(P * 4) + 2 * al(P * s.FF * 2) + al(P * 4);
    // x and h as int8 levels (+ scales, 32-value sums) for the integer-dot path
    const size_t dt = al(P * 3 * s.FF) + al(P * 3 * (s.FF / 64 + 1) * 4) + al(P * (s.FF / 32) * 4) +
                      al((size_t)nb * 3 * s.D) + al((size_t)nb * 3 * (s.D / 64 + 1) * 4) + al((size_t)nb * (s.D / 32) * 4);
    // + the work lists: integer-dot items, their counts, gate/up and down passes
    return base + mf + dt + al(P * 8) + al(4 * 4) + al((size_t)tile_cap(P, n_expert, 1, kMfmaGuTok) * 16) +
           al((size_t)tile_cap(P, n_expert, 1, kMfmaDnTok) * 16) + al((size_t)n_expert * 16);
}

// A second stream per device on which the per-wave matrix-core kernels (the
// small groups) run beside the workgroup kernels (the large groups) of the
// same matmul: the two write disjoint rows of h / yp, and each alone leaves
// the CUs waiting on memory latency (one 8-wave workgroup per CU for the
// workgroup kernels).  Fork: an event on the caller's stream that the side
// stream waits for; join: an event on the side stream that the caller's
// stream waits for.  Both streams keep the default priority.  Kept per device
// until the process ends.
struct SideStream {
    hipStream_t st = nullptr;
    hipEvent_t fork = nullptr, join = nullptr;
};
static std::mutex g_side_mu;
static SideStream g_side[64];

static SideStream* side_stream() {
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return nullptr;
    std::lock_guard<std::mutex> g(g_side_mu);
    SideStream& ss = g_side[dev];
    if (!ss.st) {
        hipStream_t st = nullptr;
        hipEvent_t a = nullptr, b = nullptr;
        if (hipStreamCreateWithFlags(&st, hipStreamNonBlocking) != hipSuccess) return nullptr;
        if (hipEventCreateWithFlags(&a, hipEventDisableTiming) != hipSuccess ||
            hipEventCreateWithFlags(&b, hipEventDisableTiming) != hipSuccess) {
            if (a) (void)hipEventDestroy(a);
            (void)hipStreamDestroy(st);
            return nullptr;
        }
        ss.st = st;
        ss.fork = a;
        ss.join = b;
    }
    return &ss;
}

// Runs small(side) and large(st) concurrently when a side stream exists
// (else both on st, in order), then joins: work queued on st afterwards waits
// for both.
template <class Small, class Large>
static hipError_t fork_join(hipStream_t st, bool any_small, bool any_large, Small small, Large large) {
    SideStream* ss = any_small && any_large ? side_stream() : nullptr;
    hipError_t e;
    if (!ss) {
        if (any_small && (e = small(st)) != hipSuccess) return e;
        if (any_large && (e = large(st)) != hipSuccess) return e;
        return hipSuccess;
    }
    if ((e = hipEventRecord(ss->fork, st)) != hipSuccess || (e = hipStreamWaitEvent(ss->st, ss->fork, 0)) != hipSuccess)
        return e;
    const hipError_t es = small(ss->st);
    // the join is recorded whatever the launch returned, so st never waits on a stale event
    if ((e = hipEventRecord(ss->join, ss->st)) != hipSuccess) return e;
    const hipError_t el = large(st);
    if ((e = hipStreamWaitEvent(st, ss->join, 0)) != hipSuccess) return e;
    return es != hipSuccess ? es : el;
}

bool grouped_supported(const MoeShape& s, int nb, int k, int n_expert) {
    return moe_shape_ok(s) && nb > 0 && k > 0 && k <= kMaxSlots && n_expert > 0 && n_expert <= kGroupMaxE &&
           s.D % 32 == 0 && s.FF % 32 == 0 && s.D % 4 == 0;
}

hipError_t launch_moe_grouped(const MoeShape& s, const ExpertEntry* table, int n_expert, const int* ids,
                              const float* w, int nb, int k, const float* x, int ldx, float* y, int ldy,
                              void* scratch, hipStream_t st) {
    if (!grouped_supported(s, nb, k, n_expert) || ldx < s.D || ldy < s.D || ldx % 4 || ldy % 4 || !scratch)
        return hipErrorInvalidValue;
    const size_t P = (size_t)nb * k, nchunks = ((size_t)nb + 63) / 64;
    auto al = [](size_t b) { return (b + 255) & ~(size_t)255; };
    uint8_t* b = static_cast<uint8_t*>(scratch);
    int* cnt = reinterpret_cast<int*>(b); b += al(nchunks * n_expert * 4);
    int* offs = reinterpret_cast<int*>(b); b += al(((size_t)n_expert + 1) * 4);
    int* tok = reinterpret_cast<int*>(b); b += al(P * 4);
    float* pw = reinterpret_cast<float*>(b); b += al(P * 4);
    int* pos = reinterpret_cast<int*>(b); b += al(P * 4);
    float* h = reinterpret_cast<float*>(b); b += al(P * s.FF * 4);
    float* yp = reinterpret_cast<float*>(b); b += al(P * s.D * 4);
    _Float16* xh = reinterpret_cast<_Float16*>(b); b += al(P * s.D * 2);
    _Float16* xl = reinterpret_cast<_Float16*>(b); b += al(P * s.D * 2);
    _Float16* xsh = reinterpret_cast<_Float16*>(b); b += al(P * (s.D / 32) * 2);
    _Float16* xsl = reinterpret_cast<_Float16*>(b); b += al(P * (s.D / 32) * 2);
    float* xsc = reinterpret_cast<float*>(b); b += al(P * 4);
    _Float16* hh = reinterpret_cast<_Float16*>(b); b += al(P * s.FF * 2);
    _Float16* hl = reinterpret_cast<_Float16*>(b); b += al(P * s.FF * 2);
    float* hsc = reinterpret_cast<float*>(b); b += al(P * 4);
    int8_t* dq = reinterpret_cast<int8_t*>(b); b += al(P * 3 * s.FF);
    float* dsc = reinterpret_cast<float*>(b); b += al(P * 3 * (s.FF / 64 + 1) * 4);
    float* ds32 = reinterpret_cast<float*>(b); b += al(P * (s.FF / 32) * 4);
    int8_t* xq = reinterpret_cast<int8_t*>(b); b += al((size_t)nb * 3 * s.D);
    float* xqs = reinterpret_cast<float*>(b); b += al((size_t)nb * 3 * (s.D / 64 + 1) * 4);
    float* xq32 = reinterpret_cast<float*>(b); b += al((size_t)nb * (s.D / 32) * 4);
    int2* items = reinterpret_cast<int2*>(b); b += al(P * 8);
    int* nitems = reinterpret_cast<int*>(b); b += al(4 * 4);  // the three lists' counts
    const int gcap = tile_cap(P, n_expert, 1, kMfmaGuTok), dcap = tile_cap(P, n_expert, 1, kMfmaDnTok);
    int4* gitems = reinterpret_cast<int4*>(b); b += al((size_t)gcap * 16);
    int4* ditems = reinterpret_cast<int4*>(b); b += al((size_t)dcap * 16);
    int4* vitems = reinterpret_cast<int4*>(b);
    const bool mf_gu = g_grouped_mfma && grouped_mfma_gate_up_ok(s);
    const bool mf_dn = g_grouped_mfma && grouped_mfma_down_ok(s);
    // Group sizes by path: 1..dmax the integer-dot kernels, then the per-wave
    // matrix-core kernels up to wave_max, then the workgroup kernels (or the
    // vector-ALU kernels for everything above dmax).  A group holds at most nb
    // tokens, so launches whose range starts above nb are skipped.
    const int dmax = !(g_dot_on && grouped_dot_gate_up_ok(s) && grouped_dot_down_ok(s)) ? 0
                     : (nb <= kDotWhole ? nb : g_dot_max);
    const bool dot = dmax > 0;
    const int rest = dmax + 1;  // smallest group left to the other kernels
    const int wave_max = g_wave_max;
    const int wg_min = wave_max + 1 > rest ? wave_max + 1 : rest;
    clear_stale_error();
    const size_t lds = (size_t)kGroupWaves * n_expert * 8 + (size_t)n_expert * 4 +
                       (nchunks <= (size_t)kGroupWaves ? nchunks * n_expert * 4 : 0);
    // the workgroup kernels' pass lists only where they run (a group holds at most nb tokens)
    const bool wg_gu = mf_gu && nb >= rest && nb >= wg_min, wg_dn = mf_dn && nb >= rest && nb >= wg_min;
    const bool wv = (mf_gu || mf_dn) && nb >= rest && wave_max >= rest;
    const GroupLists gl{dmax, wg_gu || wg_dn ? wg_min : INT_MAX, wv ? rest : INT_MAX, wave_max, items, nitems, gitems,
                        nitems + 1, ditems, nitems + 2, vitems, nitems + 3};
    group_pairs_kernel<<<1, kGroupThreads, lds, st>>>(ids, w, nb, k, n_expert, cnt, offs, tok, pw, pos, gl);
    // item slots: every item holds a pair, and an expert at most (dmax + 1) / 2
    const size_t cap_e = (size_t)n_expert * ((dmax + 1) / 2);
    const DotItems di{items, nitems, (int)(P < cap_e ? P : cap_e)};
    const TileItems gi{gitems, nitems + 1, tile_cap(P, n_expert, wg_min, kMfmaGuTok)};
    const TileItems dni{ditems, nitems + 2, tile_cap(P, n_expert, wg_min, kMfmaDnTok)};
    const TileItems vi{vitems, nitems + 3, (int)(P < (size_t)n_expert ? P : (size_t)n_expert)};
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return e;
    if (dot && ((e = launch_levels_rows(x, ldx, nb, s.D, xq, xqs, xq32, st)) != hipSuccess ||
                (e = launch_gate_up_dot(s, table, n_expert, di, tok, xq, xqs, xq32, h, 1, dmax, st)) != hipSuccess))
        return e;
    if (nb >= rest) {
        if (mf_gu) {
            if ((e = launch_prep_rows(offs, n_expert, tok, x, ldx, s.D, (int)P, xh, xl, xsh, xsl, xsc, st)) !=
                hipSuccess)
                return e;
            e = fork_join(
                st, wave_max >= rest, nb >= wg_min,
                [&](hipStream_t q) {
                    return launch_gate_up_wave(s, table, vi, xh, xl, xsh, xsl, xsc, h, rest, wave_max, q);
                },
                [&](hipStream_t q) {
                    return launch_gate_up_mfma(s, table, gi, xh, xl, xsh, xsl, xsc, h, wg_min, q);
                });
            if (e != hipSuccess) return e;
        } else {
            const dim3 ga((unsigned)((s.FF + 3) / 4), (unsigned)n_expert);
            switch (s.gate_type) {
                case kQ4_K: e = gate_up_for<kQ4_K>(s.up_type, s, ga, table, offs, tok, x, ldx, h, rest, st); break;
                case kQ5_K: e = gate_up_for<kQ5_K>(s.up_type, s, ga, table, offs, tok, x, ldx, h, rest, st); break;
                case kQ6_K: e = gate_up_for<kQ6_K>(s.up_type, s, ga, table, offs, tok, x, ldx, h, rest, st); break;
                case kQ8_0: e = gate_up_for<kQ8_0>(s.up_type, s, ga, table, offs, tok, x, ldx, h, rest, st); break;
                default: e = hipErrorInvalidValue;
            }
            if (e != hipSuccess) return e;
            if ((e = hipGetLastError()) != hipSuccess) return e;
        }
    }
    if (dot && ((e = launch_levels_rows(h, s.FF, (int)P, s.FF, dq, dsc, ds32, st)) != hipSuccess ||
                (e = launch_down_dot(s, table, n_expert, di, dq, dsc, ds32, yp, 1, dmax, st)) != hipSuccess))
        return e;
    if (nb >= rest) {
        if (mf_dn) {
            if ((e = launch_prep_rows(offs, n_expert, nullptr, h, s.FF, s.FF, (int)P, hh, hl, nullptr, nullptr, hsc,
                                      st)) != hipSuccess)
                return e;
            e = fork_join(
                st, wave_max >= rest, nb >= wg_min,
                [&](hipStream_t q) { return launch_down_wave(s, table, vi, hh, hl, hsc, yp, rest, wave_max, q); },
                [&](hipStream_t q) { return launch_down_mfma(s, table, dni, hh, hl, hsc, yp, wg_min, q); });
            if (e != hipSuccess) return e;
        } else {
            const dim3 gd((unsigned)((s.D + 3) / 4), (unsigned)n_expert);
            switch (s.down_type) {
                case kQ4_K: grouped_down_kernel<kQ4_K><<<gd, 256, 0, st>>>(s, table, offs, h, yp, rest); break;
                case kQ5_K: grouped_down_kernel<kQ5_K><<<gd, 256, 0, st>>>(s, table, offs, h, yp, rest); break;
                case kQ6_K: grouped_down_kernel<kQ6_K><<<gd, 256, 0, st>>>(s, table, offs, h, yp, rest); break;
                case kQ8_0: grouped_down_kernel<kQ8_0><<<gd, 256, 0, st>>>(s, table, offs, h, yp, rest); break;
                default: return hipErrorInvalidValue;
            }
            if ((e = hipGetLastError()) != hipSuccess) return e;
        }
    }
    const size_t nthr = (size_t)nb * (s.D / 4);
    grouped_combine_kernel<<<(unsigned)((nthr + 255) / 256), 256, 0, st>>>(pos, pw, nb, k, s.D, yp, y, ldy);
    return hipGetLastError();
}

}  // namespace eahmmf
