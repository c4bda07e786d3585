// kernels_grouped_wave.hip - the ragged grouped expert block's matrix-core
// matmuls for experts holding few tokens (up to 32: one 16-token tile up to
// 16 tokens, two above).
//
// The workgroup-per-row-block kernels of kernels_grouped_mfma.hip decode a
// 64- or 128-row block's weight fragments once and share them through LDS
// with eight waves, one 16-token tile each; for an expert that holds one or
// two tiles' worth of tokens most of those waves have no tokens, and the
// per-sub-block LDS hand-off and barrier set the pace.  Here a wave is
// independent: it owns 16 rows, decodes its own A fragments from bytes it
// loads a super-block ahead, reads its B fragments (the tokens' fp16 hi/lo
// activations) straight from memory three sub-blocks ahead, and runs the
// MFMAs for its NT tiles.  No LDS, no barriers; the exactness argument of
// kernels_grouped_mfma.hip is unchanged (integer weight fragments, hi + lo
// activations, scales and the min term applied in fp32 per super-block).
#include "internal.h"
#include "kquant.h"
#include "mfma_frag.h"

namespace eahmmf {

constexpr int kWaveWaves = 4;  // waves per workgroup (independent)
constexpr int kBAhead = 3;     // B fragments loaded this many sub-blocks ahead (ring of 4)

template <int T>
struct KRowSb {   // one lane's bytes of one row for one super-block (Q4_K / Q5_K)
    uint4 hdr;    // d, dmin, scales
    uint2 qh;     // Q5_K high bits of the lane's 8 columns
    uint2 q[4];   // 4-bit codes of the lane's columns, groups 0..3 (both nibbles)
};

template <int T>
__device__ __forceinline__ void krow_load(const uint8_t* row, int b, int kq, KRowSb<T>& r) {
    constexpr int QS = T == kQ5_K ? 48 : 16;
    const uint8_t* sb = row + (size_t)b * Fmt<T>::bytes;
    r.hdr = gld16(sb);
    if (T == kQ5_K) r.qh = ld8(sb + 16 + kq * 8);
#pragma unroll
    for (int g = 0; g < 4; g++) r.q[g] = ld8(sb + QS + 32 * g + kq * 8);
}

// A fragment of sub-block j: sc_j * q (exact small integers)
template <int T>
__device__ __forceinline__ f16x8 krow_frag(const KRowSb<T>& r, int j) {
    uint32_t sc, mn;
    scale_min_k4(j, r.hdr.y, r.hdr.z, r.hdr.w, sc, mn);
    const int g = j >> 1, hh = j & 1;
    uint2 c = make_uint2((r.q[g].x >> (4 * hh)) & 0x0F0F0F0Fu, (r.q[g].y >> (4 * hh)) & 0x0F0F0F0Fu);
    if (T == kQ5_K) {
        c.x |= ((r.qh.x >> j) & 0x01010101u) << 4;
        c.y |= ((r.qh.y >> j) & 0x01010101u) << 4;
    }
    return codes_times(c, (_Float16)(float)sc, (_Float16)0.0f);
}

// Min-term A fragment of a super-block: m_0..m_7 on the lanes with kq == 0.
template <int T>
__device__ __forceinline__ f16x8 krow_mins(const KRowSb<T>& r, int kq) {
    f16x8 mv = {};
    if (kq == 0) {
#pragma unroll
        for (int j = 0; j < 8; j++) {
            uint32_t sc, mn;
            scale_min_k4(j, r.hdr.y, r.hdr.z, r.hdr.w, sc, mn);
            mv[j] = (_Float16)(float)mn;
        }
    }
    return mv;
}

// gate/up of one expert's 16-row strip for its (at most 16 * NT) tokens:
// h[q][r] = silu(g) * u.  Experts outside [tmin, tmax] tokens leave at once.
template <int T, int NT>
__device__ __forceinline__ void gate_up_wave_body(const MoeShape& s, const ExpertEntry* __restrict__ table, int e,
                                                  int p0, int p1, const _Float16* __restrict__ xh,
                                                  const _Float16* __restrict__ xl, const _Float16* __restrict__ xsh,
                                                  const _Float16* __restrict__ xsl, const float* __restrict__ xscale,
                                                  float* __restrict__ h) {
    const int w = __builtin_amdgcn_readfirstlane(threadIdx.x / 64), l = threadIdx.x % 64;
    const int lr = l & 15, kq = l >> 4;
    const int r0 = (blockIdx.x * kWaveWaves + w) * 16;
    if (r0 >= s.FF) return;
    const int D = s.D, nsub = D / 32, nsb = D / 256;
    const ExpertEntry ent = table[e];
    const uint8_t* grow = ent.gate + (size_t)(r0 + lr) * s.gate_rb;
    const uint8_t* urow = ent.up + (size_t)(r0 + lr) * s.up_rb;
    int qv[NT];
#pragma unroll
    for (int t = 0; t < NT; t++) {
        const int q = p0 + 16 * t + lr;
        qv[t] = q < p1 ? q : p1 - 1;  // a valid row for the loads; masked at the end
    }
    f16x8 bh[kBAhead + 1][NT], bl[kBAhead + 1][NT];
    auto bload = [&](int jj, int slot) {
#pragma unroll
        for (int t = 0; t < NT; t++) {
            bh[slot][t] = *reinterpret_cast<const f16x8*>(xh + (size_t)qv[t] * D + jj * 32 + kq * 8);
            bl[slot][t] = *reinterpret_cast<const f16x8*>(xl + (size_t)qv[t] * D + jj * 32 + kq * 8);
        }
    };
    KRowSb<T> gc, uc, gn, un;
    krow_load<T>(grow, 0, kq, gc);
    krow_load<T>(urow, 0, kq, uc);
#pragma unroll
    for (int j = 0; j < kBAhead; j++) bload(j, j);
    f32x4 og[NT], ou[NT];
#pragma unroll
    for (int t = 0; t < NT; t++) og[t] = ou[t] = (f32x4){0.f, 0.f, 0.f, 0.f};
    for (int b = 0; b < nsb; b++) {
        if (b + 1 < nsb) {
            krow_load<T>(grow, b + 1, kq, gn);
            krow_load<T>(urow, b + 1, kq, un);
        }
        // the tokens' sub-block sums of this super-block (lanes kq == 0)
        f16x8 sh8[NT], sl8[NT];
#pragma unroll
        for (int t = 0; t < NT; t++) {
            const f16x8 zero8 = {};
            sh8[t] = kq == 0 ? *reinterpret_cast<const f16x8*>(xsh + (size_t)qv[t] * nsub + 8 * b) : zero8;
            sl8[t] = kq == 0 ? *reinterpret_cast<const f16x8*>(xsl + (size_t)qv[t] * nsub + 8 * b) : zero8;
        }
        f32x4 ag[NT], au[NT];
#pragma unroll
        for (int t = 0; t < NT; t++) ag[t] = au[t] = (f32x4){0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int j = 0; j < 8; j++) {
            const int jj = 8 * b + j;
            if (jj + kBAhead < nsub) bload(jj + kBAhead, (j + kBAhead) % (kBAhead + 1));
            const int slot = j % (kBAhead + 1);
            const f16x8 Ag = krow_frag<T>(gc, j), Au = krow_frag<T>(uc, j);
#pragma unroll
            for (int t = 0; t < NT; t++) {
                ag[t] = mfma(Ag, bh[slot][t], ag[t]);
                au[t] = mfma(Au, bh[slot][t], au[t]);
            }
#pragma unroll
            for (int t = 0; t < NT; t++) {
                ag[t] = mfma(Ag, bl[slot][t], ag[t]);
                au[t] = mfma(Au, bl[slot][t], au[t]);
            }
        }
        // end of the super-block: min term, then d / dmin of the C rows 4kq + i
        const f16x8 Mg = krow_mins<T>(gc, kq), Mu = krow_mins<T>(uc, kq);
        float dg[4], dmg[4], du[4], dmu[4];
#pragma unroll
        for (int i = 0; i < 4; i++) {
            const uint32_t hg = (uint32_t)__shfl((int)gc.hdr.x, 4 * kq + i, 64);
            const uint32_t hu = (uint32_t)__shfl((int)uc.hdr.x, 4 * kq + i, 64);
            dg[i] = (float)__builtin_bit_cast(_Float16, (uint16_t)(hg & 0xFFFFu));
            dmg[i] = (float)__builtin_bit_cast(_Float16, (uint16_t)(hg >> 16)) / kSumScale;
            du[i] = (float)__builtin_bit_cast(_Float16, (uint16_t)(hu & 0xFFFFu));
            dmu[i] = (float)__builtin_bit_cast(_Float16, (uint16_t)(hu >> 16)) / kSumScale;
        }
#pragma unroll
        for (int t = 0; t < NT; t++) {
            f32x4 zg = mfma(Mg, sh8[t], (f32x4){0.f, 0.f, 0.f, 0.f});
            f32x4 zu = mfma(Mu, sh8[t], (f32x4){0.f, 0.f, 0.f, 0.f});
            zg = mfma(Mg, sl8[t], zg);
            zu = mfma(Mu, sl8[t], zu);
#pragma unroll
            for (int i = 0; i < 4; i++) {
                og[t][i] += dg[i] * ag[t][i] - dmg[i] * zg[i];
                ou[t][i] += du[i] * au[t][i] - dmu[i] * zu[i];
            }
        }
        gc = gn;
        uc = un;
    }
#pragma unroll
    for (int t = 0; t < NT; t++) {
        const int q = p0 + 16 * t + lr;
        if (q >= p1) continue;
        const float xs = xscale[q];
#pragma unroll
        for (int i = 0; i < 4; i++) {
            const int r = r0 + 4 * kq + i;
            const float gv = og[t][i] * xs, uv = ou[t][i] * xs;
            h[(size_t)q * s.FF + r] = gv / (1.0f + expf(-gv)) * uv;
        }
    }
}

// One launch for groups of tmin..tmax tokens: one 16-token tile for groups of
// at most 16, two above.
// The workgroup's expert (blockIdx.y of the list): false past the list's end.
__device__ __forceinline__ bool expert_item(const TileItems& g, int& e, int& p0, int& p1) {
    const int i = (int)blockIdx.y;
    const int total = *g.n;
    const int4 v = g.items[i];  // in bounds: the grid has cap rows, the list cap slots
    if (i >= total) return false;
    e = v.x;
    p0 = v.w;
    p1 = v.z;
    return true;
}

template <int T>
__global__ __launch_bounds__(kWaveWaves * 64) void gate_up_wave_kernel(
    MoeShape s, const ExpertEntry* __restrict__ table, TileItems wi, const _Float16* __restrict__ xh,
    const _Float16* __restrict__ xl, const _Float16* __restrict__ xsh, const _Float16* __restrict__ xsl,
    const float* __restrict__ xscale, float* __restrict__ h, int tmin, int tmax) {
    int e, p0, p1;
    if (!expert_item(wi, e, p0, p1)) return;
    const int n = p1 - p0;
    if (n < tmin || n > tmax || n <= 0) return;
    if (n <= 16)
        gate_up_wave_body<T, 1>(s, table, e, p0, p1, xh, xl, xsh, xsl, xscale, h);
    else
        gate_up_wave_body<T, 2>(s, table, e, p0, p1, xh, xl, xsh, xsl, xscale, h);
}

// down (Q6_K) of one expert's 16-row strip: yp[q][r] = down_r . h[q], h as
// scaled fp16 hi/lo.  A Q6_K 32-value quarter's weights (q - 32) * sc are
// split into the exact parts 16 * (q - 32) * (sc >> 4) and (q - 32) * (sc & 15).
struct Q6Lane {  // one lane's bytes of one row for one 64-value chunk (quarters u0, u0 + 1 of half n)
    uint2 ql0, ql1, qh;
    int sc0, sc1;
};

__device__ __forceinline__ void q6_load(const uint8_t* row, int c, int kq, Q6Lane& a) {
    const int b = c >> 2, g = c & 3, n = g >> 1, u0 = 2 * (g & 1);
    const uint8_t* blk = row + (size_t)b * 210;
    a.ql0 = ld8_a2(blk + 64 * n + kq * 8);
    a.ql1 = ld8_a2(blk + 64 * n + 32 + kq * 8);
    a.qh = ld8_a2(blk + 128 + 32 * n + kq * 8);
    a.sc0 = ld_i8(blk + 192 + 8 * n + (kq >> 1) + 2 * u0);
    a.sc1 = ld_i8(blk + 192 + 8 * n + (kq >> 1) + 2 * (u0 + 1));
}

template <int NT>
__device__ __forceinline__ void down_wave_q6k_body(const MoeShape& s, const ExpertEntry* __restrict__ table, int e,
                                                   int p0, int p1, const _Float16* __restrict__ hh,
                                                   const _Float16* __restrict__ hl, const float* __restrict__ hscale,
                                                   float* __restrict__ yp) {
    const int w = __builtin_amdgcn_readfirstlane(threadIdx.x / 64), l = threadIdx.x % 64;
    const int lr = l & 15, kq = l >> 4;
    const int r0 = (blockIdx.x * kWaveWaves + w) * 16;
    if (r0 >= s.D) return;
    const int FF = s.FF, nq = FF / 32, nch = FF / 64;
    const uint8_t* dbase = table[e].down;
    const uint8_t* arow = dbase + (size_t)(r0 + lr) * s.down_rb;
    int qv[NT];
#pragma unroll
    for (int t = 0; t < NT; t++) {
        const int q = p0 + 16 * t + lr;
        qv[t] = q < p1 ? q : p1 - 1;
    }
    // B ring over quarters (32 K values)
    f16x8 bh[kBAhead + 1][NT], bl[kBAhead + 1][NT];
    auto bload = [&](int qq, int slot) {
#pragma unroll
        for (int t = 0; t < NT; t++) {
            bh[slot][t] = *reinterpret_cast<const f16x8*>(hh + (size_t)qv[t] * FF + qq * 32 + kq * 8);
            bl[slot][t] = *reinterpret_cast<const f16x8*>(hl + (size_t)qv[t] * FF + qq * 32 + kq * 8);
        }
    };
#pragma unroll
    for (int j = 0; j < kBAhead; j++) bload(j, j);
    Q6Lane cur, nx;
    q6_load(arow, 0, kq, cur);
    f32x4 out[NT];
#pragma unroll
    for (int t = 0; t < NT; t++) out[t] = (f32x4){0.f, 0.f, 0.f, 0.f};
    for (int b = 0; b < nch / 4; b++) {  // super-blocks: four 64-value chunks
        float dsb[4];
#pragma unroll
        for (int i = 0; i < 4; i++) dsb[i] = half_at(dbase + (size_t)(r0 + 4 * kq + i) * s.down_rb + (size_t)b * 210 + 208);
        f32x4 acc[NT];
#pragma unroll
        for (int t = 0; t < NT; t++) acc[t] = (f32x4){0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int g = 0; g < 4; g++) {
            const int c = 4 * b + g;
            if (c + 1 < nch) q6_load(arow, c + 1, kq, nx);
#pragma unroll
            for (int qq = 0; qq < 2; qq++) {  // the chunk's two quarters
                const int jq = 2 * c + qq, jl = 2 * g + qq;  // quarter index (global, in the super-block)
                if (jq + kBAhead < nq) bload(jq + kBAhead, (jl + kBAhead) % (kBAhead + 1));
                const int slot = jl % (kBAhead + 1);
                const int u = 2 * (g & 1) + qq;
                const uint2 ql = qq ? cur.ql1 : cur.ql0;
                const int sc = qq ? cur.sc1 : cur.sc0;
                const int sh4 = u >= 2 ? 4 : 0;
                const uint2 code =
                    make_uint2(((ql.x >> sh4) & 0x0F0F0F0Fu) | (((cur.qh.x >> (2 * u)) & 0x03030303u) << 4),
                               ((ql.y >> sh4) & 0x0F0F0F0Fu) | (((cur.qh.y >> (2 * u)) & 0x03030303u) << 4));
                const f16x8 A1 = codes_times(code, (_Float16)(float)(16 * (sc >> 4)), (_Float16)-32.0f);
                const f16x8 A2 = codes_times(code, (_Float16)(float)(sc & 15), (_Float16)-32.0f);
#pragma unroll
                for (int t = 0; t < NT; t++) {
                    acc[t] = mfma(A1, bh[slot][t], acc[t]);
                    acc[t] = mfma(A2, bh[slot][t], acc[t]);
                    acc[t] = mfma(A1, bl[slot][t], acc[t]);
                    acc[t] = mfma(A2, bl[slot][t], acc[t]);
                }
            }
            cur = nx;
        }
#pragma unroll
        for (int t = 0; t < NT; t++)
#pragma unroll
            for (int i = 0; i < 4; i++) out[t][i] += dsb[i] * acc[t][i];
    }
#pragma unroll
    for (int t = 0; t < NT; t++) {
        const int q = p0 + 16 * t + lr;
        if (q >= p1) continue;
        const float hs = hscale[q];
#pragma unroll
        for (int i = 0; i < 4; i++) yp[(size_t)q * s.D + r0 + 4 * kq + i] = out[t][i] * hs;
    }
}

__global__ __launch_bounds__(kWaveWaves * 64) void down_wave_q6k_kernel(
    MoeShape s, const ExpertEntry* __restrict__ table, TileItems wi, const _Float16* __restrict__ hh,
    const _Float16* __restrict__ hl, const float* __restrict__ hscale, float* __restrict__ yp, int tmin, int tmax) {
    int e, p0, p1;
    if (!expert_item(wi, e, p0, p1)) return;
    const int n = p1 - p0;
    if (n < tmin || n > tmax || n <= 0) return;
    if (n <= 16)
        down_wave_q6k_body<1>(s, table, e, p0, p1, hh, hl, hscale, yp);
    else
        down_wave_q6k_body<2>(s, table, e, p0, p1, hh, hl, hscale, yp);
}

// ---------------------------------------------------------------------------

bool grouped_wave_gate_up_ok(const MoeShape& s) { return grouped_mfma_gate_up_ok(s); }
bool grouped_wave_down_ok(const MoeShape& s) { return grouped_mfma_down_ok(s); }

hipError_t launch_gate_up_wave(const MoeShape& s, const ExpertEntry* table, TileItems wi, const _Float16* xh,
                               const _Float16* xl, const _Float16* xsh, const _Float16* xsl, const float* xscale,
                               float* h, int tmin, int tmax, hipStream_t st) {
    if (wi.cap < 1) return hipErrorInvalidValue;
    const dim3 g((unsigned)((s.FF / 16 + kWaveWaves - 1) / kWaveWaves), (unsigned)wi.cap);
    if (s.gate_type == kQ4_K)
        gate_up_wave_kernel<kQ4_K><<<g, kWaveWaves * 64, 0, st>>>(s, table, wi, xh, xl, xsh, xsl, xscale, h, tmin, tmax);
    else
        gate_up_wave_kernel<kQ5_K><<<g, kWaveWaves * 64, 0, st>>>(s, table, wi, xh, xl, xsh, xsl, xscale, h, tmin, tmax);
    return hipGetLastError();
}

hipError_t launch_down_wave(const MoeShape& s, const ExpertEntry* table, TileItems wi, const _Float16* hh,
                            const _Float16* hl, const float* hscale, float* yp, int tmin, int tmax,
                            hipStream_t st) {
    if (wi.cap < 1) return hipErrorInvalidValue;
    const dim3 g((unsigned)((s.D / 16 + kWaveWaves - 1) / kWaveWaves), (unsigned)wi.cap);
    down_wave_q6k_kernel<<<g, kWaveWaves * 64, 0, st>>>(s, table, wi, hh, hl, hscale, yp, tmin, tmax);
    return hipGetLastError();
}

}  // namespace eahmmf
