// kernels_grouped_mfma.hip - matrix-core (MFMA) matmuls of the ragged grouped
// expert block for the K-quant formats of Q4_K_M layers: gate/up in Q4_K or
// Q5_K, down in Q6_K.
//
// Exactness.  v_mfma_f32_16x16x32_f16 multiplies fp16 operands exactly and
// accumulates in fp32, so it is fed only values that fp16 holds exactly:
//   weights      small integers: Q4_K/Q5_K q*sc (<= 31*63 = 1953); Q6_K
//                (q-32)*sc split as 16*(q-32)*(sc>>4) (a multiple of 16 with
//                |.| <= 4096) plus (q-32)*(sc&15) (|.| <= 480)
//   activations  each row scaled by a power of two so that max|v| < 2^13,
//                then split v = hi + lo with hi = fp16(v), lo = fp16(v - hi)
//                (about 22 significant bits)
// The per-super-block factors (d, dmin: fp16 values) and the row's power of
// two are applied in fp32 after each super-block, and the Q4_K/Q5_K min term
// sum_j m_j * sum(x over sub-block j) is a second, small MFMA over the
// sub-block sums.  So the products equal the reference's dequantized weight
// times activation up to the fp32 rounding of the sums (the same bar as any
// fp32 matmul).
//
// Operand layout (16x16x32): lane l holds A[l%16][8*(l/16) + i],
// B[8*(l/16) + i][l%16] and C[4*(l/16) + i][l%16], i < 8 (C: i < 4).
//
// Work split: a workgroup covers 64 of an expert's grouped tokens (four
// 16-token tiles) and a block of its output rows (16 per wave); grid.z walks
// the expert's tokens in passes of 64 and workgroups past the end leave at
// once.
#include "internal.h"
#include "kquant.h"
#include "mfma_frag.h"

namespace eahmmf {

// ---------------------------------------------------------------------------
// Activation rows -> scaled fp16 hi/lo (+ 32-value sums).  One workgroup per
// position q < offs[E]; the row is src + (tok ? tok[q] : q) * ld, n values.
__global__ __launch_bounds__(256) void prep_rows_kernel(const int* __restrict__ offs, int E,
                                                        const int* __restrict__ tok, const float* __restrict__ src,
                                                        int ld, int n, _Float16* __restrict__ vh,
                                                        _Float16* __restrict__ vl, _Float16* __restrict__ sh,
                                                        _Float16* __restrict__ sl, float* __restrict__ vscale) {
    __shared__ float wmax[4];
    const int q = blockIdx.x;
    if (q >= offs[E]) return;
    const float* row = src + (size_t)(tok ? tok[q] : q) * ld;
    const int tid = threadIdx.x;
    float m = 0.f;
    for (int c = tid; c < n / 8; c += 256) {
        const float4 a = reinterpret_cast<const float4*>(row)[2 * c], b = reinterpret_cast<const float4*>(row)[2 * c + 1];
        m = fmaxf(m, fmaxf(fmaxf(fabsf(a.x), fabsf(a.y)), fmaxf(fabsf(a.z), fabsf(a.w))));
        m = fmaxf(m, fmaxf(fmaxf(fabsf(b.x), fabsf(b.y)), fmaxf(fabsf(b.z), fabsf(b.w))));
    }
    for (int off = 32; off > 0; off >>= 1) m = fmaxf(m, __shfl_xor(m, off, 64));
    if ((tid & 63) == 0) wmax[tid >> 6] = m;
    __syncthreads();
    m = fmaxf(fmaxf(wmax[0], wmax[1]), fmaxf(wmax[2], wmax[3]));
    int ex = 0;
    if (m > 0.f) (void)frexpf(m, &ex);  // m < 2^ex
    const float up = ldexpf(1.0f, 13 - ex), down = ldexpf(1.0f, ex - 13);
    if (tid == 0) vscale[q] = m > 0.f ? down : 1.0f;
    const float sc = m > 0.f ? up : 1.0f;
    for (int c = tid; c < n / 8; c += 256) {  // a 32-value block is four consecutive c (lanes)
        const float4 a = reinterpret_cast<const float4*>(row)[2 * c], b = reinterpret_cast<const float4*>(row)[2 * c + 1];
        const float v[8] = {a.x * sc, a.y * sc, a.z * sc, a.w * sc, b.x * sc, b.y * sc, b.z * sc, b.w * sc};
        f16x8 hi, lo;
        float s = 0.f;
#pragma unroll
        for (int i = 0; i < 8; i++) {
            hi[i] = (_Float16)v[i];
            lo[i] = (_Float16)(v[i] - (float)hi[i]);
            s += v[i];
        }
        *reinterpret_cast<f16x8*>(vh + (size_t)q * n + 8 * c) = hi;
        *reinterpret_cast<f16x8*>(vl + (size_t)q * n + 8 * c) = lo;
        if (sh) {
            s += __shfl_xor(s, 1, 64);
            s += __shfl_xor(s, 2, 64);
            if ((c & 3) == 0) {
                const float ss = s * kSumScale;
                const _Float16 h = (_Float16)ss;
                sh[(size_t)q * (n / 32) + c / 4] = h;
                sl[(size_t)q * (n / 32) + c / 4] = (_Float16)(ss - (float)h);
            }
        }
    }
}

// ---------------------------------------------------------------------------
// gate/up (Q4_K or Q5_K, same type) for one expert: h[q][r] = silu(g) * u.
//
// Weights stationary: a workgroup of 8 waves covers 64 rows (4 row tiles of
// 16) and 128 of the expert's tokens, one 16-token tile per wave.  For every
// 32-value sub-block all 512 threads decode the 64 rows' exact-integer fp16
// A fragments (gate and up) into LDS, double-buffered, so each fragment is
// built once per workgroup and read by every wave; each wave then runs 4 row
// tiles x (gate, up) x (hi, lo) MFMAs against its own token tile, whose
// activations stream from global memory three sub-blocks ahead.  Per
// super-block the rows' mins (as A fragments of the min-term MFMA) and their
// (d, dmin) are staged the same way.  The weight bytes a thread decodes are
// loaded one super-block ahead.
constexpr int kGuWaves = 8;
constexpr int kGuRowTiles = 4;
constexpr int kGuRows = 16 * kGuRowTiles;  // 64
constexpr int kGuFrags = 2 * kGuRowTiles * 64 / 512;  // A fragments each thread decodes per sub-block
constexpr int kGuTok = 16 * kGuWaves;      // 128 tokens per workgroup pass
constexpr int kChunkK = 64;                // the down kernel's LDS chunk
constexpr int kBRow = kChunkK + 8;         // halfs per token row in the down kernel's LDS: 144 B

struct GuLds {
    uint4 a[2][2][kGuRowTiles][64];     // [sub-block parity][gate, up][row tile][lane]: A fragments
    uint4 amin[2][2][kGuRowTiles][64];  // [super-block parity][gate, up][row tile][lane]: min-term A
    uint32_t dd[2][2][kGuRows];         // [super-block parity][gate, up][row]: d | dmin << 16
};

template <int T>
struct GuRowSb {  // the weight bytes one thread decodes for a super-block (one row of one matrix)
    uint4 hdr;     // d, dmin, scales
    uint2 qh;      // Q5_K high bits of the thread's 8 columns
    uint2 q[4];    // 4-bit codes of the thread's columns for g = 0..3 (both nibbles)
};

static_assert(kGuTok == kMfmaGuTok && kPassTok == kMfmaDnTok, "pass lists: tile sizes");

// The workgroup's pass (blockIdx.y of the list): false past the list's end.
__device__ __forceinline__ bool tile_item(const TileItems& g, int& e, int& pb, int& p1, int& p0) {
    const int i = (int)blockIdx.y;
    const int total = *g.n;
    const int4 v = g.items[i];  // in bounds: the grid has cap rows, the list cap slots
    if (i >= total) return false;
    e = v.x;
    pb = v.y;
    p1 = v.z;
    p0 = v.w;
    return true;
}

template <int T>
__global__ __launch_bounds__(512) void gate_up_mfma_kernel(MoeShape s, const ExpertEntry* __restrict__ table,
                                                           TileItems gi,
                                                           const _Float16* __restrict__ xh,
                                                           const _Float16* __restrict__ xl,
                                                           const _Float16* __restrict__ xsh,
                                                           const _Float16* __restrict__ xsl,
                                                           const float* __restrict__ xscale, float* __restrict__ h,
                                                           int tmin) {
    static_assert(T == kQ4_K || T == kQ5_K, "gate/up MFMA path: Q4_K or Q5_K");
    constexpr int BB = Fmt<T>::bytes;
    constexpr int QS = T == kQ5_K ? 48 : 16;  // offset of the 4-bit codes in a super-block
    __shared__ GuLds L;
    int e, p0, p1, pb;
    if (!tile_item(gi, e, pb, p1, p0) || pb >= p1 || p1 - p0 < tmin) return;  // whole workgroup
    const int tid = threadIdx.x, wave = tid >> 6, l = tid & 63;
    const int lr = l & 15, kq = l >> 4;
    const int rw = blockIdx.x * kGuRows;
    const int D = s.D, nsub = D / 32, nsb = D / 256;
    const ExpertEntry ent = table[e];
    // this wave's tokens; a wave whose tile starts past the group only decodes
    const int q = pb + wave * 16 + lr;
    const bool qok = q < p1;
    const bool busy = pb + wave * 16 < p1;  // wave-uniform
    const int qc = qok ? q : p1 - 1;        // a valid row for the activation loads
    // decode assignment: thread -> (matrix, row tile, lane) fragment(s), fixed for the whole K loop
    int dm[kGuFrags], drt[kGuFrags], dll[kGuFrags], drow[kGuFrags];
    bool dok[kGuFrags];
    const uint8_t* drp[kGuFrags];
#pragma unroll
    for (int i = 0; i < kGuFrags; i++) {
        const int f = tid + 512 * i;
        dm[i] = f / (kGuRowTiles * 64);
        drt[i] = (f >> 6) % kGuRowTiles;
        dll[i] = f & 63;
        drow[i] = rw + drt[i] * 16 + (dll[i] & 15);
        dok[i] = drow[i] < s.FF;
        drp[i] = (dm[i] ? ent.up : ent.gate) + (size_t)(dok[i] ? drow[i] : 0) * (dm[i] ? s.up_rb : s.gate_rb);
    }
    auto rload = [&](int b, int i, GuRowSb<T>& r) {
        const uint8_t* sb = drp[i] + (size_t)b * BB;
        const int dkq = dll[i] >> 4;
        r.hdr = gld16(sb);
        if (T == kQ5_K) r.qh = ld8(sb + 16 + dkq * 8);
#pragma unroll
        for (int g = 0; g < 4; g++) r.q[g] = ld8(sb + QS + 32 * g + dkq * 8);
    };
    // the fragment of sub-block j for fragment slot i, written to parity buffer par
    auto decode = [&](int j, int i, const GuRowSb<T>& r, int par) {
        uint32_t sc, mn;
        scale_min_k4(j, r.hdr.y, r.hdr.z, r.hdr.w, sc, mn);
        const int g = j >> 1, hh = j & 1;
        uint2 c = make_uint2((r.q[g].x >> (4 * hh)) & 0x0F0F0F0Fu, (r.q[g].y >> (4 * hh)) & 0x0F0F0F0Fu);
        if (T == kQ5_K) {
            c.x |= ((r.qh.x >> j) & 0x01010101u) << 4;
            c.y |= ((r.qh.y >> j) & 0x01010101u) << 4;
        }
        const f16x8 A = codes_times(c, (_Float16)(float)sc, (_Float16)0.0f);
        L.a[par][dm[i]][drt[i]][dll[i]] = __builtin_bit_cast(uint4, A);
    };
    // per super-block: min-term fragments (m_0..m_7 on lanes with kq == 0) and (d, dmin)
    auto sbstage = [&](int b, int i, const GuRowSb<T>& r) {
        f16x8 mv = {};
        if ((dll[i] >> 4) == 0) {
#pragma unroll
            for (int j = 0; j < 8; j++) {
                uint32_t sc, mn;
                scale_min_k4(j, r.hdr.y, r.hdr.z, r.hdr.w, sc, mn);
                mv[j] = (_Float16)(float)mn;
            }
        }
        L.amin[b & 1][dm[i]][drt[i]][dll[i]] = __builtin_bit_cast(uint4, mv);
        if ((dll[i] >> 4) == 0) L.dd[b & 1][dm[i]][drt[i] * 16 + (dll[i] & 15)] = r.hdr.x;
    };

    GuRowSb<T> rc[kGuFrags], rn[kGuFrags];
#pragma unroll
    for (int i = 0; i < kGuFrags; i++) {
        rload(0, i, rc[i]);
        sbstage(0, i, rc[i]);
        decode(0, i, rc[i], 0);
    }
    // activations of the wave's token tile, kBAhead sub-blocks ahead in a
    // ring of kBAhead + 1 (a sub-block's compute is shorter than an L2 load:
    // one sub-block ahead, every sub-block waited for its activations).
    // Every sub-block issues its load (the last ones reload the last
    // sub-block) so the compiler's counts of loads in flight stay exact.
    constexpr int kBAhead = 3;
    auto xload = [&](int jj, f16x8& bh, f16x8& bl) {
        const int kk = min(jj, nsub - 1) * 32;
        bh = *reinterpret_cast<const f16x8*>(xh + (size_t)qc * D + kk + kq * 8);
        bl = *reinterpret_cast<const f16x8*>(xl + (size_t)qc * D + kk + kq * 8);
    };
    f16x8 bh[kBAhead + 1], bl[kBAhead + 1];
#pragma unroll
    for (int a = 0; a < kBAhead; a++) xload(a, bh[a], bl[a]);
    lds_barrier();

    f32x4 og[kGuRowTiles], ou[kGuRowTiles], ag[kGuRowTiles], au[kGuRowTiles];
#pragma unroll
    for (int rt = 0; rt < kGuRowTiles; rt++) og[rt] = ou[rt] = ag[rt] = au[rt] = (f32x4){0.f, 0.f, 0.f, 0.f};
    // super-blocks run-time, their 8 sub-blocks unrolled (every register-array
    // index below is a compile-time constant)
    for (int b = 0; b < nsb; b++) {
        const bool more_sb = b + 1 < nsb;
        if (more_sb) {  // next super-block's weight bytes, a super-block ahead
#pragma unroll
            for (int i = 0; i < kGuFrags; i++) rload(b + 1, i, rn[i]);
        }
#pragma unroll
        for (int j = 0; j < 8; j++) {
            const int jj = 8 * b + j, par = j & 1, slot = j & kBAhead;  // 8 * b + j == j modulo 4
            xload(jj + kBAhead, bh[(j + kBAhead) & kBAhead], bl[(j + kBAhead) & kBAhead]);
            if (busy) {
#pragma unroll
                for (int rt = 0; rt < kGuRowTiles; rt++) {
                    const f16x8 Ag = __builtin_bit_cast(f16x8, L.a[par][0][rt][l]);
                    const f16x8 Au = __builtin_bit_cast(f16x8, L.a[par][1][rt][l]);
                    ag[rt] = mfma(Ag, bh[slot], ag[rt]);
                    au[rt] = mfma(Au, bh[slot], au[rt]);
                }
#pragma unroll
                for (int rt = 0; rt < kGuRowTiles; rt++) {
                    const f16x8 Ag = __builtin_bit_cast(f16x8, L.a[par][0][rt][l]);
                    const f16x8 Au = __builtin_bit_cast(f16x8, L.a[par][1][rt][l]);
                    ag[rt] = mfma(Ag, bl[slot], ag[rt]);
                    au[rt] = mfma(Au, bl[slot], au[rt]);
                }
                if (j == 7) {  // end of the super-block: min term, then d / dmin
                    const f16x8 zero8 = {};
                    const f16x8 sh8 = kq == 0 && qok ? *reinterpret_cast<const f16x8*>(xsh + (size_t)q * nsub + 8 * b) : zero8;
                    const f16x8 sl8 = kq == 0 && qok ? *reinterpret_cast<const f16x8*>(xsl + (size_t)q * nsub + 8 * b) : zero8;
#pragma unroll
                    for (int rt = 0; rt < kGuRowTiles; rt++) {
                        const f16x8 Mg = __builtin_bit_cast(f16x8, L.amin[b & 1][0][rt][l]);
                        const f16x8 Mu = __builtin_bit_cast(f16x8, L.amin[b & 1][1][rt][l]);
                        f32x4 zg = mfma(Mg, sh8, (f32x4){0.f, 0.f, 0.f, 0.f});
                        f32x4 zu = mfma(Mu, sh8, (f32x4){0.f, 0.f, 0.f, 0.f});
                        zg = mfma(Mg, sl8, zg);
                        zu = mfma(Mu, sl8, zu);
                        const uint4 dg4 = *reinterpret_cast<const uint4*>(&L.dd[b & 1][0][rt * 16 + 4 * kq]);
                        const uint4 du4 = *reinterpret_cast<const uint4*>(&L.dd[b & 1][1][rt * 16 + 4 * kq]);
                        const uint32_t dgv[4] = {dg4.x, dg4.y, dg4.z, dg4.w}, duv[4] = {du4.x, du4.y, du4.z, du4.w};
#pragma unroll
                        for (int i = 0; i < 4; i++) {
                            const float dg = (float)__builtin_bit_cast(_Float16, (uint16_t)(dgv[i] & 0xFFFFu));
                            const float dmg = (float)__builtin_bit_cast(_Float16, (uint16_t)(dgv[i] >> 16)) / kSumScale;
                            const float du = (float)__builtin_bit_cast(_Float16, (uint16_t)(duv[i] & 0xFFFFu));
                            const float dmu = (float)__builtin_bit_cast(_Float16, (uint16_t)(duv[i] >> 16)) / kSumScale;
                            og[rt][i] += dg * ag[rt][i] - dmg * zg[i];
                            ou[rt][i] += du * au[rt][i] - dmu * zu[i];
                        }
                        ag[rt] = au[rt] = (f32x4){0.f, 0.f, 0.f, 0.f};
                    }
                }
            }
            // decode the next sub-block (the next super-block's first one from the prefetched bytes)
            if (j < 7) {
#pragma unroll
                for (int i = 0; i < kGuFrags; i++) decode(j + 1, i, rc[i], par ^ 1);
            } else if (more_sb) {
#pragma unroll
                for (int i = 0; i < kGuFrags; i++) {
                    rc[i] = rn[i];
                    sbstage(b + 1, i, rc[i]);
                    decode(0, i, rc[i], par ^ 1);
                }
            }
            lds_barrier();
        }
    }
    if (!qok) return;
    const float xs = xscale[q];
#pragma unroll
    for (int rt = 0; rt < kGuRowTiles; rt++) {
#pragma unroll
        for (int i = 0; i < 4; i++) {
            const int r = rw + rt * 16 + 4 * kq + i;
            if (r >= s.FF) continue;
            const float gv = og[rt][i] * xs, uv = ou[rt][i] * xs;
            h[(size_t)q * s.FF + r] = gv / (1.0f + expf(-gv)) * uv;
        }
    }
}

// ---------------------------------------------------------------------------
// down (Q6_K) for one expert: yp[q][r] = down_r . h[q].  Same organisation
// as gate/up: 8 waves x 16 rows, 64 tokens, h staged through LDS in chunks of
// 64 K values (two Q6_K quarters), the next chunk prefetched into registers.
constexpr int kDnRows = 128;  // down: 8 waves x 16 rows

struct DnA {          // one lane's Q6_K bytes for a chunk (quarters u0 = 2(g&1), u0 + 1 of half n = g/2)
    uint2 ql0, ql1;   // low-nibble sources of the two quarters
    uint2 qh;         // high bits (shared by the quarters)
    int sc0, sc1;     // the quarters' 16-value group scales for this lane's columns
};

__global__ __launch_bounds__(512) void down_mfma_q6k_kernel(MoeShape s, const ExpertEntry* __restrict__ table,
                                                            TileItems gi,
                                                            const _Float16* __restrict__ hh,
                                                            const _Float16* __restrict__ hl,
                                                            const float* __restrict__ hscale,
                                                            float* __restrict__ yp, int tmin) {
    __shared__ _Float16 LB[2][2][kPassTok][kBRow];  // [stage][hi, lo][token][k]
    int e, p0, p1, pb;
    if (!tile_item(gi, e, pb, p1, p0) || pb >= p1 || p1 - p0 < tmin) return;
    const int tid = threadIdx.x, wave = tid >> 6, l = tid & 63;
    const int lr = l & 15, kq = l >> 4;
    const int r0 = blockIdx.x * kDnRows + wave * 16;
    const bool on = r0 < s.D;
    const int FF = s.FF, nch = FF / kChunkK, nsb = FF / 256;
    const uint8_t* dbase = table[e].down;
    const uint8_t* da = dbase + (size_t)(on ? r0 + lr : 0) * s.down_rb;
    const int st_t = tid >> 3, st_k = (tid & 7) * 8;
    const bool st_ok = pb + st_t < p1;
    const size_t st_row = (size_t)(pb + st_t) * FF;
    auto gload = [&](int c, uint4& vh, uint4& vl) {
        if (st_ok) {
            vh = *reinterpret_cast<const uint4*>(hh + st_row + (size_t)c * kChunkK + st_k);
            vl = *reinterpret_cast<const uint4*>(hl + st_row + (size_t)c * kChunkK + st_k);
        } else {
            vh = vl = make_uint4(0, 0, 0, 0);
        }
    };
    auto aload = [&](int c, DnA& a) {
        const int b = c >> 2, g = c & 3, n = g >> 1, u0 = 2 * (g & 1);
        const uint8_t* blk = da + (size_t)b * 210;
        a.ql0 = ld8_a2(blk + 64 * n + kq * 8);
        a.ql1 = ld8_a2(blk + 64 * n + 32 + kq * 8);
        a.qh = ld8_a2(blk + 128 + 32 * n + kq * 8);
        a.sc0 = ld_i8(blk + 192 + 8 * n + (kq >> 1) + 2 * u0);
        a.sc1 = ld_i8(blk + 192 + 8 * n + (kq >> 1) + 2 * (u0 + 1));
    };
    auto dload = [&](int b, float (&d)[4]) {
#pragma unroll
        for (int i = 0; i < 4; i++)
            d[i] = half_at(dbase + (size_t)(on ? r0 + 4 * kq + i : 0) * s.down_rb + (size_t)b * 210 + 208);
    };
    DnA cur{}, nx1{}, nx2{};
    float dc[4] = {}, dn[4] = {};
    uint4 vh, vl, vh1, vl1, vh2 = {}, vl2 = {};
    if (on) {
        aload(0, cur);
        dload(0, dc);
        if (nch > 1) aload(1, nx1);
    }
    gload(0, vh, vl);
    if (nch > 1) gload(1, vh1, vl1);
    *reinterpret_cast<uint4*>(&LB[0][0][st_t][st_k]) = vh;
    *reinterpret_cast<uint4*>(&LB[0][1][st_t][st_k]) = vl;
    lds_barrier();
    f32x4 out[4];
#pragma unroll
    for (int nt = 0; nt < 4; nt++) out[nt] = (f32x4){0.f, 0.f, 0.f, 0.f};
    for (int b = 0; b < nsb; b++) {
        f32x4 acc[4];
#pragma unroll
        for (int nt = 0; nt < 4; nt++) acc[nt] = (f32x4){0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int g = 0; g < 4; g++) {
            const int c = 4 * b + g;
            const int stg = c & 1;
            const bool more = c + 1 < nch;
            const bool next_sb = more && g == 3;
            if (c + 2 < nch) {
                gload(c + 2, vh2, vl2);
                if (on) aload(c + 2, nx2);
            }
            if (next_sb && on) dload(b + 1, dn);
            if (on) {
#pragma unroll
                for (int qq = 0; qq < 2; qq++) {  // the chunk's two quarters
                    const int u = 2 * (g & 1) + qq;
                    const uint2 ql = qq ? cur.ql1 : cur.ql0;
                    const int sc = qq ? cur.sc1 : cur.sc0;
                    const int sh4 = u >= 2 ? 4 : 0;
                    const uint2 code =
                        make_uint2(((ql.x >> sh4) & 0x0F0F0F0Fu) | (((cur.qh.x >> (2 * u)) & 0x03030303u) << 4),
                                   ((ql.y >> sh4) & 0x0F0F0F0Fu) | (((cur.qh.y >> (2 * u)) & 0x03030303u) << 4));
                    const f16x8 A1 = codes_times(code, (_Float16)(float)(16 * (sc >> 4)), (_Float16)-32.0f);
                    const f16x8 A2 = codes_times(code, (_Float16)(float)(sc & 15), (_Float16)-32.0f);
                    f16x8 bh[4], bl[4];
#pragma unroll
                    for (int nt = 0; nt < 4; nt++) {
                        bh[nt] = *reinterpret_cast<const f16x8*>(&LB[stg][0][nt * 16 + lr][qq * 32 + kq * 8]);
                        bl[nt] = *reinterpret_cast<const f16x8*>(&LB[stg][1][nt * 16 + lr][qq * 32 + kq * 8]);
                    }
#pragma unroll
                    for (int nt = 0; nt < 4; nt++) acc[nt] = mfma(A1, bh[nt], acc[nt]);
#pragma unroll
                    for (int nt = 0; nt < 4; nt++) acc[nt] = mfma(A2, bh[nt], acc[nt]);
#pragma unroll
                    for (int nt = 0; nt < 4; nt++) acc[nt] = mfma(A1, bl[nt], acc[nt]);
#pragma unroll
                    for (int nt = 0; nt < 4; nt++) acc[nt] = mfma(A2, bl[nt], acc[nt]);
                }
                if (g == 3) {
#pragma unroll
                    for (int i = 0; i < 4; i++)
#pragma unroll
                        for (int nt = 0; nt < 4; nt++) out[nt][i] += dc[i] * acc[nt][i];
                }
            }
            if (more) {
                *reinterpret_cast<uint4*>(&LB[stg ^ 1][0][st_t][st_k]) = vh1;
                *reinterpret_cast<uint4*>(&LB[stg ^ 1][1][st_t][st_k]) = vl1;
            }
            lds_barrier();
            vh1 = vh2;
            vl1 = vl2;
            if (more && on) {
                cur = nx1;
                nx1 = nx2;
                if (next_sb) {
#pragma unroll
                    for (int i = 0; i < 4; i++) dc[i] = dn[i];
                }
            }
        }
    }
    if (!on) return;
#pragma unroll
    for (int nt = 0; nt < 4; nt++) {
        const int q = pb + nt * 16 + lr;
        if (q >= p1) continue;
        const float hs = hscale[q];
#pragma unroll
        for (int i = 0; i < 4; i++) yp[(size_t)q * s.D + r0 + 4 * kq + i] = out[nt][i] * hs;
    }
}

// ---------------------------------------------------------------------------
bool grouped_mfma_gate_up_ok(const MoeShape& s) {
    return (s.gate_type == kQ4_K || s.gate_type == kQ5_K) && s.up_type == s.gate_type && s.FF % 16 == 0 &&
           s.D % 256 == 0 && s.gate_rb % 16 == 0 && s.up_rb % 16 == 0;
}
bool grouped_mfma_down_ok(const MoeShape& s) { return s.down_type == kQ6_K && s.D % 16 == 0 && s.FF % 256 == 0; }

hipError_t launch_prep_rows(const int* offs, int E, const int* tok, const float* src, int ld, int n, int P,
                            _Float16* vh, _Float16* vl, _Float16* sh, _Float16* sl, float* vscale, hipStream_t st) {
    prep_rows_kernel<<<(unsigned)P, 256, 0, st>>>(offs, E, tok, src, ld, n, vh, vl, sh, sl, vscale);
    return hipGetLastError();
}

hipError_t launch_gate_up_mfma(const MoeShape& s, const ExpertEntry* table, TileItems gi,
                               const _Float16* xh, const _Float16* xl, const _Float16* xsh, const _Float16* xsl,
                               const float* xscale, float* h, int tmin, hipStream_t st) {
    if (gi.cap < 1) return hipErrorInvalidValue;
    const dim3 g((unsigned)((s.FF + kGuRows - 1) / kGuRows), (unsigned)gi.cap);
    if (s.gate_type == kQ4_K)
        gate_up_mfma_kernel<kQ4_K><<<g, 512, 0, st>>>(s, table, gi, xh, xl, xsh, xsl, xscale, h, tmin);
    else
        gate_up_mfma_kernel<kQ5_K><<<g, 512, 0, st>>>(s, table, gi, xh, xl, xsh, xsl, xscale, h, tmin);
    return hipGetLastError();
}

hipError_t launch_down_mfma(const MoeShape& s, const ExpertEntry* table, TileItems gi,
                            const _Float16* hh, const _Float16* hl, const float* hscale, float* yp, int tmin,
                            hipStream_t st) {
    if (gi.cap < 1) return hipErrorInvalidValue;
    const dim3 g((unsigned)((s.D + kDnRows - 1) / kDnRows), (unsigned)gi.cap);
    down_mfma_q6k_kernel<<<g, 512, 0, st>>>(s, table, gi, hh, hl, hscale, yp, tmin);
    return hipGetLastError();
}

}  // namespace eahmmf
