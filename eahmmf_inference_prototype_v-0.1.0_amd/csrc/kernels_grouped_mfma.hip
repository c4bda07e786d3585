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

namespace eahmmf {

typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
typedef _Float16 f16x2 __attribute__((ext_vector_type(2)));
typedef float f32x4 __attribute__((ext_vector_type(4)));

constexpr int kPassTok = 64;  // tokens per pass: four 16-token tiles
constexpr float kSumScale = 1.0f / 16.0f;  // sub-block sums (32 values) kept below 2^14

struct __attribute__((packed, aligned(2))) Bytes8A2 { uint32_t x, y; };
__device__ __forceinline__ uint2 ld8_a2(const uint8_t* p) {
    const Bytes8A2 v = *reinterpret_cast<const Bytes8A2*>(p);
    return make_uint2(v.x, v.y);
}
__device__ __forceinline__ uint2 ld8(const uint8_t* p) { return *reinterpret_cast<const uint2*>(p); }

// Two fp16 values b0, b1 from bytes 2m, 2m+1 of w (each < 256): the byte is
// placed under the exponent of 1024 (0x64XX = 1024 + XX) and 1024 removed.
template <int M>
__device__ __forceinline__ f16x2 byte_pair(uint32_t w) {
    constexpr uint32_t sel = M == 0 ? 0x04010400u : 0x04030402u;
    const f16x2 v = __builtin_bit_cast(f16x2, __builtin_amdgcn_perm(0x64646464u, w, sel));
    return v - (f16x2){(_Float16)1024.0f, (_Float16)1024.0f};
}

// Eight codes (bytes of c) times an integer factor f (|code * f| exact in fp16).
__device__ __forceinline__ f16x8 codes_times(uint2 c, _Float16 f, _Float16 bias) {
    const f16x2 fv = {f, f}, bv = {bias, bias};
    const f16x2 a = (byte_pair<0>(c.x) + bv) * fv, b = (byte_pair<1>(c.x) + bv) * fv;
    const f16x2 d = (byte_pair<0>(c.y) + bv) * fv, e = (byte_pair<1>(c.y) + bv) * fv;
    return (f16x8){a.x, a.y, b.x, b.y, d.x, d.y, e.x, e.y};
}

__device__ __forceinline__ f32x4 mfma(f16x8 a, f16x8 b, f32x4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_f16(a, b, c, 0, 0, 0);
}

__device__ __forceinline__ float half_at(const uint8_t* p) {
    return (float)__builtin_bit_cast(_Float16, *reinterpret_cast<const uint16_t*>(p));
}

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
// A workgroup of 8 waves covers 128 rows (16 per wave) and 64 tokens.  The
// tokens' fp16 hi/lo activations are staged through LDS in chunks of 64 K
// values (double-buffered, shared by the 8 waves); the next chunk's
// activations and weight bytes are loaded into registers while the current
// chunk runs on the matrix cores.  The sub-block sums of the min term are
// staged once per super-block.
constexpr int kGuWaves = 8;
constexpr int kGuRows = 16 * kGuWaves;
constexpr int kChunkK = 64;
constexpr int kBRow = kChunkK + 8;  // halfs per token row in LDS: 144 B, so 16 lanes' 16-B reads hit distinct banks

struct GuLds {
    _Float16 b[2][2][kPassTok][kBRow];  // [stage][hi, lo][token][k]
    _Float16 sm[2][2][kPassTok][8];     // [super-block parity][hi, lo][token][sub-block]: scaled sums
};

template <int T>
struct GuA {  // one lane's weight bytes for a chunk (gate and up)
    uint4 gh, uh;    // super-block headers (d, dmin, scales)
    uint2 gqh, uqh;  // Q5_K high bits of the lane's 8 columns
    uint2 gq, uq;    // 4-bit codes of the lane's 8 columns, both nibbles (sub-blocks 2g, 2g+1)
};

template <int T>
__global__ __launch_bounds__(512) void gate_up_mfma_kernel(MoeShape s, const ExpertEntry* __restrict__ table,
                                                           const int* __restrict__ offs,
                                                           const _Float16* __restrict__ xh,
                                                           const _Float16* __restrict__ xl,
                                                           const _Float16* __restrict__ xsh,
                                                           const _Float16* __restrict__ xsl,
                                                           const float* __restrict__ xscale, float* __restrict__ h) {
    static_assert(T == kQ4_K || T == kQ5_K, "gate/up MFMA path: Q4_K or Q5_K");
    constexpr int BB = Fmt<T>::bytes;
    constexpr int QS = T == kQ5_K ? 48 : 16;  // offset of the 4-bit codes in a super-block
    __shared__ GuLds L;
    const int e = blockIdx.y;
    const int p0 = offs[e], p1 = offs[e + 1];
    const int pb = p0 + (int)blockIdx.z * kPassTok;
    if (pb >= p1) return;  // whole workgroup
    const int tid = threadIdx.x, wave = tid >> 6, l = tid & 63;
    const int lr = l & 15, kq = l >> 4;
    const int r0 = blockIdx.x * kGuRows + wave * 16;
    const bool on = r0 < s.FF;  // wave-uniform; idle waves still stage and synchronise
    const int D = s.D, nsub = D / 32, nch = D / kChunkK;
    const ExpertEntry ent = table[e];
    const uint8_t* ga = ent.gate + (size_t)(on ? r0 + lr : 0) * s.gate_rb;
    const uint8_t* ua = ent.up + (size_t)(on ? r0 + lr : 0) * s.up_rb;
    // staging: thread -> (token, 8 k values) of a chunk, hi and lo
    const int st_t = tid >> 3, st_k = (tid & 7) * 8;
    const bool st_ok = pb + st_t < p1;
    const size_t st_row = (size_t)(pb + st_t) * D;
    auto gload = [&](int c, uint4& vh, uint4& vl) {
        if (st_ok) {
            vh = *reinterpret_cast<const uint4*>(xh + st_row + (size_t)c * kChunkK + st_k);
            vl = *reinterpret_cast<const uint4*>(xl + st_row + (size_t)c * kChunkK + st_k);
        } else {
            vh = vl = make_uint4(0, 0, 0, 0);
        }
    };
    // sums of a super-block: threads 0..127 stage one 16-B piece each
    auto sload = [&](int b, uint4& v) {
        v = make_uint4(0, 0, 0, 0);
        if (tid < 2 * kPassTok) {
            const int t = tid & (kPassTok - 1);
            if (pb + t < p1)
                v = *reinterpret_cast<const uint4*>((tid < kPassTok ? xsh : xsl) + (size_t)(pb + t) * nsub + 8 * b);
        }
    };
    auto swrite_sums = [&](int b, uint4 v) {
        if (tid < 2 * kPassTok)
            *reinterpret_cast<uint4*>(&L.sm[b & 1][tid >= kPassTok][tid & (kPassTok - 1)][0]) = v;
    };
    auto aload = [&](int c, GuA<T>& a) {
        const int b = c >> 2, g = c & 3;
        const uint8_t* gb = ga + (size_t)b * BB;
        const uint8_t* ub = ua + (size_t)b * BB;
        if (g == 0) {
            a.gh = *reinterpret_cast<const uint4*>(gb);
            a.uh = *reinterpret_cast<const uint4*>(ub);
            if (T == kQ5_K) {
                a.gqh = ld8(gb + 16 + kq * 8);
                a.uqh = ld8(ub + 16 + kq * 8);
            }
        }
        a.gq = ld8(gb + QS + 32 * g + kq * 8);
        a.uq = ld8(ub + QS + 32 * g + kq * 8);
    };
    // (d, dmin) of the rows this lane's accumulators hold, for super-block b
    auto dload = [&](int b, uint32_t (&dg)[4], uint32_t (&du)[4]) {
#pragma unroll
        for (int i = 0; i < 4; i++) {
            const size_t row = (size_t)(on ? r0 + 4 * kq + i : 0);
            dg[i] = *reinterpret_cast<const uint32_t*>(ent.gate + row * s.gate_rb + (size_t)b * BB);
            du[i] = *reinterpret_cast<const uint32_t*>(ent.up + row * s.up_rb + (size_t)b * BB);
        }
    };

    // Prefetch distance 2: chunk c computes while chunks c+1 (registers, written
    // to LDS at the end of the iteration) and c+2 (loads in flight) arrive.
    GuA<T> cur{}, nx1{}, nx2{};
    uint32_t dgc[4], duc[4], dgn[4] = {}, dun[4] = {};
    uint4 vh, vl, vs, vh1, vl1, vh2 = {}, vl2 = {};
    if (on) {
        aload(0, cur);
        dload(0, dgc, duc);
        if (nch > 1) aload(1, nx1);
    }
    gload(0, vh, vl);
    sload(0, vs);
    if (nch > 1) gload(1, vh1, vl1);
    *reinterpret_cast<uint4*>(&L.b[0][0][st_t][st_k]) = vh;
    *reinterpret_cast<uint4*>(&L.b[0][1][st_t][st_k]) = vl;
    swrite_sums(0, vs);
    __syncthreads();

    // Tokens past the group's end were staged as zeros, so every tile runs
    // unconditionally (no branches around the matrix instructions).
    const f16x8 zero8 = {};
    f32x4 og[4], ou[4];
#pragma unroll
    for (int nt = 0; nt < 4; nt++) og[nt] = ou[nt] = (f32x4){0.f, 0.f, 0.f, 0.f};
    const int nsb = D / 256;
    for (int b = 0; b < nsb; b++) {
        f32x4 ag[4], au[4];
#pragma unroll
        for (int nt = 0; nt < 4; nt++) ag[nt] = au[nt] = (f32x4){0.f, 0.f, 0.f, 0.f};
        // scales and mins of this lane's row for the 8 sub-blocks (static indices)
        uint32_t scg[8], mng[8], scu[8], mnu[8];
#pragma unroll
        for (int j = 0; j < 8; j++) {
            scale_min_k4(j, cur.gh.y, cur.gh.z, cur.gh.w, scg[j], mng[j]);
            scale_min_k4(j, cur.uh.y, cur.uh.z, cur.uh.w, scu[j], mnu[j]);
        }
        const uint2 gqh = cur.gqh, uqh = cur.uqh;
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
            if (next_sb) {
                sload(b + 1, vs);
                if (on) dload(b + 1, dgn, dun);
            }
            if (on) {
#pragma unroll
                for (int hh = 0; hh < 2; hh++) {
                    const int j = 2 * g + hh;
                    uint2 cg = make_uint2((cur.gq.x >> (4 * hh)) & 0x0F0F0F0Fu, (cur.gq.y >> (4 * hh)) & 0x0F0F0F0Fu);
                    uint2 cu = make_uint2((cur.uq.x >> (4 * hh)) & 0x0F0F0F0Fu, (cur.uq.y >> (4 * hh)) & 0x0F0F0F0Fu);
                    if (T == kQ5_K) {
                        cg.x |= ((gqh.x >> j) & 0x01010101u) << 4;
                        cg.y |= ((gqh.y >> j) & 0x01010101u) << 4;
                        cu.x |= ((uqh.x >> j) & 0x01010101u) << 4;
                        cu.y |= ((uqh.y >> j) & 0x01010101u) << 4;
                    }
                    const f16x8 Ag = codes_times(cg, (_Float16)(float)scg[j], (_Float16)0.0f);
                    const f16x8 Au = codes_times(cu, (_Float16)(float)scu[j], (_Float16)0.0f);
                    f16x8 bh[4], bl[4];
#pragma unroll
                    for (int nt = 0; nt < 4; nt++) {
                        bh[nt] = *reinterpret_cast<const f16x8*>(&L.b[stg][0][nt * 16 + lr][hh * 32 + kq * 8]);
                        bl[nt] = *reinterpret_cast<const f16x8*>(&L.b[stg][1][nt * 16 + lr][hh * 32 + kq * 8]);
                    }
                    // independent accumulators back to back
#pragma unroll
                    for (int nt = 0; nt < 4; nt++) {
                        ag[nt] = mfma(Ag, bh[nt], ag[nt]);
                        au[nt] = mfma(Au, bh[nt], au[nt]);
                    }
#pragma unroll
                    for (int nt = 0; nt < 4; nt++) {
                        ag[nt] = mfma(Ag, bl[nt], ag[nt]);
                        au[nt] = mfma(Au, bl[nt], au[nt]);
                    }
                }
                if (g == 3) {  // end of the super-block: min term, then d / dmin
                    f16x8 mgv = zero8, muv = zero8;
                    if (kq == 0) {
#pragma unroll
                        for (int j = 0; j < 8; j++) {
                            mgv[j] = (_Float16)(float)mng[j];
                            muv[j] = (_Float16)(float)mnu[j];
                        }
                    }
                    f32x4 zg[4], zu[4];
#pragma unroll
                    for (int nt = 0; nt < 4; nt++) {
                        const f16x8 sh8 = *reinterpret_cast<const f16x8*>(&L.sm[b & 1][0][nt * 16 + lr][0]);
                        const f16x8 sl8 = *reinterpret_cast<const f16x8*>(&L.sm[b & 1][1][nt * 16 + lr][0]);
                        zg[nt] = mfma(mgv, sh8, (f32x4){0.f, 0.f, 0.f, 0.f});
                        zu[nt] = mfma(muv, sh8, (f32x4){0.f, 0.f, 0.f, 0.f});
                        zg[nt] = mfma(mgv, sl8, zg[nt]);
                        zu[nt] = mfma(muv, sl8, zu[nt]);
                    }
#pragma unroll
                    for (int i = 0; i < 4; i++) {
                        const float dg = (float)__builtin_bit_cast(_Float16, (uint16_t)(dgc[i] & 0xFFFFu));
                        const float dmg = (float)__builtin_bit_cast(_Float16, (uint16_t)(dgc[i] >> 16)) / kSumScale;
                        const float du = (float)__builtin_bit_cast(_Float16, (uint16_t)(duc[i] & 0xFFFFu));
                        const float dmu = (float)__builtin_bit_cast(_Float16, (uint16_t)(duc[i] >> 16)) / kSumScale;
#pragma unroll
                        for (int nt = 0; nt < 4; nt++) {
                            og[nt][i] += dg * ag[nt][i] - dmg * zg[nt][i];
                            ou[nt][i] += du * au[nt][i] - dmu * zu[nt][i];
                        }
                    }
                }
            }
            if (more) {
                *reinterpret_cast<uint4*>(&L.b[stg ^ 1][0][st_t][st_k]) = vh1;
                *reinterpret_cast<uint4*>(&L.b[stg ^ 1][1][st_t][st_k]) = vl1;
                if (next_sb) swrite_sums(b + 1, vs);
            }
            __syncthreads();
            vh1 = vh2;
            vl1 = vl2;
            if (more && on) {
                cur.gq = nx1.gq;
                cur.uq = nx1.uq;
                if (next_sb) {
                    cur.gh = nx1.gh;
                    cur.uh = nx1.uh;
                    cur.gqh = nx1.gqh;
                    cur.uqh = nx1.uqh;
#pragma unroll
                    for (int i = 0; i < 4; i++) {
                        dgc[i] = dgn[i];
                        duc[i] = dun[i];
                    }
                }
                nx1 = nx2;
            }
        }
    }
    if (!on) return;
#pragma unroll
    for (int nt = 0; nt < 4; nt++) {
        const int q = pb + nt * 16 + lr;
        if (q >= p1) continue;
        const float xs = xscale[q];
#pragma unroll
        for (int i = 0; i < 4; i++) {
            const float gv = og[nt][i] * xs, uv = ou[nt][i] * xs;
            h[(size_t)q * s.FF + r0 + 4 * kq + i] = gv / (1.0f + expf(-gv)) * uv;
        }
    }
}

// ---------------------------------------------------------------------------
// down (Q6_K) for one expert: yp[q][r] = down_r . h[q].  Same organisation
// as gate/up: 8 waves x 16 rows, 64 tokens, h staged through LDS in chunks of
// 64 K values (two Q6_K quarters), the next chunk prefetched into registers.
struct DnA {          // one lane's Q6_K bytes for a chunk (quarters u0 = 2(g&1), u0 + 1 of half n = g/2)
    uint2 ql0, ql1;   // low-nibble sources of the two quarters
    uint2 qh;         // high bits (shared by the quarters)
    int sc0, sc1;     // the quarters' 16-value group scales for this lane's columns
};

__global__ __launch_bounds__(512) void down_mfma_q6k_kernel(MoeShape s, const ExpertEntry* __restrict__ table,
                                                            const int* __restrict__ offs,
                                                            const _Float16* __restrict__ hh,
                                                            const _Float16* __restrict__ hl,
                                                            const float* __restrict__ hscale,
                                                            float* __restrict__ yp) {
    __shared__ _Float16 LB[2][2][kPassTok][kBRow];  // [stage][hi, lo][token][k]
    const int e = blockIdx.y;
    const int p0 = offs[e], p1 = offs[e + 1];
    const int pb = p0 + (int)blockIdx.z * kPassTok;
    if (pb >= p1) return;
    const int tid = threadIdx.x, wave = tid >> 6, l = tid & 63;
    const int lr = l & 15, kq = l >> 4;
    const int r0 = blockIdx.x * kGuRows + wave * 16;
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
        a.sc0 = (int)(int8_t)blk[192 + 8 * n + (kq >> 1) + 2 * u0];
        a.sc1 = (int)(int8_t)blk[192 + 8 * n + (kq >> 1) + 2 * (u0 + 1)];
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
    __syncthreads();
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
            __syncthreads();
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

hipError_t launch_gate_up_mfma(const MoeShape& s, const ExpertEntry* table, int E, const int* offs, int nb,
                               const _Float16* xh, const _Float16* xl, const _Float16* xsh, const _Float16* xsl,
                               const float* xscale, float* h, hipStream_t st) {
    const dim3 g((unsigned)((s.FF + kGuRows - 1) / kGuRows), (unsigned)E, (unsigned)((nb + kPassTok - 1) / kPassTok));
    if (s.gate_type == kQ4_K)
        gate_up_mfma_kernel<kQ4_K><<<g, 512, 0, st>>>(s, table, offs, xh, xl, xsh, xsl, xscale, h);
    else
        gate_up_mfma_kernel<kQ5_K><<<g, 512, 0, st>>>(s, table, offs, xh, xl, xsh, xsl, xscale, h);
    return hipGetLastError();
}

hipError_t launch_down_mfma(const MoeShape& s, const ExpertEntry* table, int E, const int* offs, int nb,
                            const _Float16* hh, const _Float16* hl, const float* hscale, float* yp, hipStream_t st) {
    const dim3 g((unsigned)((s.D + kGuRows - 1) / kGuRows), (unsigned)E, (unsigned)((nb + kPassTok - 1) / kPassTok));
    down_mfma_q6k_kernel<<<g, 512, 0, st>>>(s, table, offs, hh, hl, hscale, yp);
    return hipGetLastError();
}

}  // namespace eahmmf
