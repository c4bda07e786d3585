// kernels_dense_mfma.hip - matrix-core matmul of a quantized weight matrix
// with a small batch of activation rows (2..64 tokens): the model's batched
// projections (Q, K, V, O, the output head) and the drop-in matmul at nb > 1.
// Same contract as matmul_kernel: out[t*ldo + r] = sum_k W[r,k] x[t*ldx + k]
// (qwen3moe.cpp:397-419), for Q4_K, Q5_K, Q6_K and Q8_0 rows.
//
// Exactness.  v_mfma_f32_16x16x32_f16 multiplies fp16 operands exactly and
// accumulates in fp32.  Activations: each row scaled by a power of two so
// that max|v| < 2^13 and split v = hi + lo (fp16 each, about 22 significant
// bits).  Weights: the integer codes of one 32-value sub-block, exact in fp16:
//   Q8_0  q (-128..127), factor d
//   Q4_K  q (0..15), factor d*sc, min term dmin*m * sum(x over the sub-block)
//   Q5_K  q (0..31), the same
//   Q6_K  (q-32)*sc with a per-16 scale, as two exact parts 16*(q-32)*(sc>>4)
//         (|.| <= 4096, a multiple of 16) and (q-32)*(sc&15) (|.| <= 480),
//         factor d
// The sub-block's MFMA sum C = sum q*x is then scaled in fp32: y += f*C - dm*S
// (S the sub-block's activation sum).  So each product is the reference's
// dequantized weight times the activation up to the fp32 rounding of the
// sums (the bar of any fp32 matmul).
//
// Operands (16x16x32, lane l): A = activations, lane holds x[t0 + l%16]
// values 8*(l/16)..+7 of the sub-block; B = weights, lane holds the codes of
// row r0 + l%16 at the same 8 positions; C[4*(l/16) + i][l%16] = tokens
// t0 + 4*(l/16) + i of row r0 + l%16, so a lane's output factors are those
// of the row whose codes it decoded.
//
// Work split: a workgroup of 4 waves covers 64 rows (16 per wave) and 16
// tokens over a range of super-blocks (256 values; grid.z splits the K range
// so that a launch has at least 512 workgroups); the 16 tokens' hi/lo values
// of a super-block are staged in LDS once for the 4 waves, double-buffered,
// and each wave's weight bytes of the next super-block are loaded while it
// works on the current one.  With one split the workgroup writes out; with
// several each writes its partial sums and a second kernel adds the splits
// in order (deterministic).
#include "internal.h"
#include "kquant.h"
#include "mfma_frag.h"

namespace eahmmf {

namespace {

constexpr int kDmWaves = 4;
constexpr int kDmRows = 16 * kDmWaves;  // rows per workgroup
constexpr int kDmRow = 256 + 8;         // halfs per token row in LDS (16-byte pad: conflict-free b128 reads)
constexpr int kDmMinGroups = 512;       // workgroups a launch aims for (split-K below that)
constexpr int kDmMaxSplit = 16;

// ---------------------------------------------------------------------------
// Activations -> scaled fp16 hi/lo rows [nbp][n], 32-value sums [n/32][nbp]
// (scaled, fp32) and the per-row factor 2^(e-13) that undoes the scaling.
// One workgroup per row q < nbp; rows past nb are zeros.
__global__ __launch_bounds__(256) void dense_prep_kernel(const float* __restrict__ x, int ldx, int nb, int n, int nbp,
                                                         _Float16* __restrict__ xh, _Float16* __restrict__ xl,
                                                         float* __restrict__ xs, float* __restrict__ vs) {
    __shared__ float wmax[4];
    const int q = blockIdx.x, tid = threadIdx.x;
    const bool live = q < nb;
    const float* row = x + (size_t)(live ? q : 0) * ldx;
    float m = 0.f;
    if (live)
        for (int c = tid; c < n / 8; c += 256) {
            const float4 a = reinterpret_cast<const float4*>(row)[2 * c];
            const float4 b = reinterpret_cast<const float4*>(row)[2 * c + 1];
            m = fmaxf(m, fmaxf(fmaxf(fabsf(a.x), fabsf(a.y)), fmaxf(fabsf(a.z), fabsf(a.w))));
            m = fmaxf(m, fmaxf(fmaxf(fabsf(b.x), fabsf(b.y)), fmaxf(fabsf(b.z), fabsf(b.w))));
        }
    for (int off = 32; off > 0; off >>= 1) m = fmaxf(m, __shfl_xor(m, off, 64));
    if ((tid & 63) == 0) wmax[tid >> 6] = m;
    __syncthreads();
    m = fmaxf(fmaxf(wmax[0], wmax[1]), fmaxf(wmax[2], wmax[3]));
    int ex = 0;
    if (m > 0.f) (void)frexpf(m, &ex);  // m < 2^ex
    const float sc = m > 0.f ? ldexpf(1.0f, 13 - ex) : 0.f;
    if (tid == 0) vs[q] = m > 0.f ? ldexpf(1.0f, ex - 13) : 0.f;
    for (int c = tid; c < n / 8; c += 256) {  // a 32-value sub-block is four consecutive c (lanes)
        float v[8];
        if (live) {
            const float4 a = reinterpret_cast<const float4*>(row)[2 * c];
            const float4 b = reinterpret_cast<const float4*>(row)[2 * c + 1];
            v[0] = a.x * sc; v[1] = a.y * sc; v[2] = a.z * sc; v[3] = a.w * sc;
            v[4] = b.x * sc; v[5] = b.y * sc; v[6] = b.z * sc; v[7] = b.w * sc;
        } else {
#pragma unroll
            for (int i = 0; i < 8; i++) v[i] = 0.f;
        }
        f16x8 hi, lo;
        float s = 0.f;
#pragma unroll
        for (int i = 0; i < 8; i++) {
            hi[i] = (_Float16)v[i];
            lo[i] = (_Float16)(v[i] - (float)hi[i]);
            s += v[i];
        }
        *reinterpret_cast<f16x8*>(xh + (size_t)q * n + 8 * c) = hi;
        *reinterpret_cast<f16x8*>(xl + (size_t)q * n + 8 * c) = lo;
        s += __shfl_xor(s, 1, 64);
        s += __shfl_xor(s, 2, 64);
        if ((c & 3) == 0) xs[(size_t)(c / 4) * nbp + q] = s;
    }
}

// ---------------------------------------------------------------------------
// One lane's weight bytes of a super-block (256 values of its row) and the B
// fragments and factors of its sub-blocks.
__device__ __forceinline__ uint2 nib(uint2 w, int sh) {
    return make_uint2((w.x >> sh) & 0x0F0F0F0Fu, (w.y >> sh) & 0x0F0F0F0Fu);
}

template <int T>
struct Sb;

template <>
struct Sb<kQ8_0> {  // eight 34-byte blocks
    static constexpr bool kMin = false;
    static constexpr size_t kBytes = 8 * 34;
    uint2 q[8];
    uint32_t d[4];  // two fp16 scales per word
    __device__ __forceinline__ void load(const uint8_t* sb, int c) {
#pragma unroll
        for (int j = 0; j < 8; j++) q[j] = ld8_a2(sb + 34 * j + 2 + 8 * c);
#pragma unroll
        for (int j = 0; j < 4; j++) d[j] = (uint32_t)gld_u16(sb + 68 * j) | ((uint32_t)gld_u16(sb + 68 * j + 34) << 16);
    }
    __device__ __forceinline__ float factor(int j) const { return half_to_float((d[j >> 1] >> (16 * (j & 1))) & 0xFFFFu); }
    __device__ __forceinline__ float min_factor(int) const { return 0.f; }
    __device__ __forceinline__ f16x8 frag(int j, int) const {
        const uint2 u = make_uint2(q[j].x ^ 0x80808080u, q[j].y ^ 0x80808080u);  // q + 128
        return codes_times(u, (_Float16)1.0f, (_Float16)-128.0f);
    }
};

template <>
struct Sb<kQ4_K> {
    static constexpr bool kMin = true;
    static constexpr size_t kBytes = 144;
    uint4 hdr;  // d, dmin, 12 scale bytes
    uint2 q[4];
    __device__ __forceinline__ void load(const uint8_t* sb, int c) {
        hdr = gld16(sb);
#pragma unroll
        for (int g = 0; g < 4; g++) q[g] = ld8(sb + 16 + 32 * g + 8 * c);
    }
    __device__ __forceinline__ float factor(int j) const {
        uint32_t sc, mn;
        scale_min_k4(j, hdr.y, hdr.z, hdr.w, sc, mn);
        return half_to_float(hdr.x & 0xFFFFu) * (float)sc;
    }
    __device__ __forceinline__ float min_factor(int j) const {
        uint32_t sc, mn;
        scale_min_k4(j, hdr.y, hdr.z, hdr.w, sc, mn);
        return half_to_float(hdr.x >> 16) * (float)mn;
    }
    __device__ __forceinline__ f16x8 frag(int j, int) const {
        return codes_times(nib(q[j >> 1], (j & 1) * 4), (_Float16)1.0f, (_Float16)0.0f);
    }
};

template <>
struct Sb<kQ5_K> {
    static constexpr bool kMin = true;
    static constexpr size_t kBytes = 176;
    uint4 hdr;
    uint2 h;  // high bits of this lane's 8 positions (bit j: sub-block j)
    uint2 q[4];
    __device__ __forceinline__ void load(const uint8_t* sb, int c) {
        hdr = gld16(sb);
        h = ld8(sb + 16 + 8 * c);
#pragma unroll
        for (int g = 0; g < 4; g++) q[g] = ld8(sb + 48 + 32 * g + 8 * c);
    }
    __device__ __forceinline__ float factor(int j) const {
        uint32_t sc, mn;
        scale_min_k4(j, hdr.y, hdr.z, hdr.w, sc, mn);
        return half_to_float(hdr.x & 0xFFFFu) * (float)sc;
    }
    __device__ __forceinline__ float min_factor(int j) const {
        uint32_t sc, mn;
        scale_min_k4(j, hdr.y, hdr.z, hdr.w, sc, mn);
        return half_to_float(hdr.x >> 16) * (float)mn;
    }
    __device__ __forceinline__ f16x8 frag(int j, int) const {
        const uint2 lo = nib(q[j >> 1], (j & 1) * 4);
        const uint2 v = make_uint2(lo.x | (((h.x >> j) & 0x01010101u) << 4), lo.y | (((h.y >> j) & 0x01010101u) << 4));
        return codes_times(v, (_Float16)1.0f, (_Float16)0.0f);
    }
};

template <>
struct Sb<kQ6_K> {  // ql[128], qh[64], scales[16] (int8, per 16 values), d
    static constexpr bool kMin = false;
    static constexpr size_t kBytes = 210;
    uint2 ql[4];  // [half n][sub-block parity]
    uint2 qh[2];  // [half n]
    uint2 s[2];   // scales 0-7, 8-15
    uint32_t d;
    __device__ __forceinline__ void load(const uint8_t* sb, int c) {
#pragma unroll
        for (int n = 0; n < 2; n++) {
            ql[2 * n] = ld8_a2(sb + 64 * n + 8 * c);
            ql[2 * n + 1] = ld8_a2(sb + 64 * n + 32 + 8 * c);
            qh[n] = ld8_a2(sb + 128 + 32 * n + 8 * c);
            s[n] = ld8_a2(sb + 192 + 8 * n);
        }
        d = gld_u16(sb + 208);
    }
    __device__ __forceinline__ float factor(int) const { return half_to_float(d); }
    __device__ __forceinline__ float min_factor(int) const { return 0.f; }
    // codes q + 32 (0..63) of sub-block j = 4n + u at this lane's positions
    __device__ __forceinline__ uint2 codes(int j) const {
        const int n = j >> 2, u = j & 3;
        const uint2 l4 = nib(ql[2 * n + (u & 1)], (u >> 1) * 4);
        const uint2 hb = qh[n];
        return make_uint2(l4.x | (((hb.x >> (2 * u)) & 0x03030303u) << 4),
                          l4.y | (((hb.y >> (2 * u)) & 0x03030303u) << 4));
    }
    // this lane's scale: scales[8n + 2u + (c >= 2)]
    __device__ __forceinline__ int scale(int j, int c) const {
        const int n = j >> 2, u = j & 3, b = 2 * u + (c >> 1);
        const uint32_t w = b < 4 ? s[n].x : s[n].y;
        return (int)(int8_t)((w >> (8 * (b & 3))) & 0xFFu);
    }
};

template <int T>
__global__ __launch_bounds__(256) void dense_mfma_kernel(const uint8_t* __restrict__ w, int ne0, int ne1, size_t rb,
                                                         const _Float16* __restrict__ xh,
                                                         const _Float16* __restrict__ xl, const float* __restrict__ xs,
                                                         const float* __restrict__ vs, int nbp, int nb, int per_split,
                                                         float* __restrict__ out, int ldo, float* __restrict__ part) {
    __shared__ __align__(16) _Float16 xa[2][2][16][kDmRow];  // [buffer][hi, lo][token][value]
    const int tid = threadIdx.x, wv = tid >> 6, l = tid & 63, c = l >> 4;
    const int nsb = ne0 / 256;
    const int sb0 = blockIdx.z * per_split, sb1 = min(nsb, sb0 + per_split);
    const int t0 = blockIdx.y * 16;
    const int row = blockIdx.x * kDmRows + wv * 16 + (l & 15);
    const uint8_t* wr = w + (size_t)min(row, ne1 - 1) * rb;  // rows past the end read the last row (unused)
    // activation tile of super-block sb: 16 tokens x 256 values x (hi, lo) =
    // 1024 pieces of 16 bytes, four per thread
    auto xload = [&](int sb, uint4 (&r)[4]) {
#pragma unroll
        for (int k = 0; k < 4; k++) {
            const int p = tid + 256 * k, part_ = p >> 9, tok = (p >> 5) & 15, c8 = p & 31;
            const _Float16* src = (part_ ? xl : xh) + (size_t)(t0 + tok) * ne0 + (size_t)sb * 256 + 8 * c8;
            r[k] = gld16(reinterpret_cast<const uint8_t*>(src));
        }
    };
    auto xstore = [&](int buf, const uint4 (&r)[4]) {
#pragma unroll
        for (int k = 0; k < 4; k++) {
            const int p = tid + 256 * k, part_ = p >> 9, tok = (p >> 5) & 15, c8 = p & 31;
            *reinterpret_cast<uint4*>(&xa[buf][part_][tok][8 * c8]) = r[k];
        }
    };
    uint4 xr[4];
    xload(sb0, xr);
    Sb<T> cur;
    cur.load(wr + (size_t)sb0 * Sb<T>::kBytes, c);
    xstore(0, xr);
    lds_barrier();
    f32x4 y = {0.f, 0.f, 0.f, 0.f};
    for (int sb = sb0; sb < sb1; sb++) {
        const int buf = (sb - sb0) & 1;
        const int nx = min(sb + 1, sb1 - 1);  // unconditional (clamped) prefetch
        xload(nx, xr);
        Sb<T> nxt;
        nxt.load(wr + (size_t)nx * Sb<T>::kBytes, c);
#pragma unroll
        for (int j = 0; j < 8; j++) {
            const f16x8 ah = *reinterpret_cast<const f16x8*>(&xa[buf][0][l & 15][32 * j + 8 * c]);
            const f16x8 al = *reinterpret_cast<const f16x8*>(&xa[buf][1][l & 15][32 * j + 8 * c]);
            f32x4 acc = {0.f, 0.f, 0.f, 0.f};
            if constexpr (T == kQ6_K) {
                const uint2 q = cur.codes(j);
                const int s = cur.scale(j, c);
                const f16x8 b1 = codes_times(q, (_Float16)(float)(16 * (s >> 4)), (_Float16)-32.0f);
                const f16x8 b2 = codes_times(q, (_Float16)(float)(s & 15), (_Float16)-32.0f);
                acc = mfma(ah, b1, acc);
                acc = mfma(al, b1, acc);
                acc = mfma(ah, b2, acc);
                acc = mfma(al, b2, acc);
            } else {
                const f16x8 b = cur.frag(j, c);
                acc = mfma(ah, b, acc);
                acc = mfma(al, b, acc);
            }
            const float f = cur.factor(j);
            if constexpr (Sb<T>::kMin) {
                const float dm = cur.min_factor(j);
                const uint4 s4u = gld16(reinterpret_cast<const uint8_t*>(xs + (size_t)(sb * 8 + j) * nbp + t0 + 4 * c));
                const float4 s4 = make_float4(__uint_as_float(s4u.x), __uint_as_float(s4u.y), __uint_as_float(s4u.z),
                                              __uint_as_float(s4u.w));
                y[0] = __builtin_fmaf(f, acc[0], __builtin_fmaf(-dm, s4.x, y[0]));
                y[1] = __builtin_fmaf(f, acc[1], __builtin_fmaf(-dm, s4.y, y[1]));
                y[2] = __builtin_fmaf(f, acc[2], __builtin_fmaf(-dm, s4.z, y[2]));
                y[3] = __builtin_fmaf(f, acc[3], __builtin_fmaf(-dm, s4.w, y[3]));
            } else {
#pragma unroll
                for (int i = 0; i < 4; i++) y[i] = __builtin_fmaf(f, acc[i], y[i]);
            }
        }
        cur = nxt;
        // buffer buf ^ 1 was last read in the previous step, which every wave
        // finished before the barrier that ended it
        xstore(buf ^ 1, xr);
        lds_barrier();
    }
    if (row >= ne1) return;
#pragma unroll
    for (int i = 0; i < 4; i++) {
        const int t = t0 + 4 * c + i;
        if (part) {
            part[((size_t)blockIdx.z * nbp + t) * ne1 + row] = y[i];
        } else if (t < nb) {
            out[(size_t)t * ldo + row] = y[i] * vs[t];
        }
    }
}

// out[t][r] = vs[t] * sum over splits (in order) of part[z][t][r]
__global__ __launch_bounds__(256) void dense_splits_kernel(const float* __restrict__ part, int ns, int nbp, int nb,
                                                           int ne1, const float* __restrict__ vs,
                                                           float* __restrict__ out, int ldo) {
    const size_t i = (size_t)blockIdx.x * 256 + threadIdx.x;
    if (i >= (size_t)nb * ne1) return;
    const int t = (int)(i / ne1), r = (int)(i % ne1);
    float s = 0.f;
    for (int z = 0; z < ns; z++) s += part[((size_t)z * nbp + t) * ne1 + r];
    out[(size_t)t * ldo + r] = s * vs[t];
}

struct DensePlan {
    int nbp, row_groups, splits, per_split;
    size_t xh, xl, xs, vs, part, total;  // byte offsets in the workspace
};

DensePlan plan_dense(int ne0, int ne1, int nb) {
    DensePlan p{};
    p.nbp = (nb + 15) / 16 * 16;
    p.row_groups = (ne1 + kDmRows - 1) / kDmRows;
    const int nsb = ne0 / 256;
    const int groups = p.row_groups * (p.nbp / 16);
    int ks = (kDmMinGroups + groups - 1) / groups;
    ks = ks < 1 ? 1 : ks > kDmMaxSplit ? kDmMaxSplit : ks;
    if (ks > nsb) ks = nsb;
    p.per_split = (nsb + ks - 1) / ks;
    p.splits = (nsb + p.per_split - 1) / p.per_split;
    auto al = [](size_t b) { return (b + 255) / 256 * 256; };
    p.xh = 0;
    p.xl = al((size_t)p.nbp * ne0 * 2);
    p.xs = p.xl + al((size_t)p.nbp * ne0 * 2);
    p.vs = p.xs + al((size_t)(ne0 / 32) * p.nbp * 4);
    p.part = p.vs + al((size_t)p.nbp * 4);
    p.total = p.part + (p.splits > 1 ? al((size_t)p.splits * p.nbp * ne1 * 4) : 0);
    return p;
}

}  // namespace

bool matmul_mfma_ok(int type, const uint8_t* w, int ne0, size_t row_bytes, const float* x, int nb, int ldx) {
    if (type != kQ4_K && type != kQ5_K && type != kQ6_K && type != kQ8_0) return false;
    if (nb < 2 || nb > kMaxMfmaMatmulTokens || ne0 <= 0 || ne0 % 256) return false;
    if (((uintptr_t)x & 15) || (ldx & 3)) return false;  // 16-byte activation loads
    const size_t sbb = type == kQ4_K ? 144 : type == kQ5_K ? 176 : type == kQ6_K ? 210 : 8 * 34;
    if (row_bytes < (size_t)(ne0 / 256) * sbb) return false;  // a longer stride: the padding is skipped
    if (type == kQ4_K || type == kQ5_K) return ((uintptr_t)w & 15) == 0 && row_bytes % 16 == 0;
    return ((uintptr_t)w & 1) == 0 && row_bytes % 2 == 0;  // Q8_0, Q6_K: 2-byte aligned rows
}

size_t matmul_mfma_ws_bytes(int ne0, int ne1, int nb) { return plan_dense(ne0, ne1, nb).total; }

hipError_t launch_matmul_mfma(int type, const uint8_t* w, int ne0, int ne1, size_t row_bytes, const float* x, int nb,
                              int ldx, float* out, int ldo, void* ws, size_t ws_bytes, hipStream_t st) {
    if (!matmul_mfma_ok(type, w, ne0, row_bytes, x, nb, ldx) || ne1 <= 0 || !ws) return hipErrorInvalidValue;
    const DensePlan p = plan_dense(ne0, ne1, nb);
    if (p.total > ws_bytes || ((uintptr_t)ws & 255)) return hipErrorInvalidValue;
    uint8_t* b = static_cast<uint8_t*>(ws);
    _Float16* xh = reinterpret_cast<_Float16*>(b + p.xh);
    _Float16* xl = reinterpret_cast<_Float16*>(b + p.xl);
    float* xs = reinterpret_cast<float*>(b + p.xs);
    float* vs = reinterpret_cast<float*>(b + p.vs);
    float* part = p.splits > 1 ? reinterpret_cast<float*>(b + p.part) : nullptr;
    clear_stale_error();
    dense_prep_kernel<<<p.nbp, 256, 0, st>>>(x, ldx, nb, ne0, p.nbp, xh, xl, xs, vs);
    const dim3 grid((unsigned)p.row_groups, (unsigned)(p.nbp / 16), (unsigned)p.splits), block(256);
    switch (type) {
        case kQ4_K:
            dense_mfma_kernel<kQ4_K><<<grid, block, 0, st>>>(w, ne0, ne1, row_bytes, xh, xl, xs, vs, p.nbp, nb,
                                                             p.per_split, out, ldo, part);
            break;
        case kQ5_K:
            dense_mfma_kernel<kQ5_K><<<grid, block, 0, st>>>(w, ne0, ne1, row_bytes, xh, xl, xs, vs, p.nbp, nb,
                                                             p.per_split, out, ldo, part);
            break;
        case kQ6_K:
            dense_mfma_kernel<kQ6_K><<<grid, block, 0, st>>>(w, ne0, ne1, row_bytes, xh, xl, xs, vs, p.nbp, nb,
                                                             p.per_split, out, ldo, part);
            break;
        default:
            dense_mfma_kernel<kQ8_0><<<grid, block, 0, st>>>(w, ne0, ne1, row_bytes, xh, xl, xs, vs, p.nbp, nb,
                                                             p.per_split, out, ldo, part);
            break;
    }
    if (part) {
        const size_t n = (size_t)nb * ne1;
        dense_splits_kernel<<<(unsigned)((n + 255) / 256), 256, 0, st>>>(part, p.splits, p.nbp, nb, ne1, vs, out, ldo);
    }
    return hipGetLastError();
}

namespace {
int g_dense_mfma = 1;
}

bool dense_mfma_enabled() { return g_dense_mfma != 0; }

int set_dense_mfma(int on) {
    const int prev = g_dense_mfma;
    g_dense_mfma = on ? 1 : 0;
    return prev;
}

hipError_t launch_matmul_auto(int type, const uint8_t* w, int ne0, int ne1, size_t row_bytes, const float* x, int nb,
                              int ldx, float* out, int ldo, void* ws, size_t ws_bytes, hipStream_t st) {
    if (g_dense_mfma && ws && matmul_mfma_ok(type, w, ne0, row_bytes, x, nb, ldx) &&
        matmul_mfma_ws_bytes(ne0, ne1, nb) <= ws_bytes)
        return launch_matmul_mfma(type, w, ne0, ne1, row_bytes, x, nb, ldx, out, ldo, ws, ws_bytes, st);
    return launch_matmul(type, w, ne0, ne1, row_bytes, x, nb, ldx, out, ldo, st);
}

}  // namespace eahmmf
