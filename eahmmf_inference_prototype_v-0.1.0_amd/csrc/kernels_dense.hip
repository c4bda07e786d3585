// kernels_dense.hip - the dense (non-expert) part of a Qwen3-MoE decode step
// on the device: token embedding, RMSNorm, per-head Q/K RMSNorm with NeoX
// RoPE and the KV-cache append, causal attention over the fp32 KV cache, and
// the residual add.
//
// Each kernel restates one step of the reference's forward
// (qwen3moe.cpp:932-1075) for nb <= 64 tokens at positions p0 .. p0+nb-1,
// with the same expression order per element; the sums run in parallel
// (tree order instead of the reference's sequential one).  The single-token
// projections and their norms are in kernels_gemv.hip.
#include "dpp.h"
#include "internal.h"
#include "kquant.h"

namespace eahmmf {

constexpr int kDenseThreads = 256;

__device__ __forceinline__ float block_sum(float v, float* red) {
    v = wave_sum(v);
    const int w = threadIdx.x / 64, lane = threadIdx.x % 64, nw = blockDim.x / 64;
    __syncthreads();  // red is free (an earlier call's readers are done)
    if (lane == 0) red[w] = v;
    __syncthreads();
    float t = 0.f;
    for (int i = 0; i < nw; i++) t += red[i];
    return t;
}

__device__ __forceinline__ float wave_max(float v) {
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) v = fmaxf(v, __shfl_xor(v, off, 64));
    return v;
}

__device__ __forceinline__ float block_max(float v, float* red) {
    v = wave_max(v);
    const int w = threadIdx.x / 64, lane = threadIdx.x % 64, nw = blockDim.x / 64;
    __syncthreads();
    if (lane == 0) red[w] = v;
    __syncthreads();
    float t = -INFINITY;
    for (int i = 0; i < nw; i++) t = fmaxf(t, red[i]);
    return t;
}

// x[t] = row toks[t] of the embedding table, dequantized (qwen3moe.cpp:924-929).
// With key set (one token): the id is the argmax held in the key (the index
// field of a gemv argmax key); the block clears the key and stores the id in
// *hist when given.
template <int T>
__global__ __launch_bounds__(kDenseThreads) void embed_kernel(const uint8_t* __restrict__ tab, size_t row_bytes,
                                                              int n_vocab, int D, const int* __restrict__ toks,
                                                              unsigned long long* key, int* hist,
                                                              float* __restrict__ x, int* __restrict__ bad) {
    const int t = blockIdx.x;
    const int id = key ? (int)(0xFFFFFFFFu - (unsigned)(*key & 0xFFFFFFFFull)) : toks[t];
    if (key) {
        __syncthreads();  // every thread has read the key
        if (threadIdx.x == 0) {
            *key = 0ull;
            if (hist) *hist = id;
        }
    }
    if (id < 0 || id >= n_vocab) {
        if (threadIdx.x == 0) *bad = 1;
        return;
    }
    const uint8_t* row = tab + (size_t)id * row_bytes;
    for (int s = threadIdx.x; s < D / 32; s += blockDim.x) {
        float v[32];
        decode_row_seg<T>(row, s, v);
#pragma unroll
        for (int i = 0; i < 32; i++) x[(size_t)t * D + s * 32 + i] = v[i];
    }
}

// out[t] = x[t] / sqrt(mean(x[t]^2) + eps) * w (qwen3moe.cpp:527-532), as
// x * (1 / sqrtf(ss / n + eps)) * w.
__global__ __launch_bounds__(kDenseThreads) void rmsnorm_kernel(const float* __restrict__ x, const float* __restrict__ w,
                                                                float* __restrict__ out, int n, float eps) {
    __shared__ float red[kDenseThreads / 64];
    const float* xr = x + (size_t)blockIdx.x * n;
    float ss = 0.f;
    for (int i = threadIdx.x; i < n; i += blockDim.x) ss += xr[i] * xr[i];
    ss = block_sum(ss, red);
    const float sc = 1.0f / sqrtf(ss / (float)n + eps);
    for (int i = threadIdx.x; i < n; i += blockDim.x) out[(size_t)blockIdx.x * n + i] = xr[i] * sc * w[i];
}

// Causal attention (qwen3moe.cpp:950-1000) for nb tokens at positions
// p0 .. p0+nb-1, from the raw Q/K/V projections.  Query head h reads KV head
// h / GRP; token t sees positions 0 .. p0 + t.
//
// Grid (nb * n_kv, n_split): a block takes one token, one KV head (its GRP
// query heads) and a range of positions.  Lane l of a wave works for head
// l / LPH on DPL = HD / LPH consecutive dimensions (LPH = 64 / GRP lanes per
// head), so a wave holds all GRP query heads in registers.  The waves take
// chunks of C positions in turn; a chunk's K and V rows (this KV head's part
// of each cached position) are copied into the wave's LDS slot by DMA while
// the wave works on its previous chunk, and each wave keeps its own running
// max m, sum l of expf(s - m) and o = sum expf(s - m) v over its positions
// (s = (q . k) * scale); the block then merges its waves in LDS.  The
// batch's own positions (>= p0) come from the raw K/V, given the head RMSNorm
// and NeoX rotation in registers, and the block of the row's own token stores
// them in the KV cache.  With one split the block writes o / l; otherwise
// the last block of the (token, KV head) to finish (a counter it resets for
// the next launch) merges the splits: M = max m,
// out = sum o * expf(m - M) / sum l * expf(m - M), which equals the
// reference's sum_j (expf(s_j - M) / sum) * v_j up to rounding.  The split
// records are exchanged with agent-scope stores and loads (coherent across
// XCDs without a cache writeback).
constexpr int kMaxSplit = 32;  // a power of two of at most 64 (lanes of one wave merge a head)
constexpr int kMinSplitPos = 64;

struct AttnArgs {
    const float* q;  // [nb][n_head * HD] raw
    const float* k;  // [nb][n_kv * HD] raw
    const float* v;  // [nb][n_kv * HD]
    const float* q_norm;
    const float* k_norm;
    const float* rope;  // [pos][HD/2] (cos, sin)
    float* kc;          // this layer's cache [n_ctx][n_kv * HD]
    float* vc;
    float* out;  // [nb][n_head * HD]
    float* part;
    unsigned* cnt;
    int n_head, n_kv, p0, n_split, span;  // span: positions per split
    // several sequences, one token each (null for one sequence's batch):
    // token t is at position tpos[t] of the sequence whose cache starts
    // tseq[t] * seq_stride floats past kc / vc
    const int* tpos;
    const int* tseq;
    size_t seq_stride;
    float eps, scale;
};

// Head RMSNorm + NeoX rotation of a head held DPL values per lane (lane
// group of LPH lanes): x holds dims g*DPL .. g*DPL+DPL-1 (g = lane % LPH);
// the partner holding dim d + HD/2 is lane ^ (LPH/2).  cs: the position's
// rope row (HD/2 cos/sin pairs).
template <int HD, int LPH, int DPL>
__device__ __forceinline__ void norm_rope(float (&x)[DPL], const float* __restrict__ nw, const float* __restrict__ cs,
                                          float eps, int g) {
    const bool lo = g < LPH / 2;
    const int i0 = (lo ? g : g - LPH / 2) * DPL;  // pair index of element 0
    float wv[DPL], cv[DPL], sv[DPL];  // loaded first: in flight during the reduction
#pragma unroll
    for (int e = 0; e < DPL; e++) {
        wv[e] = nw[g * DPL + e];
        cv[e] = cs[2 * (i0 + e)];
        sv[e] = cs[2 * (i0 + e) + 1];
    }
    float ss = 0.f;
#pragma unroll
    for (int e = 0; e < DPL; e++) ss += x[e] * x[e];
    ss = group_sum_all<LPH>(ss);
    const float sc = 1.0f / sqrtf(ss / (float)HD + eps);
#pragma unroll
    for (int e = 0; e < DPL; e++) x[e] = x[e] * sc * wv[e];
#pragma unroll
    for (int e = 0; e < DPL; e++) {
        const float other = __shfl_xor(x[e], LPH / 2, 64);
        x[e] = lo ? x[e] * cv[e] - other * sv[e] : other * sv[e] + x[e] * cv[e];
    }
}

template <int HD, int GRP>
struct AttnShape {
    static constexpr int LPH = 64 / GRP, DPL = HD / LPH;
    static constexpr int C = 4;                         // positions per chunk
    static constexpr int W = GRP * HD <= 1024 ? 8 : 4;  // waves per block
    static constexpr int RPI = 1024 / (HD * 4);         // rows per 1 KiB DMA instruction
    static constexpr int NI = 2 * C / RPI;              // DMA instructions per chunk (K and V)
    static constexpr int SLOT = 2 * C * HD;             // floats per chunk slot: K rows then V rows
};

// Copies the K and V rows of positions c0 .. c0+C-1 (clamped to row `safe`
// where a position is not cached) into slot (floats [2][C][HD]).
template <int HD, int GRP>
__device__ __forceinline__ void issue_chunk(const float* kc, const float* vc, int KD, int kvh, int c0, int old_end,
                                            int safe, float* slot, int lane) {
    using S = AttnShape<HD, GRP>;
    constexpr int LPR = 64 / S::RPI;  // lanes per row
#pragma unroll
    for (int i = 0; i < S::NI; i++) {
        const bool is_v = i >= S::NI / 2;
        const int j = (i % (S::NI / 2)) * S::RPI + lane / LPR;
        int pos = c0 + j;
        if (pos >= old_end) pos = safe;
        const float* src = (is_v ? vc : kc) + (size_t)pos * KD + kvh * HD + (lane % LPR) * 4;
        lds_dma16((uintptr_t)src, reinterpret_cast<const uint8_t*>(slot + i * 256));
    }
}

template <int HD, int GRP>
__global__ __launch_bounds__((AttnShape<HD, GRP>::W * 64)) void attention_kernel(AttnArgs a) {
    using S = AttnShape<HD, GRP>;
    constexpr int LPH = S::LPH, DPL = S::DPL, C = S::C, W = S::W;
    __shared__ __align__(16) float smem[W * 2 * S::SLOT > W * GRP * HD ? W * 2 * S::SLOT : W * GRP * HD];
    __shared__ float wm[W][GRP], wl[W][GRP];
    __shared__ unsigned last;
    const int n_kv = a.n_kv, KD = n_kv * HD, QD = a.n_head * HD;
    const int t = blockIdx.x / n_kv, kvh = blockIdx.x % n_kv, s = blockIdx.y;
    const int tid = threadIdx.x, w = __builtin_amdgcn_readfirstlane(tid / 64), lane = tid % 64;
    const int h = lane / LPH, g = lane % LPH, d0 = g * DPL;
    // the token's batch starts at pfirst (its own sequence); the token sits at own
    const bool multi = a.tpos != nullptr;
    const int pfirst = multi ? a.tpos[t] : a.p0;
    const int own = multi ? pfirst : a.p0 + t;
    const size_t sbase = multi ? (size_t)a.tseq[t] * a.seq_stride : 0;
    float* const kc = a.kc + sbase;
    float* const vc = a.vc + sbase;
    const int np = own + 1;
    const int pos0 = s * a.span, pos1 = min(pos0 + a.span, np);
    const int old_end = min(pos1, pfirst);  // cached rows end here
    const int safe = 0;                     // a row that always exists (its data is not used)
    float* slots = smem + w * 2 * S::SLOT;
    int c0 = pos0 + w * C;
    if (c0 < pos1) issue_chunk<HD, GRP>(kc, vc, KD, kvh, c0, old_end, safe, slots, lane);
    // query head (kvh * GRP + h), normed and rotated at the token's position
    float q[DPL];
    {
        const float* src = a.q + (size_t)t * QD + (size_t)(kvh * GRP + h) * HD + d0;
#pragma unroll
        for (int e = 0; e < DPL; e++) q[e] = src[e];
        norm_rope<HD, LPH, DPL>(q, a.q_norm, a.rope + (size_t)own * HD, a.eps, g);
    }
    float o[DPL];
#pragma unroll
    for (int e = 0; e < DPL; e++) o[e] = 0.f;
    float m = -INFINITY, l = 0.f;
    for (int k = 0; c0 < pos1; c0 += W * C, k++) {
        float* cur = slots + (k & 1) * S::SLOT;
        if (c0 + W * C < pos1) {
            issue_chunk<HD, GRP>(kc, vc, KD, kvh, c0 + W * C, old_end, safe, slots + ((k + 1) & 1) * S::SLOT, lane);
            wait_vm_upto<S::NI>();
        } else {
            wait_vm();
        }
        const int nc = min(C, pos1 - c0);
        // the batch's own rows of this chunk: normed, rotated, into the slot
        for (int j = max(0, old_end - c0); j < nc; j++) {
            const int pos = c0 + j, tt = multi ? t : pos - a.p0;  // (a single-token batch: its own row)
            float kr[DPL], vr[DPL];
            const float* kp = a.k + (size_t)tt * KD + kvh * HD + d0;
            const float* vp = a.v + (size_t)tt * KD + kvh * HD + d0;
#pragma unroll
            for (int e = 0; e < DPL; e++) {
                kr[e] = kp[e];
                vr[e] = vp[e];
            }
            norm_rope<HD, LPH, DPL>(kr, a.k_norm, a.rope + (size_t)pos * HD, a.eps, g);
            if (h == 0) {
#pragma unroll
                for (int e = 0; e < DPL; e++) {
                    cur[j * HD + d0 + e] = kr[e];
                    cur[(C + j) * HD + d0 + e] = vr[e];
                }
                if (pos == np - 1) {  // this token's own row: one block stores it
#pragma unroll
                    for (int e = 0; e < DPL; e++) {
                        kc[(size_t)pos * KD + kvh * HD + d0 + e] = kr[e];
                        vc[(size_t)pos * KD + kvh * HD + d0 + e] = vr[e];
                    }
                }
            }
        }
        float sc[C];
        float mc = -INFINITY;
#pragma unroll
        for (int j = 0; j < C; j++) {
            const float* kr = cur + j * HD + d0;
            float p = 0.f;
#pragma unroll
            for (int e = 0; e < DPL; e++) p = __builtin_fmaf(q[e], kr[e], p);
            p = group_sum_all<LPH>(p) * a.scale;
            sc[j] = j < nc ? p : -INFINITY;
            mc = fmaxf(mc, sc[j]);
        }
        const float mn = fmaxf(m, mc);
        const float al = m == -INFINITY ? 0.f : expf(m - mn);
        l *= al;
#pragma unroll
        for (int e = 0; e < DPL; e++) o[e] *= al;
#pragma unroll
        for (int j = 0; j < C; j++) {
            const float ej = j < nc ? expf(sc[j] - mn) : 0.f;
            l += ej;
            const float* vr = cur + (C + j) * HD + d0;
#pragma unroll
            for (int e = 0; e < DPL; e++) o[e] = __builtin_fmaf(ej, vr[e], o[e]);
        }
        m = mn;
    }
    // merge the block's waves (their LDS slots are reused for the partials)
    __syncthreads();
    float* wo = smem;  // [W][GRP * HD]
#pragma unroll
    for (int e = 0; e < DPL; e++) wo[w * GRP * HD + h * HD + d0 + e] = o[e];
    if (g == 0) {
        wm[w][h] = m;
        wl[w][h] = l;
    }
    __syncthreads();
    // per (wave, head): the wave's factor expf(m - M) (kept in wm) and the
    // head's M and L (kept in wl[0] / wl[1])
    if (tid < GRP) {
        float M = -INFINITY;
#pragma unroll
        for (int u = 0; u < W; u++) M = fmaxf(M, wm[u][tid]);
        float L = 0.f;
#pragma unroll
        for (int u = 0; u < W; u++) {
            const float f = wm[u][tid] == -INFINITY ? 0.f : expf(wm[u][tid] - M);
            L = __builtin_fmaf(wl[u][tid], f, L);
            wm[u][tid] = f;
        }
        wl[0][tid] = M;
        wl[1][tid] = L;
    }
    __syncthreads();
    const size_t rec = HD + 4;  // split record per (t, head, split): o, m, l (16-byte records)
    float* base = a.part + ((size_t)t * a.n_head + kvh * GRP) * a.n_split * rec;
    for (int i = tid; i < GRP * HD; i += W * 64) {
        const int hh = i / HD, d = i % HD;
        const float M = wl[0][hh], L = wl[1][hh];
        float acc = 0.f;
#pragma unroll
        for (int u = 0; u < W; u++) acc = __builtin_fmaf(wo[u * GRP * HD + i], wm[u][hh], acc);
        if (a.n_split == 1) {
            a.out[(size_t)t * QD + (size_t)(kvh * GRP + hh) * HD + d] = acc / L;
        } else {
            float* r = base + ((size_t)hh * a.n_split + s) * rec;
            __hip_atomic_store(r + d, acc, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            if (d == 0) {
                __hip_atomic_store(r + HD, M, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                __hip_atomic_store(r + HD + 1, L, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            }
        }
    }
    if (a.n_split == 1) return;
    wait_vm();  // this wave's records are stored
    __syncthreads();
    if (tid == 0)
        last = __hip_atomic_fetch_add(&a.cnt[t * n_kv + kvh], 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) ==
               (unsigned)(a.n_split - 1);
    __syncthreads();
    if (!last) return;
    // the other blocks' records: drop this XCD's cached copies of older
    // contents (the records of earlier launches), then ordinary loads.  A
    // thread takes four dimensions of one head and loads, in one round, the
    // head's m and l and its four o values of every split.
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "agent");
    if constexpr (GRP * HD / 4 <= W * 64) {
        // One round of loads: thread (head, four dimensions) takes the o
        // values of every split, thread (head, split) that split's m and l.
        // The split factors expf(m_u - M) are then formed once per (head,
        // split) and shared through LDS instead of by every thread of the
        // head (32 expf each).
        __shared__ float msh[GRP][kMaxSplit], lsh[GRP][kMaxSplit];
        const int hh = tid / (HD / 4), d = (tid % (HD / 4)) * 4;
        const bool mine = tid < GRP * HD / 4;
        const float* r = base + (size_t)(mine ? hh : 0) * a.n_split * rec;
        float4 ov[kMaxSplit];
#pragma unroll
        for (int u = 0; u < kMaxSplit; u++)
            ov[u] = mine && u < a.n_split ? *reinterpret_cast<const float4*>(r + (size_t)u * rec + d)
                                          : make_float4(0.f, 0.f, 0.f, 0.f);
        const int fh = tid / kMaxSplit, fu = tid % kMaxSplit;
        if (tid < GRP * kMaxSplit) {
            float2 ml = make_float2(-INFINITY, 0.f);
            if (fu < a.n_split) ml = *reinterpret_cast<const float2*>(base + ((size_t)fh * a.n_split + fu) * rec + HD);
            msh[fh][fu] = ml.x;
            lsh[fh][fu] = ml.y;
        }
        __syncthreads();
        float fac = 0.f;
        if (tid < GRP * kMaxSplit) {
            float M = -INFINITY;
#pragma unroll
            for (int u = 0; u < kMaxSplit; u++) M = fmaxf(M, msh[fh][u]);
            const float mu = msh[fh][fu];
            fac = mu == -INFINITY ? 0.f : expf(mu - M);
        }
        __syncthreads();  // every M is formed before the factors overwrite the maxima
        if (tid < GRP * kMaxSplit) msh[fh][fu] = fac;
        __syncthreads();
        if (mine) {
            float L = 0.f;
            float4 acc = make_float4(0.f, 0.f, 0.f, 0.f);
#pragma unroll
            for (int u = 0; u < kMaxSplit; u++) {
                const float fu_ = msh[hh][u];
                L = __builtin_fmaf(lsh[hh][u], fu_, L);
                acc.x = __builtin_fmaf(ov[u].x, fu_, acc.x);
                acc.y = __builtin_fmaf(ov[u].y, fu_, acc.y);
                acc.z = __builtin_fmaf(ov[u].z, fu_, acc.z);
                acc.w = __builtin_fmaf(ov[u].w, fu_, acc.w);
            }
            float* o = a.out + (size_t)t * QD + (size_t)(kvh * GRP + hh) * HD + d;
            o[0] = acc.x / L;
            o[1] = acc.y / L;
            o[2] = acc.z / L;
            o[3] = acc.w / L;
        }
    } else {
        for (int i = tid; i < GRP * HD / 4; i += W * 64) {
            const int hh = i / (HD / 4), d = (i % (HD / 4)) * 4;
            const float* r = base + (size_t)hh * a.n_split * rec;
            float4 ov[kMaxSplit];
            float2 ml[kMaxSplit];
#pragma unroll
            for (int u = 0; u < kMaxSplit; u++) {
                if (u < a.n_split) {
                    ov[u] = *reinterpret_cast<const float4*>(r + (size_t)u * rec + d);
                    ml[u] = *reinterpret_cast<const float2*>(r + (size_t)u * rec + HD);
                } else {
                    ov[u] = make_float4(0.f, 0.f, 0.f, 0.f);
                    ml[u] = make_float2(-INFINITY, 0.f);
                }
            }
            float M = -INFINITY;
#pragma unroll
            for (int u = 0; u < kMaxSplit; u++) M = fmaxf(M, ml[u].x);
            float L = 0.f;
            float4 acc = make_float4(0.f, 0.f, 0.f, 0.f);
#pragma unroll
            for (int u = 0; u < kMaxSplit; u++) {
                const float f = ml[u].x == -INFINITY ? 0.f : expf(ml[u].x - M);
                L = __builtin_fmaf(ml[u].y, f, L);
                acc.x = __builtin_fmaf(ov[u].x, f, acc.x);
                acc.y = __builtin_fmaf(ov[u].y, f, acc.y);
                acc.z = __builtin_fmaf(ov[u].z, f, acc.z);
                acc.w = __builtin_fmaf(ov[u].w, f, acc.w);
            }
            float* o = a.out + (size_t)t * QD + (size_t)(kvh * GRP + hh) * HD + d;
            o[0] = acc.x / L;
            o[1] = acc.y / L;
            o[2] = acc.z / L;
            o[3] = acc.w / L;
        }
    }
    if (tid == 0) __hip_atomic_store(&a.cnt[t * n_kv + kvh], 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

__global__ void add_kernel(float* __restrict__ x, const float* __restrict__ y, size_t n) {
    for (size_t i = blockIdx.x * (size_t)blockDim.x + threadIdx.x; i < n; i += (size_t)gridDim.x * blockDim.x)
        x[i] += y[i];
}

// ---------------------------------------------------------------------------

hipError_t launch_embed(int type, const uint8_t* tab, size_t row_bytes, int n_vocab, int D, const int* toks,
                        unsigned long long* key, int* hist, int nb, float* x, int* bad, hipStream_t st) {
    if ((key && nb != 1) || (!key && !toks)) return hipErrorInvalidValue;
    clear_stale_error();
    const dim3 g(nb), b(kDenseThreads);
    switch (type) {
        case kF32: embed_kernel<kF32><<<g, b, 0, st>>>(tab, row_bytes, n_vocab, D, toks, key, hist, x, bad); break;
        case kQ8_0: embed_kernel<kQ8_0><<<g, b, 0, st>>>(tab, row_bytes, n_vocab, D, toks, key, hist, x, bad); break;
        case kQ4_K: embed_kernel<kQ4_K><<<g, b, 0, st>>>(tab, row_bytes, n_vocab, D, toks, key, hist, x, bad); break;
        case kQ5_K: embed_kernel<kQ5_K><<<g, b, 0, st>>>(tab, row_bytes, n_vocab, D, toks, key, hist, x, bad); break;
        case kQ6_K: embed_kernel<kQ6_K><<<g, b, 0, st>>>(tab, row_bytes, n_vocab, D, toks, key, hist, x, bad); break;
        default: return hipErrorInvalidValue;
    }
    return hipGetLastError();
}

hipError_t launch_rmsnorm(const float* x, const float* w, float* out, int rows, int n, float eps, hipStream_t st) {
    clear_stale_error();
    rmsnorm_kernel<<<rows, kDenseThreads, 0, st>>>(x, w, out, n, eps);
    return hipGetLastError();
}

size_t attention_part_floats(int nb, int n_head, int hd, int n_pos) {
    return (size_t)nb * n_head * kMaxSplit * (hd + 4);
}

template <int HD, int GRP>
static void attn_launch(const AttnArgs& a, int nb, hipStream_t st) {
    const dim3 g((unsigned)(nb * a.n_kv), (unsigned)a.n_split);
    attention_kernel<HD, GRP><<<g, AttnShape<HD, GRP>::W * 64, 0, st>>>(a);
}

template <int HD>
static bool attn_dispatch(const AttnArgs& a, int grp, int nb, hipStream_t st) {
    switch (grp) {
        case 1: attn_launch<HD, 1>(a, nb, st); return true;
        case 2: attn_launch<HD, 2>(a, nb, st); return true;
        case 4: attn_launch<HD, 4>(a, nb, st); return true;
        case 8: attn_launch<HD, 8>(a, nb, st); return true;
        case 16: attn_launch<HD, 16>(a, nb, st); return true;
        default: return false;
    }
}

bool attention_supported(int n_head, int n_kv, int hd) {
    if (n_kv <= 0 || n_head % n_kv) return false;
    const int grp = n_head / n_kv;
    return (hd == 64 || hd == 128) && (grp == 1 || grp == 2 || grp == 4 || grp == 8 || grp == 16);
}

hipError_t launch_attention(const float* q, const float* k, const float* v, const float* q_norm, const float* k_norm,
                            const float* rope, float* kc, float* vc, float* out, int nb, int n_head, int n_kv, int hd,
                            int p0, float eps, float scale, float* part, unsigned* cnt, hipStream_t st) {
    if (!attention_supported(n_head, n_kv, hd) || nb <= 0 || p0 < 0) return hipErrorInvalidValue;
    AttnArgs a{q, k, v, q_norm, k_norm, rope, kc, vc, out, part, cnt, n_head, n_kv, p0, 0, 0, nullptr, nullptr, 0,
               eps, scale};
    // splits of at least kMinSplitPos positions, at most kMaxSplit (the
    // merge reads one record per split in a single round)
    const int n_pos = p0 + nb;  // of the last token
    int n_split = (n_pos + kMinSplitPos - 1) / kMinSplitPos;
    if (n_split > kMaxSplit) n_split = kMaxSplit;
    a.span = (n_pos + n_split - 1) / n_split;
    a.n_split = (n_pos + a.span - 1) / a.span;
    clear_stale_error();
    const bool ok = hd == 64 ? attn_dispatch<64>(a, n_head / n_kv, nb, st) : attn_dispatch<128>(a, n_head / n_kv, nb, st);
    if (!ok) return hipErrorInvalidValue;
    return hipGetLastError();
}

hipError_t launch_attention_multi(const float* q, const float* k, const float* v, const float* q_norm,
                                  const float* k_norm, const float* rope, float* kc, float* vc, float* out, int nb,
                                  int n_head, int n_kv, int hd, const int* tpos, const int* tseq, size_t seq_stride,
                                  int max_pos, float eps, float scale, float* part, unsigned* cnt, hipStream_t st) {
    if (!attention_supported(n_head, n_kv, hd) || nb <= 0 || max_pos < 0 || !tpos || !tseq) return hipErrorInvalidValue;
    AttnArgs a{q, k, v, q_norm, k_norm, rope, kc, vc, out, part, cnt, n_head, n_kv, 0, 0, 0, tpos, tseq, seq_stride,
               eps, scale};
    const int n_pos = max_pos + 1;  // positions of the longest sequence, its new token included
    int n_split = (n_pos + kMinSplitPos - 1) / kMinSplitPos;
    if (n_split > kMaxSplit) n_split = kMaxSplit;
    a.span = (n_pos + n_split - 1) / n_split;
    a.n_split = (n_pos + a.span - 1) / a.span;
    clear_stale_error();
    const bool ok = hd == 64 ? attn_dispatch<64>(a, n_head / n_kv, nb, st) : attn_dispatch<128>(a, n_head / n_kv, nb, st);
    if (!ok) return hipErrorInvalidValue;
    return hipGetLastError();
}

hipError_t launch_add(float* x, const float* y, size_t n, hipStream_t st) {
    clear_stale_error();
    const size_t blocks = (n + 255) / 256;
    add_kernel<<<(unsigned)(blocks < 1024 ? blocks : 1024), 256, 0, st>>>(x, y, n);
    return hipGetLastError();
}

}  // namespace eahmmf
