// model.hip - whole-model decode on one device behind the C ABI
// (eahmmf_hip_model_*, include/eahmmf_hip.h).
//
// The reference's Engine (qwen3moe.cpp:859-1084) keeps the model in host
// memory and runs everything but the expert matmuls on the CPU.  Here every
// tensor lives in HBM and one forward is a chain of launches on the model's
// own stream:
//
//   embed -> per layer { rmsnorm, Q/K/V matmuls, head norm + RoPE + KV append,
//   split attention, output matmul, residual add, rmsnorm, router matmul,
//   expert block, residual add } -> final rmsnorm -> output head [-> argmax]
//
// One token per forward uses the fused routed layer kernel (routing and the
// k experts in one launch, routing ids/weights written out for the trace); a
// batch uses the routing kernel and the grouped expert kernels.  The host
// waits once per forward, for the logits, the trace and the error words.
#include <math.h>
#include <stdarg.h>

#include <algorithm>
#include <stdio.h>
#include <string.h>

#include <vector>

#include "../../include/eahmmf_hip.h"
#include "internal.h"
#include "kquant.h"

using namespace eahmmf;

namespace {

constexpr int kMaxBatch = 64;  // tokens per forward (the reference's MAXB, qwen3moe.cpp:39)

void fail(const char* fmt, ...) {
    char buf[512];
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(buf, sizeof buf, fmt, ap);
    va_end(ap);
    set_last_error(buf);
}

bool ok(hipError_t e, const char* what) {
    if (e == hipSuccess) return true;
    fail("%s: %s (%d)", what, hipGetErrorString(e), (int)e);
    return false;
}

struct Tens {
    const uint8_t* p = nullptr;
    int type = 0;
    int64_t ne0 = 0, ne1 = 0;
    size_t rb = 0;
};

struct LayerDev {
    const float *attn_norm, *ffn_norm, *q_norm, *k_norm;
    Tens wq, wk, wv, wo, router;
    eahmmf_hip_moe_shape shape;
    eahmmf_hip_expert_ptrs* table;  // device [n_expert]
};

struct Model {
    int dev = 0;
    hipStream_t st = nullptr;
    int n_layer, D, n_head, n_kv, hd, E, K, FF, V, n_ctx, QD, KD;
    float eps, rope_base, scale;
    Tens tok, out;
    const float* out_norm = nullptr;
    std::vector<LayerDev> L;
    std::vector<void*> owned;  // device allocations freed with the model
    float *rope, *kc, *vc, *x, *h, *xn, *q, *k, *v, *att, *tmp, *rl, *logits, *part;
    unsigned long long* key;  // argmax key of the greedy loop
    int *toks, *ids, *bad, *gen;
    // sequences: KV cache [n_layer][n_seq][n_ctx][KD]; a decode step over
    // several sequences takes token t at position tpos[t] of sequence tseq[t]
    // (device arrays beside toks) and leaves logits [t][V] (lg_rows rows)
    int n_seq = 1, lg_rows = 1;
    int *tpos, *tseq;
    void* ws = nullptr;  // workspace of the batched matrix-core matmuls
    size_t ws_bytes = 0;
    float* wts;
    unsigned* cnt;
    // pinned host staging
    int* h_toks = nullptr;
    float* h_logits = nullptr;  // [lg_rows][V]
    int* h_ids = nullptr;
    float* h_w = nullptr;
    unsigned* h_status = nullptr;  // [0] before, [1] after; [2] bad-token flag
    int* h_gen = nullptr;
    int gen_cap = 0;
    bool trace = false;
    std::vector<int> tr_ids;
    std::vector<float> tr_w;
};

struct DeviceGuard {
    int prev = -1;
    explicit DeviceGuard(int d) {
        if (hipGetDevice(&prev) != hipSuccess) prev = -1;
        if (prev != d) (void)hipSetDevice(d);
    }
    ~DeviceGuard() {
        int cur = -1;
        if (prev >= 0 && hipGetDevice(&cur) == hipSuccess && cur != prev) (void)hipSetDevice(prev);
    }
};

size_t fmt_row_bytes(int type, int64_t ne0) {
    const int b = type_blck(type);
    if (b <= 0 || ne0 % b) return 0;
    return (size_t)(ne0 / b) * type_bytes(type);
}

void* dalloc(Model* m, size_t bytes, bool zero) {
    void* p = nullptr;
    if (!ok(hipMalloc(&p, bytes ? bytes : 4), "hipMalloc")) return nullptr;
    m->owned.push_back(p);
    if (zero && !ok(hipMemset(p, 0, bytes ? bytes : 4), "hipMemset")) return nullptr;
    return p;
}

// A tensor on the device: host data is copied into memory the model owns,
// device data is borrowed.  Checks type, row length and row count.
bool place(Model* m, const eahmmf_hip_tensor& t, const char* name, int64_t ne0, int64_t ne1, bool f32_only,
           Tens& o) {
    if (!t.data) return fail("%s: null data", name), false;
    if ((t.type != kF32 && !type_supported(t.type)) || (f32_only && t.type != kF32))
        return fail("%s: unsupported type %d", name, t.type), false;
    if (t.ne0 != ne0 || t.ne1 != ne1)
        return fail("%s: shape %lld x %lld, expected %lld x %lld", name, (long long)t.ne0, (long long)t.ne1,
                    (long long)ne0, (long long)ne1),
               false;
    // the matmul kernel's loads: Q4_K/Q5_K rows 16-byte aligned, F32 rows 16 bytes, others 2
    const size_t need = fmt_row_bytes(t.type, t.ne0);
    const size_t align = (t.type == kQ4_K || t.type == kQ5_K || t.type == kF32) ? 16 : 2;
    if (!need || t.row_bytes < need || t.row_bytes % align)
        return fail("%s: row_bytes %zu (need >= %zu, a multiple of %zu)", name, t.row_bytes, need, align), false;
    o.type = t.type;
    o.ne0 = t.ne0;
    o.ne1 = t.ne1;
    o.rb = t.row_bytes;
    if (t.on_device) {
        o.p = static_cast<const uint8_t*>(t.data);
        return true;
    }
    const size_t bytes = t.row_bytes * (size_t)t.ne1;
    void* d = dalloc(m, bytes, false);
    if (!d || !ok(hipMemcpy(d, t.data, bytes, hipMemcpyHostToDevice), "copy weights")) return false;
    o.p = static_cast<const uint8_t*>(d);
    return true;
}

bool place_vec(Model* m, const eahmmf_hip_tensor& t, const char* name, int64_t n, const float** o) {
    Tens tt;
    if (!place(m, t, name, n, 1, true, tt)) return false;
    *o = reinterpret_cast<const float*>(tt.p);
    return true;
}

void release(Model* m) {
    if (!m) return;
    DeviceGuard g(m->dev);
    if (m->st) {
        (void)hipStreamSynchronize(m->st);
        (void)hipStreamDestroy(m->st);
    }
    for (void* p : m->owned) (void)hipFree(p);
    for (void* p : {(void*)m->h_toks, (void*)m->h_logits, (void*)m->h_ids, (void*)m->h_w, (void*)m->h_status,
                    (void*)m->h_gen})
        if (p) (void)hipHostFree(p);
    delete m;
}

bool mm(Model* m, const Tens& w, const float* x, int nb, int ldx, float* out, int ldo, hipStream_t st,
        const char* what) {
    return ok(launch_matmul_auto(w.type, w.p, (int)w.ne0, (int)w.ne1, w.rb, x, nb, ldx, out, ldo, m->ws, m->ws_bytes,
                                 st),
              what);
}

// Workspace for the batched matmuls of every matrix the model multiplies
// with nb = 2..kMaxBatch tokens.
size_t mm_ws_bytes(const Model* m) {
    size_t need = 0;
    auto fit = [&](const Tens& w) {
        for (int nb = 2; nb <= kMaxBatch && nb <= kMaxMfmaMatmulTokens; nb++)
            if (w.ne0 % 256 == 0) need = std::max(need, matmul_mfma_ws_bytes((int)w.ne0, (int)w.ne1, nb));
    };
    for (const LayerDev& L : m->L)
        for (const Tens* w : {&L.wq, &L.wk, &L.wv, &L.wo, &L.router}) fit(*w);
    fit(m->out);
    return need;
}

// out = W in with the input formed in the kernel (kernels_gemv.hip).
GemvArgs gemv_in(const float* x, const float* x_add, const float* norm_w, float eps) {
    GemvArgs g{};
    g.x = x;
    g.x_add = x_add;
    g.norm_w = norm_w;
    g.eps = eps;
    return g;
}

bool gemv1(const Tens& w, GemvArgs g, float* out, const float* resid, hipStream_t st, const char* what) {
    g.seg[0] = GemvSeg{w.p, out, resid, (int)w.ne1};
    g.nseg = 1;
    g.ne0 = (int)w.ne0;
    g.rb = (int)w.rb;
    return ok(launch_gemv(w.type, g, st), what);
}

// The Q, K and V projections of one token: one launch when the three share a
// type and row size, else one launch each (the input is formed identically).
bool gemv_qkv(Model* m, const LayerDev& L, GemvArgs g, hipStream_t st) {
    if (L.wq.type == L.wk.type && L.wk.type == L.wv.type && L.wq.rb == L.wk.rb && L.wk.rb == L.wv.rb) {
        g.seg[0] = GemvSeg{L.wq.p, m->q, nullptr, (int)L.wq.ne1};
        g.seg[1] = GemvSeg{L.wk.p, m->k, nullptr, (int)L.wk.ne1};
        g.seg[2] = GemvSeg{L.wv.p, m->v, nullptr, (int)L.wv.ne1};
        g.nseg = 3;
        g.ne0 = (int)L.wq.ne0;
        g.rb = (int)L.wq.rb;
        return ok(launch_gemv(L.wq.type, g, st), "q/k/v projections");
    }
    if (!gemv1(L.wq, g, m->q, nullptr, st, "q projection")) return false;
    g.x_sum_out = nullptr;
    return gemv1(L.wk, g, m->k, nullptr, st, "k projection") && gemv1(L.wv, g, m->v, nullptr, st, "v projection");
}

size_t seq_floats(const Model* m) { return (size_t)m->n_ctx * m->KD; }

// nb tokens of sequence `seq` at p0..
bool attention(Model* m, int l, int nb, int p0, int seq, hipStream_t st) {
    const LayerDev& L = m->L[l];
    const size_t off = ((size_t)l * m->n_seq + seq) * seq_floats(m);
    return ok(launch_attention(m->q, m->k, m->v, L.q_norm, L.k_norm, m->rope, m->kc + off, m->vc + off, m->att, nb,
                               m->n_head, m->n_kv, m->hd, p0, m->eps, m->scale, m->part, m->cnt, st),
              "attention");
}

// one token each of nb sequences (m->tpos / m->tseq), positions up to max_pos
bool attention_seqs(Model* m, int l, int nb, int max_pos, hipStream_t st) {
    const LayerDev& L = m->L[l];
    const size_t off = (size_t)l * m->n_seq * seq_floats(m);
    return ok(launch_attention_multi(m->q, m->k, m->v, L.q_norm, L.k_norm, m->rope, m->kc + off, m->vc + off, m->att,
                                     nb, m->n_head, m->n_kv, m->hd, m->tpos, m->tseq, seq_floats(m), max_pos, m->eps,
                                     m->scale, m->part, m->cnt, st),
              "attention");
}

// One token (nb = 1), five launches per layer.  The residual stream is kept
// as r (m->x: the layer's input), h = r + attention (m->h) and the expert
// block's output y (m->tmp); the next layer's Q/K/V launch forms r' = h + y
// (block 0 stores it) and its norm itself:
//   QKV(r or h + y, norm) -> attention -> O-proj (+ r) -> h
//   -> expert block from h (norm, F32 router matmul and routing inside the
//      fused launch; a quantized router runs as its own matrix-vector launch
//      first) -> y
// amax: the output head also tracks the argmax key when set.
bool enqueue_decode(Model* m, int p0, int seq, bool want_logits, unsigned long long* amax) {
    hipStream_t st = m->st;
    for (int l = 0; l < m->n_layer; l++) {
        const LayerDev& L = m->L[l];
        GemvArgs g = l == 0 ? gemv_in(m->x, nullptr, L.attn_norm, m->eps) : gemv_in(m->h, m->tmp, L.attn_norm, m->eps);
        if (l > 0) g.x_sum_out = m->x;
        if (!gemv_qkv(m, L, g, st) || !attention(m, l, 1, p0, seq, st) ||
            !gemv1(L.wo, gemv_in(m->att, nullptr, nullptr, 0.f), m->h, m->x, st, "output projection"))
            return false;
        int* ids = m->ids + (size_t)l * kMaxBatch * m->K;
        float* wts = m->wts + (size_t)l * kMaxBatch * m->K;
        if (L.router.type == kF32 && L.router.rb == (size_t)m->D * 4) {
            // norm, F32 router matmul, routing and experts: one launch where
            // the fused kernel takes the shape (the entry point's own choice)
            if (eahmmf_hip_moe_layer_decode_xn_async(&L.shape, L.table, m->E, (const float*)L.router.p, L.ffn_norm,
                                                     m->eps, m->h, m->K, m->tmp, ids, wts, nullptr, nullptr, st) != 0)
                return false;  // the entry point set the message
            continue;
        }
        GemvArgs gr = gemv_in(m->h, nullptr, L.ffn_norm, m->eps);
        gr.xn_out = m->xn;
        if (!gemv1(L.router, gr, m->rl, nullptr, st, "router")) return false;
        if (eahmmf_hip_moe_layer_decode_async(&L.shape, L.table, m->E, m->rl, m->K, m->xn, m->tmp, ids, wts, st) != 0)
            return false;  // the entry point set the message
    }
    if (!want_logits) return true;
    GemvArgs gh = gemv_in(m->h, m->tmp, m->out_norm, m->eps);
    gh.amax = amax;
    return gemv1(m->out, gh, m->logits, nullptr, st, "output head");
}

// A batch of nb > 1 tokens: per-step kernels over the batch (norm, the
// matmul kernel, attention, add, routing + the grouped expert block).  The
// tokens are nb consecutive positions p0.. of sequence seq, or (seqs) one
// token of each of nb sequences (m->tpos / m->tseq, positions up to
// max_pos), whose logits all come out ([nb][V]).
bool enqueue_batch(Model* m, int nb, int p0, int seq, bool want_logits, bool seqs = false, int max_pos = 0) {
    hipStream_t st = m->st;
    const int D = m->D;
    for (int l = 0; l < m->n_layer; l++) {
        const LayerDev& L = m->L[l];
        int* ids = m->ids + (size_t)l * kMaxBatch * m->K;
        float* wts = m->wts + (size_t)l * kMaxBatch * m->K;
        if (!ok(launch_rmsnorm(m->x, L.attn_norm, m->xn, nb, D, m->eps, st), "attn rmsnorm") ||
            !mm(m, L.wq, m->xn, nb, D, m->q, m->QD, st, "q matmul") ||
            !mm(m, L.wk, m->xn, nb, D, m->k, m->KD, st, "k matmul") ||
            !mm(m, L.wv, m->xn, nb, D, m->v, m->KD, st, "v matmul") ||
            !(seqs ? attention_seqs(m, l, nb, max_pos, st) : attention(m, l, nb, p0, seq, st)) ||
            !mm(m, L.wo, m->att, nb, m->QD, m->tmp, D, st, "output matmul") ||
            !ok(launch_add(m->x, m->tmp, (size_t)nb * D, st), "residual add") ||
            !ok(launch_rmsnorm(m->x, L.ffn_norm, m->xn, nb, D, m->eps, st), "ffn rmsnorm") ||
            !mm(m, L.router, m->xn, nb, D, m->rl, m->E, st, "router matmul"))
            return false;
        if (eahmmf_hip_route_topk_async(m->rl, nb, m->E, m->K, ids, wts, st) != 0 ||
            eahmmf_hip_moe_grouped_async(&L.shape, L.table, m->E, ids, wts, nb, m->K, m->xn, m->tmp, st) != 0)
            return false;
        if (!ok(launch_add(m->x, m->tmp, (size_t)nb * D, st), "residual add")) return false;
    }
    if (!want_logits) return true;
    if (seqs)
        return ok(launch_rmsnorm(m->x, m->out_norm, m->xn, nb, D, m->eps, st), "output rmsnorm") &&
               mm(m, m->out, m->xn, nb, D, m->logits, m->V, st, "output head");
    return gemv1(m->out, gemv_in(m->x + (size_t)(nb - 1) * D, nullptr, m->out_norm, m->eps), m->logits, nullptr, st,
                 "output head");
}

// Enqueues one forward of nb tokens at positions p0...: ids from toks (device)
// or, when key is set (nb = 1), the argmax held in the key, which the
// embedding step clears and also stores in hist when given.
bool enqueue_forward(Model* m, const int* toks, unsigned long long* key, int* hist, int nb, int p0, int seq,
                     bool want_logits, unsigned long long* amax) {
    if (!ok(launch_embed(m->tok.type, m->tok.p, m->tok.rb, (int)m->tok.ne1, m->D, toks, key, hist, nb, m->x, m->bad,
                         m->st),
            "embed"))
        return false;
    return nb == 1 ? enqueue_decode(m, p0, seq, want_logits, amax) : enqueue_batch(m, nb, p0, seq, want_logits);
}

// Queues the error-word and bad-token reads, waits, and judges the forward.
bool finish(Model* m, bool enqueued) {
    bool good = enqueued;
    if (good)
        good = eahmmf_hip_fused_status_async(&m->h_status[1], m->st) == 0 &&
               ok(hipMemcpyAsync(&m->h_status[2], m->bad, sizeof(int), hipMemcpyDeviceToHost, m->st), "read flag");
    const bool synced = ok(hipStreamSynchronize(m->st), "model stream");
    if (!good || !synced) return false;
    if (m->h_status[1] != m->h_status[0]) {
        fail("model forward: a fused expert launch gave up a wait (launch %u); outputs invalid", m->h_status[1]);
        (void)eahmmf_hip_device_flags();  // resets the fused kernel's counters and error word
        return false;
    }
    if (m->h_status[2]) return fail("model forward: token id out of range"), false;
    return true;
}

bool begin(Model* m) {
    return eahmmf_hip_fused_status_async(&m->h_status[0], m->st) == 0 &&
           ok(hipMemsetAsync(m->bad, 0, sizeof(int), m->st), "clear flag");
}

void record_trace(Model* m, int nb) {
    const int K = m->K;
    for (int l = 0; l < m->n_layer; l++)
        for (int t = 0; t < nb; t++)
            for (int j = 0; j < K; j++) {
                const size_t i = ((size_t)l * kMaxBatch + t) * K + j;
                m->tr_ids.push_back(m->h_ids[i]);
                m->tr_w.push_back(m->h_w[i]);
            }
}

bool queue_trace_read(Model* m) {
    const size_t n = (size_t)m->n_layer * kMaxBatch * m->K;
    return ok(hipMemcpyAsync(m->h_ids, m->ids, n * sizeof(int), hipMemcpyDeviceToHost, m->st), "read trace") &&
           ok(hipMemcpyAsync(m->h_w, m->wts, n * sizeof(float), hipMemcpyDeviceToHost, m->st), "read trace");
}

int forward(Model* m, const int* toks, int nb, int p0, int seq, float* logits) {
    if (nb < 1 || nb > kMaxBatch) return fail("batch size %d outside 1..%d", nb, kMaxBatch), -1;
    if (seq < 0 || seq >= m->n_seq) return fail("sequence %d outside 0..%d", seq, m->n_seq - 1), -1;
    if (p0 < 0 || p0 + nb > m->n_ctx) return fail("context overflow (%d > %d)", p0 + nb, m->n_ctx), -1;
    for (int t = 0; t < nb; t++)
        if (toks[t] < 0 || toks[t] >= (int)m->tok.ne1) return fail("token id %d out of range", toks[t]), -1;
    DeviceGuard g(m->dev);
    memcpy(m->h_toks, toks, sizeof(int) * nb);
    bool e = begin(m) &&
             ok(hipMemcpyAsync(m->toks, m->h_toks, sizeof(int) * nb, hipMemcpyHostToDevice, m->st), "copy tokens") &&
             enqueue_forward(m, m->toks, nullptr, nullptr, nb, p0, seq, logits != nullptr, nullptr);
    if (e && logits)
        e = ok(hipMemcpyAsync(m->h_logits, m->logits, sizeof(float) * m->V, hipMemcpyDeviceToHost, m->st),
               "read logits");
    if (e && m->trace) e = queue_trace_read(m);
    if (!finish(m, e)) return -3;
    if (logits) memcpy(logits, m->h_logits, sizeof(float) * m->V);
    if (m->trace) record_trace(m, nb);
    return 0;
}

// One token of each of n distinct sequences; logits [n][V] when given.
int decode_seqs(Model* m, int n, const int* toks, const int* seqs, const int* pos, float* logits) {
    if (n < 1 || n > m->n_seq) return fail("sequence count %d outside 1..%d", n, m->n_seq), -1;
    int max_pos = 0;
    for (int t = 0; t < n; t++) {
        if (toks[t] < 0 || toks[t] >= (int)m->tok.ne1) return fail("token id %d out of range", toks[t]), -1;
        if (seqs[t] < 0 || seqs[t] >= m->n_seq) return fail("sequence %d outside 0..%d", seqs[t], m->n_seq - 1), -1;
        if (pos[t] < 0 || pos[t] >= m->n_ctx) return fail("context overflow (%d > %d)", pos[t] + 1, m->n_ctx), -1;
        for (int u = 0; u < t; u++)
            if (seqs[u] == seqs[t]) return fail("sequence %d given twice in one step", seqs[t]), -1;
        max_pos = pos[t] > max_pos ? pos[t] : max_pos;
    }
    DeviceGuard g(m->dev);
    // tokens, positions and sequences staged together (m->tpos / m->tseq follow m->toks)
    memcpy(m->h_toks, toks, sizeof(int) * n);
    memcpy(m->h_toks + kMaxBatch, pos, sizeof(int) * n);
    memcpy(m->h_toks + 2 * kMaxBatch, seqs, sizeof(int) * n);
    bool e = begin(m) &&
             ok(hipMemcpyAsync(m->toks, m->h_toks, sizeof(int) * 3 * kMaxBatch, hipMemcpyHostToDevice, m->st),
                "copy tokens") &&
             ok(launch_embed(m->tok.type, m->tok.p, m->tok.rb, (int)m->tok.ne1, m->D, m->toks, nullptr, nullptr, n,
                             m->x, m->bad, m->st),
                "embed") &&
             enqueue_batch(m, n, 0, 0, logits != nullptr, true, max_pos);
    if (e && logits)
        e = ok(hipMemcpyAsync(m->h_logits, m->logits, sizeof(float) * n * m->V, hipMemcpyDeviceToHost, m->st),
               "read logits");
    if (e && m->trace) e = queue_trace_read(m);
    if (!finish(m, e)) return -3;
    if (logits) memcpy(logits, m->h_logits, sizeof(float) * n * m->V);
    if (m->trace) record_trace(m, n);
    return 0;
}

}  // namespace

extern "C" {

void* eahmmf_hip_model_create(const eahmmf_hip_model_desc* d) {
    if (!d || !d->layers) return fail("null model description"), nullptr;
    Model* m = new Model();
    if (!ok(hipGetDevice(&m->dev), "hipGetDevice")) return delete m, nullptr;
    m->n_layer = d->n_layer;
    m->D = d->D;
    m->n_head = d->n_head;
    m->n_kv = d->n_kv;
    m->hd = d->hd;
    m->E = d->n_expert;
    m->K = d->n_used;
    m->FF = d->FF;
    m->V = d->n_vocab;
    m->n_ctx = d->n_ctx;
    m->eps = d->eps;
    m->rope_base = d->rope_base;
    m->QD = m->n_head * m->hd;
    m->KD = m->n_kv * m->hd;
    m->scale = 1.0f / sqrtf((float)m->hd);
    auto bad = [&](const char* why) {
        fail("model: %s", why);
        release(m);
        return nullptr;
    };
    if (m->n_layer <= 0 || m->D <= 0 || m->n_head <= 0 || m->n_kv <= 0 || m->n_ctx <= 0 || m->V <= 0)
        return bad("non-positive dimension");
    if (m->hd != 64 && m->hd != 128) return bad("head dimension must be 64 or 128");
    if (!attention_supported(m->n_head, m->n_kv, m->hd)) return bad("n_head / n_kv must be 1, 2, 4, 8 or 16");
    if (m->D % 32 || m->FF % 32 || m->QD % 32) return bad("dimensions must be multiples of 32");
    if (m->E <= 0 || m->E > 512 || m->K <= 0 || m->K > kMaxSlots || m->K > m->E) return bad("bad expert count / top-k");
    if (!ok(hipStreamCreateWithFlags(&m->st, hipStreamNonBlocking), "hipStreamCreate")) return release(m), nullptr;

    const int D = m->D, FF = m->FF, E = m->E;
    if (!place(m, d->tok_embd, "token_embd", D, d->tok_embd.ne1, false, m->tok)) return release(m), nullptr;
    if (d->output.data) {
        if (!place(m, d->output, "output", D, m->V, false, m->out)) return release(m), nullptr;
    } else {
        if (m->tok.ne1 != m->V) return bad("tied output: token_embd rows != n_vocab");
        m->out = m->tok;
    }
    if (!place_vec(m, d->output_norm, "output_norm", D, &m->out_norm)) return release(m), nullptr;
    m->L.resize(m->n_layer);
    for (int l = 0; l < m->n_layer; l++) {
        const eahmmf_hip_layer_desc& s = d->layers[l];
        LayerDev& L = m->L[l];
        Tens g, u, dn;
        if (!place_vec(m, s.attn_norm, "attn_norm", D, &L.attn_norm) ||
            !place_vec(m, s.ffn_norm, "ffn_norm", D, &L.ffn_norm) ||
            !place_vec(m, s.q_norm, "attn_q_norm", m->hd, &L.q_norm) ||
            !place_vec(m, s.k_norm, "attn_k_norm", m->hd, &L.k_norm) ||
            !place(m, s.wq, "attn_q", D, m->QD, false, L.wq) || !place(m, s.wk, "attn_k", D, m->KD, false, L.wk) ||
            !place(m, s.wv, "attn_v", D, m->KD, false, L.wv) ||
            !place(m, s.wo, "attn_output", m->QD, D, false, L.wo) ||
            !place(m, s.router, "ffn_gate_inp", D, E, false, L.router) ||
            !place(m, s.gate_exps, "ffn_gate_exps", D, (int64_t)E * FF, false, g) ||
            !place(m, s.up_exps, "ffn_up_exps", D, (int64_t)E * FF, false, u) ||
            !place(m, s.down_exps, "ffn_down_exps", FF, (int64_t)E * D, false, dn))
            return release(m), nullptr;
        L.shape = eahmmf_hip_moe_shape{g.type, u.type, dn.type, D, FF, g.rb, u.rb, dn.rb};
        MoeShape ms{g.type, u.type, dn.type, D, FF, g.rb, u.rb, dn.rb};
        if (!moe_shape_ok(ms)) return bad("unsupported expert shape/type combination");
        std::vector<eahmmf_hip_expert_ptrs> tab(E);
        for (int e = 0; e < E; e++)
            tab[e] = eahmmf_hip_expert_ptrs{g.p + (size_t)e * FF * g.rb, u.p + (size_t)e * FF * u.rb,
                                            dn.p + (size_t)e * D * dn.rb};
        L.table = static_cast<eahmmf_hip_expert_ptrs*>(dalloc(m, sizeof(eahmmf_hip_expert_ptrs) * E, false));
        if (!L.table || !ok(hipMemcpy(L.table, tab.data(), sizeof(eahmmf_hip_expert_ptrs) * E, hipMemcpyHostToDevice),
                            "copy expert table"))
            return release(m), nullptr;
    }
    // RoPE table as the reference computes it: inv_freq[i] = (float)base^(-2i/hd),
    // then cos/sin of (double)pos * inv_freq[i] rounded to float (qwen3moe.cpp:906-907, 936-941).
    const int half = m->hd / 2;
    std::vector<float> inv(half), rope((size_t)m->n_ctx * half * 2);
    for (int i = 0; i < half; i++) inv[i] = (float)pow((double)m->rope_base, -2.0 * i / m->hd);
    for (int p = 0; p < m->n_ctx; p++)
        for (int i = 0; i < half; i++) {
            const double ang = (double)p * inv[i];
            rope[((size_t)p * half + i) * 2] = (float)cos(ang);
            rope[((size_t)p * half + i) * 2 + 1] = (float)sin(ang);
        }
    const size_t kvn = (size_t)m->n_layer * m->n_ctx * m->KD;
    const int B = kMaxBatch, Kk = m->K;
    m->rope = (float*)dalloc(m, rope.size() * sizeof(float), false);
    m->kc = (float*)dalloc(m, kvn * sizeof(float), true);
    m->vc = (float*)dalloc(m, kvn * sizeof(float), true);
    m->x = (float*)dalloc(m, (size_t)B * D * 4, false);
    m->xn = (float*)dalloc(m, (size_t)B * D * 4, false);
    m->h = (float*)dalloc(m, (size_t)D * 4, false);
    m->key = (unsigned long long*)dalloc(m, 8, true);
    m->q = (float*)dalloc(m, (size_t)B * m->QD * 4, false);
    m->k = (float*)dalloc(m, (size_t)B * m->KD * 4, false);
    m->v = (float*)dalloc(m, (size_t)B * m->KD * 4, false);
    m->att = (float*)dalloc(m, (size_t)B * m->QD * 4, false);
    m->tmp = (float*)dalloc(m, (size_t)B * D * 4, false);
    m->rl = (float*)dalloc(m, (size_t)B * E * 4, false);
    m->logits = (float*)dalloc(m, (size_t)m->V * 4, false);  // one row until more sequences are set
    m->part = (float*)dalloc(m, attention_part_floats(B, m->n_head, m->hd, m->n_ctx) * 4, false);
    m->cnt = (unsigned*)dalloc(m, (size_t)B * m->n_kv * 4, true);
    m->toks = (int*)dalloc(m, (size_t)3 * B * 4, false);  // tokens, then positions, then sequences
    m->ids = (int*)dalloc(m, (size_t)m->n_layer * B * Kk * 4, true);
    m->wts = (float*)dalloc(m, (size_t)m->n_layer * B * Kk * 4, true);
    m->bad = (int*)dalloc(m, 4, true);
    m->gen = (int*)dalloc(m, 4, true);
    if (!m->rope || !m->kc || !m->vc || !m->x || !m->xn || !m->h || !m->key || !m->q || !m->k || !m->v || !m->att || !m->tmp || !m->rl ||
        !m->logits || !m->part || !m->cnt || !m->toks || !m->ids || !m->wts || !m->bad || !m->gen)
        return release(m), nullptr;
    m->tpos = m->toks + B;
    m->tseq = m->toks + 2 * B;
    m->ws_bytes = mm_ws_bytes(m);
    if (m->ws_bytes && !(m->ws = dalloc(m, m->ws_bytes, false))) return release(m), nullptr;
    if (!ok(hipMemcpy(m->rope, rope.data(), rope.size() * sizeof(float), hipMemcpyHostToDevice), "copy rope"))
        return release(m), nullptr;
    const size_t trn = (size_t)m->n_layer * B * Kk;
    if (!ok(hipHostMalloc((void**)&m->h_toks, 3 * B * sizeof(int), 0), "hipHostMalloc") ||
        !ok(hipHostMalloc((void**)&m->h_logits, (size_t)m->V * sizeof(float), 0), "hipHostMalloc") ||
        !ok(hipHostMalloc((void**)&m->h_ids, trn * sizeof(int), 0), "hipHostMalloc") ||
        !ok(hipHostMalloc((void**)&m->h_w, trn * sizeof(float), 0), "hipHostMalloc") ||
        !ok(hipHostMalloc((void**)&m->h_status, 4 * sizeof(unsigned), 0), "hipHostMalloc"))
        return release(m), nullptr;
    return m;
}

int eahmmf_hip_model_forward(void* model, const int* toks, int nb, int p0, float* logits) {
    if (!model || !toks) return fail("null argument"), -1;
    return forward(static_cast<Model*>(model), toks, nb, p0, 0, logits);
}

int eahmmf_hip_model_set_sequences(void* model, int n_seq) {
    Model* m = static_cast<Model*>(model);
    if (!m) return fail("null model"), -1;
    if (n_seq < 1 || n_seq > kMaxBatch) return fail("sequence count %d outside 1..%d", n_seq, kMaxBatch), -1;
    DeviceGuard g(m->dev);
    if (!ok(hipStreamSynchronize(m->st), "model stream")) return -3;
    const size_t kvn = (size_t)m->n_layer * n_seq * seq_floats(m);
    float* kc = (float*)dalloc(m, kvn * sizeof(float), true);
    float* vc = kc ? (float*)dalloc(m, kvn * sizeof(float), true) : nullptr;
    float* lg = nullptr;
    float* hlg = nullptr;
    const int rows = n_seq > m->lg_rows ? n_seq : m->lg_rows;
    if (vc && rows > m->lg_rows) {
        lg = (float*)dalloc(m, (size_t)rows * m->V * 4, false);
        if (lg && !ok(hipHostMalloc((void**)&hlg, (size_t)rows * m->V * sizeof(float), 0), "hipHostMalloc"))
            hlg = nullptr;
    }
    // drops device allocations made here or replaced (they are in m->owned)
    auto drop = [m](void* p) {
        if (!p) return;
        for (size_t i = 0; i < m->owned.size(); i++)
            if (m->owned[i] == p) {
                m->owned.erase(m->owned.begin() + i);
                break;
            }
        (void)hipFree(p);
    };
    if (!kc || !vc || (rows > m->lg_rows && (!lg || !hlg))) {
        drop(kc);
        drop(vc);
        drop(lg);
        return -3;  // dalloc / hipHostMalloc set the message; the model is as it was
    }
    drop(m->kc);
    drop(m->vc);
    m->kc = kc;
    m->vc = vc;
    if (lg) {
        drop(m->logits);
        (void)hipHostFree(m->h_logits);
        m->logits = lg;
        m->h_logits = hlg;
        m->lg_rows = rows;
    }
    m->n_seq = n_seq;
    return 0;
}

int eahmmf_hip_model_forward_seq(void* model, int seq, const int* toks, int nb, int p0, float* logits) {
    if (!model || !toks) return fail("null argument"), -1;
    return forward(static_cast<Model*>(model), toks, nb, p0, seq, logits);
}

int eahmmf_hip_model_decode_seqs(void* model, int n, const int* toks, const int* seqs, const int* pos,
                                 float* logits) {
    if (!model || !toks || !seqs || !pos) return fail("null argument"), -1;
    return decode_seqs(static_cast<Model*>(model), n, toks, seqs, pos, logits);
}

int eahmmf_hip_model_eval(void* model, const int* toks, int n, int p0, int n_batch, float* logits) {
    if (!model || !toks || n <= 0) return fail("null argument or empty input"), -1;
    if (n_batch < 1 || n_batch > kMaxBatch) return fail("n_batch %d outside 1..%d", n_batch, kMaxBatch), -1;
    Model* m = static_cast<Model*>(model);
    for (int i = 0; i < n; i += n_batch) {
        const int nb = n - i < n_batch ? n - i : n_batch;
        const int rc = forward(m, toks + i, nb, p0 + i, 0, i + nb == n ? logits : nullptr);
        if (rc) return rc;
    }
    return 0;
}

int eahmmf_hip_model_generate_greedy(void* model, int first, int p0, int n, int* out_toks, float* last_logits) {
    Model* m = static_cast<Model*>(model);
    if (!m || !out_toks || n <= 0) return fail("null argument or n <= 0"), -1;
    if (p0 < 0 || p0 + n > m->n_ctx) return fail("context overflow (%d > %d)", p0 + n, m->n_ctx), -1;
    if (first < 0 || first >= (int)m->tok.ne1) return fail("token id %d out of range", first), -1;
    DeviceGuard g(m->dev);
    if (n > m->gen_cap) {
        if (m->h_gen) (void)hipHostFree(m->h_gen);
        m->h_gen = nullptr;
        m->gen_cap = 0;
        void* p = nullptr;
        if (!ok(hipMalloc(&p, (size_t)n * sizeof(int)), "hipMalloc")) return -3;
        m->owned.push_back(p);
        m->gen = static_cast<int*>(p);
        if (!ok(hipHostMalloc((void**)&m->h_gen, (size_t)n * sizeof(int), 0), "hipHostMalloc")) return -3;
        m->gen_cap = n;
    }
    m->h_toks[0] = first;
    bool e = begin(m) &&
             ok(hipMemcpyAsync(m->toks, m->h_toks, sizeof(int), hipMemcpyHostToDevice, m->st), "copy token");
    // step i embeds token i (the first from the host, then the argmax key of
    // step i - 1, stored as output i - 1) and leaves its argmax in the key
    for (int i = 0; e && i < n; i++) {
        e = enqueue_forward(m, i == 0 ? m->toks : nullptr, i == 0 ? nullptr : m->key, i == 0 ? nullptr : m->gen + i - 1,
                            1, p0 + i, 0, true, m->key);
        if (e && m->trace) {
            // the trace of this step is read before the next step overwrites it
            e = queue_trace_read(m) && ok(hipStreamSynchronize(m->st), "model stream");
            if (e) record_trace(m, 1);
        }
    }
    // the last argmax: through the embedding step once more (its row is not used)
    if (e)
        e = ok(launch_embed(m->tok.type, m->tok.p, m->tok.rb, (int)m->tok.ne1, m->D, nullptr, m->key, m->gen + n - 1, 1,
                            m->x, m->bad, m->st),
               "last token");
    if (e) e = ok(hipMemcpyAsync(m->h_gen, m->gen, (size_t)n * sizeof(int), hipMemcpyDeviceToHost, m->st), "read tokens");
    if (e && last_logits)
        e = ok(hipMemcpyAsync(m->h_logits, m->logits, sizeof(float) * m->V, hipMemcpyDeviceToHost, m->st),
               "read logits");
    if (!finish(m, e)) return -3;
    memcpy(out_toks, m->h_gen, (size_t)n * sizeof(int));
    if (last_logits) memcpy(last_logits, m->h_logits, sizeof(float) * m->V);
    return 0;
}

int eahmmf_hip_model_set_trace(void* model, int on) {
    if (!model) return -1;
    Model* m = static_cast<Model*>(model);
    const int prev = m->trace ? 1 : 0;
    m->trace = on != 0;
    return prev;
}

int eahmmf_hip_model_trace(void* model, int* ids, float* w, int cap) {
    if (!model) return -1;
    Model* m = static_cast<Model*>(model);
    const int n = (int)m->tr_ids.size();
    for (int i = 0; i < n && i < cap; i++) {
        if (ids) ids[i] = m->tr_ids[i];
        if (w) w[i] = m->tr_w[i];
    }
    return n;
}

void eahmmf_hip_model_trace_clear(void* model) {
    if (!model) return;
    static_cast<Model*>(model)->tr_ids.clear();
    static_cast<Model*>(model)->tr_w.clear();
}

void* eahmmf_hip_model_stream(void* model) { return model ? (void*)static_cast<Model*>(model)->st : nullptr; }

void eahmmf_hip_model_free(void* model) { release(static_cast<Model*>(model)); }

}  // extern "C"
