// ref_harness.cpp - exposes the compiled reference's CPU primitives through a
// C ABI so tests and fixture scripts can call them.
//
// TEST INFRASTRUCTURE ONLY.  This file is ours; it compiles the reference's
// own qwen3moe.cpp in place (REF_SRC points at it, it is never copied) with
// the reference's QWEN3MOE_NO_MAIN switch, the same way the reference's
// tests/test_eahmmf.cpp:5-6 does.  The output goes to oracle/_ref/ only.
// Without /root/reference the library is simply not built.
#define QWEN3MOE_NO_MAIN
#include REF_SRC

#include <omp.h>

extern "C" {

void ref_init() { init_types(); }

// One block of `type` through the reference's dq_* table (qwen3moe.cpp:204-218).
int ref_dequant_block(int type, const uint8_t* src, float* dst) {
    if (type < 0 || type >= 40 || !g_types[type].dq) return -1;
    g_types[type].dq(src, dst);
    return 0;
}

// The reference's block-wise matmul (qwen3moe.cpp:397-419); nb <= MAXB.
int ref_matmul(int type, int64_t ne0, int64_t ne1, size_t row_bytes, const uint8_t* w,
               const float* x, int nb, int ldx, float* out, int ldo) {
    if (type < 0 || type >= 40 || !g_types[type].dq || nb < 1 || nb > MAXB) return -1;
    WeightView v;
    v.data = w;
    v.type = (uint32_t)type;
    v.ne0 = ne0;
    v.ne1 = ne1;
    v.row_bytes = row_bytes;
    v.bytes = row_bytes * (size_t)ne1;
    matmul(v, x, nb, ldx, out, ldo);
    return 0;
}

void ref_rmsnorm(const float* x, const float* w, float* out, int n, float eps) { rmsnorm(x, w, out, n, eps); }

// The timed CPU baseline: the reference's single-token expert block
// (qwen3moe.cpp:1024-1067 at nb = 1: for each routed expert in ascending id,
// the gate and up matmuls, SiLU, the down matmul, y += w * out) over n_tok
// tokens per repetition, with `threads` OpenMP threads.  Experts are stacked:
// expert e's gate at gate + e * FF * grb, its down at down + e * D * drb.
// ids/w [n_tok][k], ids ascending per token.  secs[i] receives the wall time
// of timed repetition i; `warmup` untimed repetitions run first.
int ref_time_expert_tokens(int gt, int dt, int D, int FF, size_t grb, size_t drb, const uint8_t* gate,
                           const uint8_t* up, const uint8_t* down, const float* xs, const int* ids, const float* w,
                           int k, int n_tok, int threads, int warmup, int reps, double* secs) {
    if (!g_types[gt].dq || !g_types[dt].dq || threads < 1) return -1;
    omp_set_num_threads(threads);
    std::vector<float> g(FF), u(FF), yd(D), y(D);
    auto view = [](int t, const uint8_t* p, int64_t ne0, int64_t ne1, size_t rb) {
        WeightView v;
        v.data = p;
        v.type = (uint32_t)t;
        v.ne0 = ne0;
        v.ne1 = ne1;
        v.row_bytes = rb;
        v.bytes = rb * (size_t)ne1;
        return v;
    };
    for (int rep = 0; rep < warmup + reps; rep++) {
        const auto t0 = std::chrono::steady_clock::now();
        for (int t = 0; t < n_tok; t++) {
            const float* x = xs + (size_t)t * D;
            std::fill(y.begin(), y.end(), 0.f);
            for (int j = 0; j < k; j++) {
                const int e = ids[(size_t)t * k + j];
                matmul(view(gt, gate + (size_t)e * FF * grb, D, FF, grb), x, 1, D, g.data(), FF);
                matmul(view(gt, up + (size_t)e * FF * grb, D, FF, grb), x, 1, D, u.data(), FF);
                for (int i = 0; i < FF; i++) {
                    float gv = g[i];
                    g[i] = gv / (1.0f + expf(-gv)) * u[i];
                }
                matmul(view(dt, down + (size_t)e * D * drb, FF, D, drb), g.data(), 1, FF, yd.data(), D);
                const float wj = w[(size_t)t * k + j];
                for (int r = 0; r < D; r++) y[r] += wj * yd[r];
            }
        }
        const double el = std::chrono::duration<double>(std::chrono::steady_clock::now() - t0).count();
        if (rep >= warmup) secs[rep - warmup] = el;
    }
    return 0;
}

// Whole engine over a GGUF file (qwen3moe.cpp:859-922, 932-1084).
void* ref_engine_new(const char* path, int ctx) {
    Engine* e = new Engine();
    e->load(path, ctx, false);
    e->trace_routing = true;
    return e;
}
void ref_engine_free(void* h) { delete (Engine*)h; }
int ref_engine_vocab(void* h) { return ((Engine*)h)->n_vocab; }
void ref_engine_eval(void* h, const int* toks, int n, int p0, int n_batch, float* logits) {
    std::vector<int> t(toks, toks + n);
    ((Engine*)h)->eval(t, p0, n_batch, logits);
}
void ref_engine_forward(void* h, const int* toks, int nb, int p0, float* logits) {
    ((Engine*)h)->forward(toks, nb, p0, logits);
}
int ref_engine_trace(void* h, int* ids, float* w, int cap) {
    Engine* e = (Engine*)h;
    int n = (int)e->trace_ids.size();
    for (int i = 0; i < n && i < cap; i++) {
        ids[i] = e->trace_ids[i];
        w[i] = e->trace_w[i];
    }
    return n;
}
void ref_engine_trace_clear(void* h) {
    ((Engine*)h)->trace_ids.clear();
    ((Engine*)h)->trace_w.clear();
}

}  // extern "C"
