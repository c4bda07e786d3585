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
