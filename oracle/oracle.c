/*
 * oracle.c - CPU restatement of the reference's quantized expert-FFN path.
 *
 * TEST INFRASTRUCTURE ONLY: the parity checker for the HIP path (see oracle.h
 * for who may load it and how each function is pinned).  Built with the
 * reference's arithmetic flags (-O3 -march=native -ffp-contract=fast) but the
 * two places where the reference binary's rounding matters are written out
 * explicitly so they do not depend on the compiler:
 *   - Q4_K / Q5_K values use a single-rounding fmaf(d*sc, q, -(dmin*m)), which
 *     is what the reference binary computes after GCC contracts
 *     `d1 * q - m1` (qwen3moe.cpp:155-156, 175-176);
 *   - Q6_K values are two separate products (d*sc)*q (qwen3moe.cpp:193-196).
 */
#include "oracle.h"

#include <math.h>
#include <omp.h>
#include <time.h>
#include <stdlib.h>
#include <string.h>

static float g_half[65536];
static int g_ready = 0;

/* qwen3moe.cpp:55-62: exact half -> float, NaN canonicalised with its sign. */
static float half_closed_form(uint16_t h) {
    unsigned sign = (h >> 15) & 1u, expo = (h >> 10) & 31u, mant = h & 1023u;
    float v;
    if (expo == 0)
        v = ldexpf((float)mant, -24);
    else if (expo == 31)
        v = mant ? NAN : INFINITY;
    else
        v = ldexpf((float)(mant | 1024u), (int)expo - 25);
    return sign ? -v : v;
}

void orc_init(void) {
    if (g_ready) return;
    for (int i = 0; i < 65536; i++) g_half[i] = half_closed_form((uint16_t)i);
    g_ready = 1;
}

float orc_f16(uint16_t h) {
    orc_init();
    return g_half[h];
}

static inline float rd16(const uint8_t* p) { return g_half[(uint16_t)(p[0] | (p[1] << 8))]; }

/* qwen3moe.cpp:133-141: eight 6-bit (scale, min) pairs packed in 12 bytes. */
void orc_scale_min_k4(int j, const uint8_t* q, uint8_t* d, uint8_t* m) {
    if (j < 4) {
        *d = (uint8_t)(q[j] & 63);
        *m = (uint8_t)(q[j + 4] & 63);
    } else {
        *d = (uint8_t)((q[j + 4] & 15) | ((q[j - 4] >> 6) << 4));
        *m = (uint8_t)((q[j + 4] >> 4) | ((q[j] >> 6) << 4));
    }
}

int orc_blck(int type) {
    switch (type) {
        case ORC_F32: return 32;
        case ORC_Q8_0: return 32;
        case ORC_Q4_K: case ORC_Q5_K: case ORC_Q6_K: return 256;
        default: return 0;
    }
}

int orc_type_bytes(int type) {
    switch (type) {
        case ORC_F32: return 128;
        case ORC_Q8_0: return 34;
        case ORC_Q4_K: return 144;
        case ORC_Q5_K: return 176;
        case ORC_Q6_K: return 210;
        default: return 0;
    }
}

/* qwen3moe.cpp:128-132 */
static void dq_q8_0(const uint8_t* b, float* y) {
    const float d = rd16(b);
    const int8_t* q = (const int8_t*)(b + 2);
    for (int i = 0; i < 32; i++) y[i] = d * (float)q[i];
}

/* qwen3moe.cpp:142-158.  Values are laid out as four 64-value chunks; chunk g
 * uses qs[32g .. 32g+32): low nibbles are sub-block 2g, high nibbles 2g+1. */
static void dq_q4_k(const uint8_t* b, float* y) {
    const float d = rd16(b), dmin = rd16(b + 2);
    const uint8_t* scales = b + 4;
    const uint8_t* qs = b + 16;
    for (int g = 0; g < 4; g++) {
        for (int h = 0; h < 2; h++) {
            uint8_t sc, mn;
            orc_scale_min_k4(2 * g + h, scales, &sc, &mn);
            const float ds = d * (float)sc, dm = dmin * (float)mn;
            for (int l = 0; l < 32; l++) {
                const int q = h ? (qs[32 * g + l] >> 4) : (qs[32 * g + l] & 15);
                y[64 * g + 32 * h + l] = fmaf(ds, (float)q, -dm);
            }
        }
    }
}

/* qwen3moe.cpp:159-179: Q4_K plus a fifth bit from qh (bit 2g+h of qh[l]). */
static void dq_q5_k(const uint8_t* b, float* y) {
    const float d = rd16(b), dmin = rd16(b + 2);
    const uint8_t* scales = b + 4;
    const uint8_t* qh = b + 16;
    const uint8_t* qs = b + 48;
    for (int g = 0; g < 4; g++) {
        for (int h = 0; h < 2; h++) {
            uint8_t sc, mn;
            orc_scale_min_k4(2 * g + h, scales, &sc, &mn);
            const float ds = d * (float)sc, dm = dmin * (float)mn;
            for (int l = 0; l < 32; l++) {
                int q = h ? (qs[32 * g + l] >> 4) : (qs[32 * g + l] & 15);
                q += ((qh[l] >> (2 * g + h)) & 1) ? 16 : 0;
                y[64 * g + 32 * h + l] = fmaf(ds, (float)q, -dm);
            }
        }
    }
}

/* qwen3moe.cpp:180-202.  Half n (128 values) uses ql[64n..], qh[32n..],
 * sc[8n..]; quarter u of the half takes the low (u<2) or high nibble of
 * ql[l + 32*(u&1)] and bits 2u..2u+1 of qh[l]. */
static void dq_q6_k(const uint8_t* b, float* y) {
    const float d = rd16(b + 208);
    for (int n = 0; n < 2; n++) {
        const uint8_t* ql = b + 64 * n;
        const uint8_t* qh = b + 128 + 32 * n;
        const int8_t* sc = (const int8_t*)(b + 192 + 8 * n);
        for (int u = 0; u < 4; u++) {
            for (int l = 0; l < 32; l++) {
                const uint8_t lo = ql[l + 32 * (u & 1)];
                const int lo4 = (u < 2) ? (lo & 15) : (lo >> 4);
                const int q = (lo4 | (((qh[l] >> (2 * u)) & 3) << 4)) - 32;
                const float ds = d * (float)sc[l / 16 + 2 * u];
                y[128 * n + 32 * u + l] = ds * (float)q;
            }
        }
    }
}

static void dq_f32(const uint8_t* b, float* y) { memcpy(y, b, 128); }

int orc_dequant_block(int type, const uint8_t* b, float* y) {
    orc_init();
    switch (type) {
        case ORC_F32: dq_f32(b, y); return 0;
        case ORC_Q8_0: dq_q8_0(b, y); return 0;
        case ORC_Q4_K: dq_q4_k(b, y); return 0;
        case ORC_Q5_K: dq_q5_k(b, y); return 0;
        case ORC_Q6_K: dq_q6_k(b, y); return 0;
        default: return -1;
    }
}

int orc_dequant_rows(int type, const uint8_t* w, int64_t ne0, int64_t nrows, size_t row_bytes, float* out) {
    const int blck = orc_blck(type), bytes = orc_type_bytes(type);
    if (!blck || ne0 % blck) return -1;
    for (int64_t r = 0; r < nrows; r++)
        for (int64_t b = 0; b < ne0 / blck; b++)
            orc_dequant_block(type, w + (size_t)r * row_bytes + (size_t)b * bytes, out + (size_t)r * ne0 + b * blck);
    return 0;
}

/* qwen3moe.cpp:376-381 */
static float dotf(const float* a, const float* b, int n) {
    float s = 0.f;
    for (int i = 0; i < n; i++) s += a[i] * b[i];
    return s;
}

/* qwen3moe.cpp:397-419: one block is dequantized, then dotted with every
 * token's slice; block partial sums accumulate per token in fp32. */
int orc_matmul(int type, int64_t ne0, int64_t ne1, size_t row_bytes, const uint8_t* w,
               const float* x, int nb, int ldx, float* out, int ldo) {
    const int blck = orc_blck(type), bytes = orc_type_bytes(type);
    if (!blck || ne0 % blck || nb <= 0) return -1;
    orc_init();
    const int64_t nblk = ne0 / blck;
#pragma omp parallel for schedule(dynamic, 16) if (ne1 * ne0 > 65536)
    for (int64_t r = 0; r < ne1; r++) {
        float tmp[256];
        float accl[64];
        float* heap = nb > 64 ? (float*)malloc(sizeof(float) * (size_t)nb) : NULL;
        float* a = heap ? heap : accl;
        for (int t = 0; t < nb; t++) a[t] = 0.f;
        const uint8_t* wr = w + (size_t)r * row_bytes;
        for (int64_t b = 0; b < nblk; b++) {
            orc_dequant_block(type, wr + (size_t)b * bytes, tmp);
            for (int t = 0; t < nb; t++) a[t] += dotf(tmp, x + (size_t)t * ldx + b * blck, blck);
        }
        for (int t = 0; t < nb; t++) out[(size_t)t * ldo + r] = a[t];
        free(heap);
    }
    return 0;
}

static float silu_mul(float g, float u) { return g / (1.0f + expf(-g)) * u; }

/* The timed CPU baseline when the compiled reference is absent: the expert
 * block of qwen3moe.cpp:1024-1067 at nb = 1 over n_tok tokens per
 * repetition through orc_matmul (stacked experts: e's gate at
 * gate + e*FF*grb, its down at down + e*D*drb; ids ascending per token);
 * secs[i] = wall time of timed repetition i after `warmup` untimed ones. */
int orc_time_expert_tokens(int gt, int dt, int D, int FF, size_t grb, size_t drb, const uint8_t* gate,
                           const uint8_t* up, const uint8_t* down, const float* xs, const int* ids, const float* w,
                           int k, int n_tok, int threads, int warmup, int reps, double* secs) {
    if (!orc_blck(gt) || !orc_blck(dt) || threads < 1) return -1;
    omp_set_num_threads(threads);
    float* g = (float*)malloc(sizeof(float) * (size_t)FF);
    float* u = (float*)malloc(sizeof(float) * (size_t)FF);
    float* yd = (float*)malloc(sizeof(float) * (size_t)D);
    float* y = (float*)malloc(sizeof(float) * (size_t)D);
    for (int rep = 0; rep < warmup + reps; rep++) {
        struct timespec t0, t1;
        clock_gettime(CLOCK_MONOTONIC, &t0);
        for (int t = 0; t < n_tok; t++) {
            const float* x = xs + (size_t)t * D;
            memset(y, 0, sizeof(float) * (size_t)D);
            for (int j = 0; j < k; j++) {
                const int e = ids[(size_t)t * k + j];
                orc_matmul(gt, D, FF, grb, gate + (size_t)e * FF * grb, x, 1, D, g, FF);
                orc_matmul(gt, D, FF, grb, up + (size_t)e * FF * grb, x, 1, D, u, FF);
                for (int i = 0; i < FF; i++) g[i] = silu_mul(g[i], u[i]);
                orc_matmul(dt, FF, D, drb, down + (size_t)e * D * drb, g, 1, FF, yd, D);
                const float wj = w[(size_t)t * k + j];
                for (int r = 0; r < D; r++) y[r] += wj * yd[r];
            }
        }
        clock_gettime(CLOCK_MONOTONIC, &t1);
        if (rep >= warmup) secs[rep - warmup] = (double)(t1.tv_sec - t0.tv_sec) + 1e-9 * (double)(t1.tv_nsec - t0.tv_nsec);
    }
    free(g);
    free(u);
    free(yd);
    free(y);
    return 0;
}

/* qwen3moe.cpp:527-532 */
void orc_rmsnorm(const float* x, const float* w, float* out, int n, float eps) {
    float ss = 0.f;
    for (int i = 0; i < n; i++) ss += x[i] * x[i];
    const float sc = 1.0f / sqrtf(ss / (float)n + eps);
    for (int i = 0; i < n; i++) out[i] = x[i] * sc * w[i];
}

/* qwen3moe.cpp:1011-1023.  e_i = expf(l_i - max); ranking by (e desc, index
 * asc) via k selection passes (same result as partial_sort with that
 * comparator); the normaliser sums the chosen e in rank order. */
void orc_route_topk(const float* logits, int nb, int n_expert, int k, int* ids, float* wts) {
    float* e = (float*)malloc(sizeof(float) * (size_t)n_expert);
    char* taken = (char*)malloc((size_t)n_expert);
    for (int t = 0; t < nb; t++) {
        const float* l = logits + (size_t)t * n_expert;
        float mx = l[0];
        for (int i = 1; i < n_expert; i++)
            if (l[i] > mx) mx = l[i];
        for (int i = 0; i < n_expert; i++) e[i] = expf(l[i] - mx);
        memset(taken, 0, (size_t)n_expert);
        for (int r = 0; r < k; r++) {
            int best = -1;
            for (int i = 0; i < n_expert; i++) {
                if (taken[i]) continue;
                if (best < 0 || e[i] > e[best]) best = i; /* ties keep the lower index */
            }
            taken[best] = 1;
            ids[(size_t)t * k + r] = best;
        }
        float tot = 0.f;
        for (int r = 0; r < k; r++) tot += e[ids[(size_t)t * k + r]];
        for (int r = 0; r < k; r++) wts[(size_t)t * k + r] = e[ids[(size_t)t * k + r]] / tot;
    }
    free(taken);
    free(e);
}

void orc_expf_array(const float* x, float* y, int64_t n) {
    for (int64_t i = 0; i < n; i++) y[i] = expf(x[i]);
}


/* qwen3moe.cpp:1024-1067 */
int orc_moe_layer(const orc_experts* ex, const float* xn, int nb, int k,
                  const int* ids, const float* wts, float* out) {
    const int D = ex->D, FF = ex->FF;
    float* xs = (float*)malloc(sizeof(float) * (size_t)nb * D);
    float* gb = (float*)malloc(sizeof(float) * (size_t)nb * FF);
    float* ub = (float*)malloc(sizeof(float) * (size_t)nb * FF);
    float* yb = (float*)malloc(sizeof(float) * (size_t)nb * D);
    int* tok = (int*)malloc(sizeof(int) * (size_t)nb);
    float* tw = (float*)malloc(sizeof(float) * (size_t)nb);
    int rc = 0;
    memset(out, 0, sizeof(float) * (size_t)nb * D);
    for (int e = 0; e < ex->n_expert && rc == 0; e++) {
        int m = 0;
        for (int t = 0; t < nb; t++)
            for (int r = 0; r < k; r++)
                if (ids[(size_t)t * k + r] == e) {
                    tok[m] = t;
                    tw[m] = wts[(size_t)t * k + r];
                    m++;
                }
        if (!m) continue;
        for (int i = 0; i < m; i++) memcpy(xs + (size_t)i * D, xn + (size_t)tok[i] * D, sizeof(float) * D);
        const orc_view* v = ex->views + (size_t)e * 3;
        rc |= orc_matmul(v[0].type, v[0].ne0, v[0].ne1, v[0].row_bytes, v[0].data, xs, m, D, gb, FF);
        rc |= orc_matmul(v[1].type, v[1].ne0, v[1].ne1, v[1].row_bytes, v[1].data, xs, m, D, ub, FF);
        for (int i = 0; i < m * FF; i++) gb[i] = silu_mul(gb[i], ub[i]);
        rc |= orc_matmul(v[2].type, v[2].ne0, v[2].ne1, v[2].row_bytes, v[2].data, gb, m, FF, yb, D);
        for (int i = 0; i < m; i++) {
            float* dst = out + (size_t)tok[i] * D;
            const float* src = yb + (size_t)i * D;
            const float w = tw[i];
            for (int d = 0; d < D; d++) dst[d] = fmaf(w, src[d], dst[d]);
        }
    }
    free(xs); free(gb); free(ub); free(yb); free(tok); free(tw);
    return rc;
}

/* ------------------------------------------------------------------------- */
/* Tiny-model forward (qwen3moe.cpp:932-1075), one token at a time: every
 * per-token quantity in the reference is independent of the batch size. */

struct orc_state {
    orc_model m;
    float *kc, *vc;
    float* inv_freq;
    int* trace_ids;
    float* trace_w;
    int trace_cap, trace_n;
    orc_moe_hook hook;  /* optional replacement of the expert block */
    void* hook_ctx;
};

void orc_state_set_moe_hook(orc_state* s, orc_moe_hook fn, void* ctx) {
    s->hook = fn;
    s->hook_ctx = ctx;
}

orc_state* orc_state_new(const orc_model* m) {
    orc_init();
    orc_state* s = (orc_state*)calloc(1, sizeof(orc_state));
    s->m = *m;
    const size_t kvn = (size_t)m->n_layer * m->n_ctx * m->n_kv * m->hd;
    s->kc = (float*)calloc(kvn, sizeof(float));
    s->vc = (float*)calloc(kvn, sizeof(float));
    s->inv_freq = (float*)malloc(sizeof(float) * (size_t)(m->hd / 2));
    for (int i = 0; i < m->hd / 2; i++) s->inv_freq[i] = (float)pow((double)m->rope_base, -2.0 * i / m->hd);
    return s;
}

void orc_state_free(orc_state* s) {
    if (!s) return;
    free(s->kc); free(s->vc); free(s->inv_freq); free(s->trace_ids); free(s->trace_w);
    free(s);
}

void orc_state_trace(orc_state* s, int* ids, float* wts, int cap, int* count) {
    if (ids && wts) {
        const int n = s->trace_n < cap ? s->trace_n : cap;
        memcpy(ids, s->trace_ids, sizeof(int) * (size_t)n);
        memcpy(wts, s->trace_w, sizeof(float) * (size_t)n);
    }
    if (count) *count = s->trace_n;
}

static void trace_push(orc_state* s, int id, float w) {
    if (s->trace_n == s->trace_cap) {
        s->trace_cap = s->trace_cap ? 2 * s->trace_cap : 1024;
        s->trace_ids = (int*)realloc(s->trace_ids, sizeof(int) * (size_t)s->trace_cap);
        s->trace_w = (float*)realloc(s->trace_w, sizeof(float) * (size_t)s->trace_cap);
    }
    s->trace_ids[s->trace_n] = id;
    s->trace_w[s->trace_n] = w;
    s->trace_n++;
}

static void mm_view(const orc_view* v, const float* x, int nb, int ldx, float* out, int ldo) {
    orc_matmul(v->type, v->ne0, v->ne1, v->row_bytes, v->data, x, nb, ldx, out, ldo);
}

static void rope_neox(float* p, int half, const float* c, const float* sn) {
    for (int i = 0; i < half; i++) {
        const float a = p[i], b = p[i + half];
        p[i] = a * c[i] - b * sn[i];
        p[i + half] = a * sn[i] + b * c[i];
    }
}

int orc_forward(orc_state* s, const int* toks, int nb, int p0, float* logits) {
    const orc_model* m = &s->m;
    const int D = m->D, hd = m->hd, half = hd / 2, QD = m->n_head * hd, KD = m->n_kv * hd;
    const int grp = m->n_head / m->n_kv, E = m->n_expert, K = m->n_used;
    const float scale = 1.0f / sqrtf((float)hd);
    if (nb < 1 || p0 + nb > m->n_ctx) return -1;
    float* x = (float*)malloc(sizeof(float) * (size_t)nb * D);
    float* xn = (float*)malloc(sizeof(float) * (size_t)nb * D);
    float* q = (float*)malloc(sizeof(float) * QD);
    float* kk = (float*)malloc(sizeof(float) * KD);
    float* vv = (float*)malloc(sizeof(float) * KD);
    float* att = (float*)malloc(sizeof(float) * QD);
    float* tmp = (float*)malloc(sizeof(float) * (size_t)nb * D);
    float* rl = (float*)malloc(sizeof(float) * (size_t)nb * E);
    float* sc = (float*)malloc(sizeof(float) * (size_t)m->n_ctx);
    float* rc = (float*)malloc(sizeof(float) * (size_t)nb * half);
    float* rs = (float*)malloc(sizeof(float) * (size_t)nb * half);
    int* ids = (int*)malloc(sizeof(int) * (size_t)nb * K);
    float* wts = (float*)malloc(sizeof(float) * (size_t)nb * K);
    orc_view* ev = (orc_view*)malloc(sizeof(orc_view) * (size_t)E * 3);
    const int blck = orc_blck(m->tok_embd.type), bb = orc_type_bytes(m->tok_embd.type);
    for (int t = 0; t < nb; t++) {
        const uint8_t* er = m->tok_embd.data + (size_t)toks[t] * m->tok_embd.row_bytes;
        for (int b = 0; b < D / blck; b++) orc_dequant_block(m->tok_embd.type, er + (size_t)b * bb, x + (size_t)t * D + b * blck);
        for (int i = 0; i < half; i++) {
            const double ang = (double)(p0 + t) * s->inv_freq[i];
            rc[t * half + i] = (float)cos(ang);
            rs[t * half + i] = (float)sin(ang);
        }
    }
    /* layer-major over the batch, as Engine::forward (the routing trace order
     * depends on it: per layer, tokens in batch order) */
    for (int l = 0; l < m->n_layer; l++) {
        float* lk = s->kc + (size_t)l * m->n_ctx * KD;
        float* lv = s->vc + (size_t)l * m->n_ctx * KD;
        for (int t = 0; t < nb; t++) {
            const int pos = p0 + t;
            float* xt = x + (size_t)t * D;
            float* xnt = xn + (size_t)t * D;
            orc_rmsnorm(xt, m->attn_norm[l], xnt, D, m->eps);
            mm_view(&m->wq[l], xnt, 1, D, q, QD);
            mm_view(&m->wk[l], xnt, 1, D, kk, KD);
            mm_view(&m->wv[l], xnt, 1, D, vv, KD);
            for (int h = 0; h < m->n_head; h++) {
                float* p = q + h * hd;
                orc_rmsnorm(p, m->q_norm[l], p, hd, m->eps);
                rope_neox(p, half, rc + t * half, rs + t * half);
            }
            for (int h = 0; h < m->n_kv; h++) {
                float* p = kk + h * hd;
                orc_rmsnorm(p, m->k_norm[l], p, hd, m->eps);
                rope_neox(p, half, rc + t * half, rs + t * half);
            }
            memcpy(lk + (size_t)pos * KD, kk, sizeof(float) * KD);
            memcpy(lv + (size_t)pos * KD, vv, sizeof(float) * KD);
            /* the reference writes every token's K/V before attending; a token
             * only attends to positions <= its own, so doing it per token is
             * the same computation */
            for (int h = 0; h < m->n_head; h++) {
                const int np = pos + 1, kvh = h / grp;
                const float* qh = q + h * hd;
                float mx = -INFINITY;
                for (int j = 0; j < np; j++) {
                    const float sj = dotf(qh, lk + (size_t)j * KD + kvh * hd, hd) * scale;
                    sc[j] = sj;
                    if (sj > mx) mx = sj;
                }
                float sum = 0.f;
                for (int j = 0; j < np; j++) {
                    sc[j] = expf(sc[j] - mx);
                    sum += sc[j];
                }
                const float inv = 1.0f / sum;
                float* o = att + h * hd;
                for (int d = 0; d < hd; d++) o[d] = 0.f;
                for (int j = 0; j < np; j++) {
                    const float w = sc[j] * inv;
                    const float* vj = lv + (size_t)j * KD + kvh * hd;
                    for (int d = 0; d < hd; d++) o[d] += w * vj[d];
                }
            }
            mm_view(&m->wo[l], att, 1, QD, tmp, D);
            for (int i = 0; i < D; i++) xt[i] += tmp[i];
        }
        for (int t = 0; t < nb; t++) orc_rmsnorm(x + (size_t)t * D, m->ffn_norm[l], xn + (size_t)t * D, D, m->eps);
        mm_view(&m->router[l], xn, nb, D, rl, E);
        orc_route_topk(rl, nb, E, K, ids, wts);
        for (int i = 0; i < nb * K; i++) trace_push(s, ids[i], wts[i]);
        for (int e = 0; e < E * 3; e++) ev[e] = m->experts[(size_t)l * E * 3 + e];
        orc_experts ex = {E, D, m->FF, ev};
        if (s->hook) {
            if (s->hook(s->hook_ctx, l, xn, nb, K, ids, wts, tmp) != 0) {
                free(x); free(xn); free(q); free(kk); free(vv); free(att); free(tmp); free(rl); free(sc);
                free(rc); free(rs); free(ids); free(wts); free(ev);
                return -2;
            }
        } else {
            orc_moe_layer(&ex, xn, nb, K, ids, wts, tmp);
        }
        for (int i = 0; i < nb * D; i++) x[i] += tmp[i];
    }
    if (logits) {
        orc_rmsnorm(x + (size_t)(nb - 1) * D, m->output_norm, xn, D, m->eps);
        mm_view(&m->output, xn, 1, D, logits, m->n_vocab);
    }
    free(x); free(xn); free(q); free(kk); free(vv); free(att); free(tmp); free(rl); free(sc);
    free(rc); free(rs); free(ids); free(wts); free(ev);
    return 0;
}
