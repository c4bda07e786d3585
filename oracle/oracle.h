/*
 * oracle.h - CPU restatement of the reference's quantized expert-FFN path.
 *
 * TEST INFRASTRUCTURE ONLY.  This library is the parity checker for the HIP
 * path: only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg
 * may load it.  Nothing in the shipped library links it or falls back to it.
 *
 * Every function follows a named region of the reference (jonny14-bro/
 * EAHMMF_inference_prototype_V-0.1.0) and is written in plain C:
 *   fp16 decode            qwen3moe.cpp:54-67
 *   block formats          qwen3moe.cpp:128-218 (Q8_0, Q4_K, Q5_K, Q6_K, F32)
 *   dotf / matmul          qwen3moe.cpp:376-381, 397-419
 *   rmsnorm                qwen3moe.cpp:527-532
 *   routing / MoE block    qwen3moe.cpp:1006-1069
 *   forward (tiny model)   qwen3moe.cpp:932-1075
 *
 * Pinning (how each function is checked, see tests/test_oracle_*.py):
 *   orc_f16            exhaustive over all 65536 codes vs a closed form
 *   orc_scale_min_k4   exhaustive over all byte pairs vs a closed form
 *   orc_dequant_*      bit-exact vs the compiled reference's dq_* (golden
 *                      fixtures), plus brute-force identities (e.g. Q4_K with
 *                      sc=1,m=0 reproduces d*q exactly)
 *   orc_matmul         fp64 brute force on dequantized rows, and the compiled
 *                      reference's matmul (golden fixtures)
 *   orc_route_topk     brute force sort, and the compiled reference's routing
 *                      trace on the tiny model (ids exact, weights exact)
 *   orc_moe_layer      closed-form fp64 restatement + tiny-model logits
 *   orc_forward        the reference's own baseline/logits.txt (2e-6)
 */
#ifndef EAHMMF_ORACLE_H
#define EAHMMF_ORACLE_H
#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

enum { ORC_F32 = 0, ORC_Q8_0 = 8, ORC_Q4_K = 12, ORC_Q5_K = 13, ORC_Q6_K = 14 };

void orc_init(void);
float orc_f16(uint16_t h);
void orc_scale_min_k4(int j, const uint8_t* q, uint8_t* d, uint8_t* m);
int orc_blck(int type);        /* values per block, 0 if unsupported */
int orc_type_bytes(int type);  /* bytes per block, 0 if unsupported */
int orc_dequant_block(int type, const uint8_t* b, float* y);
/* rows of a component: out[r*ne0 + k] */
int orc_dequant_rows(int type, const uint8_t* w, int64_t ne0, int64_t nrows, size_t row_bytes, float* out);
/* out[t*ldo + r] = sum_k W[r,k] * x[t*ldx + k], block-wise fp32 like the reference */
int orc_matmul(int type, int64_t ne0, int64_t ne1, size_t row_bytes, const uint8_t* w,
               const float* x, int nb, int ldx, float* out, int ldo);
int orc_time_expert_tokens(int gt, int dt, int D, int FF, size_t grb, size_t drb, const uint8_t* gate,
                           const uint8_t* up, const uint8_t* down, const float* xs, const int* ids, const float* w,
                           int k, int n_tok, int threads, int warmup, int reps, double* secs);
void orc_rmsnorm(const float* x, const float* w, float* out, int n, float eps);

/* softmax -> top-k (e desc, index asc) -> renorm in rank order.
 * logits[nb][n_expert] (not modified); ids/wts [nb][k] in rank order. */
void orc_route_topk(const float* logits, int nb, int n_expert, int k, int* ids, float* wts);
/* y[i] = expf(x[i]) with the host libm's expf, the function the routing
 * keys use (qwen3moe.cpp:1013). */
void orc_expf_array(const float* x, float* y, int64_t n);

/* One quantized component view (a WeightView without the device pointer). */
typedef struct {
    const uint8_t* data;
    int type;
    int64_t ne0, ne1;
    size_t row_bytes;
} orc_view;

/* One MoE layer's experts: views[e*3 + c], c = 0 gate, 1 up, 2 down. */
typedef struct {
    int n_expert, D, FF;
    const orc_view* views;
} orc_experts;

/* MoE expert block (qwen3moe.cpp:1024-1067): given normalized activations
 * xn[nb][D] and the routing (ids, wts)[nb][k], writes out[nb][D] =
 * sum over the token's experts of w * down(silu(gate x) * up x), experts
 * visited in ascending id, tokens of one expert batched together. */
int orc_moe_layer(const orc_experts* ex, const float* xn, int nb, int k,
                  const int* ids, const float* wts, float* out);

/* Qwen3-MoE model for the end-to-end tiny-model check. */
typedef struct {
    int n_layer, D, n_head, n_kv, hd, n_expert, n_used, FF, n_vocab, n_ctx;
    float eps, rope_base;
    orc_view tok_embd, output;
    const float* output_norm;
    /* per layer arrays [n_layer] */
    const float* const* attn_norm;
    const float* const* ffn_norm;
    const float* const* q_norm;
    const float* const* k_norm;
    const orc_view* wq;
    const orc_view* wk;
    const orc_view* wv;
    const orc_view* wo;
    const orc_view* router;     /* F32 [n_expert][D] */
    const orc_view* experts;    /* [n_layer][n_expert][3] */
} orc_model;

typedef struct orc_state orc_state;
orc_state* orc_state_new(const orc_model* m);
/* Optional replacement of the expert block inside orc_forward, so that another
 * implementation of qwen3moe.cpp:1024-1067 can be checked end to end against
 * the reference's logits: called per layer with the normalised activations
 * xn[nb][D], the routing ids/wts[nb][k] and out[nb][D]; nonzero aborts the
 * forward (orc_forward then returns -2). */
typedef int (*orc_moe_hook)(void* ctx, int layer, const float* xn, int nb, int k, const int* ids,
                            const float* wts, float* out);
void orc_state_set_moe_hook(orc_state* s, orc_moe_hook fn, void* ctx);
void orc_state_free(orc_state* s);
/* Optional routing trace: every (id, w) chosen, in token/rank order. */
void orc_state_trace(orc_state* s, int* ids, float* wts, int cap, int* count);
/* Evaluate nb tokens at positions p0..; writes the last token's logits when
 * logits != NULL.  Mirrors Engine::forward (qwen3moe.cpp:932-1075). */
int orc_forward(orc_state* s, const int* toks, int nb, int p0, float* logits);

#ifdef __cplusplus
}
#endif
#endif
