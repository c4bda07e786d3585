/*
 * eahmmf_hip.h - C ABI of the MI355X (gfx950) expert-FFN library,
 * libeahmmf_hip.so.
 *
 * Plain pointers and sizes only.  "device" pointers are HIP device memory on
 * the current device (hipSetDevice / the caller's choice), "host" pointers are
 * ordinary pageable host memory.  Weight pointers address row 0 of one expert
 * component; rows are contiguous at stride row_bytes (the GGUF layout, bytes
 * never repacked).  Supported ggml types: 8 (Q8_0), 12 (Q4_K), 13 (Q5_K),
 * 14 (Q6_K).
 *
 * Error convention (same as the reference's CUDA C ABI): the bool entry points
 * return false on invalid arguments or any HIP error and never abort; queued
 * work is drained before returning, even after an error.  The int entry points
 * return 0 on success and a negative code otherwise.  eahmmf_hip_last_error()
 * describes the most recent failure on the calling thread.
 *
 * Threading: like the reference's ABI, one caller thread per device is
 * assumed; each device has one internal stream and one set of scratch and
 * pinned staging buffers that grow on demand and are kept until
 * eahmmf_hip_shutdown().  The *_async entry points run on the caller's
 * stream but use that same per-device scratch, so calls that may overlap in
 * time on one device (streams without an order between them) race: order
 * them on one stream.
 */
#ifndef EAHMMF_HIP_H
#define EAHMMF_HIP_H
#include <stdbool.h>
#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* ---- drop-in replacements for the reference's CUDA C ABI -------------- */

/* out[t*ldo + r] = sum_k W[r,k] * x[t*ldx + k], r < ne1, t < nb; host x/out,
 * synchronous.  Only r < ne1 of each output row is written.
 * Replaces eahmmf_cuda_matmul (expert_cuda.cu:251-261, declared
 * qwen3moe.cpp:422-423, called by gpu_matmul qwen3moe.cpp:471-474). */
bool eahmmf_hip_matmul(const uint8_t* device_weights, int type, int ne0, int ne1, size_t row_bytes,
                       const float* host_x, int nb, int ldx, float* host_out, int ldo);

/* Gate and up projections of one expert sharing one input transfer and one
 * synchronisation.  Requires equal (ne0, ne1).  Replaces
 * eahmmf_cuda_matmul_pair (expert_cuda.cu:344-348, declared qwen3moe.cpp:424,
 * called by gpu_matmul_pair qwen3moe.cpp:476-491). */
bool eahmmf_hip_matmul_pair(const uint8_t* gw, int gt, int gne0, int gne1, size_t grb,
                            const uint8_t* uw, int ut, int une0, int une1, size_t urb,
                            const float* host_x, int nb, int ldx,
                            float* host_g, int ldg, float* host_u, int ldu);

/* ---- fused MoE expert block (additions, same conventions) ------------- */

/* One expert component as the kernels see it: the device fields of the
 * reference's WeightView (eahmmf.h:54-62). */
typedef struct {
    const uint8_t* dev;
    int type;
    int ne0, ne1;
    size_t row_bytes;
} eahmmf_hip_weight;

/* One routed expert: its three leased components (ExpertViews, eahmmf.h:263-267). */
typedef struct {
    eahmmf_hip_weight gate, up, down;
} eahmmf_hip_expert;

/* Device-resident table entry, one per expert id of a layer. */
typedef struct {
    const uint8_t* gate;
    const uint8_t* up;
    const uint8_t* down;
} eahmmf_hip_expert_ptrs;

/* Shape of a layer's experts: gate/up are FF x D (ne0 = D), down is D x FF. */
typedef struct {
    int gate_type, up_type, down_type;
    int D, FF;
    size_t gate_row_bytes, up_row_bytes, down_row_bytes;
} eahmmf_hip_moe_shape;

/* Maximum routed experts per token in one fused call. */
#define EAHMMF_HIP_MAX_TOPK 16

/* Single-token expert block, synchronous, host x[D] -> host y[D]:
 *   y = sum_j w[j] * down_j( silu(gate_j x) * (up_j x) ).
 * All k experts must share one shape.  The caller holds the k leases across
 * the call.  Replaces the per-expert loop of qwen3moe.cpp:1024-1067 for one
 * token (gate/up pair, SiLU, down, weighted sum). */
bool eahmmf_hip_moe_decode(const eahmmf_hip_expert* experts, const float* w, int k,
                           const float* host_x, float* host_y);

/* The same under partial residency: a slot whose expert has no device copy
 * (a null gate/up/down dev pointer: the store served that lease from RAM or
 * the SSD mapping, eahmmf.h:721-742, e.g. when the VRAM budget is full of
 * pinned experts) is skipped, and bit j of *skipped_mask is set for skipped
 * slot j.  host_y[D] is then the weighted sum over the resident slots only
 * (all zeros if none is resident; D is taken from experts[0].gate.ne0), and
 * the caller adds the skipped experts' contributions on the CPU.  The
 * resident slots must share one shape, as for eahmmf_hip_moe_decode. */
bool eahmmf_hip_moe_decode_resident(const eahmmf_hip_expert* experts, const float* w, int k, const float* host_x,
                                    float* host_y, uint32_t* skipped_mask);

/* Same on device buffers, asynchronous on `stream` (a hipStream_t, 0 for the
 * null stream).  experts/w are read on the host during the call. */
int eahmmf_hip_moe_decode_async(const eahmmf_hip_moe_shape* shape, const eahmmf_hip_expert_ptrs* experts,
                                const float* w, int k, const float* dev_x, float* dev_y, void* stream);

/* Routed variant: routing results and the expert table live on the device
 * (dev_table [n_expert], dev_ids/dev_w [k]); no host round trip between
 * routing and the expert block. */
int eahmmf_hip_moe_decode_routed_async(const eahmmf_hip_moe_shape* shape, const eahmmf_hip_expert_ptrs* dev_table,
                                       int n_expert, const int* dev_ids, const float* dev_w, int k,
                                       const float* dev_x, float* dev_y, void* stream);

/* One launch for a whole layer-token: routing from device router logits
 * (dev_logits [n_expert], n_expert <= 256 for the fused kernel) and the
 * expert block over the device table.  The chosen ids and weights are also
 * written to dev_ids_out/dev_w_out [k] when those are non-null.  Replaces the
 * routing and expert loop of qwen3moe.cpp:1011-1067 for one token. */
int eahmmf_hip_moe_layer_decode_async(const eahmmf_hip_moe_shape* shape, const eahmmf_hip_expert_ptrs* dev_table,
                                      int n_expert, const float* dev_logits, int k, const float* dev_x, float* dev_y,
                                      int* dev_ids_out, float* dev_w_out, void* stream);

/* No counterpart in the reference.  For callers that cannot allocate device
 * memory (code under HIP graph capture, tight serving loops, harnesses that
 * forbid hipMalloc): eahmmf_hip_moe_layer_decode_async with the same
 * arguments and results, calling no hipMalloc/hipFree.  Its scratch (the
 * single-launch kernel's exchange and sync words, or the two-kernel path's h
 * and routing results) is one file-scope device array of about 1 MiB that
 * every GPU the library runs on holds until the process ends.  Limits:
 * k * FF <= 65536 and D <= 4096 (else -1 and a message).  All calls on one
 * GPU share the array, which keeps the last call's contents: calls that
 * overlap in time on one device race (order them on one stream).  The first
 * call on a device sets the array up (its address, one fill kernel and a
 * synchronisation of `stream`), so make it outside graph capture.  A launch
 * whose bounded wait gave up writes NaN to dev_y and is reported by
 * eahmmf_hip_device_flags(). */
int eahmmf_hip_moe_layer_decode_noalloc(const eahmmf_hip_moe_shape* shape, const eahmmf_hip_expert_ptrs* dev_table,
                                        int n_expert, const float* dev_logits, int k, const float* dev_x,
                                        float* dev_y, int* dev_ids_out, float* dev_w_out, void* stream);

/* Single-token MoE block from the layer's residual stream, on the device:
 * RMSNorm of dev_x [D] with dev_norm_w [D] (eps; dev_norm_w null: dev_x is
 * already normalized), the router matmul with dev_router (F32, n_expert rows
 * of D values), softmax/top-k routing and the expert block, as the
 * reference's nb = 1 step does (qwen3moe.cpp:1020-1067: rmsnorm, matmul
 * router, partial_sort, experts).  One launch on `stream` where the fused
 * kernel takes the shape (the norm in every workgroup, the router matmul
 * split over the workgroups and exchanged between them, then routing and
 * experts), else two (the router matmul, then the fused routed layer
 * kernel).  dev_xn_out / dev_logits_out
 * (optional, device) receive the normalized input and the router logits;
 * dev_ids_out / dev_w_out as in eahmmf_hip_moe_layer_decode_async.  The
 * logits sum in a different order than the reference's sequential loop, so
 * two experts whose logits differ by a few ulps may rank the other way round
 * (the ids then differ from the reference's; the output stays within
 * tolerance of the reference's for the ids it reports).  No single
 * counterpart in the reference (its router runs on the CPU); 0, or -1/-2/-3
 * as the other async entry points. */
int eahmmf_hip_moe_layer_decode_xn_async(const eahmmf_hip_moe_shape* shape, const eahmmf_hip_expert_ptrs* dev_table,
                                         int n_expert, const float* dev_router, const float* dev_norm_w, float eps,
                                         const float* dev_x, int k, float* dev_y, int* dev_ids_out, float* dev_w_out,
                                         float* dev_xn_out, float* dev_logits_out, void* stream);

/* Ragged grouped expert block for a batch of nb tokens (prefill, batched
 * decode), in the reference's by_exp form: group g (ascending expert id) is
 * experts[g] applied to tokens[group_offsets[g] .. group_offsets[g+1]) with
 * router weights weights[same range]; host x[nb][D] -> host y[nb][D],
 *   y[t] = sum over the groups holding t, ascending, of w * down(silu(gate x_t) * up x_t).
 * A token may appear in at most EAHMMF_HIP_MAX_TOPK groups; all groups share
 * one shape.  Synchronous.  Replaces the per-expert loop of
 * qwen3moe.cpp:1024-1067 for a batch (gather, batched matmuls, SiLU,
 * weighted scatter-add). */
bool eahmmf_hip_moe_grouped(const eahmmf_hip_expert* experts, int n_groups, const int* group_offsets,
                            const int* tokens, const float* weights, int nb, const float* host_x, float* host_y);

/* Same with the routing on the device: dev_ids/dev_w [nb][k] (e.g. from
 * eahmmf_hip_route_topk_async; ids outside 0..n_expert-1 are skipped) over
 * the device table [n_expert <= 256]; dev_x/dev_y [nb][D], asynchronous on
 * `stream`.  Above 32 tokens the (token, expert) pairs are grouped on the
 * device (stable, in token order) and each token's results are added in
 * ascending expert id, as qwen3moe.cpp:1009-1067 does.  A batch of up to 32
 * tokens (a decode step of a few sequences) where the single-launch kernel
 * covers the shape runs as one such launch per token instead, its results
 * added in the routing's rank order (the same output tolerance). */
int eahmmf_hip_moe_grouped_async(const eahmmf_hip_moe_shape* shape, const eahmmf_hip_expert_ptrs* dev_table,
                                 int n_expert, const int* dev_ids, const float* dev_w, int nb, int k,
                                 const float* dev_x, float* dev_y, void* stream);

/* Softmax -> top-k -> renormalise (qwen3moe.cpp:1011-1023), synchronous on
 * host buffers: logits[nb][n_expert] -> ids[nb][k], w[nb][k] in rank order
 * (e = expf(l - max) descending, lower id first on ties). */
bool eahmmf_hip_route_topk(const float* host_logits, int nb, int n_expert, int k, int* host_ids, float* host_w);
int eahmmf_hip_route_topk_async(const float* dev_logits, int nb, int n_expert, int k, int* dev_ids, float* dev_w,
                                void* stream);

/* The routing's exponential on the device: dev_y[i] = expf(dev_x[i]) with
 * the bits glibc's expf gives (the method of expf_ref.h), so routing keys
 * e = expf(l - max) and their ties match the reference host's
 * (qwen3moe.cpp:1013-1016).  No counterpart in the reference; for callers
 * that form routing keys in their own kernels.  Asynchronous on stream; 0 on
 * success, -1 on bad arguments, -3 on a launch error. */
int eahmmf_hip_expf_ref_async(const float* dev_x, float* dev_y, int64_t n, void* stream);

/* ---- measurement ------------------------------------------------------ */

/* Streaming read of bytes from dev_buf (16-byte aligned, bytes a multiple of
 * 16).  dev_sink holds EAHMMF_HIP_STREAM_SINK_WORDS words; afterwards their
 * XOR is the XOR of every 32-bit word read.  No counterpart in the reference:
 * it measures the achievable HBM read rate that the decode kernels are
 * compared with (nontemporal 16-byte loads, eight per thread in flight, at
 * most 4096 workgroups of 512 threads, no atomics).  Asynchronous on stream;
 * 0 on success (also for 0 bytes, which writes nothing), -1 on bad arguments,
 * -3 on a launch error. */
#define EAHMMF_HIP_STREAM_SINK_WORDS 4096
int eahmmf_hip_stream_read_async(const void* dev_buf, size_t bytes, uint32_t* dev_sink, void* stream);

/* ---- format utilities ------------------------------------------------- */

/* Dequantize nrows rows of ne0 values into dev_out[r*ne0 + k], bit-identical
 * to the reference CPU decoder (qwen3moe.cpp:128-202). */
int eahmmf_hip_dequantize(const uint8_t* dev_w, int type, int64_t ne0, int64_t nrows, size_t row_bytes,
                          float* dev_out, void* stream);

/* Row bytes of a row of ne0 values, 0 if the type/length is unsupported. */
size_t eahmmf_hip_row_bytes(int type, int64_t ne0);

/* Host-side quantizer (synthetic weights): src[nrows][ne0] fp32 -> dst rows of
 * eahmmf_hip_row_bytes(type, ne0) bytes.  Returns bytes written or -1. */
int64_t eahmmf_hip_quantize_rows(int type, const float* src, int64_t nrows, int64_t ne0, uint8_t* dst);

/* ---- device memory for DeviceBackend implementations ----------------- */

/* Thin wrappers used by the C++ HipDevice (hipMalloc/hipFree/async copies on
 * the library stream/hipMemGetInfo).  Return 0 on success. */
int eahmmf_hip_alloc(void** dev_ptr, size_t bytes);
int eahmmf_hip_free(void* dev_ptr);
int eahmmf_hip_h2d(void* dev_dst, const void* host_src, size_t n);
int eahmmf_hip_d2h(void* host_dst, const void* dev_src, size_t n);
int eahmmf_hip_sync(void);
int eahmmf_hip_mem_info(size_t* free_bytes, size_t* total_bytes);

/* One host-to-device copy of a batch. */
typedef struct {
    void* dev_dst;
    const void* host_src; /* pageable host memory */
    size_t bytes;
} eahmmf_hip_copy;

/* Bulk staging: performs n host-to-device copies through a ring of four
 * 32 MiB pinned buffers, so that CPU threads fill one buffer while the DMA
 * engine drains the others (EAHMMF_HIP_STAGE_THREADS threads, default half
 * the host's hardware threads, at most 16).  Small copies share a buffer.
 * Work already queued on the library stream finishes first; the call returns
 * when every byte is on the device (copies are then valid for compute, as
 * after h2d() + sync()).  The reference moves an expert with three h2d()
 * calls and a sync() (ExpertPager::stage_to_vram, eahmmf.h:959-1031, the
 * copies at :1009-1013) and lists asynchronous prefetch as not implemented
 * (README.md:379); this is the batch form its store can use to make many
 * experts resident at once.  Single-threaded caller per device.  0 on
 * success, -1 on bad arguments, -2 on a HIP error. */
int eahmmf_hip_h2d_batch(const eahmmf_hip_copy* copies, int n);
/* Asynchronous bulk staging (no counterpart in the reference, whose README.md:379
 * lists asynchronous prefetch as not implemented): queues the same copies to
 * a per-device worker thread and returns at once with a ticket (> 0) in
 * *ticket.  The worker stages batches in order through the ring above while
 * the caller goes on (e.g. computing a layer while the next layer's experts
 * are made resident).  The host sources must stay valid and unchanged, and
 * the destinations unused, until the batch has landed.  Unlike the
 * synchronous form it does not wait for work queued on the library stream.
 * 0 on success, -1 on bad arguments, -2 on a HIP error. */
int eahmmf_hip_h2d_batch_async(const eahmmf_hip_copy* copies, int n, uint64_t* ticket);
/* Waits for batch `ticket`.  With a stream, the host waits only until the
 * batch's copies are all queued, and the stream waits (on the device) until
 * they have landed, so work queued on it afterwards sees the bytes; with a
 * null stream the host waits until they have landed.  0 on success, -1 for a
 * ticket never handed out, -2 when the batch failed (eahmmf_hip_last_error()
 * names the cause). */
int eahmmf_hip_h2d_batch_wait(uint64_t ticket, void* stream);
/* 1 when batch `ticket` has landed, 0 while it is pending, -1 for a ticket
 * never handed out, -2 when it failed. */
int eahmmf_hip_h2d_batch_query(uint64_t ticket);

/* ---- diagnostics / lifetime ------------------------------------------- */
/* Selects the single-launch fused expert block (1, the default) or the
 * routing + two-kernel path (0); a negative argument only queries.  Returns
 * the previous setting.  EAHMMF_HIP_UNFUSED=1 selects 0 at start-up (like the
 * reference's EAHMMF_OLD_KERNEL switch, expert_cuda.cu:307-308). */
int eahmmf_hip_set_fused(int enable);
/* How the fused kernel's partitions exchange their gate/up results on the
 * current device: 1 through each XCD's own L2 (eight XCDs that each receive
 * an equal share of a launch, checked once per device; workgroups then rank
 * themselves per XCD with an atomic ticket), 0 through device-coherent
 * memory, -1 on error. */
int eahmmf_hip_fused_exchange(void);
/* Selects matrix-core (MFMA) matmuls in the grouped block where the formats
 * allow (1, the default: Q4_K/Q5_K gate/up, Q6_K down) or the vector-ALU
 * kernels only (0); a negative argument only queries.  Returns the previous
 * setting. */
int eahmmf_hip_set_grouped_mfma(int enable);
/* Largest expert group, in tokens, that the grouped block's matrix-core
 * matmuls run on the per-wave kernels (each wave its own 16 rows, one or two
 * 16-token tiles); larger groups use the workgroup kernels.  0 disables the
 * per-wave kernels, at most 32 (default 32); a negative argument only
 * queries.  Returns the previous value.  No counterpart in the reference. */
int eahmmf_hip_set_grouped_wave_max(int max_tokens);
/* The grouped block's integer-dot kernels (each weight row streamed once and
 * dotted in int32 against int8 levels of each of the group's tokens): 0
 * turns them off; any positive value turns them on for blocks of at most 32
 * tokens, which then run on them whole; 1..32 also sends the groups of at
 * most that many tokens of larger blocks to them (above 32, the default,
 * reported as 33: none).  A negative argument only queries.  Returns the
 * previous setting.  No counterpart in the reference. */
int eahmmf_hip_set_grouped_dot_max(int max_tokens);
/* Matrix-core path of the batched matmuls (the drop-in eahmmf_hip_matmul /
 * _pair at 2..64 tokens and the model's projections and output head at
 * batch 2..64) for Q4_K, Q5_K, Q6_K and Q8_0 rows of a multiple of 256
 * values: 1 on (default), 0 the general kernel.  Returns the previous
 * setting.  No counterpart in the reference (a switch for A/B checks). */
int eahmmf_hip_set_dense_mfma(int on);
/* The single-launch expert block's workgroups wait for each other's words
 * (h, per-partition partials).  Every wait is bounded; when one gives up the
 * launch writes NaN where the missing words were needed and records its
 * epoch in a per-device error word, and the kernel still exits.  The
 * synchronous entry points read that word with their output and then return
 * false (as on any HIP error, expert_cuda.cu:332-335, so the caller falls back
 * to the CPU, qwen3moe.cpp:515-521).  For the *_async entry points:
 *
 * eahmmf_hip_device_flags: 1 if a fused launch on the current device gave up
 * a wait since the last call (its output is then not valid), else 0; -2 on a
 * HIP error.  Synchronises the device and clears the word. */
int eahmmf_hip_device_flags(void);
/* Cheap check for *_async callers: enqueues on `stream` a copy of the error
 * word (0: no launch gave up a wait since the word was last cleared) into
 * dst, device or pinned host memory, valid once the stream reaches it.  Does
 * not clear the word (eahmmf_hip_device_flags does).  0 on success, -1 on a
 * null dst, -3 on a HIP error. */
int eahmmf_hip_fused_status_async(unsigned* dst, void* stream);
/* Test knob, no counterpart in the reference: the number of polls after which
 * a fused-kernel wait gives up (0: the default, 2^18), and one partition
 * (0-7) whose h words are never stored (-1: none), so that tests can make the
 * kernel's own bounded waits give up while every kernel still exits
 * normally.  Not for production use. */
void eahmmf_hip_set_fault_injection(unsigned spin_limit, int drop_partition);
/* ---------------------------------------------------------------------------
 * Whole-model decode on the device.  The reference's Engine
 * (qwen3moe.cpp:859-1084) runs embedding, attention, norms, RoPE, the KV
 * cache, the router and the output head on the CPU and sends expert matmuls
 * to the GPU; this engine keeps the entire forward on one device: token
 * embedding, RMSNorm, the Q/K/V/output projections and the router and output
 * head (the quantized matmul kernel, any supported type incl. F32), per-head
 * Q/K RMSNorm with NeoX RoPE, an fp32 KV cache [n_layer][n_ctx][n_kv * hd],
 * causal attention, and the expert block (the fused routed layer kernel for
 * one token, routing + grouped kernels for a batch).  No counterpart entry
 * point exists in the reference; the arguments mirror Engine::load /
 * forward / eval and the routing trace (qwen3moe.cpp:862-922, 932-1084). */
typedef struct {
    const void* data;  /* the tensor's bytes: rows of row_bytes */
    int on_device;     /* 0: host memory, copied at create; 1: device memory, borrowed */
    int type;          /* 0 F32, 8 Q8_0, 12 Q4_K, 13 Q5_K, 14 Q6_K */
    int64_t ne0, ne1;  /* values per row, rows (stacked expert tensors: n_expert * rows) */
    size_t row_bytes;
} eahmmf_hip_tensor;

/* One layer's tensors (GGUF names blk.N.*, qwen3moe.cpp:883-905).  The
 * norm weights are F32 vectors (ne1 = 1); gate/up/down_exps hold the
 * n_expert experts back to back (expert e's gate at e * FF * row_bytes). */
typedef struct {
    eahmmf_hip_tensor attn_norm, ffn_norm, q_norm, k_norm;
    eahmmf_hip_tensor wq, wk, wv, wo, router;
    eahmmf_hip_tensor gate_exps, up_exps, down_exps;
} eahmmf_hip_layer_desc;

typedef struct {
    int n_layer, D, n_head, n_kv, hd, n_expert, n_used, FF, n_vocab, n_ctx;
    float eps, rope_base;
    eahmmf_hip_tensor tok_embd, output_norm, output; /* output.data null: tied to tok_embd */
    const eahmmf_hip_layer_desc* layers;             /* n_layer entries */
} eahmmf_hip_model_desc;

/* Builds a model on the current device: copies host tensors, builds the
 * expert tables, the RoPE table (cos/sin of pos * inv_freq as the reference
 * computes them, in double) and a zeroed KV cache.  NULL on failure
 * (eahmmf_hip_last_error says why): unsupported shape or type, out of memory. */
void* eahmmf_hip_model_create(const eahmmf_hip_model_desc* desc);
/* Engine::forward: nb (1..64) host tokens at positions p0 .. p0+nb-1; if
 * logits is non-null, the host receives the last token's n_vocab logits.
 * Synchronous.  0 on success; -1 bad arguments (batch size, context overflow,
 * token id out of range); -3 a HIP error or a fused expert launch that gave
 * up a wait (outputs invalid). */
int eahmmf_hip_model_forward(void* model, const int* toks, int nb, int p0, float* logits);
/* Engine::eval: n tokens from p0 in chunks of n_batch (1..64); logits of the last. */
int eahmmf_hip_model_eval(void* model, const int* toks, int n, int p0, int n_batch, float* logits);
/* Greedy decoding without host round trips: feeds `first` at position p0,
 * then n - 1 times the argmax (first largest) of the last logits; out_toks
 * receives the n argmax tokens; last_logits (may be null) the final logits.
 * One synchronisation at the end.  Same return codes as forward. */
int eahmmf_hip_model_generate_greedy(void* model, int first, int p0, int n, int* out_toks, float* last_logits);
/* Sequences (the reference's Engine keeps one: a single KV cache
 * [n_layer][n_ctx][KD] written at p0 + t, qwen3moe.cpp:791, 910-913, 969-971).
 * Sets the model to n_seq (1..64) independent sequences, each with its own KV
 * rows [n_layer][n_seq][n_ctx][KD]; every cache row is cleared (all sequences
 * start empty).  Sequence 0 is the one forward / eval / generate_greedy use.
 * Synchronous; 0, -1 bad count, -3 out of device memory (the model is then
 * unchanged). */
int eahmmf_hip_model_set_sequences(void* model, int n_seq);
/* Engine::forward (qwen3moe.cpp:910-913) on sequence seq: nb tokens at
 * positions p0 .. p0+nb-1 of that sequence; same arguments and return codes
 * as eahmmf_hip_model_forward, plus -1 for seq outside 0..n_seq-1. */
int eahmmf_hip_model_forward_seq(void* model, int seq, const int* toks, int nb, int p0, float* logits);
/* One decode step of n (1..n_seq) different sequences, batched: token toks[i]
 * at position pos[i] of sequence seqs[i]; each token attends to its own
 * sequence's rows 0..pos[i] and its row is written there.  Equals n calls of
 * Engine::forward(&toks[i], 1, pos[i], ...) each on its own sequence's
 * engine, in one pass whose matmuls and expert block see all n tokens.
 * logits (may be null): [n][n_vocab], row i for toks[i].  -1 for a sequence
 * given twice, outside 0..n_seq-1, pos outside 0..n_ctx-1 or a bad token;
 * otherwise as eahmmf_hip_model_forward. */
int eahmmf_hip_model_decode_seqs(void* model, int n, const int* toks, const int* seqs, const int* pos,
                                 float* logits);
/* Routing trace (Engine::trace_routing): when on, every forward appends, per
 * layer and token, the n_used expert ids and weights in routing order. */
int eahmmf_hip_model_set_trace(void* model, int on);
/* Copies up to cap trace entries; returns the number recorded. */
int eahmmf_hip_model_trace(void* model, int* ids, float* w, int cap);
void eahmmf_hip_model_trace_clear(void* model);
/* The model's stream (a hipStream_t), for callers that time or order work around it. */
void* eahmmf_hip_model_stream(void* model);
void eahmmf_hip_model_free(void* model);

const char* eahmmf_hip_last_error(void);
int eahmmf_hip_device_count(void);
/* Frees the calling device's scratch, staging buffers and stream. */
void eahmmf_hip_shutdown(void);

#ifdef __cplusplus
}
#endif
#endif
