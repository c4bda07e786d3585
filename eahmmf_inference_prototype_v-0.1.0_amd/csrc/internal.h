// internal.h - launchers shared between the kernel files and the C ABI.
#pragma once
#include <hip/hip_runtime.h>
#include <stddef.h>
#include <stdint.h>

namespace eahmmf {

constexpr int kMaxSlots = 16;  // routed experts per token handled by one fused launch

// Shape of one MoE layer's expert components (all experts of a layer share it).
struct MoeShape {
    int gate_type, up_type, down_type;
    int D, FF;
    size_t gate_rb, up_rb, down_rb;  // row bytes
};

// The k routed experts of one token, by value in the kernel arguments.
struct DecodeSlots {
    const uint8_t* gate[kMaxSlots];
    const uint8_t* up[kMaxSlots];
    const uint8_t* down[kMaxSlots];
    float w[kMaxSlots];
    int k;
};

// Device-resident per-layer table, one entry per expert id (for routed launches).
struct ExpertEntry {
    const uint8_t* gate;
    const uint8_t* up;
    const uint8_t* down;
};

// hipGetLastError() reports the last failure of any runtime call on this
// thread, including ones made by other libraries in the process; launchers
// clear it first so a launch is judged by its own status only.
inline void clear_stale_error() { (void)hipGetLastError(); }

hipError_t launch_dequant(int type, const uint8_t* w, int64_t ne0, int64_t nrows, size_t row_bytes, float* out,
                          hipStream_t st);
hipError_t launch_matmul(int type, const uint8_t* w, int ne0, int ne1, size_t row_bytes, const float* x, int nb,
                         int ldx, float* out, int ldo, hipStream_t st);
// The same product on the matrix cores for 2..kMaxMfmaMatmulTokens tokens of
// Q4_K / Q5_K / Q6_K / Q8_0 rows with ne0 % 256 == 0 (kernels_dense_mfma.hip);
// ws: device workspace of matmul_mfma_ws_bytes(ne0, ne1, nb) bytes, 256-byte
// aligned.  launch_matmul_auto takes that path when matmul_mfma_ok, the
// switch is on and ws is large enough, else launch_matmul.
constexpr int kMaxMfmaMatmulTokens = 64;
bool matmul_mfma_ok(int type, const uint8_t* w, int ne0, size_t row_bytes, const float* x, int nb, int ldx);
size_t matmul_mfma_ws_bytes(int ne0, int ne1, int nb);
hipError_t launch_matmul_mfma(int type, const uint8_t* w, int ne0, int ne1, size_t row_bytes, const float* x, int nb,
                              int ldx, float* out, int ldo, void* ws, size_t ws_bytes, hipStream_t st);
hipError_t launch_matmul_auto(int type, const uint8_t* w, int ne0, int ne1, size_t row_bytes, const float* x, int nb,
                              int ldx, float* out, int ldo, void* ws, size_t ws_bytes, hipStream_t st);
bool dense_mfma_enabled();
int set_dense_mfma(int on);  // returns the previous setting

// Fused single-token decode: h[k][FF] scratch, y[D] = sum_j w_j down_j(silu(gate_j x) * up_j x).
hipError_t launch_moe_decode(const MoeShape& s, const DecodeSlots& slots, const float* x, float* h, float* y,
                             hipStream_t st);
// Same with the routing taken from device memory: ids/w [k], table [n_expert].
hipError_t launch_moe_decode_routed(const MoeShape& s, const ExpertEntry* table, int n_expert, const int* ids,
                                    const float* w, int k, const float* x, float* h, float* y, hipStream_t st);

// Host description of one fused expert-block launch (kernels_fused.hip).
struct FusedArgsHost {
    MoeShape shape;
    int k = 0, n_expert = 0;
    int mode = 0;  // 0: direct slots, 1: logits + table (routing in the kernel), 2: ids/w + table,
                   // 3: residual stream + router + table (norm, router matmul and routing in the kernel;
                   // hipErrorNotSupported when the launch has fewer workgroups than experts)
    DecodeSlots direct{};
    const ExpertEntry* table = nullptr;
    const float* logits = nullptr;
    const int* ids_in = nullptr;
    const float* w_in = nullptr;
    int* ids_out = nullptr;
    float* w_out = nullptr;
    const float* x = nullptr;
    float* y = nullptr;
    // mode 3: F32 router rows [n_expert][D], the input's RMSNorm weights (null:
    // none) and eps, optional outputs (normalized input, logits)
    const float* router = nullptr;
    const float* norm_w = nullptr;
    float eps = 0.f;
    float* xn_out = nullptr;
    float* logits_out = nullptr;
};

// Sync buffer of a fused scratch set: kSyncWords words, zero before the first
// launch.  Word kSyncFlagWord is the error word (the epoch of the last launch
// whose bounded wait gave up, 0 if none); the eight per-XCD ticket counters
// sit kTicketStride words apart (one 128-byte line each) from kTicketWord.
constexpr int kSyncWords = 4096;
constexpr int kSyncFlagWord = 1020;
constexpr int kTicketWord = 1024;
constexpr int kTicketStride = 32;

// One set of the fused kernel's scratch and its launch bookkeeping.  The
// exchange words (h and the per-partition partials) carry the epoch of the
// launch that wrote them, so they are zeroed once, when allocated, and never
// again; every launch on the set gets a new epoch.
struct FusedState {
    uint64_t* hx = nullptr;     // hx_words words: h value bits | epoch << 32
    size_t hx_words = 0;
    uint64_t* ypart = nullptr;  // ypart_words words: 8 partitions x D partials, same form
    size_t ypart_words = 0;
    unsigned* sync = nullptr;   // kSyncWords words
    unsigned epoch = 0;         // epoch of the last launch (0: none yet; launches skip 0 when it wraps)
    unsigned ticket_base = 0;   // tickets each XCD counter handed out so far
};

bool fused_supported(const MoeShape& s, int k, int n_expert_for_routing);
// 1 if the fused kernel's partitions exchange h through their own XCD's L2 on
// this device (eight XCDs, a launch spread evenly over them), 0 if it uses the
// device-coherent protocol.
int fused_exchange_mode(int device);
// The same, running the one-time placement probe (first call per device) with
// probe_buf (4 KiB of device memory) instead of a buffer of its own.
int fused_exchange_probe(int device, int* probe_buf);
// Enqueues one fused launch on st with the next epoch of `fs`; its scratch
// must hold k * FF h words and 8 * D partials.
hipError_t launch_moe_fused(const FusedArgsHost& h, FusedState& fs, hipStream_t st);
// Enqueues the reset of fs's ticket counters, and of its error word when
// clear_error (a fill kernel, no memset node), and restarts the host's ticket
// count; after a launch whose wait gave up.
hipError_t reset_fused_sync(FusedState& fs, hipStream_t st, bool clear_error);
// Test knobs of the fused kernel (0 / -1 restore the defaults): the polls
// before a wait gives up, and one partition whose h words are never stored,
// so that the kernel's own bounded waits give up.
void set_fused_fault_injection(unsigned spin_limit, int drop_partition);

// Ragged grouped expert block (kernels_grouped.hip): nb tokens routed by
// ids/w [nb][k] over table [n_expert]; x [nb][ldx] -> y [nb][ldy].  scratch
// holds grouped_scratch_bytes() bytes of device memory.
bool grouped_supported(const MoeShape& s, int nb, int k, int n_expert);
size_t grouped_scratch_bytes(const MoeShape& s, int nb, int k, int n_expert);
hipError_t launch_moe_grouped(const MoeShape& s, const ExpertEntry* table, int n_expert, const int* ids,
                              const float* w, int nb, int k, const float* x, int ldx, float* y, int ldy,
                              void* scratch, hipStream_t st);

// Matrix-core matmuls of the grouped block (kernels_grouped_mfma.hip).
bool grouped_mfma_gate_up_ok(const MoeShape& s);
bool grouped_mfma_down_ok(const MoeShape& s);
hipError_t launch_prep_rows(const int* offs, int E, const int* tok, const float* src, int ld, int n, int P,
                            _Float16* vh, _Float16* vl, _Float16* sh, _Float16* sl, float* vscale, hipStream_t st);
// (experts holding fewer than tmin tokens are left to the per-wave kernels)
// The matrix-core launches' work lists, written by the grouping kernel:
// item i < *n is {e, first pair of the pass, end of the expert's pairs, start
// of the expert's pairs} (the per-wave kernels: one pass per expert); cap
// item slots (the launches' grid).
struct TileItems {
    const int4* items;
    const int* n;
    int cap;
};
constexpr int kMfmaGuTok = 128;  // tokens of a gate/up workgroup pass
constexpr int kMfmaDnTok = 64;   // tokens of a down workgroup pass
// Item slots of a pass list: passes of tile tokens over the experts holding
// at least wmin of P pairs.
inline int tile_cap(size_t P, int E, int wmin, int tile) {
    const size_t ge = P / (size_t)(wmin > 0 ? wmin : 1);
    return (int)(P / tile + (ge < (size_t)E ? ge : (size_t)E) + 1);
}
hipError_t launch_gate_up_mfma(const MoeShape& s, const ExpertEntry* table, TileItems gi,
                               const _Float16* xh, const _Float16* xl, const _Float16* xsh, const _Float16* xsl,
                               const float* xscale, float* h, int tmin, hipStream_t st);
hipError_t launch_down_mfma(const MoeShape& s, const ExpertEntry* table, TileItems gi,
                            const _Float16* hh, const _Float16* hl, const float* hscale, float* yp, int tmin,
                            hipStream_t st);
// Per-wave matrix-core matmuls for experts holding tmin..tmax tokens, tmax <= 32
// (kernels_grouped_wave.hip); the same formats as the workgroup kernels.
hipError_t launch_gate_up_wave(const MoeShape& s, const ExpertEntry* table, TileItems wi, const _Float16* xh,
                               const _Float16* xl, const _Float16* xsh, const _Float16* xsl, const float* xscale,
                               float* h, int tmin, int tmax, hipStream_t st);
hipError_t launch_down_wave(const MoeShape& s, const ExpertEntry* table, TileItems wi, const _Float16* hh,
                            const _Float16* hl, const float* hscale, float* yp, int tmin, int tmax, hipStream_t st);
// Largest expert (in tokens) the per-wave kernels take (0: none, at most 32);
// a negative argument only queries.  Returns the previous value.
int set_grouped_wave_max(int tmax);
// Integer-dot matmuls for experts holding tmin..tmax tokens, tmax <= 32
// (kernels_grouped_dot.hip).  levels: rows of n values as int8 levels
// (q [rows][3][n], sc [rows][3][n/64], s32 [rows][n/32]).  gate/up from the
// tokens' x levels to h [P][FF] fp32, down from h's levels.
bool grouped_dot_gate_up_ok(const MoeShape& s);
bool grouped_dot_down_ok(const MoeShape& s);
hipError_t launch_levels_rows(const float* src, int ld, int rows, int n, int8_t* q, float* sc, float* s32,
                              hipStream_t st);
// The integer-dot launches' work list, written by the grouping kernel: item
// i < *n is (expert e, pair j of its n tokens), packed as
// e | j << 16 | n << 24 in .x, with the expert's first pair position in .y;
// cap item slots (the launches' grid).
struct DotItems {
    const int2* items;
    const int* n;
    int cap;
};
hipError_t launch_gate_up_dot(const MoeShape& s, const ExpertEntry* table, int E, DotItems gr, const int* tok,
                              const int8_t* xq, const float* xsc, const float* xs32, float* h, int tmin, int tmax,
                              hipStream_t st);
hipError_t launch_down_dot(const MoeShape& s, const ExpertEntry* table, int E, DotItems gr, const int8_t* hq,
                           const float* hsc, const float* hs32, float* yp, int tmin, int tmax, hipStream_t st);
// The integer-dot kernels: 0 off; 1..32 on, and in batches of more than 32
// tokens also for groups of at most that many tokens; above 32 on for
// batches of at most 32 tokens only (the default, reported as 33).  A
// negative argument only queries.  Returns the previous setting.
int set_grouped_dot_max(int tmax);
// 1 (default): the grouped block uses the matrix-core matmuls where the formats
// allow; 0: the vector-ALU kernels only.  A negative argument only queries.
int set_grouped_mfma(int enable);

// y[i] = expf(x[i]) bit for bit as glibc's (expf_ref.h), i < n.
hipError_t launch_expf_ref(const float* x, float* y, int64_t n, hipStream_t st);
// softmax -> top-k (e desc, index asc) -> renormalise; logits [nb][n_expert].
hipError_t launch_route_topk(const float* logits, int nb, int n_expert, int k, int* ids, float* w, hipStream_t st);
// Streaming read of bytes (a multiple of 16, 16-byte aligned buffer); the
// XOR of sink[0..4096) becomes the XOR of every 32-bit word read.
// hipErrorInvalidValue on bad arguments.
hipError_t launch_stream_read(const void* buf, size_t bytes, uint32_t* sink, hipStream_t st);

bool moe_shape_ok(const MoeShape& s);

// Sets the message eahmmf_hip_last_error() returns on this thread (capi.hip).
void set_last_error(const char* msg);
// The eahmmf_hip_set_fused() setting (capi.hip).
bool fused_path_enabled();
// Error word of the no-allocation entry point's scratch on the current device
// (noalloc.hip): 1 if a launch gave up a wait since the last call, then
// cleared; 0 if not or never set up; -2 on a HIP error.
int noalloc_device_flags();
bool type_supported(int t);

// Dense decode steps (kernels_dense.hip), nb tokens at positions p0 ...
// x[t] = dequantized row toks[t] of tab (or, with key, nb = 1: the argmax id
// held in the key, which is cleared and stored in *hist if given); a token id
// outside [0, n_vocab) sets *bad.
hipError_t launch_embed(int type, const uint8_t* tab, size_t row_bytes, int n_vocab, int D, const int* toks,
                        unsigned long long* key, int* hist, int nb, float* x, int* bad, hipStream_t st);
hipError_t launch_rmsnorm(const float* x, const float* w, float* out, int rows, int n, float eps, hipStream_t st);
// Floats of partial-result scratch launch_attention needs for nb tokens whose
// last position is n_pos - 1.
size_t attention_part_floats(int nb, int n_head, int hd, int n_pos);
// Causal attention of nb tokens at p0.. from raw q [nb][n_head*hd], k/v
// [nb][n_kv*hd]: head RMSNorm + NeoX RoPE (rope [pos][hd/2] cos/sin pairs),
// the batch's K/V rows appended to kc/vc (this layer's [n_ctx][n_kv*hd]),
// out [nb][n_head*hd].  cnt: nb * n_kv counters, zero before the first
// launch (each launch leaves them zero).  hd 64 or 128, n_head / n_kv in
// {1, 2, 4, 8, 16}.
bool attention_supported(int n_head, int n_kv, int hd);
hipError_t launch_attention(const float* q, const float* k, const float* v, const float* q_norm, const float* k_norm,
                            const float* rope, float* kc, float* vc, float* out, int nb, int n_head, int n_kv, int hd,
                            int p0, float eps, float scale, float* part, unsigned* cnt, hipStream_t st);
// The same for nb tokens of nb different sequences: token t is at position
// tpos[t] (device) of the sequence whose cache rows start tseq[t] (device) *
// seq_stride floats past kc / vc, and attends to that sequence's rows
// 0 .. tpos[t]; max_pos >= every tpos[t] sizes the splits.
hipError_t launch_attention_multi(const float* q, const float* k, const float* v, const float* q_norm,
                                  const float* k_norm, const float* rope, float* kc, float* vc, float* out, int nb,
                                  int n_head, int n_kv, int hd, const int* tpos, const int* tseq, size_t seq_stride,
                                  int max_pos, float eps, float scale, float* part, unsigned* cnt, hipStream_t st);
// Single-token matrix-vector products with fused input and output steps
// (kernels_gemv.hip).  Up to three weight matrices of one type and row
// length; out[r] = (resid ? resid[r] : 0) + sum_i W[r][i] * in[i] where
// in = x (+ x_add), RMS-normalized with norm_w when given.  Block 0 stores
// x + x_add in x_sum_out and the normalized input in xn_out when given.
// amax (if set) receives atomicMax of (ordered value, ~global row) keys.
struct GemvSeg {
    const uint8_t* w;
    float* out;
    const float* resid;
    int rows;
};
struct GemvArgs {
    GemvSeg seg[3];
    int nseg;
    int ne0, rb;
    int ni, rpw, nbuf, total_rows;  // set by launch_gemv
    const float* x;
    const float* x_add;
    const float* norm_w;
    float eps;
    float* x_sum_out;
    float* xn_out;
    unsigned long long* amax;
};
bool gemv_supported(int type, int ne0, size_t rb);
hipError_t launch_gemv(int type, GemvArgs a, hipStream_t st);

hipError_t launch_add(float* x, const float* y, size_t n, hipStream_t st);
// Copies two regions of 4-byte words (sizes multiples of 4) in one kernel;
// either side may be pinned host memory (kernels_basic.hip).
hipError_t launch_copy_words(void* d0, const void* s0, size_t bytes0, void* d1, const void* s1, size_t bytes1,
                             hipStream_t st);
// The same by one workgroup, then `seq` stored (system scope) to the pinned
// word `flag` once every copied word is in place.
hipError_t launch_copy_words_signal(void* d0, const void* s0, size_t bytes0, void* d1, const void* s1, size_t bytes1,
                                    unsigned* flag, unsigned seq, hipStream_t st);

}  // namespace eahmmf
