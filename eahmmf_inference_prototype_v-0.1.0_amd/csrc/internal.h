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
    int mode = 0;  // 0: direct slots, 1: logits + table (routing in the kernel), 2: ids/w + table
    DecodeSlots direct{};
    const ExpertEntry* table = nullptr;
    const float* logits = nullptr;
    const int* ids_in = nullptr;
    const float* w_in = nullptr;
    int* ids_out = nullptr;
    float* w_out = nullptr;
    const float* x = nullptr;
    float* y = nullptr;
    uint64_t* hx = nullptr;       // k * FF exchange words (h value | epoch << 32), zeroed when allocated
    uint64_t* ypart = nullptr;    // 8 * D exchange words: per-partition partial outputs, zeroed when allocated
    unsigned* sync = nullptr;     // kSyncWords words, zero before the first launch (error flag)
    unsigned epoch = 0;           // launch number on these buffers, starting at 1
};
constexpr int kSyncWords = 4096;
constexpr int kSyncFlagWord = 1020;  // error flag word inside the sync buffer
bool fused_supported(const MoeShape& s, int k, int n_expert_for_routing);
// 1 if the fused kernel's partitions exchange h through their own XCD's L2 on
// this device (workgroup b runs on XCD b % 8), 0 if it uses the
// device-coherent protocol.
int fused_exchange_mode(int device);
hipError_t launch_moe_fused(const FusedArgsHost& h, hipStream_t st);

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
hipError_t launch_gate_up_mfma(const MoeShape& s, const ExpertEntry* table, int E, const int* offs, int nb,
                               const _Float16* xh, const _Float16* xl, const _Float16* xsh, const _Float16* xsl,
                               const float* xscale, float* h, hipStream_t st);
hipError_t launch_down_mfma(const MoeShape& s, const ExpertEntry* table, int E, const int* offs, int nb,
                            const _Float16* hh, const _Float16* hl, const float* hscale, float* yp, hipStream_t st);
// 1 (default): the grouped block uses the matrix-core matmuls where the formats
// allow; 0: the vector-ALU kernels only.  A negative argument only queries.
int set_grouped_mfma(int enable);

// softmax -> top-k (e desc, index asc) -> renormalise; logits [nb][n_expert].
hipError_t launch_route_topk(const float* logits, int nb, int n_expert, int k, int* ids, float* w, hipStream_t st);
// Streaming read of bytes (a multiple of 16, 16-byte aligned buffer); the
// XOR of sink[0..4096) becomes the XOR of every 32-bit word read.
// hipErrorInvalidValue on bad arguments.
hipError_t launch_stream_read(const void* buf, size_t bytes, uint32_t* sink, hipStream_t st);

bool moe_shape_ok(const MoeShape& s);
bool type_supported(int t);

}  // namespace eahmmf
