// noalloc.hip - the single-launch expert block for callers that cannot
// allocate device memory (code under HIP graph capture, tight serving loops,
// harnesses that forbid hipMalloc).
//
// eahmmf_hip_moe_layer_decode_noalloc is eahmmf_hip_moe_layer_decode_async
// with its scratch in one file-scope device array instead of buffers the
// library allocates: the fused kernel's exchange words (h and the
// per-partition partials), its sync words (error word, ticket counters), and
// for shapes the fused kernel does not take, the two-kernel path's h and
// routing results.  Every GPU the library runs on holds its own copy of the
// array (kScratchBytes, about 1 MiB) until the process ends.  Calls on one GPU
// share it: calls that overlap in time on one device race.
//
// In host code the array's name is not a device address.  Its address on a
// device comes from hipGetSymbolAddress, once per device with that device
// current, and only that pointer is passed to kernels.
#include <mutex>

#include "../../include/eahmmf_hip.h"
#include "internal.h"

namespace eahmmf {
namespace {

// Layout of the scratch array (bytes).
constexpr size_t kHxWords = (size_t)kMaxSlots * 4096;  // k * FF <= 16 * 4096 h exchange words
constexpr size_t kYpartWords = (size_t)8 * 4096;       // 8 partitions x D <= 4096 partials
constexpr size_t kHxOff = 0;
constexpr size_t kYpartOff = kHxOff + kHxWords * 8;
constexpr size_t kSyncOff = kYpartOff + kYpartWords * 8;
constexpr size_t kHOff = kSyncOff + (size_t)kSyncWords * 4;  // two-kernel path: h [k][FF] fp32
constexpr size_t kHFloats = (size_t)kMaxSlots * 4096;
constexpr size_t kIdsOff = kHOff + kHFloats * 4;  // two-kernel path: routing ids [k], then weights [k]
constexpr size_t kWOff = kIdsOff + 256;
constexpr size_t kScratchBytes = kWOff + 256;
static_assert(kHOff % 256 == 0 && kIdsOff % 256 == 0, "aligned regions");
static_assert(kHFloats * 4 >= 4096, "the placement probe's 1024 ints fit the h region");

static __device__ __align__(256) uint8_t scratch[kScratchBytes];

constexpr int kMaxDevices = 64;

struct NoAllocDev {
    bool ready = false;
    uint8_t* base = nullptr;  // scratch's address on this device (hipGetSymbolAddress)
    FusedState fs;
};
NoAllocDev g_dev[kMaxDevices];
std::mutex g_mu;

__global__ void zero_words_kernel(uint32_t* p, size_t n) {
    for (size_t i = blockIdx.x * (size_t)blockDim.x + threadIdx.x; i < n; i += (size_t)gridDim.x * blockDim.x)
        p[i] = 0u;
}

}  // namespace

// The calling device's scratch state, set up on its first call: the array's
// device address, cleared with a fill kernel on `st` (no memset node), and the
// fused kernel's XCD placement probed with the array as its buffer.  Null on
// a HIP error (message in *err).
static NoAllocDev* noalloc_dev(hipStream_t st, const char** err) {
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= kMaxDevices) {
        *err = "no usable current device";
        return nullptr;
    }
    std::lock_guard<std::mutex> lk(g_mu);
    NoAllocDev& d = g_dev[dev];
    if (d.ready) return &d;
    void* p = nullptr;
    if (hipGetSymbolAddress(&p, HIP_SYMBOL(scratch)) != hipSuccess || !p) {
        *err = "hipGetSymbolAddress(scratch) failed";
        return nullptr;
    }
    uint8_t* base = (uint8_t*)p;
    clear_stale_error();
    hipLaunchKernelGGL(zero_words_kernel, dim3(256), dim3(256), 0, st, (uint32_t*)base, kScratchBytes / 4);
    if (hipGetLastError() != hipSuccess || hipStreamSynchronize(st) != hipSuccess) {
        *err = "clearing the scratch array failed";
        return nullptr;
    }
    // one-time probe (a no-op when an earlier call on this device ran it); it
    // uses the h region, which holds nothing yet
    (void)fused_exchange_probe(dev, (int*)(base + kHOff));
    d.base = base;
    d.fs.hx = (uint64_t*)(base + kHxOff);
    d.fs.hx_words = kHxWords;
    d.fs.ypart = (uint64_t*)(base + kYpartOff);
    d.fs.ypart_words = kYpartWords;
    d.fs.sync = (unsigned*)(base + kSyncOff);
    d.ready = true;
    return &d;
}

// Nonzero if a no-allocation launch on the current device gave up a wait
// since the last call; clears the word.  0 when the scratch was never set up.
int noalloc_device_flags() {
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= kMaxDevices) return 0;
    NoAllocDev* d = nullptr;
    {
        std::lock_guard<std::mutex> lk(g_mu);
        if (!g_dev[dev].ready) return 0;
        d = &g_dev[dev];
    }
    unsigned v = 0;
    if (hipDeviceSynchronize() != hipSuccess ||
        hipMemcpy(&v, d->fs.sync + kSyncFlagWord, sizeof v, hipMemcpyDeviceToHost) != hipSuccess)
        return -2;
    if (v) {
        (void)reset_fused_sync(d->fs, nullptr, true);
        (void)hipDeviceSynchronize();
    }
    return v ? 1 : 0;
}

}  // namespace eahmmf

using namespace eahmmf;

extern "C" int eahmmf_hip_moe_layer_decode_noalloc(const eahmmf_hip_moe_shape* shape,
                                                   const eahmmf_hip_expert_ptrs* dev_table, int n_expert,
                                                   const float* dev_logits, int k, const float* dev_x, float* dev_y,
                                                   int* dev_ids_out, float* dev_w_out, void* stream) {
    if (!shape) return set_last_error("null shape"), -1;
    MoeShape s{shape->gate_type, shape->up_type, shape->down_type, shape->D, shape->FF,
               shape->gate_row_bytes, shape->up_row_bytes, shape->down_row_bytes};
    if (!moe_shape_ok(s)) return set_last_error("unsupported expert shape/type combination"), -1;
    if (!dev_table || !dev_logits || !dev_x || !dev_y) return set_last_error("null argument"), -1;
    if (n_expert <= 0 || n_expert > 512 || k <= 0 || k > kMaxSlots || k > n_expert)
        return set_last_error("bad routing shape (need 1 <= k <= 16 and k <= n_expert <= 512)"), -1;
    if ((size_t)k * s.FF > kHxWords || s.D > 4096)
        return set_last_error("shape exceeds the scratch array (need k * FF <= 65536 and D <= 4096)"), -1;
    hipStream_t st = (hipStream_t)stream;
    const char* err = "";
    NoAllocDev* d = noalloc_dev(st, &err);
    if (!d) return set_last_error(err), -2;
    if (fused_path_enabled() && fused_supported(s, k, n_expert)) {
        FusedArgsHost f;
        f.shape = s;
        f.k = k;
        f.n_expert = n_expert;
        f.mode = 1;
        f.table = (const ExpertEntry*)dev_table;
        f.logits = dev_logits;
        f.ids_out = dev_ids_out;
        f.w_out = dev_w_out;
        f.x = dev_x;
        f.y = dev_y;
        return launch_moe_fused(f, d->fs, st) == hipSuccess ? 0 : (set_last_error("fused moe layer launch failed"), -3);
    }
    // the routing kernel and the two expert kernels, every scratch buffer in the array
    int* ids = dev_ids_out;
    float* w = dev_w_out;
    if (!ids || !w) {
        ids = (int*)(d->base + kIdsOff);
        w = (float*)(d->base + kWOff);
    }
    if (launch_route_topk(dev_logits, 1, n_expert, k, ids, w, st) != hipSuccess)
        return set_last_error("route launch failed"), -3;
    if (launch_moe_decode_routed(s, (const ExpertEntry*)dev_table, n_expert, ids, w, k, dev_x,
                                 (float*)(d->base + kHOff), dev_y, st) != hipSuccess)
        return set_last_error("routed moe decode launch failed"), -3;
    return 0;
}
