// capi.hip - the C ABI of libeahmmf_hip.so (include/eahmmf_hip.h).
//
// Per device the library keeps one non-blocking stream, device scratch for
// activations/outputs and pinned host staging buffers, all grown on demand
// and reused (the reference's wrappers keep the same kind of static scratch,
// expert_cuda.cu:269-301, 363-392).  Synchronous entry points stage pageable
// host data through the pinned buffers, enqueue copies and kernels on the
// stream, and always drain the stream before returning, also after an error,
// so a caller may release its expert leases as soon as the call returns.
#include <stdarg.h>
#include <stdlib.h>
#include <stdio.h>
#include <string.h>

#include <map>
#include <mutex>
#include <string>
#include <vector>
#include <algorithm>
#include <chrono>
#include <condition_variable>
#include <deque>
#include <thread>

#include "../../include/eahmmf_hip.h"
#include "internal.h"
#include "kquant.h"

using namespace eahmmf;

namespace {

thread_local std::string g_last_error;

void set_error(const char* fmt, ...) {
    char buf[512];
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(buf, sizeof buf, fmt, ap);
    va_end(ap);
    g_last_error = buf;
}

bool hip_ok(hipError_t e, const char* what) {
    if (e == hipSuccess) return true;
    set_error("%s: %s (%d)", what, hipGetErrorString(e), (int)e);
    return false;
}

struct DeviceBuf {
    void* p = nullptr;
    size_t cap = 0;
};

// Largest batch eahmmf_hip_moe_grouped_async runs as per-token fused launches
// (from 4 tokens the grouped block, which streams each distinct routed expert
// once, is faster).
constexpr int kFusedBatchMax = 3;

// Bulk staging ring: kRingSlots pinned slots of kRingChunk bytes each.
constexpr int kRingSlots = 4;
constexpr size_t kRingChunk = (size_t)32 << 20;

struct DevCtx {
    hipStream_t stream = nullptr;
    DeviceBuf dx, dy, dy2, dh, dids, dw, dyp, dhx, dgs, dtab, drt, dws;  // device scratch
    DeviceBuf px, py, py2;                // pinned host staging
    unsigned* dsync = nullptr;            // fused-launch error word and ticket counters (zeroed once)
    FusedState fused;                     // the fused kernel's scratch set (dhx, dyp, dsync) and epochs
    // bulk host-to-device staging (eahmmf_hip_h2d_batch), created on first use
    hipStream_t copy_stream[kRingSlots] = {};  // one per slot: slots drain on parallel DMA engines
    uint8_t* ring[kRingSlots] = {};
    hipEvent_t ring_done[kRingSlots] = {};  // recorded after the copies out of each slot
    bool ring_ready = false;
    int ring_next = 0;  // the slot the next staged batch starts in
    unsigned* hflag = nullptr;  // pinned completion word of the synchronous entry points
    unsigned hseq = 0;          // the last sequence number stored there
};

// 1: single fused launch where the shape allows it; 0: route + two-kernel path.
// EAHMMF_HIP_UNFUSED=1 in the environment selects 0 at start-up.
int g_fused = -1;
bool fused_enabled() {
    if (g_fused < 0) {
        const char* e = getenv("EAHMMF_HIP_UNFUSED");
        g_fused = (e && *e && *e != '0') ? 0 : 1;
    }
    return g_fused == 1;
}

std::mutex g_mu;
std::map<int, DevCtx> g_ctx;

DevCtx* ctx_for_current_device() {
    int dev = 0;
    if (!hip_ok(hipGetDevice(&dev), "hipGetDevice")) return nullptr;
    std::lock_guard<std::mutex> g(g_mu);
    DevCtx& c = g_ctx[dev];
    if (!c.stream && !hip_ok(hipStreamCreateWithFlags(&c.stream, hipStreamNonBlocking), "hipStreamCreate"))
        return nullptr;
    if (!c.dsync) {
        void* p = nullptr;
        if (!hip_ok(hipMalloc(&p, kSyncWords * sizeof(unsigned)), "hipMalloc(sync)")) return nullptr;
        if (!hip_ok(hipMemset(p, 0, kSyncWords * sizeof(unsigned)), "hipMemset(sync)")) {
            (void)hipFree(p);
            return nullptr;
        }
        c.dsync = (unsigned*)p;
        c.fused.sync = c.dsync;
    }
    return &c;
}

bool grow_device(DeviceBuf& b, size_t need) {
    if (need <= b.cap) return true;
    if (b.p) (void)hipFree(b.p);
    b.p = nullptr;
    b.cap = 0;
    size_t cap = need < 4096 ? 4096 : need;
    if (!hip_ok(hipMalloc(&b.p, cap), "hipMalloc(scratch)")) return false;
    b.cap = cap;
    return true;
}

bool grow_pinned(DeviceBuf& b, size_t need) {
    if (need <= b.cap) return true;
    if (b.p) (void)hipHostFree(b.p);
    b.p = nullptr;
    b.cap = 0;
    size_t cap = need < 4096 ? 4096 : need;
    if (!hip_ok(hipHostMalloc(&b.p, cap, hipHostMallocDefault), "hipHostMalloc(staging)")) return false;
    b.cap = cap;
    return true;
}

// Drain the stream; a failure here also fails the call.
bool drain(DevCtx* c, bool ok) {
    const hipError_t e = hipStreamSynchronize(c->stream);
    if (e != hipSuccess) {
        set_error("hipStreamSynchronize: %s (%d)", hipGetErrorString(e), (int)e);
        return false;
    }
    return ok;
}

// The reference's checks (expert_cuda.cu:263-267) plus two of the layout:
// ne0 a whole number of blocks (every GGUF row is), and a row stride that
// holds the row's blocks, a multiple of 16 for Q4_K/Q5_K and of 2 for
// Q6_K/Q8_0 (the block loads' alignment).  Rows may be padded: row r starts
// at w + r * row_bytes, as in the reference.
bool matmul_args_ok(const uint8_t* w, int type, int ne0, int ne1, size_t row_bytes, int ldx, int ldo) {
    if (!w) return set_error("null weight pointer"), false;
    if (!type_supported(type)) return set_error("unsupported ggml type %d", type), false;
    if (ne0 <= 0 || ne1 <= 0) return set_error("bad shape %d x %d", ne1, ne0), false;
    if (ne0 % type_blck(type)) return set_error("ne0 %d not a multiple of the block size", ne0), false;
    const size_t packed = (size_t)(ne0 / type_blck(type)) * type_bytes(type);
    const size_t align = (type == kQ4_K || type == kQ5_K) ? 16 : 2;
    if (row_bytes < packed || row_bytes % align)
        return set_error("row_bytes %zu: type %d, ne0 %d needs at least %zu, a multiple of %zu", row_bytes, type, ne0,
                         packed, align),
               false;
    if (ldx < ne0 || ldo < ne1) return set_error("ldx/ldo smaller than the row length"), false;
    return true;
}

// host x[nb][ldx] (first ne0 of each row) -> device dense [nb][ne0]
// Up to this many bytes a synchronous call's staging copies run as a copy
// kernel on the call's stream (launch_copy_words), above it on a copy engine.
constexpr size_t kKernelCopyMax = (size_t)1 << 20;

// Queues dst0 <- src0 and dst1 <- src1 (bytes multiples of 4; bytes1 may be 0)
// between pinned staging and device buffers on the context's stream.
bool queue_copies(DevCtx* c, void* d0, const void* s0, size_t b0, void* d1, const void* s1, size_t b1,
                  hipMemcpyKind kind, const char* what) {
    if (b0 + b1 <= kKernelCopyMax && ((b0 | b1) & 3) == 0)
        return hip_ok(launch_copy_words(d0, s0, b0, d1, s1, b1, c->stream), what);
    return hip_ok(hipMemcpyAsync(d0, s0, b0, kind, c->stream), what) &&
           (b1 == 0 || hip_ok(hipMemcpyAsync(d1, s1, b1, kind, c->stream), what));
}

// The synchronous entry points' results: the copies to pinned staging run as
// one workgroup that then stores a sequence number to a pinned word, and the
// host polls that word instead of synchronising the stream (a stream
// synchronisation costs about 10 us more per call here).  A launch that has
// not signalled within kPollBudget (a fault stops the queue) falls back to
// the stream synchronisation, which then reports the error.  Larger results
// take the copies and the synchronisation.
constexpr size_t kSignalMax = (size_t)256 << 10;
constexpr auto kPollBudget = std::chrono::milliseconds(50);

bool finish_copies(DevCtx* c, bool ok, void* d0, const void* s0, size_t b0, void* d1, const void* s1, size_t b1,
                   const char* what) {
    if (!ok) return drain(c, false);
    if (!c->hflag) {
        void* p = nullptr;
        if (hipHostMalloc(&p, 4096, hipHostMallocCoherent) == hipSuccess) {
            c->hflag = (unsigned*)p;
            __atomic_store_n(c->hflag, 0u, __ATOMIC_RELEASE);
        } else {
            clear_stale_error();
        }
    }
    if (!c->hflag || b0 + b1 > kSignalMax || ((b0 | b1) & 3)) {
        ok = queue_copies(c, d0, s0, b0, d1, s1, b1, hipMemcpyDeviceToHost, what);
        return drain(c, ok);
    }
    unsigned seq = ++c->hseq;
    if (seq == 0) seq = ++c->hseq;  // 0 is the word's initial value
    if (!hip_ok(launch_copy_words_signal(d0, s0, b0, d1, s1, b1, c->hflag, seq, c->stream), what))
        return drain(c, false);
    const auto t0 = std::chrono::steady_clock::now();
    for (unsigned i = 1;; i++) {
        if (__atomic_load_n(c->hflag, __ATOMIC_ACQUIRE) == seq) return true;
        if ((i & 1023) == 0 && std::chrono::steady_clock::now() - t0 > kPollBudget) break;
    }
    return drain(c, true);
}

bool stage_x(DevCtx* c, const float* host_x, int nb, int ne0, int ldx) {
    const size_t bytes = (size_t)nb * ne0 * sizeof(float);
    if (!grow_pinned(c->px, bytes) || !grow_device(c->dx, bytes)) return false;
    float* px = (float*)c->px.p;
    for (int t = 0; t < nb; t++) memcpy(px + (size_t)t * ne0, host_x + (size_t)t * ldx, sizeof(float) * ne0);
    return queue_copies(c, c->dx.p, px, bytes, nullptr, nullptr, 0, hipMemcpyHostToDevice, "stage x");
}

void unstage_rows(const float* dense, int nb, int n, float* host, int ld) {
    for (int t = 0; t < nb; t++) memcpy(host + (size_t)t * ld, dense + (size_t)t * n, sizeof(float) * n);
}

// the fused launch's per-partition partial outputs (8 partitions x D floats)
// The fused kernel's exchange words (h and the per-partition partials, each
// a value and a launch epoch): zeroed when allocated, so that no stale word
// can carry the epoch of a launch to come (epochs start at 1).
static bool grow_zeroed(DeviceBuf& b, size_t need) {
    if (need <= b.cap) return true;
    if (!grow_device(b, need)) return false;
    // complete before any launch: the fused kernel runs on non-blocking streams
    if (!hip_ok(hipMemset(b.p, 0, b.cap), "hipMemset(exchange words)") ||
        !hip_ok(hipDeviceSynchronize(), "hipDeviceSynchronize(exchange words)")) {
        (void)hipFree(b.p);
        b.p = nullptr;
        b.cap = 0;
        return false;
    }
    return true;
}

bool grow_fused(DevCtx* c, const MoeShape& s, int k) {
    if (!grow_zeroed(c->dyp, (size_t)8 * s.D * sizeof(uint64_t)) ||
        !grow_zeroed(c->dhx, (size_t)k * s.FF * sizeof(uint64_t)))
        return false;
    c->fused.hx = (uint64_t*)c->dhx.p;
    c->fused.hx_words = c->dhx.cap / sizeof(uint64_t);
    c->fused.ypart = (uint64_t*)c->dyp.p;
    c->fused.ypart_words = c->dyp.cap / sizeof(uint64_t);
    return true;
}

// After the drain: an error word equal to the call's own launch epoch means
// that launch gave up a wait and its output is invalid (NaN where words were
// missing).  The call then fails, as the reference's ABI does on any GPU
// error (expert_cuda.cu:332-335), and the ticket counters are reset for the
// next launch.  The word itself stays set for eahmmf_hip_device_flags(); a
// later launch compares it with its own epoch, so it does not fail them.
bool flag_ok(DevCtx* c, unsigned v, unsigned epoch) {
    if (v != epoch) return true;
    set_error("fused expert block: a bounded wait gave up (launch %u); output invalid", v);
    (void)reset_fused_sync(c->fused, c->stream, false);
    (void)hipStreamSynchronize(c->stream);
    return false;
}

bool weight_ok(const eahmmf_hip_weight& w) { return w.dev && type_supported(w.type) && w.ne0 > 0 && w.ne1 > 0; }

bool ensure_ring(DevCtx* c) {
    if (c->ring_ready) return true;
    for (int s = 0; s < kRingSlots; s++) {
        if (!c->copy_stream[s] &&
            !hip_ok(hipStreamCreateWithFlags(&c->copy_stream[s], hipStreamNonBlocking), "hipStreamCreate(staging)"))
            return false;
        if (!c->ring[s]) {
            void* p = nullptr;
            if (!hip_ok(hipHostMalloc(&p, kRingChunk, hipHostMallocDefault), "hipHostMalloc(staging ring)")) return false;
            c->ring[s] = (uint8_t*)p;
        }
        if (!c->ring_done[s] &&
            !hip_ok(hipEventCreateWithFlags(&c->ring_done[s], hipEventDisableTiming), "hipEventCreate(staging)"))
            return false;
    }
    c->ring_ready = true;
    return true;
}

// One piece of a staging slot: n bytes from src to dst, at offset at in the slot.
struct Piece {
    uint8_t* dst;
    const uint8_t* src;
    size_t n, at;
};

// Threads that fill a slot (pageable -> pinned copies run on the CPU).
int stage_threads() {
    static const int n = [] {
        const char* e = getenv("EAHMMF_HIP_STAGE_THREADS");
        int v = e && *e ? atoi(e) : (int)std::thread::hardware_concurrency() / 2;
        return v < 1 ? 1 : (v > 16 ? 16 : v);
    }();
    return n;
}

// Copies the pieces into the slot, splitting the slot's bytes [0, total)
// evenly over nt threads (small slots on the calling thread alone).
void fill_slot(uint8_t* slot, const std::vector<Piece>& ps, size_t total, int nt) {
    auto range = [&](size_t lo, size_t hi) {
        for (const Piece& q : ps) {
            const size_t a = std::max(lo, q.at), b = std::min(hi, q.at + q.n);
            if (a < b) memcpy(slot + a, q.src + (a - q.at), b - a);
        }
    };
    if (nt <= 1 || total < ((size_t)4 << 20)) {
        range(0, total);
        return;
    }
    const size_t per = ((total + nt - 1) / nt + 4095) & ~(size_t)4095;
    std::vector<std::thread> th;
    size_t done = per;  // [0, done) is this thread's; the rest is handed out below
    try {
        for (int t = 1; t < nt && (size_t)t * per < total; t++) {
            th.emplace_back(range, (size_t)t * per, std::min(total, (size_t)(t + 1) * per));
            done = std::min(total, (size_t)(t + 1) * per);
        }
    } catch (...) {
        // no thread could be started: the rest is copied here (no exception
        // leaves the C ABI)
    }
    range(0, std::min(total, per));
    if (done < total) range(done, total);
    for (std::thread& x : th) x.join();
}

// Every copy has both pointers unless it is empty.
bool copies_ok(const eahmmf_hip_copy* copies, int n) {
    if (n < 0 || (n > 0 && !copies)) return set_error("null argument"), false;
    for (int i = 0; i < n; i++)
        if (copies[i].bytes && (!copies[i].dev_dst || !copies[i].host_src))
            return set_error("copy %d: null pointer", i), false;
    return true;
}

// The copies of one batch through the ring: per slot, wait until its previous
// copies have left it, fill it on the CPU, then one DMA per piece on the
// slot's stream and an event behind them.  Pieces start 256-byte aligned in
// a slot; small copies share one.
bool stage_copies(DevCtx* c, const eahmmf_hip_copy* copies, int n) {
    const int nt = stage_threads();
    bool ok = true;
    int slot = c->ring_next;
    std::vector<Piece> ps;
    size_t fill = 0;
    auto flush = [&]() -> bool {
        if (ps.empty()) return true;
        if (!hip_ok(hipEventSynchronize(c->ring_done[slot]), "staging wait")) return false;
        fill_slot(c->ring[slot], ps, fill, nt);
        for (const Piece& q : ps)
            if (!hip_ok(hipMemcpyAsync(q.dst, c->ring[slot] + q.at, q.n, hipMemcpyHostToDevice,
                                       c->copy_stream[slot]),
                        "staging copy"))
                return false;
        if (!hip_ok(hipEventRecord(c->ring_done[slot], c->copy_stream[slot]), "staging record")) return false;
        slot = (slot + 1) % kRingSlots;
        ps.clear();
        fill = 0;
        return true;
    };
    for (int i = 0; ok && i < n; i++) {
        uint8_t* dst = (uint8_t*)copies[i].dev_dst;
        const uint8_t* src = (const uint8_t*)copies[i].host_src;
        for (size_t off = 0; ok && off < copies[i].bytes;) {
            const size_t m = std::min(copies[i].bytes - off, kRingChunk - fill);
            ps.push_back(Piece{dst + off, src + off, m, fill});
            off += m;
            fill = std::min(kRingChunk, (fill + m + 255) & ~(size_t)255);
            if (fill == kRingChunk) ok = flush();
        }
    }
    if (ok) ok = flush();
    c->ring_next = slot;
    return ok;
}

// Asynchronous staging (eahmmf_hip_h2d_batch_async): one worker thread per
// device takes batches in order, stages them through the ring and records a
// completion event behind every slot's copies (on a join stream that waits
// for the four slots).  A ticket's batch has landed once its event has
// completed; completed events are destroyed when the next batch is queued.
// The worker and the state live until the process ends (the thread is
// detached and idles on its condition variable).
constexpr int kMaxDev = 64;
struct Stager {
    DevCtx* c = nullptr;
    int dev = 0;
    hipStream_t join = nullptr;
    std::mutex qmu;
    std::condition_variable qcv, dcv;
    std::deque<std::pair<uint64_t, std::vector<eahmmf_hip_copy>>> q;
    uint64_t next = 1, issued = 0;  // tickets handed out; batches whose copies are all queued
    std::map<uint64_t, hipEvent_t> ev;
    std::map<uint64_t, std::string> failed;  // the worker's error message per failed batch
    bool stop = false, running = false;
};
Stager* g_stager[kMaxDev] = {};

void stager_main(Stager* st) {
    (void)hipSetDevice(st->dev);
    std::unique_lock<std::mutex> lk(st->qmu);
    for (;;) {
        st->qcv.wait(lk, [&] { return st->stop || !st->q.empty(); });
        if (st->q.empty()) break;  // stop
        auto job = std::move(st->q.front());
        st->q.pop_front();
        lk.unlock();
        hipEvent_t e = nullptr;
        bool ok = hip_ok(hipEventCreateWithFlags(&e, hipEventDisableTiming), "hipEventCreate(staging)");
        ok = ok && stage_copies(st->c, job.second.data(), (int)job.second.size());
        for (int s = 0; ok && s < kRingSlots; s++)
            ok = hip_ok(hipStreamWaitEvent(st->join, st->c->ring_done[s], 0), "staging join");
        ok = ok && hip_ok(hipEventRecord(e, st->join), "staging record");
        lk.lock();
        if (ok) {
            st->ev[job.first] = e;
        } else {
            st->failed[job.first] = g_last_error;
            if (e) (void)hipEventDestroy(e);
        }
        st->issued = job.first;
        st->dcv.notify_all();
    }
    st->running = false;
    st->dcv.notify_all();
}

// Destroys the events of landed batches (caller holds qmu).
void retire_done(Stager* st) {
    for (auto it = st->ev.begin(); it != st->ev.end();) {
        if (hipEventQuery(it->second) == hipSuccess) {
            (void)hipEventDestroy(it->second);
            it = st->ev.erase(it);
        } else {
            ++it;
        }
    }
}

Stager* stager_for(DevCtx* c) {
    int dev = 0;
    if (!hip_ok(hipGetDevice(&dev), "hipGetDevice")) return nullptr;
    if (dev < 0 || dev >= kMaxDev) return set_error("device %d out of range", dev), nullptr;
    std::lock_guard<std::mutex> g(g_mu);
    if (!ensure_ring(c)) return nullptr;
    Stager*& st = g_stager[dev];
    if (st && st->running) return st;
    if (!st) {
        st = new (std::nothrow) Stager;
        if (!st) return set_error("out of memory"), nullptr;
        st->dev = dev;
    }
    st->c = c;
    if (!st->join && !hip_ok(hipStreamCreateWithFlags(&st->join, hipStreamNonBlocking), "hipStreamCreate(join)"))
        return nullptr;
    st->stop = false;
    st->running = true;
    try {
        std::thread(stager_main, st).detach();
    } catch (...) {
        st->running = false;
        return set_error("could not start the staging thread"), nullptr;
    }
    return st;
}

// Stops the device's staging worker once its queue is empty (shutdown).
void stop_stager(int dev) {
    Stager* st = dev >= 0 && dev < kMaxDev ? g_stager[dev] : nullptr;
    if (!st) return;
    std::unique_lock<std::mutex> lk(st->qmu);
    st->stop = true;
    st->qcv.notify_all();
    st->dcv.wait(lk, [&] { return !st->running; });
    for (auto& kv : st->ev) {
        (void)hipEventSynchronize(kv.second);
        (void)hipEventDestroy(kv.second);
    }
    st->ev.clear();
    st->c = nullptr;
}

// A single token (the reference's decode calls, nb = 1) runs on the decode
// matrix-vector kernel (kernels_gemv.hip: rows DMA'd into LDS, the input held
// once per block in LDS, DPP reductions) where it takes the shape; its direct
// row reads want 16-byte aligned matrices.
bool gemv_ok(int type, const uint8_t* w, int ne0, size_t rb) {
    return gemv_supported(type, ne0, rb) && ((uintptr_t)w & 15u) == 0;
}

// The drop-in matmul's launch: the matrix-vector kernel for one token, the
// matrix cores for 2..64 tokens of a K-quant or Q8_0 matrix (workspace grown
// on demand), else the general kernel.
hipError_t matmul_launch(DevCtx* c, int type, const uint8_t* w, int ne0, int ne1, size_t rb, int nb, float* out) {
    const float* x = (const float*)c->dx.p;
    if (nb == 1 && gemv_ok(type, w, ne0, rb)) {
        GemvArgs g{};
        g.x = x;
        g.seg[0] = GemvSeg{w, out, nullptr, ne1};
        g.nseg = 1;
        g.ne0 = ne0;
        g.rb = (int)rb;
        return launch_gemv(type, g, c->stream);
    }
    if (dense_mfma_enabled() && matmul_mfma_ok(type, w, ne0, rb, x, nb, ne0) &&
        grow_device(c->dws, matmul_mfma_ws_bytes(ne0, ne1, nb)))
        return launch_matmul_mfma(type, w, ne0, ne1, rb, x, nb, ne0, out, ne1, c->dws.p, c->dws.cap, c->stream);
    return launch_matmul(type, w, ne0, ne1, rb, x, nb, ne0, out, ne1, c->stream);
}

}  // namespace

void eahmmf::set_last_error(const char* msg) { set_error("%s", msg); }
bool eahmmf::fused_path_enabled() { return fused_enabled(); }

extern "C" {

const char* eahmmf_hip_last_error(void) { return g_last_error.c_str(); }

int eahmmf_hip_device_count(void) {
    int n = 0;
    if (hipGetDeviceCount(&n) != hipSuccess) return 0;
    return n;
}

bool eahmmf_hip_matmul(const uint8_t* device_weights, int type, int ne0, int ne1, size_t row_bytes,
                       const float* host_x, int nb, int ldx, float* host_out, int ldo) {
    if (!host_x || !host_out || nb <= 0) return set_error("null host buffer or nb <= 0"), false;
    if (!matmul_args_ok(device_weights, type, ne0, ne1, row_bytes, ldx, ldo)) return false;
    DevCtx* c = ctx_for_current_device();
    if (!c) return false;
    const size_t obytes = (size_t)nb * ne1 * sizeof(float);
    bool ok = grow_device(c->dy, obytes) && grow_pinned(c->py, obytes) && stage_x(c, host_x, nb, ne0, ldx);
    if (ok) ok = hip_ok(matmul_launch(c, type, device_weights, ne0, ne1, row_bytes, nb, (float*)c->dy.p), "matmul launch");
    ok = finish_copies(c, ok, c->py.p, c->dy.p, obytes, nullptr, nullptr, 0, "copy out");
    if (ok) unstage_rows((const float*)c->py.p, nb, ne1, host_out, ldo);
    return ok;
}

bool eahmmf_hip_matmul_pair(const uint8_t* gw, int gt, int gne0, int gne1, size_t grb,
                            const uint8_t* uw, int ut, int une0, int une1, size_t urb,
                            const float* host_x, int nb, int ldx,
                            float* host_g, int ldg, float* host_u, int ldu) {
    if (!host_x || !host_g || !host_u || nb <= 0) return set_error("null host buffer or nb <= 0"), false;
    if (gne0 != une0 || gne1 != une1) return set_error("gate/up shape mismatch"), false;
    if (!matmul_args_ok(gw, gt, gne0, gne1, grb, ldx, ldg) || !matmul_args_ok(uw, ut, une0, une1, urb, ldx, ldu))
        return false;
    DevCtx* c = ctx_for_current_device();
    if (!c) return false;
    const size_t obytes = (size_t)nb * gne1 * sizeof(float);
    bool ok = grow_device(c->dy, obytes) && grow_device(c->dy2, obytes) && grow_pinned(c->py, obytes) &&
              grow_pinned(c->py2, obytes) && stage_x(c, host_x, nb, gne0, ldx);
    if (ok && nb == 1 && gt == ut && grb == urb && gemv_ok(gt, gw, gne0, grb) && gemv_ok(ut, uw, une0, urb)) {
        // one matrix-vector launch for both (the input staged in LDS once)
        GemvArgs g{};
        g.x = (const float*)c->dx.p;
        g.seg[0] = GemvSeg{gw, (float*)c->dy.p, nullptr, gne1};
        g.seg[1] = GemvSeg{uw, (float*)c->dy2.p, nullptr, une1};
        g.nseg = 2;
        g.ne0 = gne0;
        g.rb = (int)grb;
        ok = hip_ok(launch_gemv(gt, g, c->stream), "gate/up launch");
    } else {
        if (ok) ok = hip_ok(matmul_launch(c, gt, gw, gne0, gne1, grb, nb, (float*)c->dy.p), "gate launch");
        if (ok) ok = hip_ok(matmul_launch(c, ut, uw, une0, une1, urb, nb, (float*)c->dy2.p), "up launch");
    }
    ok = finish_copies(c, ok, c->py.p, c->dy.p, obytes, c->py2.p, c->dy2.p, obytes, "copy g/u");
    if (ok) {
        unstage_rows((const float*)c->py.p, nb, gne1, host_g, ldg);
        unstage_rows((const float*)c->py2.p, nb, une1, host_u, ldu);
    }
    return ok;
}

bool eahmmf_hip_moe_decode(const eahmmf_hip_expert* experts, const float* w, int k, const float* host_x,
                           float* host_y) {
    if (!experts || !w || !host_x || !host_y) return set_error("null argument"), false;
    if (k <= 0 || k > kMaxSlots) return set_error("k=%d outside 1..%d", k, kMaxSlots), false;
    const eahmmf_hip_expert& e0 = experts[0];
    MoeShape s{};
    s.gate_type = e0.gate.type;
    s.up_type = e0.up.type;
    s.down_type = e0.down.type;
    s.D = e0.gate.ne0;
    s.FF = e0.gate.ne1;
    s.gate_rb = e0.gate.row_bytes;
    s.up_rb = e0.up.row_bytes;
    s.down_rb = e0.down.row_bytes;
    DecodeSlots slots{};
    slots.k = k;
    for (int j = 0; j < k; j++) {
        const eahmmf_hip_expert& e = experts[j];
        if (!weight_ok(e.gate) || !weight_ok(e.up) || !weight_ok(e.down))
            return set_error("expert slot %d: missing device pointer or unsupported type", j), false;
        if (e.gate.type != s.gate_type || e.up.type != s.up_type || e.down.type != s.down_type ||
            e.gate.ne0 != s.D || e.gate.ne1 != s.FF || e.up.ne0 != s.D || e.up.ne1 != s.FF || e.down.ne0 != s.FF ||
            e.down.ne1 != s.D || e.gate.row_bytes != s.gate_rb || e.up.row_bytes != s.up_rb ||
            e.down.row_bytes != s.down_rb)
            return set_error("expert slot %d: shape/type differs from slot 0", j), false;
        slots.gate[j] = e.gate.dev;
        slots.up[j] = e.up.dev;
        slots.down[j] = e.down.dev;
        slots.w[j] = w[j];
    }
    if (!moe_shape_ok(s)) return set_error("unsupported expert shape/type combination"), false;
    DevCtx* c = ctx_for_current_device();
    if (!c) return false;
    const size_t ybytes = (size_t)s.D * sizeof(float);
    const size_t flag_at = (ybytes + 255) & ~(size_t)255;  // the error word's pinned slot
    bool ok = grow_device(c->dy, ybytes) && grow_pinned(c->py, flag_at + 256) &&
              grow_device(c->dh, (size_t)k * s.FF * sizeof(float)) && stage_x(c, host_x, 1, s.D, s.D);
    bool fused = false;
    if (ok) {
        if (fused_enabled() && fused_supported(s, k, 0) && grow_fused(c, s, k)) {
            FusedArgsHost f;
            f.shape = s;
            f.k = k;
            f.mode = 0;
            f.direct = slots;
            f.x = (const float*)c->dx.p;
            f.y = (float*)c->dy.p;
            fused = true;
            ok = hip_ok(launch_moe_fused(f, c->fused, c->stream), "fused moe decode launch");
        } else {
            ok = hip_ok(launch_moe_decode(s, slots, (const float*)c->dx.p, (float*)c->dh.p, (float*)c->dy.p,
                                          c->stream), "moe decode launch");
        }
    }
    unsigned* flag = (unsigned*)((uint8_t*)c->py.p + flag_at);
    // y, and for a fused launch its error word into the staging next to y
    if (ok) *flag = 0;
    ok = finish_copies(c, ok, c->py.p, c->dy.p, ybytes, flag, c->dsync + kSyncFlagWord, fused ? sizeof(unsigned) : 0,
                       "copy y");
    if (!ok) return false;
    // also after a wait gave up: y then holds NaN where it is invalid, so a
    // caller that ignores the return value still cannot take it for a result
    memcpy(host_y, c->py.p, ybytes);
    return fused ? flag_ok(c, *flag, c->fused.epoch) : true;
}

bool eahmmf_hip_moe_decode_resident(const eahmmf_hip_expert* experts, const float* w, int k, const float* host_x,
                                    float* host_y, uint32_t* skipped_mask) {
    if (!experts || !w || !host_x || !host_y || !skipped_mask) return set_error("null argument"), false;
    if (k <= 0 || k > kMaxSlots) return set_error("k=%d outside 1..%d", k, kMaxSlots), false;
    // the device-resident slots, in slot order
    eahmmf_hip_expert res[kMaxSlots];
    float wr[kMaxSlots];
    int kr = 0;
    uint32_t skipped = 0;
    for (int j = 0; j < k; j++) {
        const eahmmf_hip_expert& e = experts[j];
        if (!e.gate.dev || !e.up.dev || !e.down.dev) {
            skipped |= 1u << j;
            continue;
        }
        res[kr] = e;
        wr[kr++] = w[j];
    }
    *skipped_mask = skipped;
    if (kr == 0) {  // nothing resident: the whole block is the caller's
        memset(host_y, 0, sizeof(float) * (size_t)experts[0].gate.ne0);
        return true;
    }
    return eahmmf_hip_moe_decode(res, wr, kr, host_x, host_y);
}

static bool shape_from_abi(const eahmmf_hip_moe_shape* sh, MoeShape& s) {
    if (!sh) return set_error("null shape"), false;
    s.gate_type = sh->gate_type;
    s.up_type = sh->up_type;
    s.down_type = sh->down_type;
    s.D = sh->D;
    s.FF = sh->FF;
    s.gate_rb = sh->gate_row_bytes;
    s.up_rb = sh->up_row_bytes;
    s.down_rb = sh->down_row_bytes;
    if (!moe_shape_ok(s)) return set_error("unsupported expert shape/type combination"), false;
    return true;
}

int eahmmf_hip_moe_decode_async(const eahmmf_hip_moe_shape* shape, const eahmmf_hip_expert_ptrs* experts,
                                const float* w, int k, const float* dev_x, float* dev_y, void* stream) {
    MoeShape s{};
    if (!shape_from_abi(shape, s)) return -1;
    if (!experts || !w || !dev_x || !dev_y) return set_error("null argument"), -1;
    if (k <= 0 || k > kMaxSlots) return set_error("k=%d outside 1..%d", k, kMaxSlots), -1;
    DecodeSlots slots{};
    slots.k = k;
    for (int j = 0; j < k; j++) {
        if (!experts[j].gate || !experts[j].up || !experts[j].down)
            return set_error("expert slot %d has a null pointer", j), -1;
        slots.gate[j] = experts[j].gate;
        slots.up[j] = experts[j].up;
        slots.down[j] = experts[j].down;
        slots.w[j] = w[j];
    }
    DevCtx* c = ctx_for_current_device();
    if (!c) return -2;
    if (!grow_device(c->dh, (size_t)k * s.FF * sizeof(float))) return -2;
    if (fused_enabled() && fused_supported(s, k, 0) && grow_fused(c, s, k)) {
        FusedArgsHost f;
        f.shape = s;
        f.k = k;
        f.mode = 0;
        f.direct = slots;
        f.x = dev_x;
        f.y = dev_y;
        return hip_ok(launch_moe_fused(f, c->fused, (hipStream_t)stream), "fused moe decode launch") ? 0 : -3;
    }
    if (!hip_ok(launch_moe_decode(s, slots, dev_x, (float*)c->dh.p, dev_y, (hipStream_t)stream), "moe decode launch"))
        return -3;
    return 0;
}

int eahmmf_hip_moe_decode_routed_async(const eahmmf_hip_moe_shape* shape, const eahmmf_hip_expert_ptrs* dev_table,
                                       int n_expert, const int* dev_ids, const float* dev_w, int k,
                                       const float* dev_x, float* dev_y, void* stream) {
    MoeShape s{};
    if (!shape_from_abi(shape, s)) return -1;
    if (!dev_table || !dev_ids || !dev_w || !dev_x || !dev_y || n_expert <= 0)
        return set_error("null argument"), -1;
    if (k <= 0 || k > kMaxSlots) return set_error("k=%d outside 1..%d", k, kMaxSlots), -1;
    DevCtx* c = ctx_for_current_device();
    if (!c) return -2;
    if (!grow_device(c->dh, (size_t)k * s.FF * sizeof(float))) return -2;
    if (fused_enabled() && fused_supported(s, k, 0) && grow_fused(c, s, k)) {
        FusedArgsHost f;
        f.shape = s;
        f.k = k;
        f.n_expert = n_expert;
        f.mode = 2;
        f.table = (const ExpertEntry*)dev_table;
        f.ids_in = dev_ids;
        f.w_in = dev_w;
        f.x = dev_x;
        f.y = dev_y;
        return hip_ok(launch_moe_fused(f, c->fused, (hipStream_t)stream), "fused routed moe decode launch") ? 0 : -3;
    }
    if (!hip_ok(launch_moe_decode_routed(s, (const ExpertEntry*)dev_table, n_expert, dev_ids, dev_w, k, dev_x,
                                         (float*)c->dh.p, dev_y, (hipStream_t)stream),
                "routed moe decode launch"))
        return -3;
    return 0;
}

int eahmmf_hip_moe_layer_decode_async(const eahmmf_hip_moe_shape* shape, const eahmmf_hip_expert_ptrs* dev_table,
                                      int n_expert, const float* dev_logits, int k, const float* dev_x, float* dev_y,
                                      int* dev_ids_out, float* dev_w_out, void* stream) {
    MoeShape s{};
    if (!shape_from_abi(shape, s)) return -1;
    if (!dev_table || !dev_logits || !dev_x || !dev_y) return set_error("null argument"), -1;
    if (n_expert <= 0 || n_expert > 512 || k <= 0 || k > kMaxSlots || k > n_expert)
        return set_error("bad routing shape n_expert=%d k=%d", n_expert, k), -1;
    DevCtx* c = ctx_for_current_device();
    if (!c) return -2;
    if (!grow_device(c->dh, (size_t)k * s.FF * sizeof(float))) return -2;
    hipStream_t st = (hipStream_t)stream;
    if (fused_enabled() && fused_supported(s, k, n_expert) && grow_fused(c, s, k)) {
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
        return hip_ok(launch_moe_fused(f, c->fused, st), "fused moe layer launch") ? 0 : -3;
    }
    // two-step path: routing kernel into scratch (or the caller's buffers), then the expert block
    int* ids = dev_ids_out;
    float* w = dev_w_out;
    if (!ids || !w) {
        if (!grow_device(c->dids, (size_t)k * sizeof(int)) || !grow_device(c->dw, (size_t)k * sizeof(float))) return -2;
        ids = (int*)c->dids.p;
        w = (float*)c->dw.p;
    }
    if (!hip_ok(launch_route_topk(dev_logits, 1, n_expert, k, ids, w, st), "route launch")) return -3;
    if (!hip_ok(launch_moe_decode_routed(s, (const ExpertEntry*)dev_table, n_expert, ids, w, k, dev_x,
                                         (float*)c->dh.p, dev_y, st),
                "routed moe decode launch"))
        return -3;
    return 0;
}

int eahmmf_hip_moe_layer_decode_xn_async(const eahmmf_hip_moe_shape* shape, const eahmmf_hip_expert_ptrs* dev_table,
                                         int n_expert, const float* dev_router, const float* dev_norm_w, float eps,
                                         const float* dev_x, int k, float* dev_y, int* dev_ids_out, float* dev_w_out,
                                         float* dev_xn_out, float* dev_logits_out, void* stream) {
    MoeShape s{};
    if (!shape_from_abi(shape, s)) return -1;
    if (!dev_table || !dev_router || !dev_x || !dev_y) return set_error("null argument"), -1;
    if (n_expert <= 0 || n_expert > 512 || k <= 0 || k > kMaxSlots || k > n_expert)
        return set_error("bad routing shape n_expert=%d k=%d", n_expert, k), -1;
    if (!gemv_supported(kF32, s.D, (size_t)s.D * 4)) return set_error("router: D=%d not supported", s.D), -1;
    DevCtx* c = ctx_for_current_device();
    if (!c) return -2;
    // one launch where the fused kernel takes the shape: the norm, the router
    // matmul (split over every workgroup) and the routing in the kernel
    if (fused_enabled() && fused_supported(s, k, n_expert) && grow_device(c->dh, (size_t)k * s.FF * sizeof(float)) &&
        grow_fused(c, s, k)) {
        FusedArgsHost f;
        f.shape = s;
        f.k = k;
        f.n_expert = n_expert;
        f.mode = 3;
        f.table = (const ExpertEntry*)dev_table;
        f.router = dev_router;
        f.norm_w = dev_norm_w;
        f.eps = eps;
        f.xn_out = dev_xn_out;
        f.logits_out = dev_logits_out;
        f.ids_out = dev_ids_out;
        f.w_out = dev_w_out;
        f.x = dev_x;
        f.y = dev_y;
        const hipError_t e = launch_moe_fused(f, c->fused, (hipStream_t)stream);
        if (e != hipErrorNotSupported) return hip_ok(e, "fused moe layer launch (router in the kernel)") ? 0 : -3;
    }
    float* xn = dev_xn_out;
    float* logits = dev_logits_out;
    if ((dev_norm_w && !xn) || !logits) {
        const size_t xn_floats = ((size_t)s.D + 63) & ~(size_t)63;
        if (!grow_device(c->drt, (xn_floats + (size_t)n_expert) * sizeof(float))) return -2;
        if (dev_norm_w && !xn) xn = (float*)c->drt.p;
        if (!logits) logits = (float*)c->drt.p + xn_floats;
    }
    // the router matmul over the (normalized) input; the kernel's block 0
    // also stores the normalized input the expert block reads
    GemvArgs g{};
    g.x = dev_x;
    g.norm_w = dev_norm_w;
    g.eps = eps;
    g.xn_out = dev_norm_w ? xn : nullptr;
    g.seg[0] = GemvSeg{reinterpret_cast<const uint8_t*>(dev_router), logits, nullptr, n_expert};
    g.nseg = 1;
    g.ne0 = s.D;
    g.rb = s.D * 4;
    if (!hip_ok(launch_gemv(kF32, g, (hipStream_t)stream), "router launch")) return -3;
    return eahmmf_hip_moe_layer_decode_async(shape, dev_table, n_expert, logits, k, dev_norm_w ? xn : dev_x, dev_y,
                                             dev_ids_out, dev_w_out, stream);
}

int eahmmf_hip_moe_grouped_async(const eahmmf_hip_moe_shape* shape, const eahmmf_hip_expert_ptrs* dev_table,
                                 int n_expert, const int* dev_ids, const float* dev_w, int nb, int k,
                                 const float* dev_x, float* dev_y, void* stream) {
    MoeShape s{};
    if (!shape_from_abi(shape, s)) return -1;
    if (!dev_table || !dev_ids || !dev_w || !dev_x || !dev_y) return set_error("null argument"), -1;
    if (!grouped_supported(s, nb, k, n_expert))
        return set_error("unsupported grouped shape: nb=%d k=%d n_expert=%d D=%d FF=%d", nb, k, n_expert, s.D, s.FF),
               -1;
    DevCtx* c = ctx_for_current_device();
    if (!c) return -2;
    // A decode batch of up to three sequences runs as one fused launch per
    // token (ids and weights as given): the grouped block's fixed cost
    // (grouping, activation levels, three more launches) outweighs the shared
    // expert reads below four tokens.  Measured at D=4096/FF=1536, top-8 of
    // 128, routing included: 1 / 2 / 4 / 8 / 16 / 32 tokens take 0.043 /
    // 0.075 / 0.139 / 0.267 / 0.507 / 1.0 ms as per-token launches and
    // 0.100 / 0.117 / 0.136 / 0.190 / 0.309 / 0.525 ms as the grouped block.
    if (nb <= kFusedBatchMax && fused_enabled() && fused_supported(s, k, 0)) {
        if (!grow_fused(c, s, k)) return -2;
        for (int t = 0; t < nb; t++) {
            FusedArgsHost f;
            f.shape = s;
            f.k = k;
            f.n_expert = n_expert;
            f.mode = 2;
            f.table = (const ExpertEntry*)dev_table;
            f.ids_in = dev_ids + (size_t)t * k;
            f.w_in = dev_w + (size_t)t * k;
            f.x = dev_x + (size_t)t * s.D;
            f.y = dev_y + (size_t)t * s.D;
            if (!hip_ok(launch_moe_fused(f, c->fused, (hipStream_t)stream), "fused batch-decode launch")) return -3;
        }
        return 0;
    }
    if (!grow_device(c->dgs, grouped_scratch_bytes(s, nb, k, n_expert))) return -2;
    return hip_ok(launch_moe_grouped(s, (const ExpertEntry*)dev_table, n_expert, dev_ids, dev_w, nb, k, dev_x, s.D,
                                     dev_y, s.D, c->dgs.p, (hipStream_t)stream),
                  "grouped moe launch")
               ? 0
               : -3;
}

bool eahmmf_hip_moe_grouped(const eahmmf_hip_expert* experts, int n_groups, const int* group_offsets,
                            const int* tokens, const float* weights, int nb, const float* host_x, float* host_y) {
    if (!experts || !group_offsets || !tokens || !weights || !host_x || !host_y)
        return set_error("null argument"), false;
    if (n_groups <= 0 || nb <= 0) return set_error("n_groups=%d nb=%d", n_groups, nb), false;
    const eahmmf_hip_expert& e0 = experts[0];
    if (!weight_ok(e0.gate) || !weight_ok(e0.up) || !weight_ok(e0.down))
        return set_error("group 0: missing device pointer or unsupported type"), false;
    MoeShape s{e0.gate.type, e0.up.type, e0.down.type, e0.gate.ne0, e0.gate.ne1,
               e0.gate.row_bytes, e0.up.row_bytes, e0.down.row_bytes};
    std::vector<ExpertEntry> table((size_t)n_groups);
    for (int g = 0; g < n_groups; g++) {
        const eahmmf_hip_expert& e = experts[g];
        if (!weight_ok(e.gate) || !weight_ok(e.up) || !weight_ok(e.down))
            return set_error("group %d: missing device pointer or unsupported type", g), false;
        if (e.gate.type != s.gate_type || e.up.type != s.up_type || e.down.type != s.down_type ||
            e.gate.ne0 != s.D || e.gate.ne1 != s.FF || e.up.ne0 != s.D || e.up.ne1 != s.FF || e.down.ne0 != s.FF ||
            e.down.ne1 != s.D || e.gate.row_bytes != s.gate_rb || e.up.row_bytes != s.up_rb ||
            e.down.row_bytes != s.down_rb)
            return set_error("group %d: shape/type differs from group 0", g), false;
        table[g] = ExpertEntry{e.gate.dev, e.up.dev, e.down.dev};
        if (group_offsets[g + 1] < group_offsets[g]) return set_error("group_offsets not ascending"), false;
    }
    if (group_offsets[0] != 0) return set_error("group_offsets[0] must be 0"), false;
    // per token: its groups in ascending order (the lists are per group, in token order)
    std::vector<int> per_tok((size_t)nb, 0);
    for (int g = 0; g < n_groups; g++)
        for (int i = group_offsets[g]; i < group_offsets[g + 1]; i++) {
            const int t = tokens[i];
            if (t < 0 || t >= nb) return set_error("token %d of group %d outside 0..%d", t, g, nb - 1), false;
            per_tok[t]++;
        }
    int k = 0;
    for (int t = 0; t < nb; t++) k = per_tok[t] > k ? per_tok[t] : k;
    if (k <= 0 || k > kMaxSlots) return set_error("a token appears in %d groups (1..%d supported)", k, kMaxSlots), false;
    if (!grouped_supported(s, nb, k, n_groups))
        return set_error("unsupported grouped shape: nb=%d k=%d groups=%d", nb, k, n_groups), false;
    std::vector<int> ids((size_t)nb * k, -1);
    std::vector<float> w((size_t)nb * k, 0.f);
    std::fill(per_tok.begin(), per_tok.end(), 0);
    for (int g = 0; g < n_groups; g++)
        for (int i = group_offsets[g]; i < group_offsets[g + 1]; i++) {
            const int t = tokens[i];
            const int j = per_tok[t]++;
            ids[(size_t)t * k + j] = g;
            w[(size_t)t * k + j] = weights[i];
        }
    DevCtx* c = ctx_for_current_device();
    if (!c) return false;
    const size_t xb = (size_t)nb * s.D * sizeof(float), tb = table.size() * sizeof(ExpertEntry);
    const size_t ib = ids.size() * sizeof(int), wb = w.size() * sizeof(float);
    bool ok = grow_device(c->dtab, tb + ib + wb) && grow_device(c->dgs, grouped_scratch_bytes(s, nb, k, n_groups)) &&
              grow_device(c->dy, xb) && grow_pinned(c->py, xb) && stage_x(c, host_x, nb, s.D, s.D);
    if (ok) {
        uint8_t* d = (uint8_t*)c->dtab.p;
        ok = hip_ok(hipMemcpyAsync(d, table.data(), tb, hipMemcpyHostToDevice, c->stream), "h2d table") &&
             hip_ok(hipMemcpyAsync(d + tb, ids.data(), ib, hipMemcpyHostToDevice, c->stream), "h2d ids") &&
             hip_ok(hipMemcpyAsync(d + tb + ib, w.data(), wb, hipMemcpyHostToDevice, c->stream), "h2d w") &&
             hip_ok(launch_moe_grouped(s, (const ExpertEntry*)d, n_groups, (const int*)(d + tb),
                                       (const float*)(d + tb + ib), nb, k, (const float*)c->dx.p, s.D,
                                       (float*)c->dy.p, s.D, c->dgs.p, c->stream),
                    "grouped moe launch") &&
             hip_ok(hipMemcpyAsync(c->py.p, c->dy.p, xb, hipMemcpyDeviceToHost, c->stream), "d2h y");
    }
    if (!drain(c, ok)) return false;
    memcpy(host_y, c->py.p, xb);
    return true;
}

int eahmmf_hip_set_grouped_mfma(int enable) { return set_grouped_mfma(enable); }

int eahmmf_hip_set_grouped_wave_max(int max_tokens) { return set_grouped_wave_max(max_tokens); }

int eahmmf_hip_set_grouped_dot_max(int max_tokens) { return set_grouped_dot_max(max_tokens); }

int eahmmf_hip_set_dense_mfma(int on) { return set_dense_mfma(on); }

int eahmmf_hip_set_fused(int enable) {
    const int prev = fused_enabled() ? 1 : 0;
    if (enable >= 0) g_fused = enable ? 1 : 0;
    return prev;
}

int eahmmf_hip_fused_exchange(void) {
    int dev = 0;
    if (!hip_ok(hipGetDevice(&dev), "get device")) return -1;
    return fused_exchange_mode(dev);
}

int eahmmf_hip_device_flags(void) {
    DevCtx* c = ctx_for_current_device();
    if (!c) return -2;
    if (!hip_ok(hipStreamSynchronize(c->stream), "sync")) return -2;
    if (!hip_ok(hipDeviceSynchronize(), "device sync")) return -2;
    unsigned v = 0;
    if (!hip_ok(hipMemcpy(&v, c->dsync + kSyncFlagWord, sizeof v, hipMemcpyDeviceToHost), "read device flags"))
        return -2;
    if (v) {
        (void)reset_fused_sync(c->fused, c->stream, true);
        (void)hipStreamSynchronize(c->stream);
    }
    const int na = noalloc_device_flags();
    if (na < 0) return set_error("reading the no-allocation scratch's error word failed"), -2;
    return (v || na) ? 1 : 0;
}

int eahmmf_hip_fused_status_async(unsigned* dst, void* stream) {
    if (!dst) return set_error("null argument"), -1;
    DevCtx* c = ctx_for_current_device();
    if (!c) return -2;
    return hip_ok(hipMemcpyAsync(dst, c->dsync + kSyncFlagWord, sizeof(unsigned), hipMemcpyDefault,
                                 (hipStream_t)stream),
                  "hipMemcpyAsync(error word)")
               ? 0
               : -3;
}

void eahmmf_hip_set_fault_injection(unsigned spin_limit, int drop_partition) {
    set_fused_fault_injection(spin_limit, drop_partition);
}

bool eahmmf_hip_route_topk(const float* host_logits, int nb, int n_expert, int k, int* host_ids, float* host_w) {
    if (!host_logits || !host_ids || !host_w) return set_error("null argument"), false;
    if (nb <= 0 || n_expert <= 0 || n_expert > 512 || k <= 0 || k > kMaxSlots || k > n_expert)
        return set_error("bad routing shape nb=%d n_expert=%d k=%d", nb, n_expert, k), false;
    DevCtx* c = ctx_for_current_device();
    if (!c) return false;
    const size_t out = (size_t)nb * k;
    bool ok = grow_device(c->dids, out * sizeof(int)) && grow_device(c->dw, out * sizeof(float)) &&
              grow_pinned(c->py, out * sizeof(int)) && grow_pinned(c->py2, out * sizeof(float)) &&
              stage_x(c, host_logits, nb, n_expert, n_expert);
    if (ok) ok = hip_ok(launch_route_topk((const float*)c->dx.p, nb, n_expert, k, (int*)c->dids.p, (float*)c->dw.p,
                                          c->stream), "route launch");
    if (ok) ok = hip_ok(hipMemcpyAsync(c->py.p, c->dids.p, out * sizeof(int), hipMemcpyDeviceToHost, c->stream), "copy ids");
    if (ok) ok = hip_ok(hipMemcpyAsync(c->py2.p, c->dw.p, out * sizeof(float), hipMemcpyDeviceToHost, c->stream), "copy w");
    ok = drain(c, ok);
    if (ok) {
        memcpy(host_ids, c->py.p, out * sizeof(int));
        memcpy(host_w, c->py2.p, out * sizeof(float));
    }
    return ok;
}

int eahmmf_hip_route_topk_async(const float* dev_logits, int nb, int n_expert, int k, int* dev_ids, float* dev_w,
                                void* stream) {
    if (!dev_logits || !dev_ids || !dev_w) return set_error("null argument"), -1;
    const hipError_t e = launch_route_topk(dev_logits, nb, n_expert, k, dev_ids, dev_w, (hipStream_t)stream);
    if (e == hipErrorInvalidValue) return set_error("bad routing shape nb=%d n_expert=%d k=%d", nb, n_expert, k), -1;
    return hip_ok(e, "route launch") ? 0 : -3;
}

int eahmmf_hip_expf_ref_async(const float* dev_x, float* dev_y, int64_t n, void* stream) {
    const hipError_t e = launch_expf_ref(dev_x, dev_y, n, (hipStream_t)stream);
    if (e == hipErrorInvalidValue) return set_error("null buffer or negative n"), -1;
    return hip_ok(e, "expf launch") ? 0 : -3;
}

int eahmmf_hip_stream_read_async(const void* dev_buf, size_t bytes, uint32_t* dev_sink, void* stream) {
    if (bytes == 0) return 0;
    if (!dev_buf || !dev_sink) return set_error("null argument"), -1;
    const hipError_t e = launch_stream_read(dev_buf, bytes, dev_sink, (hipStream_t)stream);
    if (e == hipErrorInvalidValue)
        return set_error("stream read needs a 16-byte aligned buffer and a multiple of 16 bytes (got %zu)", bytes), -1;
    return hip_ok(e, "stream read launch") ? 0 : -3;
}

int eahmmf_hip_dequantize(const uint8_t* dev_w, int type, int64_t ne0, int64_t nrows, size_t row_bytes,
                          float* dev_out, void* stream) {
    if (!dev_w || !dev_out || nrows < 0) return set_error("null argument"), -1;
    if (!(type_supported(type) || type == kF32)) return set_error("unsupported ggml type %d", type), -1;
    if (ne0 <= 0 || ne0 % type_blck(type)) return set_error("bad row length %lld", (long long)ne0), -1;
    if (row_bytes != (size_t)(ne0 / type_blck(type)) * type_bytes(type)) return set_error("row_bytes mismatch"), -1;
    return hip_ok(launch_dequant(type, dev_w, ne0, nrows, row_bytes, dev_out, (hipStream_t)stream), "dequant launch")
               ? 0
               : -3;
}

int eahmmf_hip_alloc(void** dev_ptr, size_t bytes) {
    if (!dev_ptr) return set_error("null argument"), -1;
    *dev_ptr = nullptr;
    return hip_ok(hipMalloc(dev_ptr, bytes), "hipMalloc") ? 0 : -2;
}

int eahmmf_hip_free(void* dev_ptr) { return hip_ok(hipFree(dev_ptr), "hipFree") ? 0 : -2; }

int eahmmf_hip_h2d(void* dev_dst, const void* host_src, size_t n) {
    DevCtx* c = ctx_for_current_device();
    if (!c) return -2;
    return hip_ok(hipMemcpyAsync(dev_dst, host_src, n, hipMemcpyHostToDevice, c->stream), "h2d") ? 0 : -2;
}

int eahmmf_hip_d2h(void* host_dst, const void* dev_src, size_t n) {
    DevCtx* c = ctx_for_current_device();
    if (!c) return -2;
    bool ok = hip_ok(hipMemcpyAsync(host_dst, dev_src, n, hipMemcpyDeviceToHost, c->stream), "d2h");
    return drain(c, ok) ? 0 : -2;
}

int eahmmf_hip_sync(void) {
    DevCtx* c = ctx_for_current_device();
    if (!c) return -2;
    return drain(c, true) ? 0 : -2;
}

int eahmmf_hip_mem_info(size_t* free_bytes, size_t* total_bytes) {
    size_t f = 0, t = 0;
    if (!hip_ok(hipMemGetInfo(&f, &t), "hipMemGetInfo")) return -2;
    if (free_bytes) *free_bytes = f;
    if (total_bytes) *total_bytes = t;
    return 0;
}

int eahmmf_hip_h2d_batch(const eahmmf_hip_copy* copies, int n) {
    if (!copies_ok(copies, n)) return -1;
    if (n == 0) return 0;
    DevCtx* c = ctx_for_current_device();
    if (!c) return -2;
    // work already queued on the library's stream finishes first
    if (!drain(c, true)) return -2;
    uint64_t ticket = 0;
    const int r = eahmmf_hip_h2d_batch_async(copies, n, &ticket);
    return r != 0 ? r : eahmmf_hip_h2d_batch_wait(ticket, nullptr);
}

int eahmmf_hip_h2d_batch_async(const eahmmf_hip_copy* copies, int n, uint64_t* ticket) {
    if (!ticket) return set_error("null ticket"), -1;
    if (!copies_ok(copies, n)) return -1;
    DevCtx* c = ctx_for_current_device();
    if (!c) return -2;
    Stager* st = stager_for(c);
    if (!st) return -2;
    std::lock_guard<std::mutex> lk(st->qmu);
    retire_done(st);
    const uint64_t id = st->next++;
    st->q.emplace_back(id, std::vector<eahmmf_hip_copy>(copies, copies + n));
    st->qcv.notify_all();
    *ticket = id;
    return 0;
}

int eahmmf_hip_h2d_batch_wait(uint64_t ticket, void* stream) {
    int dev = 0;
    if (!hip_ok(hipGetDevice(&dev), "hipGetDevice")) return -2;
    Stager* st = dev >= 0 && dev < kMaxDev ? g_stager[dev] : nullptr;
    if (!st || ticket == 0) return set_error("unknown staging ticket"), -1;
    std::unique_lock<std::mutex> lk(st->qmu);
    if (ticket >= st->next) return set_error("unknown staging ticket"), -1;
    st->dcv.wait(lk, [&] { return st->issued >= ticket; });
    auto f = st->failed.find(ticket);
    if (f != st->failed.end()) return set_error("staging batch %llu: %s", (unsigned long long)ticket, f->second.c_str()), -2;
    auto e = st->ev.find(ticket);
    if (e == st->ev.end()) return 0;  // landed and retired
    // held under the lock: the event is not retired meanwhile
    const hipError_t r = stream ? hipStreamWaitEvent((hipStream_t)stream, e->second, 0) : hipEventSynchronize(e->second);
    return hip_ok(r, "staging wait") ? 0 : -2;
}

int eahmmf_hip_h2d_batch_query(uint64_t ticket) {
    int dev = 0;
    if (!hip_ok(hipGetDevice(&dev), "hipGetDevice")) return -2;
    Stager* st = dev >= 0 && dev < kMaxDev ? g_stager[dev] : nullptr;
    if (!st || ticket == 0) return set_error("unknown staging ticket"), -1;
    std::lock_guard<std::mutex> lk(st->qmu);
    if (ticket >= st->next) return set_error("unknown staging ticket"), -1;
    if (st->issued < ticket) return 0;
    auto f = st->failed.find(ticket);
    if (f != st->failed.end()) return set_error("staging batch %llu: %s", (unsigned long long)ticket, f->second.c_str()), -2;
    auto e = st->ev.find(ticket);
    if (e == st->ev.end()) return 1;
    const hipError_t r = hipEventQuery(e->second);
    if (r == hipSuccess) return 1;
    if (r == hipErrorNotReady) return 0;
    return hip_ok(r, "staging query") ? 0 : -2;
}

void eahmmf_hip_shutdown(void) {
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess) return;
    stop_stager(dev);
    std::lock_guard<std::mutex> g(g_mu);
    auto it = g_ctx.find(dev);
    if (it == g_ctx.end()) return;
    DevCtx& c = it->second;
    if (c.stream) (void)hipStreamSynchronize(c.stream);
    for (DeviceBuf* b : {&c.dx, &c.dy, &c.dy2, &c.dh, &c.dids, &c.dw, &c.dyp, &c.dhx, &c.dgs, &c.dtab, &c.drt, &c.dws})
        if (b->p) (void)hipFree(b->p);
    for (DeviceBuf* b : {&c.px, &c.py, &c.py2})
        if (b->p) (void)hipHostFree(b->p);
    if (c.hflag) (void)hipHostFree(c.hflag);
    if (c.dsync) (void)hipFree(c.dsync);
    for (int s = 0; s < kRingSlots; s++) {
        if (c.copy_stream[s]) (void)hipStreamSynchronize(c.copy_stream[s]);
        if (c.ring[s]) (void)hipHostFree(c.ring[s]);
        if (c.ring_done[s]) (void)hipEventDestroy(c.ring_done[s]);
        if (c.copy_stream[s]) (void)hipStreamDestroy(c.copy_stream[s]);
    }
    if (c.stream) (void)hipStreamDestroy(c.stream);
    if (dev >= 0 && dev < kMaxDev && g_stager[dev] && g_stager[dev]->join) {
        (void)hipStreamDestroy(g_stager[dev]->join);
        g_stager[dev]->join = nullptr;
    }
    g_ctx.erase(it);
}

}  // extern "C"
