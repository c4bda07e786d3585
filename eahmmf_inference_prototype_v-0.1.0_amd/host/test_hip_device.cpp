// test_hip_device.cpp - C++ host check of HipDevice and of the expert-store
// calling pattern on one GPU, through libeahmmf_hip.so only.
//
// 1. HipDevice keeps the DeviceBackend contract of the reference's CudaDevice
//    (eahmmf.h:150-200): a round trip through h2d/sync/d2h is exact, a failed
//    allocation returns nullptr and leaves the device usable, memory figures
//    are consistent.
// 2. Experts staged through HipDevice (as ExpertStore does for VRAM-resident
//    experts, eahmmf.h:923-1032) feed the single-call expert block, whose
//    result matches the reference's per-expert sequence rebuilt from the same
//    library's drop-in calls: gate/up pair, SiLU on the host, down, weighted
//    sum in ascending expert order (qwen3moe.cpp:1024-1067).
// Exit status 0 when every check passes; every failure is printed.
#include <math.h>
#include <stdio.h>
#include <string.h>

#include <random>
#include <vector>

#include "hip_device.h"

static int g_fail = 0;
#define CHECK(c)                                                      \
    do {                                                              \
        if (!(c)) {                                                   \
            fprintf(stderr, "FAILED %s:%d: %s\n", __FILE__, __LINE__, #c); \
            g_fail++;                                                 \
        }                                                             \
    } while (0)

static void check_device(eahmmf_hip::HipDevice& dev) {
    CHECK(strcmp(dev.name(), "hip") == 0);
    CHECK(!dev.cpu_readable());
    const size_t fr = dev.free_memory();
    CHECK(dev.total_memory() > 0);
    CHECK(fr > 0);
    const size_t n = (1u << 20) + 12;  // not a multiple of the page or copy granule
    std::vector<uint8_t> src(n), back(n, 0);
    for (size_t i = 0; i < n; i++) src[i] = (uint8_t)(i * 131u + 7u);
    void* p = dev.alloc(n);
    CHECK(p != nullptr);
    if (p) {
        CHECK(dev.h2d(p, src.data(), n));
        CHECK(dev.sync());
        CHECK(dev.d2h(back.data(), p, n));
        CHECK(memcmp(src.data(), back.data(), n) == 0);
        dev.release(p, n);
    }
    // far beyond any device: nullptr, and the device keeps working
    void* huge = dev.alloc((size_t)1 << 52);
    CHECK(huge == nullptr);
    void* q = dev.alloc(4096);
    CHECK(q != nullptr);
    dev.release(q, 4096);
    CHECK(dev.sync());
}

static bool close_enough(const std::vector<float>& got, const std::vector<float>& want) {
    for (size_t i = 0; i < got.size(); i++) {
        const double err = fabs((double)got[i] - (double)want[i]);
        if (!(err <= 1e-4 + 1e-3 * fabs((double)want[i]))) {
            fprintf(stderr, "mismatch at %zu: %g vs %g\n", i, got[i], want[i]);
            return false;
        }
    }
    return true;
}

static void check_expert_block(eahmmf_hip::HipDevice& dev, int D, int FF, int k, int gt, int dt) {
    std::mt19937 rng(1234u + (unsigned)(D + FF + k));
    std::normal_distribution<float> nd(0.f, 0.02f), nx(0.f, 1.f);
    const size_t grb = eahmmf_hip_row_bytes(gt, D), drb = eahmmf_hip_row_bytes(dt, FF);
    CHECK(grb > 0 && drb > 0);
    std::vector<eahmmf_hip_expert> ex(k);
    std::vector<void*> owned;
    auto stage = [&](int type, int rows, int ne0, size_t rb) -> const uint8_t* {
        std::vector<float> w((size_t)rows * ne0);
        for (auto& v : w) v = nd(rng);
        std::vector<uint8_t> q(rb * rows);
        CHECK(eahmmf_hip_quantize_rows(type, w.data(), rows, ne0, q.data()) == (int64_t)q.size());
        void* p = dev.alloc(q.size());
        CHECK(p != nullptr);
        if (p) CHECK(dev.h2d(p, q.data(), q.size()));
        owned.push_back(p);
        return (const uint8_t*)p;
    };
    for (int j = 0; j < k; j++) {
        ex[j].gate = {stage(gt, FF, D, grb), gt, D, FF, grb};
        ex[j].up = {stage(gt, FF, D, grb), gt, D, FF, grb};
        ex[j].down = {stage(dt, D, FF, drb), dt, FF, D, drb};
    }
    CHECK(dev.sync());  // the staged experts are valid for compute
    std::vector<float> x(D), w(k), y(D, 0.f), want(D, 0.f);
    for (auto& v : x) v = nx(rng);
    float tot = 0.f;
    for (int j = 0; j < k; j++) tot += (w[j] = 1.0f + (float)j);
    for (auto& v : w) v /= tot;
    if (!eahmmf_hip_moe_decode(ex.data(), w.data(), k, x.data(), y.data())) {
        fprintf(stderr, "FAILED eahmmf_hip_moe_decode D=%d FF=%d k=%d: %s\n", D, FF, k, eahmmf_hip_last_error());
        g_fail++;
    }
    // the reference's sequence of calls, through the drop-in entry points
    std::vector<float> g(FF), u(FF), yd(D);
    for (int j = 0; j < k; j++) {
        CHECK(eahmmf_hip_matmul_pair(ex[j].gate.dev, gt, D, FF, grb, ex[j].up.dev, gt, D, FF, grb, x.data(), 1, D,
                                     g.data(), FF, u.data(), FF));
        for (int i = 0; i < FF; i++) g[i] = g[i] / (1.0f + expf(-g[i])) * u[i];
        CHECK(eahmmf_hip_matmul(ex[j].down.dev, dt, FF, D, drb, g.data(), 1, FF, yd.data(), D));
        for (int r = 0; r < D; r++) want[r] += w[j] * yd[r];
    }
    if (!close_enough(y, want)) {
        fprintf(stderr, "expert block D=%d FF=%d k=%d differs from the per-expert calls\n", D, FF, k);
        g_fail++;
    }
    for (void* p : owned) dev.release(p, 0);
}

// Bulk staging (h2d_batch): copies of assorted sizes - one byte, unaligned,
// exactly one 32 MiB ring slot, more than one slot, empty, and the C2 expert
// components - land byte for byte; a second batch reuses the ring.
static void check_batch(eahmmf_hip::HipDevice& dev) {
    std::mt19937 rng(99u);
    const size_t sizes[] = {1, 4097, (size_t)32 << 20, ((size_t)40 << 20) + 123, 0, 884736, 1290240, 884736};
    const int n = (int)(sizeof sizes / sizeof sizes[0]);
    std::vector<std::vector<uint8_t>> host(n);
    std::vector<void*> ptrs(n, nullptr);
    std::vector<eahmmf_hip_copy> cp(n);
    for (int round = 0; round < 2; round++) {
        for (int i = 0; i < n; i++) {
            host[i].resize(sizes[i]);
            for (auto& b : host[i]) b = (uint8_t)rng();
            if (round == 0 && sizes[i]) {
                ptrs[i] = dev.alloc(sizes[i]);
                CHECK(ptrs[i] != nullptr);
            }
            cp[i] = eahmmf_hip_copy{ptrs[i], host[i].data(), sizes[i]};
        }
        CHECK(dev.h2d_batch(cp.data(), n));
        for (int i = 0; i < n; i++) {
            if (!sizes[i] || !ptrs[i]) continue;
            std::vector<uint8_t> back(sizes[i]);
            CHECK(dev.d2h(back.data(), ptrs[i], sizes[i]));
            CHECK(back == host[i]);
        }
    }
    CHECK(eahmmf_hip_h2d_batch(nullptr, 1) == -1);
    CHECK(eahmmf_hip_h2d_batch(cp.data(), 0) == 0);
    // the asynchronous form: both halves queued at once, then waited for
    for (int i = 0; i < n; i++)
        for (auto& b : host[i]) b = (uint8_t)rng();
    const uint64_t t0 = dev.h2d_batch_async(cp.data(), n / 2);
    const uint64_t t1 = dev.h2d_batch_async(cp.data() + n / 2, n - n / 2);
    CHECK(t0 != 0 && t1 > t0);
    CHECK(dev.h2d_batch_wait(t1));
    CHECK(dev.h2d_batch_wait(t0));
    CHECK(eahmmf_hip_h2d_batch_query(t0) == 1 && eahmmf_hip_h2d_batch_query(t1) == 1);
    for (int i = 0; i < n; i++) {
        if (!sizes[i] || !ptrs[i]) continue;
        std::vector<uint8_t> back(sizes[i]);
        CHECK(dev.d2h(back.data(), ptrs[i], sizes[i]));
        CHECK(back == host[i]);
    }
    for (void* p : ptrs)
        if (p) dev.release(p, 0);
}

int main() {
    if (eahmmf_hip_device_count() < 1) {
        fprintf(stderr, "no HIP device\n");
        return 2;
    }
    eahmmf_hip::HipDevice dev;
    check_device(dev);
    // error contract of the drop-in call: false, never an abort
    float o[4];
    CHECK(!eahmmf_hip_matmul(nullptr, 12, 256, 4, 144, o, 1, 256, o, 4));
    check_expert_block(dev, 512, 256, 2, 12, 14);    // Q4_K gate/up, Q6_K down
    check_expert_block(dev, 2048, 768, 8, 12, 14);   // Qwen3-30B-A3B expert shape, top-8
    check_expert_block(dev, 1024, 512, 4, 8, 8);     // Q8_0 throughout
    check_batch(dev);
    eahmmf_hip_shutdown();
    if (g_fail) {
        fprintf(stderr, "%d check(s) failed\n", g_fail);
        return 1;
    }
    printf("test_hip_device: all checks passed\n");
    return 0;
}
