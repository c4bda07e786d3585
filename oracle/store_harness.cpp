// store_harness.cpp - the reference's expert store and engine with HipDevice
// (libeahmmf_hip.so) as their device backend, on one GPU.
//
// TEST INFRASTRUCTURE.  This file is ours; it compiles the reference's own
// qwen3moe.cpp (and through it eahmmf.h) in place with QWEN3MOE_NO_MAIN, as
// ref_harness.cpp does, and links the library.  The binary goes to
// oracle/_ref/ only; nothing of the reference is copied.
//
// What it checks (run with a tiny qwen3moe GGUF as argv[1]):
//  A. HipDeviceOn<eahmmf::DeviceBackend> compiles against the reference's
//     DeviceBackend (eahmmf.h:88-100) and serves as the store's device.
//  B. Tier matrix (the reference's own acceptance rule, its
//     tests/test_eahmmf.cpp section 3): prompt logits, greedy tokens, routing
//     ids and weights bitwise identical to the SSD-tier run, for VRAM tiers
//     with unlimited, 2-, 1- and sub-1-expert budgets, RAM budgets that force
//     every pager path, and gpu_compute views; store invariants hold, no pin
//     and no device allocation leaks.
//  C. A residency walk SSD -> RAM -> VRAM -> RAM -> SSD with the bytes the
//     store serves equal to the file's at every step (device copies read
//     back through HipDevice::d2h).
//  D. Pinned experts are not evicted; a full VRAM pool of pinned experts
//     degrades to RAM service, or refuses in strict mode.
//  E. The dispatch of qwen3moe.cpp:471-525 over the HIP ABI
//     (host/expert_dispatch.h): VRAM-served views go to the GPU (pair for
//     gate/up unless EAHMMF_DISABLE_PAIR), the rest to the reference's CPU
//     matmul, and every GPU result passes the reference's shadow criterion
//     (max|cpu - gpu| / max(max|cpu|, 1e-3) < 1e-4) against that matmul.
//  F. The single-call expert block (eahmmf_hip_moe_decode) over leased views
//     against the reference's own expert loop (matmuls, SiLU, weighted sum).
//  G. Partial residency: with VRAM for two experts, all of a layer's experts
//     leased at once; eahmmf_hip_moe_decode_resident computes the resident
//     subset and reports the rest, which the host adds on the CPU; the sum
//     matches the all-CPU block.
#define QWEN3MOE_NO_MAIN
#include REF_SRC

#include "expert_dispatch.h"
#include "hip_device.h"

using namespace eahmmf;

static int g_fail = 0, g_checks = 0;
#define CHECK(c, ...)                                                      \
    do {                                                                   \
        g_checks++;                                                        \
        if (!(c)) {                                                        \
            g_fail++;                                                      \
            fprintf(stderr, "  FAIL %s:%d: %s  ", __FILE__, __LINE__, #c); \
            fprintf(stderr, " " __VA_ARGS__);                              \
            fprintf(stderr, "\n");                                         \
        }                                                                  \
    } while (0)

// HipDevice with its live allocations counted, so that leaks show.
struct CountedHip : eahmmf_hip::HipDeviceOn<eahmmf::DeviceBackend> {
    size_t* live;
    explicit CountedHip(size_t* l) : live(l) {}
    void* alloc(size_t n) override {
        void* p = HipDeviceOn::alloc(n);
        if (p) *live += n;
        return p;
    }
    void release(void* p, size_t n) override {
        if (p) *live -= n;
        HipDeviceOn::release(p, n);
    }
};

static const std::vector<int> kPrompt = {3, 99, 250, 7, 42, 123, 8, 64, 200, 1, 77, 15};

struct Run {
    std::vector<float> logits;
    std::vector<int> gen, ids;
    std::vector<float> w;
};
static bool bitwise_equal(const Run& a, const Run& b) {
    return a.logits.size() == b.logits.size() && !memcmp(a.logits.data(), b.logits.data(), 4 * a.logits.size()) &&
           a.gen == b.gen && a.ids == b.ids && a.w.size() == b.w.size() &&
           !memcmp(a.w.data(), b.w.data(), 4 * a.w.size());
}
// prompt in batches of 4, then 10 greedy tokens, routing traced
static Run infer(Engine& E) {
    Run r;
    E.trace_routing = true;
    E.trace_ids.clear();
    E.trace_w.clear();
    r.logits.resize(E.n_vocab);
    E.eval(kPrompt, 0, 4, r.logits.data());
    std::vector<float> lg = r.logits;
    int pos = (int)kPrompt.size();
    for (int i = 0; i < 10; i++) {
        int t = (int)(std::max_element(lg.begin(), lg.end()) - lg.begin());
        r.gen.push_back(t);
        E.forward(&t, 1, pos++, lg.data());
    }
    r.ids = E.trace_ids;
    r.w = E.trace_w;
    E.trace_routing = false;
    return r;
}

static Config tier(Residency t, size_t ram, size_t vram, bool verify, bool gpu_compute = false) {
    Config c;
    c.exec_tier = t;
    c.ram_budget = ram;
    c.vram_budget = vram;
    c.verify = verify;
    c.gpu_compute = gpu_compute;
    return c;
}

static bool served_bytes_match_file(Engine& E, int l, int x, Residency* from) {
    ExpertLease lease = E.store->acquire_lease(l, x);
    if (!lease) return false;
    const ExpertViews& v = lease.views();
    const ExpertDescriptor& d = E.store->descriptor(l, x);
    const WeightView* w[3] = {&v.gate, &v.up, &v.down};
    bool ok = true;
    for (int c = 0; c < 3; c++) ok &= !memcmp(w[c]->data, E.g.map + d.slice[c].file_offset, d.bytes[c]);
    if (from) *from = v.served_from;
    return ok;
}

// The reference's CPU kernel as the dispatch's fallback and shadow.
static void cpu_matmul(const WeightView& W, const float* x, int nb, int ldx, float* out, int ldo) {
    matmul(W, x, nb, ldx, out, ldo);
}

// The reference's expert loop body for one token over given views
// (qwen3moe.cpp:1034-1067): gate/up, SiLU, down, y += w * down(h).
static void cpu_expert_block(const std::vector<const ExpertViews*>& vs, const std::vector<float>& w,
                             const float* x, int D, int FF, float* y) {
    std::vector<float> g(FF), u(FF), yd(D);
    for (size_t j = 0; j < vs.size(); j++) {
        matmul(vs[j]->gate, x, 1, D, g.data(), FF);
        matmul(vs[j]->up, x, 1, D, u.data(), FF);
        for (int i = 0; i < FF; i++) {
            float gv = g[i];
            g[i] = gv / (1.0f + expf(-gv)) * u[i];
        }
        matmul(vs[j]->down, g.data(), 1, FF, yd.data(), D);
        for (int r = 0; r < D; r++) y[r] += w[j] * yd[r];
    }
}

static eahmmf_hip_weight hip_view(const WeightView& w) {
    return eahmmf_hip_weight{w.dev, (int)w.type, (int)w.ne0, (int)w.ne1, w.row_bytes};
}

int main(int argc, char** argv) {
    if (argc < 2) {
        fprintf(stderr, "usage: %s tiny.gguf\n", argv[0]);
        return 2;
    }
    if (eahmmf_hip_device_count() < 1) {
        fprintf(stderr, "no HIP device\n");
        return 2;
    }
    init_types();
    Engine E;
    E.load(argv[1], 64, false);
    const size_t FP = E.store->descriptor(0, 0).footprint;
    const int D = E.D, FF = E.FF, NE = E.n_expert;
    size_t live = 0;
    auto hip = [&]() { return std::unique_ptr<DeviceBackend>(new CountedHip(&live)); };

    fprintf(stderr, "[A/B] tier matrix with HipDevice (expert footprint %zu B)\n", FP);
    const Run base = infer(E);  // SSD tier, the default store
    CHECK(!base.ids.empty() && base.ids.size() == base.w.size());
    struct Case {
        const char* name;
        Config cfg;
    };
    const Case cases[] = {
        {"vram unlimited", tier(Residency::VRAM, SIZE_MAX, SIZE_MAX, true)},
        {"vram unlimited, gpu_compute views", tier(Residency::VRAM, SIZE_MAX, SIZE_MAX, true, true)},
        {"vram 2 experts, ram unlimited", tier(Residency::VRAM, SIZE_MAX, 2 * FP, true)},
        {"vram 2, ram 2 (every pager path)", tier(Residency::VRAM, 2 * FP, 2 * FP, true)},
        {"vram 2, ram 1 (victims dropped to SSD)", tier(Residency::VRAM, 1 * FP, 2 * FP, true)},
        {"vram 1, ram 1", tier(Residency::VRAM, 1 * FP, 1 * FP, true)},
        {"vram below one expert (all fallback)", tier(Residency::VRAM, SIZE_MAX, FP / 2, false)},
        {"ram 3 experts", tier(Residency::RAM, 3 * FP, SIZE_MAX, true)},
    };
    for (const Case& c : cases) {
        CHECK(E.init_experts(c.cfg, hip()), "%s: init", c.name);
        CHECK(strcmp(E.dev->name(), "hip") == 0 && !E.dev->cpu_readable());
        const Run r = infer(E);
        CHECK(bitwise_equal(r, base), "case '%s' differs from the SSD-tier run", c.name);
        const std::string inv = E.store->check_invariants();
        CHECK(inv.empty(), "%s: %s", c.name, inv.c_str());
        const Stats& st = E.store->stats();
        CHECK(st.acquires == st.releases && st.pinned_now == 0, "pin leak in '%s'", c.name);
        CHECK(live == E.store->vram_used(), "%s: device bytes %zu, store charges %zu", c.name, live,
              E.store->vram_used());
        if (!strcmp(c.name, "vram 2, ram 2 (every pager path)"))
            CHECK(st.mig_n[SSD_RAM] > 0 && st.mig_n[RAM_VRAM] > 0 && st.mig_n[VRAM_RAM] > 0 && st.mig_n[RAM_SSD] > 0,
                  "every pager path exercised");
        if (!strcmp(c.name, "vram 2, ram 1 (victims dropped to SSD)"))
            CHECK(st.mig_n[VRAM_SSD] > 0 && st.mig_n[VRAM_RAM] == 0, "drop path used");
        fprintf(stderr, "    %-42s ssd->ram=%llu ram->vram=%llu vram->ram=%llu ram->ssd=%llu vram->ssd=%llu fb=%llu\n",
                c.name, (unsigned long long)st.mig_n[SSD_RAM], (unsigned long long)st.mig_n[RAM_VRAM],
                (unsigned long long)st.mig_n[VRAM_RAM], (unsigned long long)st.mig_n[RAM_SSD],
                (unsigned long long)st.mig_n[VRAM_SSD], (unsigned long long)st.fallbacks);
    }
    E.init_experts(Config());  // the HipDevice store is gone: every device byte returned
    CHECK(live == 0, "device bytes still allocated: %zu", live);

    fprintf(stderr, "[C] residency walk with byte checks\n");
    {
        CHECK(E.init_experts(tier(Residency::SSD, SIZE_MAX, SIZE_MAX, true), hip()));
        Residency from;
        CHECK(served_bytes_match_file(E, 1, 3, &from) && from == Residency::SSD);
        CHECK(E.store->promote(1, 3, Residency::RAM) && E.store->residency(1, 3) == Residency::RAM);
        CHECK(served_bytes_match_file(E, 1, 3, &from) && from == Residency::RAM);
        CHECK(E.store->promote(1, 3, Residency::VRAM) && E.store->residency(1, 3) == Residency::VRAM);
        CHECK(served_bytes_match_file(E, 1, 3, &from) && from == Residency::VRAM, "VRAM copy read back");
        CHECK(live == E.store->vram_used() && live >= FP);
        CHECK(E.store->demote(1, 3, Residency::RAM) && E.store->residency(1, 3) == Residency::RAM && live == 0);
        CHECK(served_bytes_match_file(E, 1, 3, &from) && from == Residency::RAM);
        CHECK(E.store->demote(1, 3, Residency::SSD) && E.store->residency(1, 3) == Residency::SSD);
        CHECK(E.store->check_invariants().empty());
    }

    fprintf(stderr, "[D] pinned experts, strict mode\n");
    {
        CHECK(E.init_experts(tier(Residency::VRAM, SIZE_MAX, 2 * FP, false), hip()));
        ExpertViews a = E.store->acquire(0, 0), b = E.store->acquire(0, 1);
        CHECK(a.ok && b.ok && a.served_from == Residency::VRAM && b.served_from == Residency::VRAM);
        ExpertViews c = E.store->acquire(0, 2);  // the pool is pinned full: served from RAM
        CHECK(c.ok && c.served_from == Residency::RAM);
        CHECK(E.store->residency(0, 0) == Residency::VRAM && E.store->residency(0, 1) == Residency::VRAM);
        CHECK(E.store->stats().refused_evictions > 0);
        E.store->release(0, 2);
        E.store->set_strict(true);
        ExpertViews d = E.store->acquire(0, 3);
        CHECK(!d.ok && E.store->descriptor(0, 3).pin_count == 0, "strict refuses, leaves no pin");
        E.store->set_strict(false);
        E.store->release(0, 0);
        ExpertViews e = E.store->acquire(0, 2);  // (0,0) is now the LRU victim
        CHECK(e.ok && e.served_from == Residency::VRAM && E.store->residency(0, 0) == Residency::RAM);
        E.store->release(0, 2);
        E.store->release(0, 1);
        CHECK(E.store->check_invariants().empty() && E.store->stats().pinned_now == 0);
    }

    std::mt19937 rng(7);
    std::normal_distribution<float> nx(0.f, 1.f);

    fprintf(stderr, "[E] expert matmul dispatch with the shadow check\n");
    {
        CHECK(E.init_experts(tier(Residency::VRAM, SIZE_MAX, SIZE_MAX, false, true), hip()));
        eahmmf_hip::DispatchStats st;
        const int nb = 5;
        std::vector<float> xs((size_t)nb * D), g((size_t)nb * FF), u((size_t)nb * FF), yd((size_t)nb * D);
        for (auto& v : xs) v = nx(rng);
        for (int l = 0; l < E.n_layer; l++)
            for (int x = 0; x < NE; x++) {
                ExpertLease lease = E.store->acquire_lease(l, x);
                CHECK(lease && lease.views().served_from == Residency::VRAM && lease.views().gate.dev);
                const ExpertViews& v = lease.views();
                eahmmf_hip::expert_matmul_gate_up(v.gate, v.up, xs.data(), nb, D, g.data(), FF, u.data(), FF,
                                                  cpu_matmul, st, true);
                for (int i = 0; i < nb * FF; i++) g[i] = g[i] / (1.0f + expf(-g[i])) * u[i];
                eahmmf_hip::expert_matmul(v.down, g.data(), nb, FF, yd.data(), D, cpu_matmul, st, true);
            }
        CHECK(st.pair_calls == (long)E.n_layer * NE && st.gpu_calls == 3L * E.n_layer * NE && st.cpu_fallbacks == 0);
        CHECK(st.shadow_calls == st.gpu_calls && st.shadow_bad == 0, "shadow: %ld of %ld bad, max rel %.3g",
              st.shadow_bad, st.shadow_calls, st.shadow_max_rel);
        // singles when the pair is disabled; the CPU for a view without a device copy
        setenv("EAHMMF_DISABLE_PAIR", "1", 1);
        eahmmf_hip::DispatchStats s2;
        {
            ExpertLease lease = E.store->acquire_lease(0, 0);
            const ExpertViews& v = lease.views();
            eahmmf_hip::expert_matmul_gate_up(v.gate, v.up, xs.data(), nb, D, g.data(), FF, u.data(), FF, cpu_matmul,
                                              s2, true);
            WeightView host_only = v.down;
            host_only.dev = nullptr;
            eahmmf_hip::expert_matmul(host_only, g.data(), nb, FF, yd.data(), D, cpu_matmul, s2, true);
        }
        unsetenv("EAHMMF_DISABLE_PAIR");
        CHECK(s2.pair_calls == 0 && s2.gpu_calls == 2 && s2.cpu_fallbacks == 1 && s2.shadow_bad == 0);
        fprintf(stderr, "    gpu calls %ld, pairs %ld, shadow max rel %.3g\n", st.gpu_calls, st.pair_calls,
                st.shadow_max_rel);
    }

    fprintf(stderr, "[F] single-call expert block over leased views\n");
    {
        CHECK(E.init_experts(tier(Residency::VRAM, SIZE_MAX, SIZE_MAX, false, true), hip()));
        const int ids[] = {6, 1, 4, 3};  // ascending id order is the reference's; any order is a valid call
        std::vector<ExpertLease> leases;
        leases.reserve(4);  // the views stay where they are while leases are added
        std::vector<const ExpertViews*> vs;
        std::vector<eahmmf_hip_expert> ex;
        std::vector<float> w;
        for (int j = 0; j < 4 && j < NE; j++) {
            leases.push_back(E.store->acquire_lease(1, ids[j] % NE));
            const ExpertViews& v = leases.back().views();
            vs.push_back(&v);
            ex.push_back(eahmmf_hip_expert{hip_view(v.gate), hip_view(v.up), hip_view(v.down)});
            w.push_back(0.1f + 0.2f * (float)j);
        }
        std::vector<float> x(D), y(D, 0.f), want(D, 0.f);
        for (auto& v : x) v = nx(rng);
        CHECK(eahmmf_hip_moe_decode(ex.data(), w.data(), (int)ex.size(), x.data(), y.data()), "%s",
              eahmmf_hip_last_error());
        cpu_expert_block(vs, w, x.data(), D, FF, want.data());
        const double rel = eahmmf_hip::shadow_rel_err(want.data(), y.data(), 1, D, D);
        CHECK(rel < 1e-4, "expert block vs the reference loop: %.3g", rel);
        fprintf(stderr, "    block rel err %.3g\n", rel);
    }

    fprintf(stderr, "[G] partial residency: the resident subset on the GPU, the rest on the CPU\n");
    {
        CHECK(E.init_experts(tier(Residency::VRAM, SIZE_MAX, 2 * FP, false, true), hip()));
        std::vector<ExpertLease> leases;
        leases.reserve(NE);
        std::vector<eahmmf_hip_expert> ex;
        std::vector<float> w;
        for (int x = 0; x < NE; x++) {
            leases.push_back(E.store->acquire_lease(0, x));  // all pinned at once
            const ExpertViews& v = leases.back().views();
            ex.push_back(eahmmf_hip_expert{hip_view(v.gate), hip_view(v.up), hip_view(v.down)});
            w.push_back(1.0f / (float)(x + 2));
        }
        uint32_t want_mask = 0;
        for (int x = 0; x < NE; x++) {
            const bool dev = leases[x].views().gate.dev != nullptr;
            CHECK(dev == (leases[x].views().served_from == Residency::VRAM));
            if (!dev) want_mask |= 1u << x;
        }
        CHECK(want_mask != 0 && want_mask != (1u << NE) - 1, "some experts resident, some not (mask %x)", want_mask);
        std::vector<float> x(D), y(D, 0.f), cpu_part(D, 0.f), all(D, 0.f);
        for (auto& v : x) v = nx(rng);
        uint32_t mask = 0;
        CHECK(eahmmf_hip_moe_decode_resident(ex.data(), w.data(), NE, x.data(), y.data(), &mask), "%s",
              eahmmf_hip_last_error());
        CHECK(mask == want_mask, "skipped %x, expected %x", mask, want_mask);
        std::vector<const ExpertViews*> skipped, every;
        std::vector<float> ws, wa;
        for (int j = 0; j < NE; j++) {
            every.push_back(&leases[j].views());
            wa.push_back(w[j]);
            if (mask >> j & 1) {
                skipped.push_back(&leases[j].views());
                ws.push_back(w[j]);
            }
        }
        cpu_expert_block(skipped, ws, x.data(), D, FF, cpu_part.data());
        for (int r = 0; r < D; r++) y[r] += cpu_part[r];
        cpu_expert_block(every, wa, x.data(), D, FF, all.data());
        const double rel = eahmmf_hip::shadow_rel_err(all.data(), y.data(), 1, D, D);
        CHECK(rel < 1e-4, "resident part + CPU part vs all on the CPU: %.3g", rel);
        fprintf(stderr, "    skipped mask %x, rel err %.3g\n", mask, rel);
        leases.clear();
        CHECK(E.store->stats().pinned_now == 0 && E.store->check_invariants().empty());
    }
    E.init_experts(Config());
    CHECK(live == 0, "device bytes still allocated: %zu", live);
    eahmmf_hip_shutdown();
    if (g_fail) {
        fprintf(stderr, "%d of %d checks failed\n", g_fail, g_checks);
        return 1;
    }
    printf("store_hip_check: all %d checks passed\n", g_checks);
    return 0;
}
