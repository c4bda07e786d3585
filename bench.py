"""Expert-FFN decode benchmark on one MI355X.

Workload (one "step"): one decode token through one MoE layer at
Qwen3-30B-A3B shape -- hidden 2048, 128 experts, expert FFN 768, top-8; gate
and up Q4_K, down Q6_K, quantized from N(0, 0.02) fp32; x ~ N(0, 1) fp32,
router logits ~ N(0, 1).  A step is the hot path on the device: softmax/top-8
routing, then the fused expert block (gate/up, SiLU, down, router-weighted
sum), inputs already resident in HBM.

The layer is replicated R times in HBM (R x 391.6 MB) and step i uses replica
i % R, so the routed experts of consecutive steps are cold in the 256 MB
Infinity Cache: the number reported is cold-HBM streaming.

value = algorithmic bytes (the 8 routed experts' weight bytes, 24,477,696 per
step) x steps / timed seconds.
"""
import argparse
import ctypes
import importlib.util
import json
import math
import os
import sys
import time

import numpy as np

ROOT = os.path.dirname(os.path.abspath(__file__))
PKG_DIR = os.path.join(ROOT, "eahmmf_inference_prototype_v-0.1.0_amd")
HBM_PEAK_GBS = 8000.0
MFMA_F16_PEAK_TFLOPS = 2500.0  # MI355X dense fp16/bf16 matrix-core peak
D, FF, E, K = 2048, 768, 128, 8
Q8_0, Q4_K, Q5_K, Q6_K = 8, 12, 13, 14
COPY_BYTES = 256 << 20


def load_binding():
    spec = importlib.util.spec_from_file_location("eahmmf_hip_bench", os.path.join(PKG_DIR, "eahmmf_hip.py"))
    mod = importlib.util.module_from_spec(spec)
    spec.loader.exec_module(mod)
    return mod


def build_layer(b, rng):
    """One layer's 128 experts: gate/up [E][FF rows x Q4_K(D)], down [E][D rows x Q6_K(FF)]."""
    grb, drb = b.row_bytes(Q4_K, D), b.row_bytes(Q6_K, FF)
    gate = np.empty((E, FF * grb), np.uint8)
    up = np.empty((E, FF * grb), np.uint8)
    down = np.empty((E, D * drb), np.uint8)
    for e in range(E):
        gate[e] = b.quantize_rows(Q4_K, rng.normal(0, .02, (FF, D)).astype(np.float32)).reshape(-1)
        up[e] = b.quantize_rows(Q4_K, rng.normal(0, .02, (FF, D)).astype(np.float32)).reshape(-1)
        down[e] = b.quantize_rows(Q6_K, rng.normal(0, .02, (D, FF)).astype(np.float32)).reshape(-1)
    return gate, up, down


def build_layer_replicated(b, rng, D, FF, E, n_unique, gt=Q4_K, dt=Q6_K):
    """E experts from n_unique distinct quantized ones (bytes of each expert
    still live at their own HBM addresses; only the values repeat)."""
    grb, drb = b.row_bytes(gt, D), b.row_bytes(dt, FF)
    uniq = []
    for _ in range(n_unique):
        uniq.append((b.quantize_rows(gt, rng.normal(0, .02, (FF, D)).astype(np.float32)).reshape(-1),
                     b.quantize_rows(gt, rng.normal(0, .02, (FF, D)).astype(np.float32)).reshape(-1),
                     b.quantize_rows(dt, rng.normal(0, .02, (D, FF)).astype(np.float32)).reshape(-1)))
    return uniq, grb, drb


def upload_layers(torch, uniq, E, R):
    """R replicas of an E-expert layer in HBM; returns the per-replica device tables."""
    n_unique = len(uniq)
    comps = []
    for c in range(3):
        host = torch.from_numpy(np.stack([uniq[e % n_unique][c] for e in range(E)])).pin_memory()
        dev = torch.empty((R,) + tuple(host.shape), dtype=torch.uint8, device="cuda")
        for r in range(R):
            dev[r].copy_(host)
        comps.append(dev)
    torch.cuda.synchronize()
    tables = []
    for r in range(R):
        t = np.array([[comps[c][r, e].data_ptr() for c in range(3)] for e in range(E)], dtype=np.uint64)
        tables.append(torch.from_numpy(t.view(np.int64)).cuda())
    return comps, tables


def zipf_routing(rng, nb, E, k, s=1.1):
    """Gumbel-top-k over log p_zipf (p ~ rank^-s on a seeded permutation of the
    ids): logits whose softmax/top-k routing is Zipf-skewed."""
    prior = np.log(np.arange(1, E + 1, dtype=np.float64) ** -s)[rng.permutation(E)]
    return (prior + rng.gumbel(size=(nb, E))).astype(np.float32)


def bench_c4(args, torch, b, hip):
    """Ragged grouped prefill: 512 tokens x top-8 over 128 Zipf-skewed experts
    at the Qwen3-30B-A3B expert shape, routing given (device ids/w), one step =
    grouping + gate/up + down + combine."""
    D_, FF_, E_, K_, NB = 2048, 768, 128, 8, 512
    rng = np.random.default_rng(4)
    uniq, grb, drb = build_layer_replicated(b, rng, D_, FF_, E_, 16)
    R = args.replicas if args.replicas else 4
    comps, tables = upload_layers(torch, uniq, E_, R)
    shape = b.MoeShape(Q4_K, Q4_K, Q6_K, D_, FF_, grb, grb, drb)
    NS = 4
    logits = zipf_routing(rng, NS * NB, E_, K_).reshape(NS, NB, E_)
    xs = rng.normal(0, 1, (NS, NB, D_)).astype(np.float32)
    dl, dx = torch.from_numpy(logits).cuda(), torch.from_numpy(xs).cuda()
    dids = torch.empty((NS, NB, K_), dtype=torch.int32, device="cuda")
    dw = torch.empty((NS, NB, K_), dtype=torch.float32, device="cuda")
    dy = torch.empty((NS, NB, D_), dtype=torch.float32, device="cuda")
    stream = torch.cuda.current_stream()
    sp, vp = ctypes.c_void_p(stream.cuda_stream), ctypes.c_void_p
    for i in range(NS):
        assert hip.eahmmf_hip_route_topk_async(vp(dl[i].data_ptr()), NB, E_, K_, vp(dids[i].data_ptr()),
                                               vp(dw[i].data_ptr()), sp) == 0
    torch.cuda.synchronize()
    ids = dids.cpu().numpy()
    exp_bytes = 2 * FF_ * grb + D_ * drb
    step_bytes = [len(np.unique(ids[i])) * exp_bytes + 2 * NB * D_ * 4 for i in range(NS)]

    def step(i):
        s_ = i % NS
        rc = hip.eahmmf_hip_moe_grouped_async(ctypes.byref(shape), vp(tables[i % R].data_ptr()), E_,
                                              vp(dids[s_].data_ptr()), vp(dw[s_].data_ptr()), NB, K_,
                                              vp(dx[s_].data_ptr()), vp(dy[s_].data_ptr()), sp)
        assert rc == 0, b.last_error()

    steps = args.steps if args.steps else 50
    for i in range(args.warmup if args.warmup else 5):
        step(i)
    torch.cuda.synchronize()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record(stream)
    for i in range(steps):
        step(i)
    e1.record(stream)
    torch.cuda.synchronize()
    el = e0.elapsed_time(e1) * 1e-3
    total = sum(step_bytes[i % NS] for i in range(steps))
    flop = NB * K_ * 2 * (3 * D_ * FF_)
    gbs = total / el / 1e9
    print(json.dumps({
        "metric": "grouped prefill expert-FFN HBM GB/s (% of peak)", "value": round(gbs, 2), "unit": "GB/s",
        "n_gpus": 1, "steps": steps, "ms_per_step": round(el * 1e3 / steps, 4), "higher_is_better": True,
        "dtype": "f32", "data": "synthetic",
        "config": {"workload": "ragged grouped prefill: 512 tokens x top-8 over 128 Zipf(1.1) experts, "
                               "D=2048 FF=768, Q4_K gate/up + Q6_K down", "layer_replicas": R,
                   "distinct_experts_per_step": [len(np.unique(ids[i])) for i in range(NS)],
                   "bytes_per_step_avg": int(np.mean(step_bytes))},
        "pct_of_hbm_peak": round(100 * gbs / HBM_PEAK_GBS, 2),
        "tflops": round(flop * steps / el / 1e12, 3),
        # useful expert FLOP over the step time against the dense fp16 matrix-core peak (the
        # grouped matmuls run v_mfma_f32_16x16x32_f16); the busy-cycle counters behind it are in
        # profiles/moe_grouped_c4_counters.md
        "mfma_util": round(flop * steps / el / 1e12 / MFMA_F16_PEAK_TFLOPS, 4),
        "mfma_peak_tflops": MFMA_F16_PEAK_TFLOPS}), flush=True)


def bench_c5_batch(args, torch, b, hip):
    """Small decode batches at the Qwen3-235B-A22B expert shape (D=4096,
    FF=1536, 128 experts top-8, Q4_K/Q6_K): nb decode tokens (one per
    sequence) through one MoE layer per step, routing on the device from fresh
    ~N(0,1) logits, then eahmmf_hip_moe_grouped_async (the headline: 16
    sequences).  Also timed per batch size: the grouped block (each distinct
    routed expert streamed once) and one single-token launch per token
    (eahmmf_hip_moe_decode_routed_async), the two paths the entry point
    chooses between."""
    D_, FF_, E_, K_, NB = 4096, 1536, 128, 8, 16
    NBMAX = 32
    rng = np.random.default_rng(6)
    uniq, grb, drb = build_layer_replicated(b, rng, D_, FF_, E_, 16)
    R = args.replicas if args.replicas else 4
    comps, tables = upload_layers(torch, uniq, E_, R)
    shape = b.MoeShape(Q4_K, Q4_K, Q6_K, D_, FF_, grb, grb, drb)
    NS = 16
    dl = torch.from_numpy(rng.normal(0, 1, (NS, NBMAX, E_)).astype(np.float32)).cuda()
    dx = torch.from_numpy(rng.normal(0, 1, (NS, NBMAX, D_)).astype(np.float32)).cuda()
    dids = torch.empty((NS, NBMAX, K_), dtype=torch.int32, device="cuda")
    dw = torch.empty((NS, NBMAX, K_), dtype=torch.float32, device="cuda")
    dy = torch.empty((NS, NBMAX, D_), dtype=torch.float32, device="cuda")
    stream = torch.cuda.current_stream()
    sp, vp = ctypes.c_void_p(stream.cuda_stream), ctypes.c_void_p
    exp_bytes = 2 * FF_ * grb + D_ * drb

    def route(s_, nb):
        assert hip.eahmmf_hip_route_topk_async(vp(dl[s_].data_ptr()), nb, E_, K_, vp(dids[s_].data_ptr()),
                                               vp(dw[s_].data_ptr()), sp) == 0

    def step(i, nb):  # routing + the batch's expert block, as a serving step runs it
        s_ = i % NS
        route(s_, nb)
        rc = hip.eahmmf_hip_moe_grouped_async(ctypes.byref(shape), vp(tables[i % R].data_ptr()), E_,
                                              vp(dids[s_].data_ptr()), vp(dw[s_].data_ptr()), nb, K_,
                                              vp(dx[s_].data_ptr()), vp(dy[s_].data_ptr()), sp)
        assert rc == 0, b.last_error()

    def step_per_token(i, nb):  # routing + one single-token launch per token
        s_ = i % NS
        route(s_, nb)
        for t in range(nb):
            rc = hip.eahmmf_hip_moe_decode_routed_async(ctypes.byref(shape), vp(tables[i % R].data_ptr()), E_,
                                                        vp(dids[s_, t].data_ptr()), vp(dw[s_, t].data_ptr()), K_,
                                                        vp(dx[s_, t].data_ptr()), vp(dy[s_, t].data_ptr()), sp)
            assert rc == 0, b.last_error()

    def timed(fn, nb, steps, warm):
        for i in range(warm):
            fn(i, nb)
        torch.cuda.synchronize()
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record(stream)
        for i in range(steps):
            fn(i, nb)
        e1.record(stream)
        torch.cuda.synchronize()
        return e0.elapsed_time(e1) * 1e-3 / steps

    for i in range(NS):
        route(i, NBMAX)
    torch.cuda.synchronize()
    ids_all = dids.cpu().numpy()
    distinct = [len(np.unique(ids_all[i, :NB])) for i in range(NS)]
    steps = args.steps if args.steps else 100
    t_api = timed(step, NB, steps, args.warmup if args.warmup else 5)
    fused_prev = hip.eahmmf_hip_set_fused(0)
    t_grouped = timed(step, NB, max(10, steps // 4), 2)
    mfma_prev = hip.eahmmf_hip_set_grouped_mfma(0)
    dot_prev = hip.eahmmf_hip_set_grouped_dot_max(0)
    t_valu = timed(step, NB, max(10, steps // 4), 2)
    hip.eahmmf_hip_set_grouped_dot_max(dot_prev)
    hip.eahmmf_hip_set_grouped_mfma(mfma_prev)
    sweep = []
    for nb in (1, 2, 4, 8, 16, 32):
        hip.eahmmf_hip_set_fused(0)
        tg = timed(step, nb, 20, 3)
        hip.eahmmf_hip_set_fused(1)
        tp = timed(step_per_token, nb, 20, 3)
        sweep.append({"tokens": nb, "grouped_ms": round(tg * 1e3, 4), "per_token_launches_ms": round(tp * 1e3, 4),
                      "distinct_experts_mean": round(float(np.mean([len(np.unique(ids_all[i, :nb])) for i in range(NS)])), 1)})
    hip.eahmmf_hip_set_fused(fused_prev)
    assert hip.eahmmf_hip_device_flags() == 0
    read_bytes = NB * K_ * exp_bytes  # each token's experts, read per token
    distinct_bytes = float(np.mean([d * exp_bytes for d in distinct]))
    gbs = distinct_bytes / t_api / 1e9  # algorithmic: each distinct routed expert once
    print(json.dumps({
        "metric": "16-sequence decode batch expert-FFN HBM GB/s (% of peak), Qwen3-235B-A22B shape",
        "value": round(gbs, 2), "unit": "GB/s", "n_gpus": 1, "steps": steps, "ms_per_step": round(t_api * 1e3, 4),
        "higher_is_better": True, "dtype": "f32", "data": "synthetic",
        "config": {"workload": "16 decode tokens (one per sequence) through one MoE layer, D=4096 FF=1536 "
                               "128 experts top-8, Q4_K gate/up + Q6_K down, routing on device, "
                               "eahmmf_hip_moe_grouped_async", "layer_replicas": R,
                   "bytes_read_if_per_token": read_bytes, "distinct_experts_mean": round(float(np.mean(distinct)), 1),
                   "distinct_expert_bytes_per_step": int(distinct_bytes)},
        "pct_of_hbm_peak": round(100 * gbs / HBM_PEAK_GBS, 2),
        "expert_only_batch_tokens_per_s_94_layers": round(NB / (94 * t_api), 1),
        "grouped_block_ms": round(t_grouped * 1e3, 4), "grouped_vector_alu_only_ms": round(t_valu * 1e3, 4),
        "batch_sweep": sweep,
        "what": "ms per layer-step including routing; grouped = eahmmf_hip_moe_grouped_async with the single-token "
                "kernel off (integer-dot kernels for every expert), per_token_launches = one single-launch "
                "expert block per token (eahmmf_hip_moe_decode_routed_async)"}), flush=True)


def bench_c5(args, torch, b, hip):
    """Single decode token through one MoE layer at the Qwen3-235B-A22B expert
    shape (D=4096, FF=1536, 128 experts, top-8, Q4_K/Q6_K), routing on device."""
    D_, FF_, E_, K_ = 4096, 1536, 128, 8
    rng = np.random.default_rng(5)
    uniq, grb, drb = build_layer_replicated(b, rng, D_, FF_, E_, 16)
    R = args.replicas if args.replicas else 4
    comps, tables = upload_layers(torch, uniq, E_, R)
    shape = b.MoeShape(Q4_K, Q4_K, Q6_K, D_, FF_, grb, grb, drb)
    NS = 64
    xs = torch.from_numpy(rng.normal(0, 1, (NS, D_)).astype(np.float32)).cuda()
    dl = torch.from_numpy(rng.normal(0, 1, (NS, E_)).astype(np.float32)).cuda()
    dy = torch.empty((NS, D_), dtype=torch.float32, device="cuda")
    stream = torch.cuda.current_stream()
    sp, vp = ctypes.c_void_p(stream.cuda_stream), ctypes.c_void_p

    def step(i):
        s_ = i % NS
        rc = hip.eahmmf_hip_moe_layer_decode_async(ctypes.byref(shape), vp(tables[i % R].data_ptr()), E_,
                                                   vp(dl[s_].data_ptr()), K_, vp(xs[s_].data_ptr()),
                                                   vp(dy[s_].data_ptr()), None, None, sp)
        assert rc == 0, b.last_error()

    steps = args.steps if args.steps else 1000
    for i in range(args.warmup if args.warmup else 50):
        step(i)
    torch.cuda.synchronize()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record(stream)
    for i in range(steps):
        step(i)
    e1.record(stream)
    torch.cuda.synchronize()
    assert hip.eahmmf_hip_device_flags() == 0
    el = e0.elapsed_time(e1) * 1e-3
    bytes_step = K_ * (2 * FF_ * grb + D_ * drb)
    gbs = bytes_step * steps / el / 1e9
    print(json.dumps({
        "metric": "expert-FFN HBM GB/s (% of peak) + decode tokens/s, Qwen3-235B-A22B shape", "value": round(gbs, 2),
        "unit": "GB/s", "n_gpus": 1, "steps": steps, "ms_per_step": round(el * 1e3 / steps, 5),
        "higher_is_better": True, "dtype": "f32", "data": "synthetic",
        "config": {"workload": "single MoE layer, one decode token, D=4096 FF=1536 128 experts top-8, "
                               "Q4_K gate/up + Q6_K down, routing on device", "bytes_per_step": bytes_step,
                   "layer_replicas": R},
        "pct_of_hbm_peak": round(100 * gbs / HBM_PEAK_GBS, 2),
        "expert_only_decode_tokens_per_s_94_layers": round(1.0 / (94 * el / steps), 1)}), flush=True)


def stream_rates(torch, hip, steps=2000):
    """Achievable HBM read rate with the library's streaming-read kernel
    (eahmmf_hip_stream_read_async: nontemporal 16-byte loads, eight per thread
    in flight).  (1) Back-to-back launches over 24,477,696-byte windows (the
    C2 layer-token's expert bytes) rotating over 16 windows (392 MB, more than
    the 256 MB Infinity Cache, so each launch reads cold HBM), event-timed on
    the launch stream exactly like the layer kernel's avg_us; (2) a 1 GiB read,
    repeated."""
    W, R = 24_477_696, 16
    buf = torch.empty(W * R, dtype=torch.uint8, device="cuda").random_(0, 256)
    big = torch.empty(1 << 30, dtype=torch.uint8, device="cuda").random_(0, 256)
    sink = torch.zeros(4096, dtype=torch.int32, device="cuda")
    stream = torch.cuda.current_stream()
    sp, vp = ctypes.c_void_p(stream.cuda_stream), ctypes.c_void_p

    def launch(base, n):
        rc = hip.eahmmf_hip_stream_read_async(vp(base), n, vp(sink.data_ptr()), sp)
        assert rc == 0, hip.eahmmf_hip_last_error()

    def timed(n_launch, fn):
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record(stream)
        for i in range(n_launch):
            fn(i)
        e1.record(stream)
        torch.cuda.synchronize()
        return e0.elapsed_time(e1) * 1e-3 / n_launch  # s per launch

    small = lambda i: launch(buf.data_ptr() + (i % R) * W, W)  # noqa: E731
    whole = lambda i: launch(buf.data_ptr(), W * R)  # noqa: E731
    large = lambda i: launch(big.data_ptr(), big.numel())  # noqa: E731
    timed(50, small)
    t_small = timed(steps, small)
    timed(3, whole)
    t_whole = timed(max(20, steps // 40), whole)
    timed(3, large)
    t_large = timed(20, large)
    del buf, big
    return {"kernel": "stream_read_kernel (nontemporal 16-byte loads, 8 in flight per thread)",
            "c2_size_cold_GB_s": round(W / t_small / 1e9, 1), "c2_size_cold_us": round(t_small * 1e6, 3),
            # the same 16 windows read by one launch: the per-window time without a launch's ramp-up and drain
            "c2_windows_in_one_launch_us_per_window": round(t_whole / R * 1e6, 3),
            "c2_windows_in_one_launch_GB_s": round(W * R / t_whole / 1e9, 1),
            "per_launch_ramp_us": round((t_small - t_whole / R) * 1e6, 3),
            "GB_s_1GiB": round((1 << 30) / t_large / 1e9, 1)}


def bench_stream(args, torch, b, hip):
    """The achievable read rate alone (the measured ceiling beside the nominal
    8 TB/s)."""
    r = stream_rates(torch, hip, args.steps or 2000)
    print(json.dumps({
        "metric": "achievable HBM read GB/s (streaming-read kernel)", "value": r["GB_s_1GiB"], "unit": "GB/s",
        "n_gpus": 1, "higher_is_better": True, "dtype": "u32", "data": "synthetic",
        "config": {"workload": "streaming read of 1 GiB; back-to-back reads of 24,477,696-byte windows "
                               "rotating over 16 (392 MB, cold in the 256 MB Infinity Cache); the 16 windows "
                               "in one launch"},
        "pct_of_hbm_peak": round(100 * r["GB_s_1GiB"] / HBM_PEAK_GBS, 2), "stream_read": r}), flush=True)


def bench_staging(args, torch, b, hip):
    """Making experts resident: one C2 layer's 128 experts (gate/up Q4_K
    884,736 B each, down Q6_K 1,290,240 B; 391.6 MB) from pageable host
    memory into HBM, (a) the reference's way - per expert three h2d() calls and
    a sync() (ExpertPager::stage_to_vram, eahmmf.h:1009-1013), through
    eahmmf_hip_h2d/eahmmf_hip_sync - (b) one eahmmf_hip_h2d_batch of all
    384 components through the pinned staging ring, and (c) the same batch
    queued with eahmmf_hip_h2d_batch_async (the caller's thread free once it
    is queued)."""
    E_, comp = 128, (884_736, 884_736, 1_290_240)
    rng = np.random.default_rng(9)
    host = [[rng.integers(0, 256, n, dtype=np.uint8) for n in comp] for _ in range(E_)]
    foot = sum((n + 4095) // 4096 * 4096 for n in comp)
    dev = torch.empty(E_ * foot, dtype=torch.uint8, device="cuda")
    base = dev.data_ptr()
    offs = [0, (comp[0] + 4095) // 4096 * 4096]
    offs.append(offs[1] + (comp[1] + 4095) // 4096 * 4096)
    total = E_ * sum(comp)
    vp = ctypes.c_void_p
    copies = (b.Copy * (3 * E_))()
    for e in range(E_):
        for c in range(3):
            copies[3 * e + c] = b.Copy(base + e * foot + offs[c], host[e][c].ctypes.data, comp[c])

    def per_expert():
        for e in range(E_):
            for c in range(3):
                assert hip.eahmmf_hip_h2d(vp(base + e * foot + offs[c]), vp(host[e][c].ctypes.data), comp[c]) == 0
            assert hip.eahmmf_hip_sync() == 0

    def batch():
        assert hip.eahmmf_hip_h2d_batch(copies, 3 * E_) == 0, b.last_error()

    def best(fn, reps):
        fn()  # first touch of the ring / driver staging
        t = []
        for _ in range(reps):
            torch.cuda.synchronize()
            t0 = time.perf_counter()
            fn()
            t.append(time.perf_counter() - t0)
        return min(t)

    t_ref, t_batch = best(per_expert, 3), best(batch, 3)
    # (c) the same batch queued asynchronously: how long the caller's thread is
    # held (the call returns once the batch is queued to the staging thread),
    # and when the bytes have landed (host wait on the ticket)
    t_ret, t_land = [], []
    for _ in range(3):
        torch.cuda.synchronize()
        ticket = ctypes.c_uint64(0)
        t0 = time.perf_counter()
        assert hip.eahmmf_hip_h2d_batch_async(copies, 3 * E_, ctypes.byref(ticket)) == 0, b.last_error()
        t_ret.append(time.perf_counter() - t0)
        assert hip.eahmmf_hip_h2d_batch_wait(ticket.value, None) == 0, b.last_error()
        t_land.append(time.perf_counter() - t0)
    probe = [(7, 2), (E_ - 1, 0)]  # spot check: two components read back exactly
    for e, c in probe:
        got = dev[e * foot + offs[c]:e * foot + offs[c] + comp[c]].cpu().numpy()
        assert np.array_equal(got, host[e][c])
    print(json.dumps({
        "metric": "expert staging GB/s, pageable host memory to HBM (one C2 layer, 128 experts)",
        "value": round(total / t_batch / 1e9, 2), "unit": "GB/s", "n_gpus": 1, "higher_is_better": True,
        "dtype": "u8", "data": "synthetic",
        "config": {"workload": "128 experts x (884,736 + 884,736 + 1,290,240 B) = 391.6 MB, pageable numpy "
                               "buffers, into one HBM allocation at 4096-byte aligned offsets",
                   "bytes": total},
        "batch_ms": round(t_batch * 1e3, 2),
        "per_expert_h2d_sync": {"GB_s": round(total / t_ref / 1e9, 2), "ms": round(t_ref * 1e3, 2),
                                "what": "3 x eahmmf_hip_h2d + eahmmf_hip_sync per expert (the reference pager)"},
        "speedup": round(t_ref / t_batch, 2),
        "async": {"return_us": round(min(t_ret) * 1e6, 1), "landed_ms": round(min(t_land) * 1e3, 2),
                  "GB_s": round(total / min(t_land) / 1e9, 2),
                  "what": "eahmmf_hip_h2d_batch_async of the same 384 copies: time until the call returns "
                          "(the caller's thread is free from then on) and until eahmmf_hip_h2d_batch_wait says "
                          "the bytes have landed"}}), flush=True)


def bench_dropin(args, torch, b, hip):
    """One C2 layer-token through the drop-in entry points, exactly as the
    reference's host loop calls them (qwen3moe.cpp:1024-1067): per routed
    expert eahmmf_hip_matmul_pair (gate/up, host x in, host g/u out), SiLU on
    the host, eahmmf_hip_matmul (down), the weighted sum on the host; every
    call synchronous with pageable host buffers.  Routing is taken as given."""
    D_, FF_, E_, K_ = 2048, 768, 128, 8
    rng = np.random.default_rng(7)
    uniq, grb, drb = build_layer_replicated(b, rng, D_, FF_, E_, 16)
    R = args.replicas if args.replicas else 4
    comps, tables = upload_layers(torch, uniq, E_, R)
    tab = [t.cpu().numpy().view(np.uint64) for t in tables]
    NS = 16
    xs = rng.normal(0, 1, (NS, D_)).astype(np.float32)
    ids = np.stack([rng.choice(E_, K_, replace=False) for _ in range(NS)])
    w = rng.uniform(0.05, 0.2, (NS, K_)).astype(np.float32)
    g = np.empty(FF_, np.float32)
    u = np.empty(FF_, np.float32)
    yd = np.empty(D_, np.float32)

    def token(i):
        s_, r = i % NS, i % R
        x = xs[s_]
        y = np.zeros(D_, np.float32)
        for j in sorted(range(K_), key=lambda jj: ids[s_, jj]):  # ascending expert id, as by_exp
            gp, up, dp = (int(v) for v in tab[r][ids[s_, j]])
            assert hip.eahmmf_hip_matmul_pair(gp, Q4_K, D_, FF_, grb, up, Q4_K, D_, FF_, grb, x.ctypes.data, 1, D_,
                                              g.ctypes.data, FF_, u.ctypes.data, FF_), b.last_error()
            h = (g / (1.0 + np.exp(-g)) * u).astype(np.float32)
            assert hip.eahmmf_hip_matmul(dp, Q6_K, FF_, D_, drb, h.ctypes.data, 1, FF_, yd.ctypes.data, D_), \
                b.last_error()
            y += w[s_, j] * yd

    steps = args.steps if args.steps else 300
    for i in range(10):
        token(i)
    t0 = time.perf_counter()
    for i in range(steps):
        token(i)
    el = (time.perf_counter() - t0) / steps
    bytes_step = K_ * (2 * FF_ * grb + D_ * drb)
    print(json.dumps({
        "metric": "expert-FFN HBM GB/s through the drop-in matmul entry points (reference calling pattern)",
        "value": round(bytes_step / el / 1e9, 2), "unit": "GB/s", "n_gpus": 1, "steps": steps,
        "ms_per_step": round(el * 1e3, 4), "higher_is_better": True, "dtype": "f32", "data": "synthetic",
        "config": {"workload": "one C2 layer-token (D=2048 FF=768, 8 routed experts, Q4_K gate/up + Q6_K down) as "
                               "8 x (eahmmf_hip_matmul_pair + host SiLU + eahmmf_hip_matmul), synchronous, pageable "
                               "host buffers", "bytes_per_step": bytes_step, "calls_per_step": 2 * K_},
        "us_per_call": round(el * 1e6 / (2 * K_), 2)}), flush=True)


def device_blocks(torch, t, nrows, ne0, gen, scale):
    """nrows rows of type t built on the device: random codes, fp16 scale
    fields uniform in [0.5, 1.5) x scale (F32: N(0, scale) values)."""
    if t == 0:
        return torch.randn((nrows, ne0), device="cuda", generator=gen).mul_(scale)
    blck, nbytes = {Q8_0: (32, 34), Q4_K: (256, 144), Q5_K: (256, 176), Q6_K: (256, 210)}[t]
    nblk = nrows * (ne0 // blck)
    raw = torch.randint(0, 256, (nblk, nbytes), dtype=torch.uint8, device="cuda", generator=gen)

    def put(off):
        d = (torch.rand(nblk, device="cuda", generator=gen) + 0.5).mul_(scale).half()
        raw[:, off:off + 2] = d.view(torch.uint8).view(nblk, 2)

    if t == Q6_K:
        put(208)
    else:
        put(0)
        if t in (Q4_K, Q5_K):
            put(2)
    return raw.view(nrows, (ne0 // blck) * nbytes)


QWEN3_30B = dict(n_layer=48, D=2048, n_head=32, n_kv=4, hd=128, n_expert=128, n_used=8, FF=768, n_vocab=151936)
QWEN3_235B = dict(n_layer=94, D=4096, n_head=64, n_kv=4, hd=128, n_expert=128, n_used=8, FF=1536, n_vocab=151936)


def c3_model(torch, b, expert_type, n_ctx, seed=3, shape=QWEN3_30B, types=None):
    """A Qwen3-MoE-shaped model in HBM (default the 48-layer Qwen3-30B-A3B
    shape: D=2048, 32 query / 4 KV heads of dim 128, 128 experts top-8, FF
    768, vocab 151936); experts all expert_type (or types = (gate, up, down)),
    attention, embedding and output head Q8_0, router F32, norm weights 1.
    Weights are generated on the device (random codes with fp16 scales sized
    for ~0.02 weights) and borrowed by the model."""
    NL, D_, NH, NKV, HD = shape["n_layer"], shape["D"], shape["n_head"], shape["n_kv"], shape["hd"]
    E_, K_, FF_, V = shape["n_expert"], shape["n_used"], shape["FF"], shape["n_vocab"]
    gt_, ut_, dt_ = types if types else (expert_type,) * 3
    gen = torch.Generator(device="cuda")
    gen.manual_seed(seed)
    sc = {Q8_0: 3e-4, Q5_K: 5e-5, Q4_K: 1e-4, Q6_K: 1e-5}
    keep, tensors = [], {}

    def add(name, t, ne0, rows, ne=None, scale=None):
        d = device_blocks(torch, t, rows, ne0, gen, sc.get(t, 0.02) if scale is None else scale)
        keep.append(d)
        tensors[name] = (t, ne if ne else [ne0, rows], d.data_ptr())

    ones = torch.ones(D_, device="cuda")
    ones_h = torch.ones(HD, device="cuda")
    keep += [ones, ones_h]
    add("token_embd.weight", Q8_0, D_, V)
    add("output.weight", Q8_0, D_, V)
    tensors["output_norm.weight"] = (0, [D_], ones.data_ptr())
    for l in range(NL):
        p = f"blk.{l}."
        for nm in ("attn_norm", "ffn_norm"):
            tensors[p + nm + ".weight"] = (0, [D_], ones.data_ptr())
        for nm in ("attn_q_norm", "attn_k_norm"):
            tensors[p + nm + ".weight"] = (0, [HD], ones_h.data_ptr())
        add(p + "attn_q.weight", Q8_0, D_, NH * HD)
        add(p + "attn_k.weight", Q8_0, D_, NKV * HD)
        add(p + "attn_v.weight", Q8_0, D_, NKV * HD)
        add(p + "attn_output.weight", Q8_0, NH * HD, D_)
        add(p + "ffn_gate_inp.weight", 0, D_, E_, scale=0.02)
        add(p + "ffn_gate_exps.weight", gt_, D_, E_ * FF_, ne=[D_, FF_, E_])
        add(p + "ffn_up_exps.weight", ut_, D_, E_ * FF_, ne=[D_, FF_, E_])
        add(p + "ffn_down_exps.weight", dt_, FF_, E_ * D_, ne=[FF_, D_, E_])
    torch.cuda.synchronize()
    hp = dict(n_layer=NL, D=D_, n_head=NH, n_kv=NKV, hd=HD, n_expert=E_, n_used=K_, FF=FF_, n_vocab=V, n_ctx=n_ctx,
              eps=1e-6, rope_base=1e6)
    m = b.DeviceModel(hp, tensors)
    return m, keep, hp


def c3_token_bytes(b, hp, expert_type, n_pos, types=None):
    """Algorithmic HBM bytes of one decode token at n_pos cached positions:
    every dense weight once (Q, K, V, output projections, router, output
    head), the 8 routed experts' three matrices per layer (all expert_type,
    or types = (gate, up, down)), the K and V rows of n_pos positions per
    layer (fp32) plus the new row, one embedding row."""
    D_, FF_, NL, KD, QD = hp["D"], hp["FF"], hp["n_layer"], hp["n_kv"] * hp["hd"], hp["n_head"] * hp["hd"]
    gt_, ut_, dt_ = types if types else (expert_type,) * 3
    q8 = lambda ne0: b.row_bytes(Q8_0, ne0)
    dense = (QD + 2 * KD) * q8(D_) + D_ * q8(QD) + hp["n_expert"] * D_ * 4
    experts = hp["n_used"] * (FF_ * (b.row_bytes(gt_, D_) + b.row_bytes(ut_, D_)) + D_ * b.row_bytes(dt_, FF_))
    kv = 2 * (n_pos + 1) * KD * 4
    return NL * (dense + experts + kv) + hp["n_vocab"] * q8(D_) + q8(D_)


def c3_decode(torch, b, et, types, CTX, steps, warm, rng):
    """Builds the 48-layer model (experts et, or types = (gate, up, down)),
    prefills CTX - warm positions (batches of 64), decodes warm tokens, then
    times one eahmmf_hip_model_generate_greedy call of `steps` tokens (one
    host wait at its end).  Returns its figures and frees the model."""
    t0 = time.perf_counter()
    m, keep, hp = c3_model(torch, b, et, CTX + warm + steps + 1, types=types)
    t_build = time.perf_counter() - t0
    prompt = rng.integers(0, hp["n_vocab"], CTX - warm).astype(np.int32)
    t0 = time.perf_counter()
    lg = m.eval(prompt, 0, 64)
    t_prefill = time.perf_counter() - t0
    assert np.isfinite(lg).all(), "non-finite logits after the prefill"
    first = int(np.argmax(lg))
    toks, lg = m.generate_greedy(first, CTX - warm, warm)
    t0 = time.perf_counter()
    toks, lg = m.generate_greedy(int(toks[-1]), CTX, steps)
    el = time.perf_counter() - t0
    assert np.isfinite(lg).all(), "non-finite logits after decode"
    bt = c3_token_bytes(b, hp, et, CTX + steps // 2, types)
    m.close()
    del keep
    torch.cuda.empty_cache()
    return {"tokens_per_s": round(steps / el, 1), "ms_per_token": round(el * 1e3 / steps, 4),
            "bytes_per_token": bt, "GB_s": round(bt * steps / el / 1e9, 1),
            "pct_of_hbm_peak": round(100 * bt * steps / el / 1e9 / HBM_PEAK_GBS, 2),
            "prefill_tokens_per_s": round(len(prompt) / t_prefill, 1), "build_s": round(t_build, 1)}


def bench_c3(args, torch, b, hip):
    """Single-token decode of the full 48-layer Qwen3-30B-A3B-shaped model at
    a 2048-token KV context (every layer on the device: attention with its
    Q8_0 projections, norms, RoPE, KV cache, router, the fused expert block,
    output head, greedy argmax), for the expert variants all-Q5_K, all-Q8_0
    and the Q4_K_M mix (Q4_K gate/up, Q6_K down).  The KV cache is filled by a
    2048-token prefill (batches of 64); the timed region is one
    eahmmf_hip_model_generate_greedy call of `steps` tokens (one host wait at
    its end).  value = tokens/s of the Q5_K variant."""
    CTX = 2048
    steps = args.steps if args.steps else 64
    warm = args.warmup if args.warmup else 8
    rng = np.random.default_rng(5)
    results = {}
    for name, et, types in (("q5_k", Q5_K, None), ("q8_0", Q8_0, None), ("q4_k_m", Q4_K, (Q4_K, Q4_K, Q6_K))):
        results[name] = c3_decode(torch, b, et, types, CTX, steps, warm, rng)
        if not args.no_cpu_baseline and name == "q5_k":  # the headline variant only (about 2 minutes)
            results[name]["cpu_baseline"] = c3_cpu_baseline(et)
        print(f"# c3 {name}: {results[name]}", file=sys.stderr, flush=True)
    r = results["q5_k"]
    print(json.dumps({
        "metric": "decode tokens/s, 48-layer Qwen3-30B-A3B-shaped model, 2048-token KV context", "unit": "tokens/s",
        "value": r["tokens_per_s"], "n_gpus": 1, "steps": steps, "warmup": warm, "ms_per_step": r["ms_per_token"],
        "higher_is_better": True, "scaling": "weak", "vs_baseline": None, "dtype": "f32", "data": "synthetic",
        "config": {"workload": "single-token greedy decode, 48 layers D=2048 32/4 heads hd=128, 128 experts top-8 "
                               "FF=768, vocab 151936, KV context 2048 (prefilled), experts Q5_K (value) / Q8_0 / "
                               "Q4_K_M (Q4_K gate/up, Q6_K down), attention + embedding + output head Q8_0, router "
                               "F32; everything on the device"},
        "roofline": {"bound": "hbm", "kernel": "whole decode token (all launches)",
                     "achieved": r["GB_s"], "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": round(r["GB_s"] / HBM_PEAK_GBS, 4), "traffic": None},
        "cpu_baseline": r.get("cpu_baseline"),
        "variants": results}), flush=True)


def bench_c5_seqs(args, torch, b, hip):
    """16 sequences decoded together through the whole 94-layer
    Qwen3-235B-A22B-shaped model (D=4096, 64 query / 4 KV heads of dim 128,
    128 experts top-8 FF=1536, Q4_K gate/up + Q6_K down, attention + embedding
    + output head Q8_0, router F32, vocab 151936; about 155 GB in HBM).  Each
    sequence is prefilled with its own prompt (lengths 32-256, so the batch is
    ragged); a timed step is one eahmmf_hip_model_decode_seqs call: one token
    of every sequence, each at its own position and attending to its own KV
    rows, all 16 logits rows back on the host, the next tokens picked there
    (greedy).  Beside it: the same 16 tokens as 16 single-sequence forwards,
    one after another (what a one-sequence engine does).  value = aggregate
    decode tokens/s."""
    NSEQ = 16
    steps = args.steps if args.steps else 20
    warm = args.warmup if args.warmup else 3
    free, _ = torch.cuda.mem_get_info()
    if free < 200e9:
        print(f"bench c5seq: needs about 170 GB of free device memory, {free / 1e9:.0f} GB free", file=sys.stderr)
        sys.exit(3)
    rng = np.random.default_rng(9)
    lens = rng.integers(32, 257, NSEQ)
    n_ctx = int(lens.max()) + warm + steps + 8
    t0 = time.perf_counter()
    m, keep, hp = c3_model(torch, b, Q4_K, n_ctx, seed=4, shape=QWEN3_235B, types=(Q4_K, Q4_K, Q6_K))
    m.set_sequences(NSEQ)
    t_build = time.perf_counter() - t0
    t0 = time.perf_counter()
    last = []
    for s_ in range(NSEQ):
        lg = m.eval(rng.integers(0, hp["n_vocab"], int(lens[s_])).astype(np.int32), 0, 64, seq=s_)
        assert np.isfinite(lg).all(), "non-finite logits after a prefill"
        last.append(int(np.argmax(lg)))
    t_prefill = time.perf_counter() - t0
    toks, pos, seqs = np.array(last, np.int32), lens.astype(np.int32).copy(), np.arange(NSEQ, dtype=np.int32)

    def step():
        nonlocal toks
        lg = m.decode_seqs(toks, seqs, pos)
        toks = np.argmax(lg, axis=1).astype(np.int32)
        pos[:] += 1

    for _ in range(warm):
        step()
    t0 = time.perf_counter()
    for _ in range(steps):
        step()
    el = time.perf_counter() - t0
    # one traced step: distinct routed experts per layer (the expert bytes of a step)
    m.set_trace(True)
    m.trace_clear()
    kv_rows = int(pos.sum()) + NSEQ
    step()
    ids, _ = m.trace()
    m.set_trace(False)
    ids = ids.reshape(hp["n_layer"], NSEQ, hp["n_used"])
    distinct = float(np.mean([len(np.unique(ids[l])) for l in range(hp["n_layer"])]))
    # the same tokens as single-sequence forwards, one after another
    n_seq_steps = 2
    t0 = time.perf_counter()
    for _ in range(n_seq_steps):
        for s_ in range(NSEQ):
            lg = m.forward([int(toks[s_])], int(pos[s_]), seq=s_)
            toks[s_] = int(np.argmax(lg))
            pos[s_] += 1
    el_seq = (time.perf_counter() - t0) / n_seq_steps
    D_, FF_, NL, KD, QD = hp["D"], hp["FF"], hp["n_layer"], hp["n_kv"] * hp["hd"], hp["n_head"] * hp["hd"]
    q8 = lambda ne0: b.row_bytes(Q8_0, ne0)
    exp_bytes = 2 * FF_ * b.row_bytes(Q4_K, D_) + D_ * b.row_bytes(Q6_K, FF_)
    dense = (QD + 2 * KD) * q8(D_) + D_ * q8(QD) + hp["n_expert"] * D_ * 4
    step_bytes = NL * (dense + distinct * exp_bytes + 2 * kv_rows * KD * 4) + hp["n_vocab"] * q8(D_)
    ms = el * 1e3 / steps
    gbs = step_bytes / (ms * 1e-3) / 1e9
    r = {"metric": "16-sequence decode tokens/s, 94-layer Qwen3-235B-A22B-shaped model (whole model on the device)",
         "unit": "tokens/s", "value": round(NSEQ * steps / el, 1), "n_gpus": 1, "steps": steps, "warmup": warm,
         "ms_per_step": round(ms, 3), "higher_is_better": True, "scaling": "weak", "vs_baseline": None,
         "dtype": "f32", "data": "synthetic",
         "config": {"workload": "one decode token of each of 16 sequences per step (eahmmf_hip_model_decode_seqs), "
                                "94 layers D=4096 64/4 heads hd=128, 128 experts top-8 FF=1536 Q4_K/Q4_K/Q6_K, "
                                "attention + embedding + output head Q8_0, router F32, vocab 151936",
                    "prompt_lengths": [int(v) for v in lens]},
         "step_bytes": int(step_bytes), "distinct_experts_per_layer": round(distinct, 1),
         "roofline": {"bound": "hbm", "kernel": "whole decode step (all launches)", "achieved": round(gbs, 1),
                      "peak": HBM_PEAK_GBS, "unit": "GB/s", "frac": round(gbs / HBM_PEAK_GBS, 4), "traffic": None},
         "one_sequence_at_a_time_ms_per_16_tokens": round(el_seq * 1e3, 2),
         "one_sequence_at_a_time_tokens_per_s": round(NSEQ / el_seq, 1),
         "prefill_tokens_per_s": round(float(lens.sum()) / t_prefill, 1), "build_s": round(t_build, 1),
         "what": "step = decode_seqs (16 tokens, logits [16][151936] to the host) + host argmax; step_bytes = "
                 "dense weights once + distinct routed experts (one traced step) + KV rows read + output head"}
    m.close()
    del keep
    torch.cuda.empty_cache()
    print(json.dumps(r), flush=True)


def bench_c3_experts(args, torch, b, hip):
    """Expert-only decode of one token through all 48 MoE layers of the
    Qwen3-30B-A3B shape (D=2048, FF=768, 128 experts, top-8), every layer
    resident at its own HBM addresses; one step = 48 layer launches (routing on
    device).  Runs the Q4_K_M variant (Q4_K gate/up, Q6_K down) and the
    config's two variants, all three components Q5_K and all Q8_0."""
    D_, FF_, E_, K_, NL = 2048, 768, 128, 8, 48
    rng = np.random.default_rng(3)
    stream = torch.cuda.current_stream()
    sp, vp = ctypes.c_void_p(stream.cuda_stream), ctypes.c_void_p
    results = {}
    for name, gt, dt in (("q4_k_m", Q4_K, Q6_K), ("q5_k", Q5_K, Q5_K), ("q8_0", Q8_0, Q8_0)):
        uniq, grb, drb = build_layer_replicated(b, rng, D_, FF_, E_, 16, gt, dt)
        comps, tables = upload_layers(torch, uniq, E_, NL)  # 48 distinct layers in HBM
        shape = b.MoeShape(gt, gt, dt, D_, FF_, grb, grb, drb)
        NS = 16
        xs = torch.from_numpy(rng.normal(0, 1, (NS, NL, D_)).astype(np.float32)).cuda()
        dl = torch.from_numpy(rng.normal(0, 1, (NS, NL, E_)).astype(np.float32)).cuda()
        dy = torch.empty((NS, NL, D_), dtype=torch.float32, device="cuda")

        def token(i):
            s_ = i % NS
            for layer in range(NL):
                rc = hip.eahmmf_hip_moe_layer_decode_async(ctypes.byref(shape), vp(tables[layer].data_ptr()), E_,
                                                           vp(dl[s_, layer].data_ptr()), K_,
                                                           vp(xs[s_, layer].data_ptr()), vp(dy[s_, layer].data_ptr()),
                                                           None, None, sp)
                assert rc == 0, b.last_error()

        steps = args.steps if args.steps else 100
        for i in range(args.warmup if args.warmup else 5):
            token(i)
        torch.cuda.synchronize()
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record(stream)
        for i in range(steps):
            token(i)
        e1.record(stream)
        torch.cuda.synchronize()
        assert hip.eahmmf_hip_device_flags() == 0
        el = e0.elapsed_time(e1) * 1e-3
        bytes_tok = NL * K_ * (2 * FF_ * grb + D_ * drb)
        results[name] = {"tokens_per_s": round(steps / el, 1), "ms_per_token": round(el * 1e3 / steps, 4),
                         "GB_s": round(bytes_tok * steps / el / 1e9, 1), "bytes_per_token": bytes_tok,
                         "pct_of_hbm_peak": round(100 * bytes_tok * steps / el / 1e9 / HBM_PEAK_GBS, 2)}
        del comps, tables
        torch.cuda.empty_cache()
    print(json.dumps({
        "metric": "expert-only decode tokens/s, 48 MoE layers of the Qwen3-30B-A3B shape", "unit": "tokens/s",
        "value": results["q4_k_m"]["tokens_per_s"], "n_gpus": 1, "higher_is_better": True, "dtype": "f32",
        "data": "synthetic",
        "config": {"workload": "one decode token through 48 resident MoE layers (D=2048 FF=768 128 experts top-8), "
                               "routing on device, one fused launch per layer; attention and the router matmul "
                               "are not part of the step"},
        "variants": results}), flush=True)


def router_variant(b, hip, torch, tables, dx, dy, dids, dw, shape, stream, R, NS, steps=400):
    """The same layer-token from the residual stream: RMSNorm + the F32
    router matmul (128 x 2048, 1 MiB) + routing + experts
    (eahmmf_hip_moe_layer_decode_xn_async, two launches); HIP events on the
    launch stream over `steps` back-to-back layer-tokens."""
    rng = np.random.default_rng(9)
    router = torch.from_numpy(rng.normal(0, 0.02, (E, D)).astype(np.float32)).cuda()
    norm_w = torch.from_numpy((1 + rng.normal(0, 0.05, D)).astype(np.float32)).cuda()
    sp, vp = ctypes.c_void_p(stream.cuda_stream), ctypes.c_void_p

    def step(i):
        s = i % NS
        rc = hip.eahmmf_hip_moe_layer_decode_xn_async(ctypes.byref(shape), vp(tables[i % R].data_ptr()), E,
                                                      vp(router.data_ptr()), vp(norm_w.data_ptr()),
                                                      ctypes.c_float(1e-6), vp(dx[s].data_ptr()), K,
                                                      vp(dy[s].data_ptr()), vp(dids[s].data_ptr()),
                                                      vp(dw[s].data_ptr()), None, None, sp)
        assert rc == 0, b.last_error()

    for i in range(50):
        step(i)
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record(stream)
    for i in range(steps):
        step(i)
    e1.record(stream)
    torch.cuda.synchronize()
    assert hip.eahmmf_hip_device_flags() == 0
    us = e0.elapsed_time(e1) * 1e3 / steps
    return {"us_per_layer_token": round(us, 3), "launches": 1,
            "what": "RMSNorm + F32 router matmul + routing + expert block from the residual stream in one "
                    "launch (eahmmf_hip_moe_layer_decode_xn_async: the router matmul split over the fused "
                    "kernel's workgroups), HIP events over back-to-back layer-tokens"}


def host_io_rate(b, hip, torch, dgate, dup, ddown, steps=2000):
    """The reference's calling convention at C2: routing on the host, then the
    synchronous eahmmf_hip_moe_decode with pageable host x / y (two 8 KB copies
    and a stream synchronisation per call).  GB/s over the routed experts' bytes."""
    rng = np.random.default_rng(7)
    xs = rng.normal(0, 1, (64, D)).astype(np.float32)
    logits = rng.normal(0, 1, (64, E)).astype(np.float32)
    grb, drb = b.row_bytes(Q4_K, D), b.row_bytes(Q6_K, FF)
    y = np.empty(D, np.float32)
    sets = []
    for s_ in range(64):
        lg = logits[s_]
        e_ = np.exp(lg - lg.max())
        ids = sorted(range(E), key=lambda i: (-e_[i], i))[:K]
        tot = np.float32(0)
        for i in ids:
            tot = np.float32(tot + np.float32(e_[i]))
        ex = (b.Expert * K)()
        w = np.array([np.float32(e_[i]) / tot for i in ids], np.float32)
        r = s_ % dgate.shape[0]
        for j, e in enumerate(ids):
            ex[j].gate = b.Weight(dgate[r, e].data_ptr(), Q4_K, D, FF, grb)
            ex[j].up = b.Weight(dup[r, e].data_ptr(), Q4_K, D, FF, grb)
            ex[j].down = b.Weight(ddown[r, e].data_ptr(), Q6_K, FF, D, drb)
        sets.append((ex, w))
    for i in range(20):
        ex, w = sets[i % 64]
        assert hip.eahmmf_hip_moe_decode(ex, w.ctypes.data, K, xs[i % 64].ctypes.data, y.ctypes.data)
    t0 = time.perf_counter()
    for i in range(steps):
        ex, w = sets[i % 64]
        assert hip.eahmmf_hip_moe_decode(ex, w.ctypes.data, K, xs[i % 64].ctypes.data, y.ctypes.data)
    el = time.perf_counter() - t0
    bytes_step = K * (2 * FF * grb + D * drb)
    return {"GB_s": round(bytes_step * steps / el / 1e9, 2), "us_per_call": round(el * 1e6 / steps, 2),
            "what": "synchronous eahmmf_hip_moe_decode, pageable host x/y, host routing outside the timed call"}


def random_blocks(rng, t, nrows, ne0):
    """Rows of valid blocks (random codes, small fp16 scales): the CPU kernel's
    time does not depend on the values."""
    blck, nbytes = {Q8_0: (32, 34), Q4_K: (256, 144), Q5_K: (256, 176), Q6_K: (256, 210)}[t]
    raw = rng.integers(0, 256, (nrows, ne0 // blck, nbytes), dtype=np.uint8)
    d = (rng.uniform(.5, 1.5, (nrows, ne0 // blck, 1)) * (3e-4 if t == Q8_0 else 3e-5)).astype(np.float16)
    d = d.view(np.uint8)
    if t == Q6_K:
        raw[:, :, 208:210] = d
    else:
        raw[:, :, 0:2] = d
        if t in (Q4_K, Q5_K):
            raw[:, :, 2:4] = d
    return raw.reshape(nrows, -1)


def c3_cpu_child(layers, etype, threads, steps, warmup=2):
    """The reference engine (oracle/_ref, compiled from the reference's
    qwen3moe.cpp) on a GGUF file of `layers` layers at the 48-layer model's
    shape (D=2048, 32/4 heads of 128, 128 experts of `etype` top-8, FF 768,
    Q8_0 attention, embedding and output head, vocab 151936): single-token
    forwards at position 2047 (a 2048-row KV cache; its contents do not change
    the work), each timed on the host clock.  In a process of its own, with
    OpenMP placement from its environment and no GPU runtime loaded."""
    import tempfile
    sys.path.insert(0, ROOT)
    sys.path.insert(0, os.path.join(ROOT, "tests"))
    import oracle
    import gguf_tools as gt
    flags = open("/proc/cpuinfo").read() if os.path.exists("/proc/cpuinfo") else ""
    avx512 = os.path.join(ROOT, "oracle", "_ref", "libref_avx512.so")
    path = avx512 if (" avx512f " in flags and os.path.exists(avx512)) else oracle.REF_PORTABLE_SO
    if not os.path.exists(path):
        print(json.dumps({"error": "the compiled reference is not built"}), flush=True)
        return
    lib = oracle.ref(path)
    D_, NH, NKV, HD, E_, K_, FF_, V = 2048, 32, 4, 128, 128, 8, 768, 151936
    rng = np.random.default_rng(21)
    spec = gt.ModelSpec(n_layer=layers, D=D_, n_head=NH, n_kv=NKV, hd=HD, n_expert=E_, n_used=K_, FF=FF_, n_vocab=V,
                        n_ctx=4096, ctx_train=4096, eps=1e-6, rope_base=1e6)

    def f32(*shape, base=0.0):
        return (base + rng.normal(0, 0.02, shape)).astype(np.float32)

    spec.add("token_embd.weight", Q8_0, [D_, V], random_blocks(rng, Q8_0, V, D_))
    spec.add("output.weight", Q8_0, [D_, V], random_blocks(rng, Q8_0, V, D_))
    spec.add("output_norm.weight", 0, [D_], f32(D_, base=1.0))
    for l in range(layers):
        p = f"blk.{l}."
        for nm, n in (("attn_norm", D_), ("ffn_norm", D_), ("attn_q_norm", HD), ("attn_k_norm", HD)):
            spec.add(p + nm + ".weight", 0, [n], f32(n, base=1.0))
        spec.add(p + "attn_q.weight", Q8_0, [D_, NH * HD], random_blocks(rng, Q8_0, NH * HD, D_))
        spec.add(p + "attn_k.weight", Q8_0, [D_, NKV * HD], random_blocks(rng, Q8_0, NKV * HD, D_))
        spec.add(p + "attn_v.weight", Q8_0, [D_, NKV * HD], random_blocks(rng, Q8_0, NKV * HD, D_))
        spec.add(p + "attn_output.weight", Q8_0, [NH * HD, D_], random_blocks(rng, Q8_0, D_, NH * HD))
        spec.add(p + "ffn_gate_inp.weight", 0, [D_, E_], f32(E_, D_))
        spec.add(p + "ffn_gate_exps.weight", etype, [D_, FF_, E_], random_blocks(rng, etype, E_ * FF_, D_))
        spec.add(p + "ffn_up_exps.weight", etype, [D_, FF_, E_], random_blocks(rng, etype, E_ * FF_, D_))
        spec.add(p + "ffn_down_exps.weight", etype, [FF_, D_, E_], random_blocks(rng, etype, E_ * D_, FF_))
    fd, gguf = tempfile.mkstemp(suffix=".gguf", dir=os.environ.get("TMPDIR", "/tmp"))
    os.close(fd)
    try:
        gt.write_gguf(spec, gguf)
        del spec
        eng = lib.ref_engine_new(gguf.encode(), 2100)
        logits = np.empty(V, np.float32)
        tok = np.array([1], np.int32)
        secs = []
        for i in range(warmup + steps):
            tok[0] = 1 + i
            t0 = time.perf_counter()
            lib.ref_engine_forward(eng, tok.ctypes.data, 1, 2047, logits.ctypes.data)
            if i >= warmup:
                secs.append(time.perf_counter() - t0)
        lib.ref_engine_free(eng)
    finally:
        os.unlink(gguf)
    print(json.dumps({"layers": layers, "threads": threads, "secs": secs, "lib": os.path.relpath(path, ROOT)}),
          flush=True)


def c3_cpu_baseline(etype, steps=8):
    """Decode tokens/s of the reference engine for the 48-layer model, from a
    bounded sample: 1- and 3-layer models of the same shape (full vocabulary
    head), median forward time each; per-layer time = (T3 - T1) / 2, the
    48-layer token = T1 + 47 x per-layer.  Every core of the host
    (OMP_PLACES=cores, OMP_PROC_BIND=close)."""
    import subprocess
    ncores = len(os.sched_getaffinity(0)) if hasattr(os, "sched_getaffinity") else (os.cpu_count() or 1)
    env = dict(os.environ, OMP_NUM_THREADS=str(ncores), OMP_PLACES="cores", OMP_PROC_BIND="close")
    med = {}
    for layers in (1, 3):
        r = subprocess.run([sys.executable, os.path.abspath(__file__), "--c3-cpu-child", str(layers),
                            "--c3-cpu-etype", str(etype), "--steps", str(steps)], env=env, capture_output=True,
                           text=True, timeout=900)
        if r.returncode != 0:
            return {"value": None, "error": r.stderr[-500:]}
        d = json.loads(r.stdout.strip().splitlines()[-1])
        if "error" in d:
            return {"value": None, "error": d["error"]}
        med[layers] = float(np.median(d["secs"]))
    per_layer = (med[3] - med[1]) / 2
    t48 = med[1] + 47 * per_layer
    return {"value": round(1.0 / t48, 3), "unit": "tokens/s", "cores": ncores, "kind": "reference",
            "sample": f"the compiled reference engine on 1- and 3-layer GGUF models of this shape (full 151936-row "
                      f"Q8_0 head), {steps} single-token forwards each at position 2047 after 2 warm-up forwards; "
                      f"median T1 {med[1] * 1e3:.2f} ms, T3 {med[3] * 1e3:.2f} ms; 48-layer token = T1 + 47 x "
                      f"(T3 - T1) / 2 = {t48 * 1e3:.1f} ms",
            "ms_per_token_48_layers": round(t48 * 1e3, 2), "ms_per_layer": round(per_layer * 1e3, 3)}


def cpu_child(threads, n_tok, reps, warmup):
    """The timed CPU leg, in a process of its own (OpenMP placement comes from
    its environment, and no GPU runtime is loaded): the reference's
    single-token expert block over n_tok C2 layer-tokens per repetition, with
    the compiled reference (oracle/_ref, AVX-512 build on an AVX-512 host) or,
    without it, the oracle's restatement."""
    sys.path.insert(0, ROOT)
    import oracle
    flags = open("/proc/cpuinfo").read() if os.path.exists("/proc/cpuinfo") else ""
    avx512 = os.path.join(ROOT, "oracle", "_ref", "libref_avx512.so")
    path = avx512 if (" avx512f " in flags and os.path.exists(avx512)) else oracle.REF_PORTABLE_SO
    dbl = ctypes.POINTER(ctypes.c_double)
    if os.path.exists(path):
        lib, kind = oracle.ref(path), "reference"
        fn = lib.ref_time_expert_tokens
    else:
        lib, kind = oracle.lib(), "port"
        fn = lib.orc_time_expert_tokens
        path = "oracle/liboracle.so"
    fn.argtypes = [ctypes.c_int] * 4 + [ctypes.c_size_t] * 2 + [ctypes.c_void_p] * 6 + [ctypes.c_int] * 5 + [dbl]
    rng = np.random.default_rng(5)
    gate = random_blocks(rng, Q4_K, E * FF, D)  # first touched here, by this process
    up = random_blocks(rng, Q4_K, E * FF, D)
    down = random_blocks(rng, Q6_K, E * D, FF)
    grb, drb = gate.shape[1], down.shape[1]
    xs = rng.normal(0, 1, (n_tok, D)).astype(np.float32)
    ids, w = oracle.route_topk(rng.normal(0, 1, (n_tok, E)).astype(np.float32), K)
    order = np.argsort(ids, axis=1, kind="stable")  # the reference's loop runs the experts in ascending id
    ids = np.ascontiguousarray(np.take_along_axis(ids, order, 1)).astype(np.int32)
    w = np.ascontiguousarray(np.take_along_axis(w, order, 1)).astype(np.float32)
    secs = np.zeros(reps, dtype=np.float64)
    rc = fn(Q4_K, Q6_K, D, FF, grb, drb, gate.ctypes.data, up.ctypes.data, down.ctypes.data, xs.ctypes.data,
            ids.ctypes.data, w.ctypes.data, K, n_tok, threads, warmup, reps, secs.ctypes.data_as(dbl))
    assert rc == 0
    print(json.dumps({"kind": kind, "lib": os.path.relpath(path, ROOT), "threads": threads, "n_tok": n_tok,
                      "secs": secs.tolist()}), flush=True)


def cpu_baseline(n_tok, reps=21, warmup=3):
    """The reference CPU expert path timed on the host's cores by the planned
    protocol: a child process per setting, (a) every core of the NUMA node
    (OMP_PLACES=cores, OMP_PROC_BIND=close) and (b) 4 threads, warm-up 3,
    median of 21 repetitions with p10/p90; a repetition is n_tok C2
    layer-tokens (routing, then 8 experts each)."""
    import subprocess
    ncores = len(os.sched_getaffinity(0)) if hasattr(os, "sched_getaffinity") else (os.cpu_count() or 1)
    bytes_tok = K * (2 * FF * (D // 256 * 144) + D * (FF // 256 * 210))
    settings = []
    for threads in dict.fromkeys((ncores, 4)):
        env = dict(os.environ, OMP_NUM_THREADS=str(threads), OMP_PLACES="cores", OMP_PROC_BIND="close")
        r = subprocess.run([sys.executable, os.path.abspath(__file__), "--cpu-child", str(threads),
                            "--cpu-tokens", str(n_tok)], env=env, capture_output=True, text=True, timeout=600)
        if r.returncode != 0:
            return {"value": None, "error": r.stderr[-500:]}
        d = json.loads(r.stdout.strip().splitlines()[-1])
        t = np.array(d["secs"])
        med = float(np.median(t))
        settings.append({"threads": threads, "median_s": round(med, 5), "p10_s": round(float(np.percentile(t, 10)), 5),
                         "p90_s": round(float(np.percentile(t, 90)), 5),
                         "GB_s": round(bytes_tok * n_tok / med / 1e9, 3),
                         "layer_tokens_per_s": round(n_tok / med, 1), "kind": d["kind"], "lib": d["lib"]})
    top = settings[0]
    return {"value": top["GB_s"], "unit": "GB/s", "cores": top["threads"], "kind": top["kind"],
            "sample": f"{reps} repetitions (after {warmup} warm-up) of {n_tok} single-token C2 layer "
                      f"evaluations (8 routed experts each, 24.5 MB of weights per token, over a 391.6 MB "
                      f"layer) timed in C++ around the reference's matmul loop; median, p10/p90 per setting",
            "settings": settings,
            "host": {"cpus": ncores, "model": cpu_model()}}


def cpu_model():
    try:
        for line in open("/proc/cpuinfo"):
            if line.startswith("model name"):
                return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return None


def measured_traffic(fused):
    """HBM bytes per launch of the fused kernel at this workload, from the
    committed rocprofv3 FETCH_SIZE/WRITE_SIZE passes (scaled by a plain copy's
    counters); None when the two-kernel path runs or no measurement exists."""
    path = os.path.join(ROOT, "profiles", "moe_decode_fused_c2_hbm_traffic.json")
    if not fused or not os.path.exists(path):
        return None
    with open(path) as f:
        return int(json.load(f)["traffic_bytes"])


def calibrate_copy(torch, steps):
    """A plain device-to-device copy of COPY_BYTES, timed with HIP events.  Under
    rocprofv3 --pmc its FETCH_SIZE / WRITE_SIZE per dispatch should read
    COPY_BYTES each; the ratio scales the same counters of the expert kernel."""
    n = COPY_BYTES // 4
    src = torch.randn(n, device="cuda")
    dst = torch.empty_like(src)
    st = torch.cuda.current_stream()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    dst.copy_(src)
    torch.cuda.synchronize()
    e0.record(st)
    for _ in range(steps):
        dst.copy_(src)
    e1.record(st)
    torch.cuda.synchronize()
    us = e0.elapsed_time(e1) * 1e3 / steps
    print(json.dumps({"copy_bytes": COPY_BYTES, "dispatches": steps + 1, "avg_us": round(us, 3),
                      "read_plus_write_GBs": round(2 * COPY_BYTES / (us * 1e-6) / 1e9, 1)}), flush=True)


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=None, help="timed steps (c2 2000, c4 50, c5 1000)")
    ap.add_argument("--warmup", type=int, default=None, help="untimed steps (c2 100, c4 5, c5 50)")
    ap.add_argument("--replicas", type=int, default=None, help="layer copies in HBM (c2 16, c4 4, c5 4)")
    ap.add_argument("--cpu-tokens", type=int, default=64, help="C2 layer-tokens per CPU-baseline repetition")
    ap.add_argument("--cpu-child", type=int, default=0, help=argparse.SUPPRESS)
    ap.add_argument("--c3-cpu-child", type=int, default=0, help=argparse.SUPPRESS)
    ap.add_argument("--c3-cpu-etype", type=int, default=Q5_K, help=argparse.SUPPRESS)
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--no-model", action="store_true", help="default line: skip the whole-model decode figure")
    ap.add_argument("--workload", choices=("c2", "c3", "c3x", "c4", "c5", "c5b16", "c5seq", "stream", "staging",
                                           "dropin"), default="c2",
                    help="c2 (default): the headline single-token layer; c3: one decode token through the whole "
                         "48-layer model; c3x: the 48 layers' expert blocks only; "
                         "c4: ragged grouped prefill; c5: single-token layer at the 235B shape; "
                         "c5b16: a 16-sequence decode batch at the 235B shape (one layer's expert block); "
                         "c5seq: 16 sequences decoded together through the whole 94-layer 235B-shaped model; "
                         "stream: the achievable HBM read rate (streaming-read kernel); "
                         "staging: making one layer's experts resident from host memory; "
                         "dropin: a C2 layer-token through the drop-in matmul calls")
    ap.add_argument("--calibrate-copy", action="store_true",
                    help="only run a plain 256 MiB device copy (the reference kernel for scaling HBM counters)")
    args = ap.parse_args()
    if args.cpu_child:
        cpu_child(args.cpu_child, args.cpu_tokens, 21, 3)
        return
    if args.c3_cpu_child:
        c3_cpu_child(args.c3_cpu_child, args.c3_cpu_etype, int(os.environ.get("OMP_NUM_THREADS", "1")),
                     args.steps or 8)
        return
    if args.workload == "c2":
        args.steps = 2000 if args.steps is None else args.steps
        args.warmup = 100 if args.warmup is None else args.warmup
        args.replicas = 16 if args.replicas is None else args.replicas
    if args.gpus != 1:
        print(f"bench.py runs on one GPU only (asked for --gpus {args.gpus}); the expert path would shard by "
              "expert across GPUs, and no multi-GPU run is made here", file=sys.stderr)
        sys.exit(2)

    import torch
    if args.calibrate_copy:
        calibrate_copy(torch, args.steps or 20)
        return
    b = load_binding()
    if args.workload != "c2":
        hip_ = b.lib()
        torch.cuda.set_device(0)
        {"c3": bench_c3, "c3x": bench_c3_experts, "c4": bench_c4, "c5": bench_c5, "c5b16": bench_c5_batch, "c5seq": bench_c5_seqs, "stream": bench_stream,
         "staging": bench_staging, "dropin": bench_dropin}[args.workload](args, torch, b, hip_)
        return
    hip = b.lib()
    torch.cuda.set_device(0)
    rng = np.random.default_rng(0)
    t_gen = time.perf_counter()
    gate, up, down = build_layer(b, rng)
    print(f"# quantized one layer ({gate.nbytes + up.nbytes + down.nbytes} B) in "
          f"{time.perf_counter() - t_gen:.1f} s", file=sys.stderr, flush=True)
    R = args.replicas
    dgate = torch.empty((R,) + gate.shape, dtype=torch.uint8, device="cuda")
    dup = torch.empty((R,) + up.shape, dtype=torch.uint8, device="cuda")
    ddown = torch.empty((R,) + down.shape, dtype=torch.uint8, device="cuda")
    hg, hu, hd = (torch.from_numpy(a).pin_memory() for a in (gate, up, down))
    for r in range(R):
        dgate[r].copy_(hg)
        dup[r].copy_(hu)
        ddown[r].copy_(hd)
    torch.cuda.synchronize()
    tables = []
    for r in range(R):
        t = np.array([[dgate[r, e].data_ptr(), dup[r, e].data_ptr(), ddown[r, e].data_ptr()] for e in range(E)],
                     dtype=np.uint64)
        tables.append(torch.from_numpy(t.view(np.int64)).cuda())
    NS = 64
    xs = rng.normal(0, 1, (NS, D)).astype(np.float32)
    logits = rng.normal(0, 1, (NS, E)).astype(np.float32)
    dx = torch.from_numpy(xs).cuda()
    dlog = torch.from_numpy(logits).cuda()
    dids = torch.empty((NS, K), dtype=torch.int32, device="cuda")
    dw = torch.empty((NS, K), dtype=torch.float32, device="cuda")
    dy = torch.empty((NS, D), dtype=torch.float32, device="cuda")
    shape = b.MoeShape(Q4_K, Q4_K, Q6_K, D, FF, b.row_bytes(Q4_K, D), b.row_bytes(Q4_K, D), b.row_bytes(Q6_K, FF))
    stream = torch.cuda.current_stream()
    sp = ctypes.c_void_p(stream.cuda_stream)
    vp = ctypes.c_void_p

    # the call's arguments per input slot, formed once (device pointers of
    # resident buffers): the timed loop is the library call itself
    period = NS * R // math.gcd(NS, R)  # step i: input slot i % NS, layer replica i % R
    call_args = [(ctypes.byref(shape), vp(tables[i % R].data_ptr()), E, vp(dlog[i % NS].data_ptr()), K,
                  vp(dx[i % NS].data_ptr()), vp(dy[i % NS].data_ptr()), vp(dids[i % NS].data_ptr()),
                  vp(dw[i % NS].data_ptr()), sp) for i in range(period)]
    layer_call = hip.eahmmf_hip_moe_layer_decode_async

    def step(i):
        rc = layer_call(*call_args[i % period])
        if rc != 0:
            raise RuntimeError(b.last_error())

    for i in range(args.warmup):
        step(i)
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for i in range(args.steps):
        step(args.warmup + i)
    torch.cuda.synchronize()
    el = time.perf_counter() - t0
    assert hip.eahmmf_hip_device_flags() == 0, "a fused launch ran out of its bounded wait"
    fused = bool(hip.eahmmf_hip_set_fused(-1))
    kernel_name = ("moe_decode_fused (routing + gate/up + down in one launch)" if fused
                   else "route_topk + moe_gate_up + moe_down")
    bytes_step = K * (2 * FF * b.row_bytes(Q4_K, D) + D * b.row_bytes(Q6_K, FF))
    value = bytes_step * args.steps / el / 1e9
    ms = el * 1e3 / args.steps

    # the layer kernel's average launch duration: HIP events on the launch
    # stream bracketing n_ev back-to-back launches (each step is one launch)
    n_ev = 400
    ev0, ev1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    ev0.record(stream)
    for i in range(n_ev):
        step(i)
    ev1.record(stream)
    torch.cuda.synchronize()
    kern_us = ev0.elapsed_time(ev1) * 1e3 / n_ev
    achieved = bytes_step / (kern_us * 1e-6) / 1e9
    # spread: per-launch event pairs (each includes the events' own overhead)
    n_sp = 200
    ev = [(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)) for _ in range(n_sp)]
    for i in range(n_sp):
        ev[i][0].record(stream)
        step(i)
        ev[i][1].record(stream)
    torch.cuda.synchronize()
    durs = np.array([a.elapsed_time(z) for a, z in ev]) * 1e3  # us

    out = {
        "metric": "expert-FFN HBM GB/s (% of peak) + decode tokens/s at Qwen3-30B-A3B Q4_K_M",
        "value": round(value, 2), "unit": "GB/s", "n_gpus": 1, "steps": args.steps, "warmup": args.warmup,
        "ms_per_step": round(ms, 5), "higher_is_better": True, "scaling": "weak", "vs_baseline": None,
        "dtype": "f32", "data": "synthetic",
        "config": {"workload": "single MoE layer, one decode token, Qwen3-30B-A3B shape: D=2048 FF=768 128 experts "
                               "top-8, gate/up Q4_K + down Q6_K (Q4_K_M), routing on device",
                   "bytes_per_step": bytes_step, "layer_replicas": R, "hbm_resident_bytes": int(
                       R * (gate.nbytes + up.nbytes + down.nbytes))},
        "pct_of_hbm_peak": round(100 * value / HBM_PEAK_GBS, 2),
        "expert_only_decode_tokens_per_s_48_layers": round(1.0 / (48 * ms * 1e-3), 1),
        "roofline": {"bound": "hbm", "kernel": kernel_name,
                     "achieved": round(achieved, 2), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": round(achieved / HBM_PEAK_GBS, 4), "traffic": measured_traffic(fused),
                     "avg_us": round(kern_us, 3),
                     "p10_us_with_event_overhead": round(float(np.percentile(durs, 10)), 3),
                     "p90_us_with_event_overhead": round(float(np.percentile(durs, 90)), 3),
                     "xcd_local_exchange": int(hip.eahmmf_hip_fused_exchange())},
    }
    out["router_from_activations"] = router_variant(b, hip, torch, tables, dx, dy, dids, dw, shape, stream, R, NS)
    out["host_io"] = host_io_rate(b, hip, torch, dgate, dup, ddown)
    # the measured read ceiling at the same launch size, timed the same way
    sr = stream_rates(torch, hip)
    sr["frac_of_c2_size_cold"] = round(achieved / sr["c2_size_cold_GB_s"], 4)
    out["stream_read"] = sr
    # the second half of the metric, measured: whole-model single-token decode at the
    # Qwen3-30B-A3B shape with Q4_K_M experts (every layer on the device, 2048-token
    # context), after the layer replicas are freed
    if not args.no_model:
        del dgate, dup, ddown, tables
        torch.cuda.empty_cache()
        r = c3_decode(torch, b, Q4_K, (Q4_K, Q4_K, Q6_K), 2048, 32, 4, np.random.default_rng(5))
        out["decode_tokens_per_s_q4_k_m_48_layers"] = r["tokens_per_s"]
        out["decode_q4_k_m"] = dict(r, what="eahmmf_hip_model_generate_greedy, 32 tokens at a 2048-token KV "
                                    "context, 48 layers (attention, norms, router, fused experts, head on the device)")
    if not args.no_cpu_baseline:
        out["cpu_baseline"] = cpu_baseline(args.cpu_tokens)
    print(json.dumps(out), flush=True)


if __name__ == "__main__":
    main()
