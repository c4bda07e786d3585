"""HIP path vs the oracle, through the C ABI (MI355X).

Bars: dequantized weights and top-k expert ids
bit-exact; outputs within 1e-3 relative / 1e-4 absolute of the oracle's fp32
result: |gpu - oracle| <= 1e-4 + 1e-3 * |oracle| elementwise.
"""
import ctypes
import os

import numpy as np
import pytest

import oracle
import synth
from conftest import GOLDEN

pytestmark = pytest.mark.gpu

RTOL, ATOL = 1e-3, 1e-4
Q8_0, Q4_K, Q5_K, Q6_K = 8, 12, 13, 14


def close(got, want):
    err = np.abs(got.astype(np.float64) - want.astype(np.float64))
    lim = ATOL + RTOL * np.abs(want.astype(np.float64))
    bad = err > lim
    assert not bad.any(), f"{bad.sum()} of {bad.size} outside tolerance; max err {err.max():.3e}"


@pytest.fixture(scope="module")
def torch_dev():
    import torch
    assert torch.cuda.is_available()
    return torch


def to_dev(torch, a):
    return torch.from_numpy(np.ascontiguousarray(a)).cuda()


def ptr(t):
    return ctypes.c_void_p(t.data_ptr())


# ---------------------------------------------------------------------------
# dequantization: bit-exact

@pytest.mark.parametrize("t", [Q8_0, Q4_K, Q5_K, Q6_K])
def test_dequant_golden_bit_exact(torch_dev, hip, t):
    torch = torch_dev
    g = np.load(os.path.join(GOLDEN, "dequant_golden.npz"))
    blocks, want = g[f"blocks_{t}"], g[f"values_{t}"]
    blck = oracle.BLOCK[t][0]
    dw = to_dev(torch, blocks)
    out = torch.empty((blocks.shape[0], blck), dtype=torch.float32, device="cuda")
    rc = hip.eahmmf_hip_dequantize(ptr(dw), t, blck, blocks.shape[0], blocks.shape[1], ptr(out), None)
    assert rc == 0, hip.eahmmf_hip_last_error()
    torch.cuda.synchronize()
    got = out.cpu().numpy()
    assert np.array_equal(got.view(np.uint32), want.view(np.uint32))


@pytest.mark.parametrize("t,rows,ne0", [(Q4_K, 768, 2048), (Q6_K, 2048, 768), (Q5_K, 768, 2048), (Q8_0, 2048, 768),
                                        (Q8_0, 37, 96), (Q6_K, 9, 1536)])
def test_dequant_expert_shapes_bit_exact(torch_dev, hip, t, rows, ne0):
    torch = torch_dev
    rng = np.random.default_rng(rows + ne0 + t)
    w = synth.random_rows(t, rows, ne0, rng)
    dw = to_dev(torch, w)
    out = torch.empty((rows, ne0), dtype=torch.float32, device="cuda")
    rc = hip.eahmmf_hip_dequantize(ptr(dw), t, ne0, rows, w.shape[1], ptr(out), None)
    assert rc == 0, hip.eahmmf_hip_last_error()
    torch.cuda.synchronize()
    want = oracle.dequant_rows(t, w, ne0)
    assert np.array_equal(out.cpu().numpy().view(np.uint32), want.view(np.uint32))


# ---------------------------------------------------------------------------
# drop-in matmul / pair (host buffers, synchronous)

MATMUL_CASES = [
    (Q4_K, 2048, 768, 1), (Q4_K, 2048, 768, 3), (Q6_K, 768, 2048, 1), (Q6_K, 768, 2048, 8), (Q5_K, 2048, 64, 13),
    (Q8_0, 2048, 96, 5), (Q8_0, 128, 256, 2), (Q8_0, 96, 17, 3), (Q6_K, 1536, 40, 64), (Q4_K, 4096, 33, 9),
    (Q5_K, 256, 256, 4),
    # the matrix-core path at its edges: 16 splits of the K range (few rows),
    # ragged token tiles (17, 33), 64 tokens, rows not a multiple of 64
    (Q4_K, 4096, 512, 16), (Q5_K, 2048, 100, 33), (Q6_K, 4096, 130, 17), (Q8_0, 8192, 70, 64),
    (Q8_0, 4096, 1000, 2), (Q6_K, 256, 4100, 48),
]


@pytest.mark.parametrize("t,ne0,ne1,nb", MATMUL_CASES)
def test_matmul_vs_oracle(torch_dev, hip, t, ne0, ne1, nb):
    torch = torch_dev
    rng = np.random.default_rng(ne0 * 7 + ne1 + nb)
    w = synth.random_rows(t, ne1, ne0, rng)
    x = rng.normal(0, 1, (nb, ne0)).astype(np.float32)
    dw = to_dev(torch, w)
    ldx, ldo = ne0 + 3, ne1 + 5
    xh = np.zeros((nb, ldx), dtype=np.float32)
    xh[:, :ne0] = x
    out = np.full((nb, ldo), 7.0, dtype=np.float32)
    ok = hip.eahmmf_hip_matmul(ptr(dw), t, ne0, ne1, w.shape[1], xh.ctypes.data, nb, ldx, out.ctypes.data, ldo)
    assert ok, hip.eahmmf_hip_last_error()
    close(out[:, :ne1], oracle.matmul(t, w, ne0, x))
    assert np.all(out[:, ne1:] == 7.0)  # padding untouched


@pytest.mark.parametrize("t,ne0,ne1,nb", [(Q4_K, 2048, 96, 5), (Q5_K, 4096, 40, 16), (Q6_K, 1536, 70, 33),
                                          (Q8_0, 2048, 130, 8)])
def test_matmul_general_kernel_vs_oracle(torch_dev, hip, t, ne0, ne1, nb):
    """The general (vector-ALU) matmul kernel, with the matrix-core path
    switched off, on shapes the matrix-core path would otherwise take."""
    prev = hip.eahmmf_hip_set_dense_mfma(0)
    try:
        test_matmul_vs_oracle(torch_dev, hip, t, ne0, ne1, nb)
    finally:
        hip.eahmmf_hip_set_dense_mfma(prev)


@pytest.mark.parametrize("t,pad", [(Q4_K, 48), (Q6_K, 6), (Q8_0, 2), (Q5_K, 16)])
def test_matmul_padded_row_stride(torch_dev, hip, t, pad):
    """Rows at a stride longer than their blocks (the reference's matmul
    takes any row_bytes, expert_cuda.cu:263-267): the padding is skipped."""
    torch = torch_dev
    ne0, ne1, nb = 512, 40, 3
    rng = np.random.default_rng(t * 100 + pad)
    w = synth.random_rows(t, ne1, ne0, rng)
    wp = np.concatenate([w, rng.integers(0, 256, (ne1, pad), dtype=np.uint8)], axis=1)
    x = rng.normal(0, 1, (nb, ne0)).astype(np.float32)
    dw = to_dev(torch, wp)
    out = np.empty((nb, ne1), dtype=np.float32)
    assert hip.eahmmf_hip_matmul(ptr(dw), t, ne0, ne1, wp.shape[1], x.ctypes.data, nb, ne0, out.ctypes.data, ne1), \
        hip.eahmmf_hip_last_error()
    close(out, oracle.matmul(t, w, ne0, x))


def test_matmul_golden_cases(torch_dev, hip):
    torch = torch_dev
    g = np.load(os.path.join(GOLDEN, "matmul_golden.npz"))
    i = 0
    while f"case{i}_meta" in g:
        t, ne0, ne1, nb = (int(v) for v in g[f"case{i}_meta"])
        w, x, want = g[f"case{i}_w"], g[f"case{i}_x"], g[f"case{i}_y"]
        dw = to_dev(torch, w)
        out = np.empty((nb, ne1), dtype=np.float32)
        assert hip.eahmmf_hip_matmul(ptr(dw), t, ne0, ne1, w.shape[1], x.ctypes.data, nb, ne0, out.ctypes.data, ne1), \
            hip.eahmmf_hip_last_error()
        # golden W carries wide random scales: compare relative to the row scale
        scale = np.abs(want).max()
        assert np.abs(out - want).max() <= 1e-5 * scale + 1e-4
        i += 1


@pytest.mark.parametrize("gt_,ut,nb", [(Q4_K, Q4_K, 1), (Q5_K, Q4_K, 4), (Q8_0, Q8_0, 7)])
def test_matmul_pair_vs_oracle(torch_dev, hip, gt_, ut, nb):
    torch = torch_dev
    ne0, ne1 = 512, 96
    rng = np.random.default_rng(nb)
    gw = synth.random_rows(gt_, ne1, ne0, rng)
    uw = synth.random_rows(ut, ne1, ne0, rng)
    x = rng.normal(0, 1, (nb, ne0)).astype(np.float32)
    dg, du = to_dev(torch, gw), to_dev(torch, uw)
    g = np.empty((nb, ne1), dtype=np.float32)
    u = np.empty((nb, ne1), dtype=np.float32)
    ok = hip.eahmmf_hip_matmul_pair(ptr(dg), gt_, ne0, ne1, gw.shape[1], ptr(du), ut, ne0, ne1, uw.shape[1],
                                    x.ctypes.data, nb, ne0, g.ctypes.data, ne1, u.ctypes.data, ne1)
    assert ok, hip.eahmmf_hip_last_error()
    close(g, oracle.matmul(gt_, gw, ne0, x))
    close(u, oracle.matmul(ut, uw, ne0, x))


# ---------------------------------------------------------------------------
# fused single-token expert block

def make_layer(binding, types, D, FF, n_expert, rng, quantized=True):
    gtp, utp, dtp = types
    ex = []
    for _ in range(n_expert):
        if quantized:
            g = synth.quantized_rows(binding, gtp, FF, D, rng)
            u = synth.quantized_rows(binding, utp, FF, D, rng)
            d = synth.quantized_rows(binding, dtp, D, FF, rng)
        else:
            g = synth.random_rows(gtp, FF, D, rng)
            u = synth.random_rows(utp, FF, D, rng)
            d = synth.random_rows(dtp, D, FF, rng)
        ex.append(((gtp, g), (utp, u), (dtp, d)))
    return ex


DECODE_CASES = [
    ("c1_q8_0", (Q8_0, Q8_0, Q8_0), 256, 128, 8, 2),
    ("tiny_mix", (Q5_K, Q4_K, Q6_K), 256, 256, 8, 2),
    ("d768_two_kernel_only", (Q4_K, Q4_K, Q6_K), 768, 256, 8, 4),
    ("q6_k_gate_up", (Q6_K, Q6_K, Q4_K), 1024, 512, 8, 4),
    ("c2_q4_k_m", (Q4_K, Q4_K, Q6_K), 2048, 768, 16, 8),
    ("c3_q5_k", (Q5_K, Q5_K, Q5_K), 2048, 768, 8, 8),
    ("c3_q8_0", (Q8_0, Q8_0, Q8_0), 2048, 768, 8, 8),
    ("c5_q4_k_m", (Q4_K, Q4_K, Q6_K), 4096, 1536, 8, 8),
    ("ff192_q8_0_odd_segments", (Q8_0, Q8_0, Q8_0), 512, 192, 8, 8),
]


@pytest.fixture(params=[1, 0], ids=["fused", "two_kernel"])
def path(request, hip):
    prev = hip.eahmmf_hip_set_fused(request.param)
    yield request.param
    hip.eahmmf_hip_set_fused(prev)
    assert hip.eahmmf_hip_device_flags() == 0  # no fused launch ran out of its bounded wait


@pytest.mark.parametrize("name,types,D,FF,E,k", DECODE_CASES, ids=[c[0] for c in DECODE_CASES])
def test_moe_decode_vs_oracle(torch_dev, binding, hip, path, name, types, D, FF, E, k):
    torch = torch_dev
    rng = np.random.default_rng(D + FF + k)
    layer = make_layer(binding, types, D, FF, E, rng)
    x = rng.normal(0, 1, (1, D)).astype(np.float32)
    logits = rng.normal(0, 1, (1, E)).astype(np.float32)
    ids, w = oracle.route_topk(logits, k)
    want = oracle.moe_layer(layer, x, ids, w)[0]
    dev = [[to_dev(torch, layer[e][c][1]) for c in range(3)] for e in range(E)]
    experts = (binding.Expert * k)()
    for j in range(k):
        e = int(ids[0, j])
        for c, (nm, ne0, ne1) in enumerate((("gate", D, FF), ("up", D, FF), ("down", FF, D))):
            t = layer[e][c][0]
            setattr(experts[j], nm, binding.Weight(dev[e][c].data_ptr(), t, ne0, ne1, binding.row_bytes(t, ne0)))
    y = np.empty(D, dtype=np.float32)
    wk = np.ascontiguousarray(w[0])
    assert hip.eahmmf_hip_moe_decode(experts, wk.ctypes.data, k, x.ctypes.data, y.ctypes.data), \
        hip.eahmmf_hip_last_error()
    close(y, want)


def test_moe_decode_resident_subset(torch_dev, binding, hip, path):
    """Partial residency (eahmmf.h:721-742): 3 of 8 routed experts have no
    device copy.  The GPU computes the resident five and reports the other
    three; their contributions added on the CPU (the oracle) give the
    oracle's whole block."""
    torch = torch_dev
    D, FF, k = 2048, 768, 8
    rng = np.random.default_rng(2024)
    layer = make_layer(binding, (Q4_K, Q4_K, Q6_K), D, FF, k, rng)
    x = rng.normal(0, 1, (1, D)).astype(np.float32)
    ids = np.arange(k, dtype=np.int32)[None, :]
    w = rng.uniform(0.05, 1.0, (1, k)).astype(np.float32)
    w /= w.sum()
    missing = [1, 4, 6]
    dev = [[to_dev(torch, layer[e][c][1]) for c in range(3)] for e in range(k)]
    experts = (binding.Expert * k)()
    for j in range(k):
        for c, (nm, ne0, ne1) in enumerate((("gate", D, FF), ("up", D, FF), ("down", FF, D))):
            t = layer[j][c][0]
            p = 0 if j in missing else dev[j][c].data_ptr()
            setattr(experts[j], nm, binding.Weight(p, t, ne0, ne1, binding.row_bytes(t, ne0)))
    y = np.full(D, np.nan, dtype=np.float32)
    mask = ctypes.c_uint32(0xFFFF)
    wk = np.ascontiguousarray(w[0])
    assert hip.eahmmf_hip_moe_decode_resident(experts, wk.ctypes.data, k, x.ctypes.data, y.ctypes.data,
                                              ctypes.byref(mask)), binding.last_error()
    assert mask.value == sum(1 << j for j in missing)
    keep = np.array([j for j in range(k) if j not in missing])
    close(y, oracle.moe_layer(layer, x, ids[:, keep], w[:, keep])[0])
    cpu = oracle.moe_layer(layer, x, ids[:, missing], w[:, missing])[0]
    close(y + cpu, oracle.moe_layer(layer, x, ids, w)[0])
    # none resident: zeros and a full mask, no launch
    for j in range(k):
        experts[j].gate.dev = 0
    assert hip.eahmmf_hip_moe_decode_resident(experts, wk.ctypes.data, k, x.ctypes.data, y.ctypes.data,
                                              ctypes.byref(mask))
    assert mask.value == (1 << k) - 1 and not y.any()


@pytest.mark.parametrize("nbytes", [16, 4096 + 48, 3 * (1 << 20) + 16 * 37, 24_477_696, (1 << 28) + 4096 + 48])
def test_stream_read_checksum(torch_dev, hip, nbytes):
    """The streaming-read kernel reads every byte once: the XOR of the 4096
    sink words (pre-filled with garbage) is the XOR of all 32-bit words of
    the buffer (sizes cover one partial batch, a ragged tail, the C2 expert
    bytes and more than 4096 full chunks)."""
    torch = torch_dev
    rng = np.random.default_rng(nbytes % 100003)
    host = rng.integers(0, 2**32, nbytes // 4, dtype=np.uint32)
    dbuf = to_dev(torch, host.view(np.int32))
    dsink = to_dev(torch, rng.integers(0, 2**32, 4096, dtype=np.uint32).view(np.int32))
    stream = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
    assert hip.eahmmf_hip_stream_read_async(ptr(dbuf), nbytes, ptr(dsink), stream) == 0, hip.eahmmf_hip_last_error()
    torch.cuda.synchronize()
    got = np.bitwise_xor.reduce(dsink.cpu().numpy().view(np.uint32))
    assert got == np.bitwise_xor.reduce(host)


def test_h2d_batch_round_trip(torch_dev, binding, hip):
    """Bulk staging through the pinned ring: copies from pageable numpy arrays
    (a C2 layer's worth of expert components plus odd sizes spanning and
    filling ring slots) land byte for byte."""
    torch = torch_dev
    rng = np.random.default_rng(11)
    sizes = [884736, 884736, 1290240] * 8 + [1, 4097, 32 << 20, (40 << 20) + 123, 0]
    host = [rng.integers(0, 256, n, dtype=np.uint8) for n in sizes]
    dev = [torch.empty(max(n, 1), dtype=torch.uint8, device="cuda") for n in sizes]
    copies = (binding.Copy * len(sizes))()
    for i, n in enumerate(sizes):
        copies[i] = binding.Copy(dev[i].data_ptr(), host[i].ctypes.data, n)
    assert hip.eahmmf_hip_h2d_batch(copies, len(sizes)) == 0, hip.eahmmf_hip_last_error()
    for h, d, n in zip(host, dev, sizes):
        assert np.array_equal(d[:n].cpu().numpy(), h)


def test_h2d_batch_async_round_trip(torch_dev, binding, hip):
    """Asynchronous staging: two batches queued back to back return at once
    with increasing tickets; one is waited for on a stream (a copy queued on
    that stream afterwards sees its bytes), the other on the host; both land
    byte for byte, query then reports them landed, and the synchronous form
    still works after them."""
    import ctypes
    torch = torch_dev
    rng = np.random.default_rng(12)
    batches = [[884736, 1290240, 1, 4097, (33 << 20) + 5], [0, 1290240, 32 << 20, 77]]
    host, dev, tickets = [], [], []
    for sizes in batches:
        h = [rng.integers(0, 256, n, dtype=np.uint8) for n in sizes]
        d = [torch.empty(max(n, 1), dtype=torch.uint8, device="cuda") for n in sizes]
        cp = (binding.Copy * len(sizes))()
        for i, n in enumerate(sizes):
            cp[i] = binding.Copy(d[i].data_ptr(), h[i].ctypes.data, n)
        t = ctypes.c_uint64(0)
        assert hip.eahmmf_hip_h2d_batch_async(cp, len(sizes), ctypes.byref(t)) == 0, hip.eahmmf_hip_last_error()
        host.append(h)
        dev.append(d)
        tickets.append(t.value)
    assert 0 < tickets[0] < tickets[1]
    assert hip.eahmmf_hip_h2d_batch_query(tickets[1] + 1000) == -1
    st = torch.cuda.Stream()
    assert hip.eahmmf_hip_h2d_batch_wait(tickets[0], ctypes.c_void_p(st.cuda_stream)) == 0
    with torch.cuda.stream(st):
        got0 = [x.clone() for x in dev[0]]
    st.synchronize()
    assert hip.eahmmf_hip_h2d_batch_wait(tickets[1], None) == 0
    for h, d in zip(host[0], got0):
        assert np.array_equal(d[:len(h)].cpu().numpy(), h)
    for h, d in zip(host[1], dev[1]):
        assert np.array_equal(d[:len(h)].cpu().numpy(), h)
    assert hip.eahmmf_hip_h2d_batch_query(tickets[0]) == 1
    assert hip.eahmmf_hip_h2d_batch_query(tickets[1]) == 1
    x = rng.integers(0, 256, 4099, dtype=np.uint8)
    y = torch.empty(4099, dtype=torch.uint8, device="cuda")
    one = (binding.Copy * 1)(binding.Copy(y.data_ptr(), x.ctypes.data, 4099))
    assert hip.eahmmf_hip_h2d_batch(one, 1) == 0
    assert np.array_equal(y.cpu().numpy(), x)


def test_route_topk_vs_oracle(torch_dev, hip):
    rng = np.random.default_rng(3)
    nb, E, k = 257, 128, 8
    logits = rng.normal(0, 1, (nb, E)).astype(np.float32)
    logits[0, 5] = logits[0, 9] = 4.0  # exact tie: lower id first
    logits[1, :] = 0.5
    ids = np.empty((nb, k), dtype=np.int32)
    w = np.empty((nb, k), dtype=np.float32)
    assert hip.eahmmf_hip_route_topk(logits.ctypes.data, nb, E, k, ids.ctypes.data, w.ctypes.data)
    oids, ow = oracle.route_topk(logits, k)
    assert np.array_equal(ids, oids)
    np.testing.assert_allclose(w, ow, rtol=1e-6, atol=0)  # device expf vs glibc expf: a few ulps


def test_moe_decode_async_and_routed(torch_dev, binding, hip, path):
    """Device-resident activations: direct slots and the routed variant (ids
    and weights produced on the device by route_topk) give the oracle's answer."""
    torch = torch_dev
    D, FF, E, k = 2048, 768, 32, 8
    rng = np.random.default_rng(99)
    layer = make_layer(binding, (Q4_K, Q4_K, Q6_K), D, FF, E, rng)
    x = rng.normal(0, 1, (1, D)).astype(np.float32)
    logits = rng.normal(0, 1, (1, E)).astype(np.float32)
    ids, w = oracle.route_topk(logits, k)
    want = oracle.moe_layer(layer, x, ids, w)[0]
    dev = [[to_dev(torch, layer[e][c][1]) for c in range(3)] for e in range(E)]
    shape = binding.MoeShape(Q4_K, Q4_K, Q6_K, D, FF, binding.row_bytes(Q4_K, D), binding.row_bytes(Q4_K, D),
                             binding.row_bytes(Q6_K, FF))
    stream = torch.cuda.current_stream().cuda_stream
    dx = to_dev(torch, x)
    dy = torch.full((D,), float("nan"), device="cuda")
    slots = (binding.ExpertPtrs * k)(*[binding.ExpertPtrs(*[dev[int(e)][c].data_ptr() for c in range(3)])
                                       for e in ids[0]])
    wk = np.ascontiguousarray(w[0])
    assert hip.eahmmf_hip_moe_decode_async(ctypes.byref(shape), slots, wk.ctypes.data, k, ptr(dx), ptr(dy),
                                           ctypes.c_void_p(stream)) == 0
    torch.cuda.synchronize()
    close(dy.cpu().numpy(), want)
    # routed: table + routing on device
    table = np.array([[dev[e][c].data_ptr() for c in range(3)] for e in range(E)], dtype=np.uint64)
    dtable = to_dev(torch, table.view(np.int64))
    dlog = to_dev(torch, logits)
    dids = torch.empty((1, k), dtype=torch.int32, device="cuda")
    dwts = torch.empty((1, k), dtype=torch.float32, device="cuda")
    dy2 = torch.full((D,), float("nan"), device="cuda")
    assert hip.eahmmf_hip_route_topk_async(ptr(dlog), 1, E, k, ptr(dids), ptr(dwts), ctypes.c_void_p(stream)) == 0
    assert hip.eahmmf_hip_moe_decode_routed_async(ctypes.byref(shape), ptr(dtable), E, ptr(dids), ptr(dwts), k,
                                                  ptr(dx), ptr(dy2), ctypes.c_void_p(stream)) == 0
    torch.cuda.synchronize()
    assert np.array_equal(dids.cpu().numpy(), ids)
    close(dy2.cpu().numpy(), want)


@pytest.mark.parametrize("name,types,D,FF,E,k", [
    ("c2_q4_k_m", (Q4_K, Q4_K, Q6_K), 2048, 768, 128, 8),
    ("c1_q8_0", (Q8_0, Q8_0, Q8_0), 256, 128, 8, 2),
    ("c3_q5_k", (Q5_K, Q5_K, Q5_K), 2048, 768, 32, 8),
    ("c5_q4_k_m", (Q4_K, Q4_K, Q6_K), 4096, 1536, 16, 8),
    ("top16_two_experts_per_partition", (Q4_K, Q4_K, Q6_K), 2048, 768, 64, 16),
    ("top6_coherent_exchange", (Q8_0, Q8_0, Q6_K), 1024, 512, 32, 6),
    ("top1", (Q6_K, Q6_K, Q5_K), 512, 256, 16, 1),
], ids=lambda c: c if isinstance(c, str) else None)
def test_moe_layer_decode_vs_oracle(torch_dev, binding, hip, path, name, types, D, FF, E, k):
    """One launch per layer-token (routing from device logits) over a device
    expert table, repeated for several tokens on one stream: ids bit-exact,
    weights to a few ulps, y within tolerance, every token."""
    torch = torch_dev
    rng = np.random.default_rng(E + D)
    n_unique = min(E, 24)
    uniq = make_layer(binding, types, D, FF, n_unique, rng)
    layer = [uniq[e % n_unique] for e in range(E)]
    dev_u = [[to_dev(torch, uniq[e][c][1]) for c in range(3)] for e in range(n_unique)]
    table = np.array([[dev_u[e % n_unique][c].data_ptr() for c in range(3)] for e in range(E)], dtype=np.uint64)
    dtable = to_dev(torch, table.view(np.int64))
    gt_, ut, dt_ = types
    shape = binding.MoeShape(gt_, ut, dt_, D, FF, binding.row_bytes(gt_, D), binding.row_bytes(ut, D),
                             binding.row_bytes(dt_, FF))
    T = 6
    xs = rng.normal(0, 1, (T, D)).astype(np.float32)
    logits = rng.normal(0, 1, (T, E)).astype(np.float32)
    dx, dl = to_dev(torch, xs), to_dev(torch, logits)
    dy = torch.full((T, D), float("nan"), device="cuda")
    dids = torch.full((T, k), -7, dtype=torch.int32, device="cuda")
    dw = torch.zeros((T, k), dtype=torch.float32, device="cuda")
    stream = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
    for t in range(T):
        rc = hip.eahmmf_hip_moe_layer_decode_async(ctypes.byref(shape), ptr(dtable), E, ptr(dl[t]), k, ptr(dx[t]),
                                                   ptr(dy[t]), ptr(dids[t]), ptr(dw[t]), stream)
        assert rc == 0, hip.eahmmf_hip_last_error()
    torch.cuda.synchronize()
    ids, w = oracle.route_topk(logits, k)
    assert np.array_equal(dids.cpu().numpy(), ids)
    np.testing.assert_allclose(dw.cpu().numpy(), w, rtol=1e-6, atol=0)
    y = dy.cpu().numpy()
    for t in range(T):
        want = oracle.moe_layer(layer, xs[t:t + 1], ids[t:t + 1], w[t:t + 1])[0]
        close(y[t], want)


@pytest.mark.parametrize("name,types,D,FF,E,k,use_norm", [
    ("c2_q4_k_m", (Q4_K, Q4_K, Q6_K), 2048, 768, 128, 8, True),
    ("c1_q8_0", (Q8_0, Q8_0, Q8_0), 256, 128, 8, 2, True),
    ("c5_q4_k_m", (Q4_K, Q4_K, Q6_K), 4096, 1536, 128, 8, True),
    ("c2_given_xn", (Q4_K, Q4_K, Q6_K), 2048, 768, 128, 8, False),
    # a format mix without an in-launch router kernel: router launch, then the fused layer
    ("c2_q5_k_q6_k", (Q5_K, Q5_K, Q6_K), 2048, 768, 128, 8, True),
    # 256 experts, one router unit per workgroup (a single slice per logit)
    ("e256_q8_0", (Q8_0, Q8_0, Q8_0), 1024, 512, 256, 8, True),
], ids=lambda c: c if isinstance(c, str) else None)
def test_moe_layer_decode_xn_vs_oracle(torch_dev, binding, hip, path, name, types, D, FF, E, k, use_norm):
    """The layer from its residual stream: RMSNorm, the F32 router matmul,
    routing and experts on the device (eahmmf_hip_moe_layer_decode_xn_async)
    against the oracle's rmsnorm -> matmul -> route_topk -> expert block
    (qwen3moe.cpp:1020-1067): normalized input and logits to fp32 rounding,
    ids bit-exact, weights to a few ulps, y within tolerance."""
    torch = torch_dev
    rng = np.random.default_rng(E + D + 7)
    n_unique = min(E, 16)
    uniq = make_layer(binding, types, D, FF, n_unique, rng)
    layer = [uniq[e % n_unique] for e in range(E)]
    dev_u = [[to_dev(torch, uniq[e][c][1]) for c in range(3)] for e in range(n_unique)]
    table = np.array([[dev_u[e % n_unique][c].data_ptr() for c in range(3)] for e in range(E)], dtype=np.uint64)
    dtable = to_dev(torch, table.view(np.int64))
    gt_, ut, dt_ = types
    shape = binding.MoeShape(gt_, ut, dt_, D, FF, binding.row_bytes(gt_, D), binding.row_bytes(ut, D),
                             binding.row_bytes(dt_, FF))
    T, eps = 4, 1e-6
    hs = (rng.normal(0, 1, (T, D)) * rng.uniform(0.5, 3.0, (T, 1))).astype(np.float32)
    norm_w = (1 + rng.normal(0, 0.05, D)).astype(np.float32)
    router = rng.normal(0, 0.05, (E, D)).astype(np.float32)
    xn_want = oracle.rmsnorm(hs, norm_w, eps) if use_norm else hs
    logits_want = oracle.matmul(0, router.view(np.uint8), D, xn_want)
    ids, w = oracle.route_topk(logits_want, k)
    dh, dnw, dr = to_dev(torch, hs), to_dev(torch, norm_w), to_dev(torch, router)
    dy = torch.full((T, D), float("nan"), device="cuda")
    dxn = torch.full((T, D), float("nan"), device="cuda")
    dlog = torch.full((T, E), float("nan"), device="cuda")
    dids = torch.full((T, k), -7, dtype=torch.int32, device="cuda")
    dw = torch.zeros((T, k), dtype=torch.float32, device="cuda")
    stream = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
    for t in range(T):
        rc = hip.eahmmf_hip_moe_layer_decode_xn_async(
            ctypes.byref(shape), ptr(dtable), E, ptr(dr), ptr(dnw) if use_norm else None, ctypes.c_float(eps),
            ptr(dh[t]), k, ptr(dy[t]), ptr(dids[t]), ptr(dw[t]), ptr(dxn[t]) if use_norm else None, ptr(dlog[t]),
            stream)
        assert rc == 0, hip.eahmmf_hip_last_error()
    torch.cuda.synchronize()
    if use_norm:
        np.testing.assert_allclose(dxn.cpu().numpy(), xn_want, rtol=2e-6, atol=1e-7)
    lg = dlog.cpu().numpy()
    assert np.abs(lg - logits_want).max() <= 1e-5 * max(1.0, np.abs(logits_want).max())
    # the drawn logits leave no near-tie at the k-th place (else the summation
    # order could swap two ids, as the entry point's declaration says)
    srt = -np.sort(-logits_want, axis=1)
    assert (srt[:, k - 1] - srt[:, k]).min() > 1e-4
    assert np.array_equal(dids.cpu().numpy(), ids)
    np.testing.assert_allclose(dw.cpu().numpy(), w, rtol=1e-5, atol=0)
    y = dy.cpu().numpy()
    for t in range(T):
        close(y[t], oracle.moe_layer(layer, xn_want[t:t + 1], ids[t:t + 1], w[t:t + 1])[0])


@pytest.mark.parametrize("n_expert,k,levels", [(128, 8, 3), (256, 16, 2), (64, 8, 1), (100, 6, 4)])
def test_layer_routing_ties(torch_dev, binding, hip, path, n_expert, k, levels):
    """Logits drawn from a few levels (many exact ties): the chosen ids follow
    (e desc, id asc) exactly, the weights the rank-order renormalisation."""
    torch = torch_dev
    rng = np.random.default_rng(n_expert * 31 + k)
    D, FF = 256, 128
    uniq = make_layer(binding, (Q8_0, Q8_0, Q8_0), D, FF, 4, rng)
    dev_u = [[to_dev(torch, uniq[e][c][1]) for c in range(3)] for e in range(4)]
    table = np.array([[dev_u[e % 4][c].data_ptr() for c in range(3)] for e in range(n_expert)], dtype=np.uint64)
    dtable = to_dev(torch, table.view(np.int64))
    rb = binding.row_bytes(Q8_0, D)
    shape = binding.MoeShape(Q8_0, Q8_0, Q8_0, D, FF, rb, rb, binding.row_bytes(Q8_0, FF))
    T = 8
    logits = rng.integers(0, levels, (T, n_expert)).astype(np.float32) * 0.5
    xs = rng.normal(0, 1, (T, D)).astype(np.float32)
    dx, dl = to_dev(torch, xs), to_dev(torch, logits)
    dy = torch.empty((T, D), device="cuda")
    dids = torch.full((T, k), -7, dtype=torch.int32, device="cuda")
    dw = torch.zeros((T, k), dtype=torch.float32, device="cuda")
    stream = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
    for t in range(T):
        rc = hip.eahmmf_hip_moe_layer_decode_async(ctypes.byref(shape), ptr(dtable), n_expert, ptr(dl[t]), k,
                                                   ptr(dx[t]), ptr(dy[t]), ptr(dids[t]), ptr(dw[t]), stream)
        assert rc == 0, hip.eahmmf_hip_last_error()
    torch.cuda.synchronize()
    ids, w = oracle.route_topk(logits, k)
    assert np.array_equal(dids.cpu().numpy(), ids)
    np.testing.assert_allclose(dw.cpu().numpy(), w, rtol=1e-6, atol=0)
    layer = [uniq[e % 4] for e in range(n_expert)]
    y = dy.cpu().numpy()
    for t in range(T):
        close(y[t], oracle.moe_layer(layer, xs[t:t + 1], ids[t:t + 1], w[t:t + 1])[0])


# ---------------------------------------------------------------------------
# ragged grouped multi-token block

def by_expert_lists(ids, w):
    """The reference's by_exp grouping (qwen3moe.cpp:1009, 1020): per expert,
    in ascending id, its (token, w) pairs in token order."""
    groups = {}
    for t in range(ids.shape[0]):
        for j in range(ids.shape[1]):
            groups.setdefault(int(ids[t, j]), []).append((t, float(w[t, j])))
    return sorted(groups.items())


GROUPED_CASES = [
    ("c1_q8_0", (Q8_0, Q8_0, Q8_0), 256, 128, 8, 2, 16),
    ("mixed_types", (Q5_K, Q4_K, Q6_K), 512, 256, 12, 3, 70),
    ("c2_shape_q4_k_m", (Q4_K, Q4_K, Q6_K), 2048, 768, 16, 8, 40),
    ("c3_q5_k", (Q5_K, Q5_K, Q5_K), 2048, 768, 8, 4, 9),
    ("q8_0_down_ne0_96", (Q8_0, Q8_0, Q8_0), 128, 96, 6, 2, 130),
    ("q5_k_gate_up_q6_k_down", (Q5_K, Q5_K, Q6_K), 1024, 512, 8, 4, 150),
    ("c5_shape", (Q4_K, Q4_K, Q6_K), 4096, 1536, 4, 2, 33),
    ("c2_shape_small_groups", (Q4_K, Q4_K, Q6_K), 2048, 768, 64, 8, 48),
    ("q8_0_d1024_small_groups", (Q8_0, Q8_0, Q8_0), 1024, 256, 32, 4, 40),
    ("q6_k_gate_up_q4_k_down", (Q6_K, Q6_K, Q4_K), 1024, 512, 16, 4, 20),
]


@pytest.fixture(params=[(1, 32, 4), (1, 32, 0), (1, 16, 0), (1, 0, 0), (0, 32, 0), (0, 32, 4)],
                ids=["dot_mfma", "mfma", "mfma_wave16", "mfma_wg", "valu", "dot_valu"])
def grouped_mode(request, hip):
    """Kernel paths of the grouped block: integer-dot kernels for small groups
    (a block of at most 32 tokens entirely, else groups of at most dot_max
    tokens) or not, then matrix-core or VALU kernels; with the matrix cores,
    groups of at most `wave_max` tokens go to the per-wave kernels (two
    16-token tiles above 16, one at or below), the rest to the workgroup
    kernels."""
    mfma, wave_max, dot_max = request.param
    prev = hip.eahmmf_hip_set_grouped_mfma(mfma)
    prev_w = hip.eahmmf_hip_set_grouped_wave_max(wave_max)
    prev_d = hip.eahmmf_hip_set_grouped_dot_max(dot_max)
    yield request.param
    hip.eahmmf_hip_set_grouped_mfma(prev)
    hip.eahmmf_hip_set_grouped_wave_max(prev_w)
    hip.eahmmf_hip_set_grouped_dot_max(prev_d)


@pytest.mark.parametrize("name,types,D,FF,E,k,nb", GROUPED_CASES, ids=[c[0] for c in GROUPED_CASES])
def test_grouped_vs_oracle(torch_dev, binding, hip, grouped_mode, name, types, D, FF, E, k, nb):
    """Host by_exp lists in, host y out: every token's y within tolerance of
    the oracle's MoE block over the same routing."""
    torch = torch_dev
    rng = np.random.default_rng(D * 3 + FF + k + nb)
    layer = make_layer(binding, types, D, FF, E, rng)
    x = rng.normal(0, 1, (nb, D)).astype(np.float32)
    logits = rng.normal(0, 1, (nb, E)).astype(np.float32)
    ids, w = oracle.route_topk(logits, k)
    want = oracle.moe_layer(layer, x, ids, w)
    dev = [[to_dev(torch, layer[e][c][1]) for c in range(3)] for e in range(E)]
    groups = by_expert_lists(ids, w)
    experts = (binding.Expert * len(groups))()
    offs, toks, wts = [0], [], []
    for g, (e, lst) in enumerate(groups):
        for c, (nm, ne0, ne1) in enumerate((("gate", D, FF), ("up", D, FF), ("down", FF, D))):
            t = layer[e][c][0]
            setattr(experts[g], nm, binding.Weight(dev[e][c].data_ptr(), t, ne0, ne1, binding.row_bytes(t, ne0)))
        toks += [t for t, _ in lst]
        wts += [wv for _, wv in lst]
        offs.append(len(toks))
    offs = np.array(offs, np.int32)
    toks = np.array(toks, np.int32)
    wts = np.array(wts, np.float32)
    y = np.full((nb, D), np.nan, np.float32)
    assert hip.eahmmf_hip_moe_grouped(experts, len(groups), offs.ctypes.data, toks.ctypes.data, wts.ctypes.data, nb,
                                      x.ctypes.data, y.ctypes.data), hip.eahmmf_hip_last_error()
    close(y, want)


@pytest.mark.parametrize("nb,E,k,skew", [(64, 32, 8, 0.0), (200, 128, 8, 1.1), (1, 16, 4, 0.0), (129, 64, 6, 2.0),
                                         (16, 128, 8, 0.0), (32, 64, 8, 1.1), (33, 128, 8, 0.0)])
def test_grouped_async_device_routing(torch_dev, binding, hip, grouped_mode, nb, E, k, skew):
    """Routing on the device (route_topk), grouping on the device, Zipf-skewed
    expert popularity: y of every token matches the oracle on the same ids
    (up to 3 tokens as per-token single-launch blocks, above as the grouped
    block)."""
    torch = torch_dev
    D, FF = 512, 256
    types = (Q4_K, Q4_K, Q6_K)
    rng = np.random.default_rng(nb * 7 + E + k)
    n_unique = min(E, 12)
    uniq = make_layer(binding, types, D, FF, n_unique, rng)
    layer = [uniq[e % n_unique] for e in range(E)]
    dev_u = [[to_dev(torch, uniq[e][c][1]) for c in range(3)] for e in range(n_unique)]
    table = np.array([[dev_u[e % n_unique][c].data_ptr() for c in range(3)] for e in range(E)], dtype=np.uint64)
    dtable = to_dev(torch, table.view(np.int64))
    shape = binding.MoeShape(Q4_K, Q4_K, Q6_K, D, FF, binding.row_bytes(Q4_K, D), binding.row_bytes(Q4_K, D),
                             binding.row_bytes(Q6_K, FF))
    # Gumbel-top-k over a Zipf prior on a seeded permutation of the ids
    prior = np.log(np.arange(1, E + 1, dtype=np.float64) ** -skew)[rng.permutation(E)]
    logits = (prior + rng.gumbel(size=(nb, E))).astype(np.float32)
    x = rng.normal(0, 1, (nb, D)).astype(np.float32)
    dl, dx = to_dev(torch, logits), to_dev(torch, x)
    dids = torch.empty((nb, k), dtype=torch.int32, device="cuda")
    dw = torch.empty((nb, k), dtype=torch.float32, device="cuda")
    dy = torch.full((nb, D), float("nan"), device="cuda")
    stream = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
    assert hip.eahmmf_hip_route_topk_async(ptr(dl), nb, E, k, ptr(dids), ptr(dw), stream) == 0
    assert hip.eahmmf_hip_moe_grouped_async(ctypes.byref(shape), ptr(dtable), E, ptr(dids), ptr(dw), nb, k, ptr(dx),
                                            ptr(dy), stream) == 0, hip.eahmmf_hip_last_error()
    torch.cuda.synchronize()
    ids, w = oracle.route_topk(logits, k)
    assert np.array_equal(dids.cpu().numpy(), ids)
    close(dy.cpu().numpy(), oracle.moe_layer(layer, x, ids, w))


@pytest.mark.parametrize("nb", [2, 16, 32])
@pytest.mark.parametrize("fused", [0, 1], ids=["grouped", "default"])
def test_decode_batch_c5_shape(torch_dev, binding, hip, nb, fused):
    """A decode batch of nb sequences at the Qwen3-235B-A22B expert shape
    (D=4096, FF=1536, 128 experts top-8, Q4_K gate/up, Q6_K down), routing on
    the device from N(0,1) logits.  With the single-token kernel off the batch
    runs as one grouped block on the integer-dot kernels (every routed
    expert's rows streamed once for all of its tokens); by default the entry
    point picks its path.  y of every token matches the oracle on the same ids
    (qwen3moe.cpp:1009-1067)."""
    torch = torch_dev
    D, FF, E, k = 4096, 1536, 128, 8
    types = (Q4_K, Q4_K, Q6_K)
    rng = np.random.default_rng(1000 + nb)
    n_unique = 6
    uniq = make_layer(binding, types, D, FF, n_unique, rng)
    layer = [uniq[e % n_unique] for e in range(E)]
    dev_u = [[to_dev(torch, uniq[e][c][1]) for c in range(3)] for e in range(n_unique)]
    table = np.array([[dev_u[e % n_unique][c].data_ptr() for c in range(3)] for e in range(E)], dtype=np.uint64)
    dtable = to_dev(torch, table.view(np.int64))
    shape = binding.MoeShape(Q4_K, Q4_K, Q6_K, D, FF, binding.row_bytes(Q4_K, D), binding.row_bytes(Q4_K, D),
                             binding.row_bytes(Q6_K, FF))
    logits = rng.normal(0, 1, (nb, E)).astype(np.float32)
    x = rng.normal(0, 1, (nb, D)).astype(np.float32)
    dl, dx = to_dev(torch, logits), to_dev(torch, x)
    dids = torch.empty((nb, k), dtype=torch.int32, device="cuda")
    dw = torch.empty((nb, k), dtype=torch.float32, device="cuda")
    dy = torch.full((nb, D), float("nan"), device="cuda")
    stream = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
    prev = hip.eahmmf_hip_set_fused(fused)
    try:
        print(f"decode batch nb={nb} fused={fused}", flush=True)
        assert hip.eahmmf_hip_route_topk_async(ptr(dl), nb, E, k, ptr(dids), ptr(dw), stream) == 0
        assert hip.eahmmf_hip_moe_grouped_async(ctypes.byref(shape), ptr(dtable), E, ptr(dids), ptr(dw), nb, k,
                                                ptr(dx), ptr(dy), stream) == 0, hip.eahmmf_hip_last_error()
        torch.cuda.synchronize()
    finally:
        hip.eahmmf_hip_set_fused(prev)
    assert hip.eahmmf_hip_device_flags() == 0
    ids, w = oracle.route_topk(logits, k)
    assert np.array_equal(dids.cpu().numpy(), ids)
    close(dy.cpu().numpy(), oracle.moe_layer(layer, x, ids, w))
