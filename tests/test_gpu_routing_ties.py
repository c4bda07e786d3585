"""Routing at its knife edges, on MI355X through the C ABI, against the
oracle (which forms e = expf(l - max) with the host libm, as
qwen3moe.cpp:1011-1023 does).

- The device exp (eahmmf_hip_expf_ref_async) equals libm's expf bit for bit
  on dense runs of inputs around the values routing meets and on random ones.
- Near-ties: logits whose k-th and (k+1)-th (and first and second) values
  are 1, 2 or 4 ulps apart, and clusters of logits that expf maps to one
  value (so the lower id must win), at magnitudes 0.1-20, in every position,
  for 128 and 256 experts: ids and weights bit-exact, through both the
  single-launch layer kernel (routing inside) and route_topk.
"""
import ctypes

import numpy as np
import pytest

import oracle
from test_gpu_parity import Q8_0, make_layer, ptr, to_dev

pytestmark = pytest.mark.gpu


def test_device_expf_matches_libm(torch_dev, hip):
    torch = torch_dev
    rng = np.random.default_rng(3)
    runs = []
    for c in (-0.0, -1e-6, -0.1, -0.5, -1.0, -3.0, -10.0, -20.0, -87.9, -88.0, -103.2, -103.97, -104.0):
        u = np.array([c], dtype=np.float32).view(np.uint32)[0]
        runs.append((np.arange(1 << 18, dtype=np.uint64) + int(u)).astype(np.uint32))  # toward -inf
    lo, hi = 0x80000000, 0xC2D00000  # -0 .. -104
    runs.append(rng.integers(lo, hi, 1 << 22, dtype=np.uint64).astype(np.uint32))
    runs.append(rng.integers(0, 1 << 32, 1 << 20, dtype=np.uint64).astype(np.uint32))  # every sign and size
    x = np.concatenate(runs).view(np.float32)
    print(f"device expf: {x.size} inputs", flush=True)
    dx = to_dev(torch, x)
    dy = torch.empty_like(dx)
    assert hip.eahmmf_hip_expf_ref_async(ptr(dx), ptr(dy), x.size, None) == 0
    torch.cuda.synchronize()
    got = dy.cpu().numpy()
    want = oracle.expf(x)
    both_nan = np.isnan(got) & np.isnan(want)
    diff = (got.view(np.uint32) != want.view(np.uint32)) & ~both_nan
    assert not diff.any(), f"{diff.sum()} differ, e.g. x={x[diff][:4]} got={got[diff][:4]} want={want[diff][:4]}"


def ulps_below(v, n):
    """v stepped n floats toward -inf."""
    out = np.float32(v)
    for _ in range(n):
        out = np.nextafter(out, np.float32(-np.inf), dtype=np.float32)
    return out


def tie_logits(rng, E, k, mag):
    """A batch of logit rows whose decisive pairs sit 0-4 ulps apart."""
    rows = []
    for gap in (1, 2, 4):
        for edge in ("kth", "first"):
            for _ in range(3):
                l = (rng.normal(0, 1, E) * mag).astype(np.float32)
                order = np.argsort(-l, kind="stable")
                if edge == "kth":
                    a, b = order[k - 1], order[k]
                else:
                    a, b = order[0], order[1]
                l[b] = ulps_below(l[a], gap)
                # put the pair at random positions (either id order)
                pa, pb = rng.choice(E, 2, replace=False)
                l[[a, pa]] = l[[pa, a]]
                l[[b, pb]] = l[[pb, b]]
                rows.append(l)
    # clusters of logits just below the maximum: expf(l - max) rounds many of
    # them to one value, and the lower ids must win
    for _ in range(4):
        l = (rng.normal(0, 1, E) * mag - 3 * mag).astype(np.float32)
        top = np.float32(rng.uniform(0.1, 1.0) * mag)
        ids = rng.choice(E, 2 * k, replace=False)
        for j, i in enumerate(ids):
            l[i] = ulps_below(top, int(rng.integers(0, 6)) if j else 0)
        rows.append(l)
    return np.stack(rows)


def layer_table(torch, binding, E, rng):
    D, FF = 256, 128
    uniq = make_layer(binding, (Q8_0, Q8_0, Q8_0), D, FF, 4, rng)
    dev_u = [[to_dev(torch, uniq[e][c][1]) for c in range(3)] for e in range(4)]
    table = np.array([[dev_u[e % 4][c].data_ptr() for c in range(3)] for e in range(E)], dtype=np.uint64)
    shape = binding.MoeShape(Q8_0, Q8_0, Q8_0, D, FF, binding.row_bytes(Q8_0, D), binding.row_bytes(Q8_0, D),
                             binding.row_bytes(Q8_0, FF))
    return D, shape, to_dev(torch, table.view(np.int64)), dev_u


@pytest.mark.parametrize("E,k", [(128, 8), (256, 8), (256, 16), (128, 1)])
@pytest.mark.parametrize("mag", [0.1, 1.0, 20.0])
def test_near_tie_routing_bit_exact(torch_dev, binding, hip, E, k, mag):
    torch = torch_dev
    rng = np.random.default_rng(E * 31 + k + int(mag * 10))
    logits = tie_logits(rng, E, k, mag)
    T = logits.shape[0]
    print(f"near ties: E={E} k={k} mag={mag} rows={T}", flush=True)
    want_ids, want_w = oracle.route_topk(logits, k)
    stream = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
    dl = to_dev(torch, logits)
    # route_topk
    dids = torch.full((T, k), -7, dtype=torch.int32, device="cuda")
    dw = torch.zeros((T, k), dtype=torch.float32, device="cuda")
    assert hip.eahmmf_hip_route_topk_async(ptr(dl), T, E, k, ptr(dids), ptr(dw), stream) == 0
    torch.cuda.synchronize()
    assert np.array_equal(dids.cpu().numpy(), want_ids)
    assert np.array_equal(dw.cpu().numpy().view(np.uint32), want_w.view(np.uint32))
    # the single-launch layer kernel, routing inside
    prev = hip.eahmmf_hip_set_fused(1)
    try:
        D, shape, dtable, _keep = layer_table(torch, binding, E, rng)
        dx = to_dev(torch, rng.normal(0, 1, (T, D)).astype(np.float32))
        dy = torch.empty((T, D), dtype=torch.float32, device="cuda")
        lids = torch.full((T, k), -7, dtype=torch.int32, device="cuda")
        lw = torch.zeros((T, k), dtype=torch.float32, device="cuda")
        for t in range(T):
            rc = hip.eahmmf_hip_moe_layer_decode_async(ctypes.byref(shape), ptr(dtable), E, ptr(dl[t]), k, ptr(dx[t]),
                                                       ptr(dy[t]), ptr(lids[t]), ptr(lw[t]), stream)
            assert rc == 0, binding.last_error()
        torch.cuda.synchronize()
        assert hip.eahmmf_hip_device_flags() == 0
    finally:
        hip.eahmmf_hip_set_fused(prev)
    assert np.array_equal(lids.cpu().numpy(), want_ids)
    assert np.array_equal(lw.cpu().numpy().view(np.uint32), want_w.view(np.uint32))
