"""A single-launch expert block whose bounded wait gives up fails loudly
(MI355X, through the C ABI).

The fused kernel's workgroups wait for each other's h words and partial
outputs.  A test knob (eahmmf_hip_set_fault_injection) makes every wait give
up after one poll and stops one partition from storing its h words, so the
kernel's own bounded waits give up while every kernel still exits normally.
Contract checked: the synchronous entry point returns false (the reference's
CPU fallback then runs, expert_cuda.cu:332-335, qwen3moe.cpp:515-521), y is
NaN, the error word is reported once by eahmmf_hip_device_flags() and by
eahmmf_hip_fused_status_async(), and the next call without the knob is
correct again.
"""
import ctypes

import numpy as np
import pytest

import oracle
from test_gpu_parity import Q4_K, Q6_K, Q8_0, close, make_layer, ptr, to_dev

pytestmark = pytest.mark.gpu


@pytest.fixture
def fused_only(hip):
    prev = hip.eahmmf_hip_set_fused(1)
    yield
    hip.eahmmf_hip_set_fault_injection(0, -1)
    hip.eahmmf_hip_set_fused(prev)
    hip.eahmmf_hip_device_flags()


def experts_for(binding, layer, dev, ids, D, FF):
    k = len(ids)
    ex = (binding.Expert * k)()
    for j, e in enumerate(ids):
        for c, (nm, ne0, ne1) in enumerate((("gate", D, FF), ("up", D, FF), ("down", FF, D))):
            t = layer[e][c][0]
            setattr(ex[j], nm, binding.Weight(dev[e][c].data_ptr(), t, ne0, ne1, binding.row_bytes(t, ne0)))
    return ex


@pytest.mark.parametrize("types,D,FF,k", [((Q4_K, Q4_K, Q6_K), 2048, 768, 8), ((Q8_0, Q8_0, Q6_K), 1024, 512, 6)],
                         ids=["c2_xcd_local_exchange", "top6_coherent_exchange"])
def test_sync_entry_fails_when_a_wait_gives_up(torch_dev, binding, hip, fused_only, types, D, FF, k):
    torch = torch_dev
    print(f"fault injection: sync entry D={D} FF={FF} k={k}", flush=True)
    rng = np.random.default_rng(5 + k)
    E = k
    layer = make_layer(binding, types, D, FF, E, rng)
    dev = [[to_dev(torch, layer[e][c][1]) for c in range(3)] for e in range(E)]
    x = rng.normal(0, 1, (1, D)).astype(np.float32)
    ids = np.arange(k, dtype=np.int32)[None, :]
    w = rng.uniform(0.05, 1.0, (1, k)).astype(np.float32)
    w /= w.sum()
    want = oracle.moe_layer(layer, x, ids, w)[0]
    ex = experts_for(binding, layer, dev, list(range(k)), D, FF)
    wk = np.ascontiguousarray(w[0])
    y = np.zeros(D, dtype=np.float32)
    assert hip.eahmmf_hip_device_flags() == 0
    # a normal call first
    assert hip.eahmmf_hip_moe_decode(ex, wk.ctypes.data, k, x.ctypes.data, y.ctypes.data), binding.last_error()
    close(y, want)
    # every wait gives up after one poll; partition 3 never stores its h
    hip.eahmmf_hip_set_fault_injection(1, 3)
    y[:] = 0
    ok = hip.eahmmf_hip_moe_decode(ex, wk.ctypes.data, k, x.ctypes.data, y.ctypes.data)
    assert not ok
    assert "bounded wait" in binding.last_error()
    assert np.isnan(y).all(), f"{np.isnan(y).sum()} of {D} NaN"
    assert hip.eahmmf_hip_device_flags() == 1
    assert hip.eahmmf_hip_device_flags() == 0  # reported once, then cleared
    # the knob off again: the same call is correct
    hip.eahmmf_hip_set_fault_injection(0, -1)
    y[:] = 0
    assert hip.eahmmf_hip_moe_decode(ex, wk.ctypes.data, k, x.ctypes.data, y.ctypes.data), binding.last_error()
    close(y, want)
    assert hip.eahmmf_hip_device_flags() == 0


def test_async_entry_reports_through_the_error_word(torch_dev, binding, hip, fused_only):
    torch = torch_dev
    D, FF, E, k = 2048, 768, 16, 8
    print(f"fault injection: async layer entry D={D} FF={FF} E={E} k={k}", flush=True)
    rng = np.random.default_rng(11)
    layer = make_layer(binding, (Q4_K, Q4_K, Q6_K), D, FF, E, rng)
    dev = [[to_dev(torch, layer[e][c][1]) for c in range(3)] for e in range(E)]
    table = np.array([[dev[e][c].data_ptr() for c in range(3)] for e in range(E)], dtype=np.uint64)
    dtable = to_dev(torch, table.view(np.int64))
    shape = binding.MoeShape(Q4_K, Q4_K, Q6_K, D, FF, binding.row_bytes(Q4_K, D), binding.row_bytes(Q4_K, D),
                             binding.row_bytes(Q6_K, FF))
    x = rng.normal(0, 1, (1, D)).astype(np.float32)
    logits = rng.normal(0, 1, (1, E)).astype(np.float32)
    ids, w = oracle.route_topk(logits, k)
    want = oracle.moe_layer(layer, x, ids, w)[0]
    dx, dl = to_dev(torch, x[0]), to_dev(torch, logits[0])
    dy = torch.zeros(D, device="cuda")
    status = torch.full((1,), 12345, dtype=torch.int32, device="cuda")
    stream = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)

    def run():
        rc = hip.eahmmf_hip_moe_layer_decode_async(ctypes.byref(shape), ptr(dtable), E, ptr(dl), k, ptr(dx), ptr(dy),
                                                   None, None, stream)
        assert rc == 0, binding.last_error()
        assert hip.eahmmf_hip_fused_status_async(ptr(status), stream) == 0
        torch.cuda.synchronize()
        return dy.cpu().numpy(), int(status.item())

    assert hip.eahmmf_hip_device_flags() == 0
    y, st = run()
    assert st == 0
    close(y, want)
    hip.eahmmf_hip_set_fault_injection(1, 5)
    y, st = run()
    assert st != 0
    assert np.isnan(y).all(), f"{np.isnan(y).sum()} of {D} NaN"
    hip.eahmmf_hip_set_fault_injection(0, -1)
    assert hip.eahmmf_hip_device_flags() == 1
    y, st = run()
    assert st == 0
    close(y, want)
