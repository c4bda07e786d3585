"""The no-allocation layer entry point (eahmmf_hip_moe_layer_decode_noalloc)
against the allocating one it varies (eahmmf_hip_moe_layer_decode_async), on
MI355X through the C ABI: ids equal, weights and outputs bit-equal (the same
kernels on the same inputs), and both within the oracle's tolerance; two calls
in a row, the second on a smaller layer, on both the single-launch kernel and
the two-kernel path."""
import ctypes

import numpy as np
import pytest

import oracle
from test_gpu_parity import Q4_K, Q5_K, Q6_K, Q8_0, close, make_layer, ptr, to_dev

pytestmark = pytest.mark.gpu

CASES = [  # (types, D, FF, E, k): the second is smaller in every dimension
    ((Q4_K, Q4_K, Q6_K), 2048, 768, 128, 8),
    ((Q5_K, Q5_K, Q8_0), 512, 256, 16, 4),
]


@pytest.mark.parametrize("fused", [1, 0], ids=["fused", "two_kernel"])
def test_noalloc_matches_the_allocating_entry(binding, hip, fused):
    import torch
    assert torch.cuda.is_available()
    prev = hip.eahmmf_hip_set_fused(fused)
    try:
        stream = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
        for i, (types, D, FF, E, k) in enumerate(CASES):
            print(f"no-alloc call {i}: fused={fused} D={D} FF={FF} E={E} k={k}", flush=True)
            rng = np.random.default_rng(100 + i)
            n_unique = min(E, 16)
            uniq = make_layer(binding, types, D, FF, n_unique, rng)
            layer = [uniq[e % n_unique] for e in range(E)]
            dev_u = [[to_dev(torch, uniq[e][c][1]) for c in range(3)] for e in range(n_unique)]
            table = np.array([[dev_u[e % n_unique][c].data_ptr() for c in range(3)] for e in range(E)],
                             dtype=np.uint64)
            dtable = to_dev(torch, table.view(np.int64))
            gt_, ut, dt_ = types
            shape = binding.MoeShape(gt_, ut, dt_, D, FF, binding.row_bytes(gt_, D), binding.row_bytes(ut, D),
                                     binding.row_bytes(dt_, FF))
            x = rng.normal(0, 1, (1, D)).astype(np.float32)
            logits = rng.normal(0, 1, (1, E)).astype(np.float32)
            dx, dl = to_dev(torch, x[0]), to_dev(torch, logits[0])
            outs = []
            for fn in (hip.eahmmf_hip_moe_layer_decode_async, hip.eahmmf_hip_moe_layer_decode_noalloc):
                dy = torch.full((D,), float("nan"), device="cuda")
                dids = torch.full((k,), -7, dtype=torch.int32, device="cuda")
                dw = torch.zeros((k,), dtype=torch.float32, device="cuda")
                rc = fn(ctypes.byref(shape), ptr(dtable), E, ptr(dl), k, ptr(dx), ptr(dy), ptr(dids), ptr(dw),
                        stream)
                assert rc == 0, binding.last_error()
                torch.cuda.synchronize()
                outs.append((dy.cpu().numpy(), dids.cpu().numpy(), dw.cpu().numpy()))
            (y0, i0, w0), (y1, i1, w1) = outs
            ids, w = oracle.route_topk(logits, k)
            assert np.array_equal(i1, ids[0]) and np.array_equal(i0, i1)
            assert np.array_equal(w0.view(np.uint32), w1.view(np.uint32))
            assert np.array_equal(y0.view(np.uint32), y1.view(np.uint32))
            close(y1, oracle.moe_layer(layer, x, ids, w)[0])
        assert hip.eahmmf_hip_device_flags() == 0
    finally:
        hip.eahmmf_hip_set_fused(prev)


def test_noalloc_rejects_sizes_beyond_its_scratch(binding, hip):
    shape = binding.MoeShape(Q8_0, Q8_0, Q8_0, 8192, 256, binding.row_bytes(Q8_0, 8192),
                             binding.row_bytes(Q8_0, 8192), binding.row_bytes(Q8_0, 256))
    one = ctypes.c_void_p(16)  # never dereferenced: the size check comes first
    rc = hip.eahmmf_hip_moe_layer_decode_noalloc(ctypes.byref(shape), one, 8, one, 2, one, one, None, None, None)
    assert rc == -1
    assert "scratch" in binding.last_error()
