"""End to end on the GPU: the reference's tiny Qwen3-MoE model (test_tiny
generator order, 2 layers, 8 Q8_0 experts, top-2) evaluated by the oracle's
forward with every layer's expert block computed by the HIP library through
the C ABI -- the batched prompt through eahmmf_hip_moe_grouped (the
reference's by_exp lists), each generated token through eahmmf_hip_moe_decode.

Checked against the reference's own numbers: baseline/logits.txt (first 16
logits, argmax 147) and the greedy continuation and per-step logits captured
from the compiled reference.  The expert block differs from the reference's
only by fp32 summation order, so logits are compared at 1e-4 absolute (the
reference's own GPU-vs-CPU shadow bar is 1e-4 relative to the largest output,
qwen3moe.cpp:449-458) and the greedy tokens exactly.
"""
import os

import numpy as np
import pytest

import gguf_tools as gt
import oracle
from conftest import GOLDEN

pytestmark = pytest.mark.gpu


class GpuExperts:
    """Device copies of every layer's experts and a hook that runs the block on them."""

    def __init__(self, torch, binding, hip, spec):
        self.b, self.hip, self.spec = binding, hip, spec
        E, D, FF = spec.n_expert, spec.D, spec.FF
        self.dev = []   # keeps device tensors alive
        self.views = []  # [layer][e] -> binding.Expert
        for l in range(spec.n_layer):
            lv = []
            comps = []
            for nm, ne0, ne1 in (("ffn_gate_exps", D, FF), ("ffn_up_exps", D, FF), ("ffn_down_exps", FF, D)):
                t, ne, data = spec.tensors[f"blk.{l}.{nm}.weight"]
                assert ne[0] == ne0 and ne[1] == ne1
                d = torch.from_numpy(np.ascontiguousarray(data).reshape(-1).copy()).cuda()
                self.dev.append(d)
                comps.append((t, d, ne0, ne1, binding.row_bytes(t, ne0)))
            for e in range(E):
                ex = binding.Expert()
                for c, nm in enumerate(("gate", "up", "down")):
                    t, d, ne0, ne1, rb = comps[c]
                    setattr(ex, nm, binding.Weight(d.data_ptr() + e * rb * ne1, t, ne0, ne1, rb))
                lv.append(ex)
            self.views.append(lv)
        self.calls = {"decode": 0, "grouped": 0}

    def __call__(self, layer, x, ids, w):
        nb, k = ids.shape
        D = self.spec.D
        y = np.empty((nb, D), np.float32)
        if nb == 1:
            ex = (self.b.Expert * k)(*[self.views[layer][int(e)] for e in ids[0]])
            wk = np.ascontiguousarray(w[0], dtype=np.float32)
            xx = np.ascontiguousarray(x[0], dtype=np.float32)
            assert self.hip.eahmmf_hip_moe_decode(ex, wk.ctypes.data, k, xx.ctypes.data, y.ctypes.data), \
                self.hip.eahmmf_hip_last_error()
            self.calls["decode"] += 1
            return y
        groups = {}
        for t in range(nb):
            for j in range(k):
                groups.setdefault(int(ids[t, j]), []).append((t, float(w[t, j])))
        groups = sorted(groups.items())
        ex = (self.b.Expert * len(groups))(*[self.views[layer][e] for e, _ in groups])
        offs, toks, wts = [0], [], []
        for _, lst in groups:
            toks += [t for t, _ in lst]
            wts += [wv for _, wv in lst]
            offs.append(len(toks))
        offs, toks, wts = (np.array(offs, np.int32), np.array(toks, np.int32), np.array(wts, np.float32))
        xx = np.ascontiguousarray(x, dtype=np.float32)
        assert self.hip.eahmmf_hip_moe_grouped(ex, len(groups), offs.ctypes.data, toks.ctypes.data, wts.ctypes.data,
                                               nb, xx.ctypes.data, y.ctypes.data), self.hip.eahmmf_hip_last_error()
        self.calls["grouped"] += 1
        return y


def baseline_logits():
    txt = open(os.path.join(GOLDEN, "baseline_logits.txt")).read().replace("argmax", "").split()
    vals = [float(v) for v in txt]
    return np.array(vals[:16]), int(vals[16])


@pytest.fixture(scope="module")
def torch_dev():
    import torch
    assert torch.cuda.is_available()
    return torch


@pytest.mark.parametrize("mfma", [1, 0], ids=["mfma", "valu"])
def test_tiny_model_with_gpu_experts(torch_dev, binding, hip, mfma):
    prev = hip.eahmmf_hip_set_grouped_mfma(mfma)
    try:
        spec = gt.test_tiny_spec()
        ref = np.load(os.path.join(GOLDEN, "tiny_ref.npz"))
        gpu = GpuExperts(torch_dev, binding, hip, spec)
        # the reference's baseline run: the 16-token prompt as one batch
        m32 = oracle.OracleModel(spec)
        m32.set_moe_hook(gpu)
        lg = m32.eval(ref["prompt"], 0, 32)
        want, am = baseline_logits()
        np.testing.assert_allclose(lg[:16], want, rtol=0, atol=1e-4)
        assert int(np.argmax(lg)) == am == 147
        np.testing.assert_allclose(lg, ref["logits_b32"], rtol=0, atol=1e-4)
        # the reference's greedy run: prompt in batches of 4, then one token at a time
        m = oracle.OracleModel(spec)
        m.set_moe_hook(gpu)
        lg = m.eval(ref["prompt"], 0, 4)
        np.testing.assert_allclose(lg, ref["logits_b4"], rtol=0, atol=1e-4)
        gen, pos = [], len(ref["prompt"])
        for i in range(len(ref["gen"])):
            t = int(np.argmax(lg))
            gen.append(t)
            lg = m.forward([t], pos)
            pos += 1
            np.testing.assert_allclose(lg, ref["step_logits"][i + 1], rtol=0, atol=1e-4)
        assert gen == list(ref["gen"])
        ids, _ = m.trace()
        assert np.array_equal(ids, ref["trace_ids"])  # the same experts routed at every layer and step
        n_prompt_batches = 1 + (len(ref["prompt"]) + 3) // 4
        assert gpu.calls["grouped"] == spec.n_layer * n_prompt_batches
        assert gpu.calls["decode"] == spec.n_layer * len(ref["gen"])
    finally:
        hip.eahmmf_hip_set_grouped_mfma(prev)


def test_config0_with_gpu_experts(torch_dev, binding, hip):
    ref = np.load(os.path.join(GOLDEN, "config0_ref.npz"))
    spec = gt.config0_spec(seed=0)
    gpu = GpuExperts(torch_dev, binding, hip, spec)
    m = oracle.OracleModel(spec)
    m.set_moe_hook(gpu)
    lg = m.eval(ref["prompt"], 0, 16)
    np.testing.assert_allclose(lg, ref["step_logits"][0], rtol=0, atol=1e-4)
    pos, gen = len(ref["prompt"]), []
    for i in range(len(ref["gen"])):
        t = int(np.argmax(lg))
        gen.append(t)
        lg = m.forward([t], pos)
        pos += 1
        # every one of the 32 decode steps' logits, not only the prompt's
        np.testing.assert_allclose(lg, ref["step_logits"][i + 1], rtol=0, atol=1e-4)
    assert gen == list(ref["gen"])
    # the routing trace of every layer, prompt token and generated token
    ids, wts = m.trace()
    assert np.array_equal(ids, ref["trace_ids"])
    np.testing.assert_allclose(wts, ref["trace_w"], rtol=5e-5, atol=0)  # the oracle's own bar vs the reference
    assert gpu.calls["decode"] == spec.n_layer * len(ref["gen"])
