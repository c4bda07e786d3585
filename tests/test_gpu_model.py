"""The whole model on the GPU (eahmmf_hip_model_*): embedding, attention,
norms, RoPE, KV cache, router, expert blocks and output head all on the
device, checked against the compiled reference's own numbers for the
reference's tiny model (tests/test_tiny.py generator order) and for the
config-0 model (Q8_0 experts, fp32 attention):

* logits of every step at 1e-4 absolute: the forward differs from the
  reference's only in fp32 summation order (parallel reductions in RMSNorm,
  attention, the matmuls and the expert block);
* the greedy tokens exactly;
* the routing trace of every layer, prompt token and generated token: ids
  exactly, weights at 5e-5 relative (the router logits come from a GPU
  matmul, so the softmax inputs carry the matmul's rounding).
"""
import os

import numpy as np
import pytest

import gguf_tools as gt
from conftest import GOLDEN

pytestmark = pytest.mark.gpu


def hp_of(spec):
    return {n: getattr(spec, n) for n in ("n_layer", "D", "n_head", "n_kv", "hd", "n_expert", "n_used", "FF",
                                          "n_vocab", "n_ctx", "eps", "rope_base")}


def baseline_logits():
    txt = open(os.path.join(GOLDEN, "baseline_logits.txt")).read().replace("argmax", "").split()
    vals = [float(v) for v in txt]
    return np.array(vals[:16]), int(vals[16])


@pytest.fixture(scope="module")
def tiny(torch_dev, binding):
    spec = gt.test_tiny_spec()
    m = binding.DeviceModel(hp_of(spec), spec.tensors)
    yield m
    m.close()


@pytest.fixture(scope="module")
def config0(torch_dev, binding):
    spec = gt.config0_spec(seed=0)
    m = binding.DeviceModel(hp_of(spec), spec.tensors)
    yield m
    m.close()


def test_tiny_prompt_one_batch(tiny):
    ref = np.load(os.path.join(GOLDEN, "tiny_ref.npz"))
    lg = tiny.eval(ref["prompt"], 0, 32)
    want, am = baseline_logits()
    np.testing.assert_allclose(lg[:16], want, rtol=0, atol=1e-4)
    assert int(np.argmax(lg)) == am == 147
    np.testing.assert_allclose(lg, ref["logits_b32"], rtol=0, atol=1e-4)


def test_tiny_greedy_steps_and_trace(tiny):
    ref = np.load(os.path.join(GOLDEN, "tiny_ref.npz"))
    tiny.trace_clear()
    tiny.set_trace(True)
    try:
        lg = tiny.eval(ref["prompt"], 0, 4)
        np.testing.assert_allclose(lg, ref["logits_b4"], rtol=0, atol=1e-4)
        gen, pos = [], len(ref["prompt"])
        for i in range(len(ref["gen"])):
            t = int(np.argmax(lg))
            gen.append(t)
            lg = tiny.forward([t], pos)
            pos += 1
            np.testing.assert_allclose(lg, ref["step_logits"][i + 1], rtol=0, atol=1e-4)
        assert gen == list(ref["gen"])
        ids, w = tiny.trace()
        assert np.array_equal(ids, ref["trace_ids"])
        np.testing.assert_allclose(w, ref["trace_w"], rtol=5e-5, atol=0)
    finally:
        tiny.set_trace(False)
        tiny.trace_clear()


def test_tiny_generate_on_device(tiny):
    """Greedy decoding with the argmax on the device and one host wait."""
    ref = np.load(os.path.join(GOLDEN, "tiny_ref.npz"))
    tiny.eval(ref["prompt"], 0, 4)
    gen = list(ref["gen"])
    toks, lg = tiny.generate_greedy(gen[0], len(ref["prompt"]), len(gen))
    assert list(toks[:-1]) == gen[1:]
    np.testing.assert_allclose(lg, ref["step_logits"][len(gen)], rtol=0, atol=1e-4)
    assert int(toks[-1]) == int(np.argmax(ref["step_logits"][len(gen)]))


def test_config0_every_step(config0):
    ref = np.load(os.path.join(GOLDEN, "config0_ref.npz"))
    config0.trace_clear()
    config0.set_trace(True)
    try:
        lg = config0.eval(ref["prompt"], 0, 16)
        np.testing.assert_allclose(lg, ref["step_logits"][0], rtol=0, atol=1e-4)
        pos, gen = len(ref["prompt"]), []
        for i in range(len(ref["gen"])):
            t = int(np.argmax(lg))
            gen.append(t)
            lg = config0.forward([t], pos)
            pos += 1
            np.testing.assert_allclose(lg, ref["step_logits"][i + 1], rtol=0, atol=1e-4)
        assert gen == list(ref["gen"])
        ids, w = config0.trace()
        assert np.array_equal(ids, ref["trace_ids"])
        np.testing.assert_allclose(w, ref["trace_w"], rtol=5e-5, atol=0)
    finally:
        config0.set_trace(False)
        config0.trace_clear()


def test_config0_generate_with_trace(config0):
    """The device greedy loop with the trace on reads each step's routing."""
    ref = np.load(os.path.join(GOLDEN, "config0_ref.npz"))
    config0.eval(ref["prompt"], 0, 16)
    gen = list(ref["gen"])
    config0.trace_clear()
    config0.set_trace(True)
    try:
        toks, lg = config0.generate_greedy(gen[0], len(ref["prompt"]), len(gen))
        ids, _ = config0.trace()
    finally:
        config0.set_trace(False)
        config0.trace_clear()
    assert list(toks[:-1]) == gen[1:]
    np.testing.assert_allclose(lg, ref["step_logits"][len(gen)], rtol=0, atol=1e-4)
    n_prompt = len(ref["prompt"]) * config0.n_layer * config0.n_used
    assert np.array_equal(ids, ref["trace_ids"][n_prompt:])


def test_model_rejects_bad_arguments(config0, binding):
    with pytest.raises(RuntimeError, match="out of range"):
        config0.forward([config0.n_vocab], 0)
    with pytest.raises(RuntimeError, match="context overflow"):
        config0.forward([1, 2], 63)
    with pytest.raises(RuntimeError, match="batch size"):
        config0.forward(list(range(65)), 0)
    # the model still works after rejected calls
    ref = np.load(os.path.join(GOLDEN, "config0_ref.npz"))
    lg = config0.eval(ref["prompt"], 0, 16)
    np.testing.assert_allclose(lg, ref["step_logits"][0], rtol=0, atol=1e-4)


def test_model_create_rejects_bad_shapes(torch_dev, binding):
    spec = gt.config0_spec(seed=0)
    hp = hp_of(spec)
    bad = dict(hp, hd=96)
    with pytest.raises(RuntimeError, match="head dimension"):
        binding.DeviceModel(bad, spec.tensors)
    t = dict(spec.tensors)
    ty, ne, data = t["blk.1.attn_q.weight"]
    t["blk.1.attn_q.weight"] = (ty, [ne[0], ne[1] - 1], data)
    with pytest.raises(RuntimeError, match="attn_q"):
        binding.DeviceModel(hp, t)
