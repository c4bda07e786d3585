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


# ---------------------------------------------------------------------------
# Long contexts and other head shapes, against the oracle's forward (the
# golden runs above stop at 48 positions: one attention split).  A 2500-token
# prompt takes 32 splits of 79 positions -- several chunks per wave, batch
# rows inside splits, the cross-block merge -- and the decode steps after it
# read a 2500-row cache.  Tolerance as above: 1e-4 absolute on the logits.

def small_spec(seed, D, NH, NKV, HD, E, K, FF, V, NL, CTX, attn_type):
    """A random model with the library's quantizer: experts Q8_0, attention
    projections attn_type, everything else F32 ~ N(0, 0.02)."""
    from conftest import load_binding
    b = load_binding()
    rng = np.random.default_rng(seed)
    spec = gt.ModelSpec(n_layer=NL, D=D, n_head=NH, n_kv=NKV, hd=HD, n_expert=E, n_used=K, FF=FF, n_vocab=V,
                        n_ctx=CTX, ctx_train=CTX, eps=1e-6, rope_base=1e6)

    def n(*shape):
        return rng.normal(0, 0.02, shape).astype(np.float32)

    def addf(name, arr):
        spec.add(name, gt.F32, list(reversed(arr.shape)), np.asarray(arr, np.float32))

    def addq(name, t, arr):
        if t == gt.F32:
            return addf(name, arr)
        spec.add(name, t, list(reversed(arr.shape)), b.quantize_rows(t, arr.reshape(-1, arr.shape[-1])))

    addf("token_embd.weight", n(V, D))
    addf("output.weight", n(V, D))
    addf("output_norm.weight", 1 + n(D))
    for l in range(NL):
        p = f"blk.{l}."
        addf(p + "attn_norm.weight", 1 + n(D))
        addf(p + "ffn_norm.weight", 1 + n(D))
        addf(p + "attn_q_norm.weight", 1 + n(HD))
        addf(p + "attn_k_norm.weight", 1 + n(HD))
        addq(p + "attn_q.weight", attn_type, n(NH * HD, D))
        addq(p + "attn_k.weight", attn_type, n(NKV * HD, D))
        addq(p + "attn_v.weight", attn_type, n(NKV * HD, D))
        addq(p + "attn_output.weight", attn_type, n(D, NH * HD))
        addf(p + "ffn_gate_inp.weight", n(E, D))
        for nm, shape in (("ffn_gate_exps", (E, FF, D)), ("ffn_up_exps", (E, FF, D)), ("ffn_down_exps", (E, D, FF))):
            spec.add(p + nm + ".weight", gt.Q8_0, list(reversed(shape)),
                     b.quantize_rows(gt.Q8_0, n(*shape).reshape(-1, shape[-1])))
    return spec


@pytest.mark.parametrize("shape", [
    dict(D=256, NH=4, NKV=2, HD=64, n_prompt=2500, attn=gt.F32),      # the config-0 heads, 32 splits
    dict(D=256, NH=16, NKV=2, HD=128, n_prompt=2100, attn=gt.Q8_0),   # 8 query heads per KV head (30B-A3B)
    dict(D=256, NH=32, NKV=2, HD=128, n_prompt=700, attn=gt.Q8_0),    # 16 per KV head (235B-A22B)
    dict(D=256, NH=2, NKV=2, HD=64, n_prompt=300, attn=gt.Q8_0),      # one per KV head
], ids=["hd64-grp2-2500", "hd128-grp8-2100", "hd128-grp16-700", "hd64-grp1-300"])
def test_long_context_against_oracle(torch_dev, binding, shape):
    import oracle
    n_prompt = shape["n_prompt"]
    spec = small_spec(3, shape["D"], shape["NH"], shape["NKV"], shape["HD"], 8, 2, 128, 512, 1, n_prompt + 8,
                      shape["attn"])
    prompt = np.random.default_rng(11).integers(0, spec.n_vocab, n_prompt).astype(np.int32)
    m = binding.DeviceModel(hp_of(spec), spec.tensors)
    try:
        o = oracle.OracleModel(spec)
        lg, lo = m.eval(prompt, 0, 64), o.eval(prompt, 0, 64)
        np.testing.assert_allclose(lg, lo, rtol=0, atol=1e-4)
        pos = n_prompt
        for _ in range(4):
            t = int(np.argmax(lo))
            lg, lo = m.forward([t], pos), o.forward([t], pos)
            pos += 1
            np.testing.assert_allclose(lg, lo, rtol=0, atol=1e-4)
        # the device greedy loop from the same state matches the host loop
        toks, lg = m.generate_greedy(int(np.argmax(lo)), pos, 3)
        want = []
        t = int(np.argmax(lo))
        for i in range(3):
            lo = o.forward([t], pos + i)
            t = int(np.argmax(lo))
            want.append(t)
        assert list(toks) == want
        np.testing.assert_allclose(lg, lo, rtol=0, atol=1e-4)
    finally:
        m.close()


# Several sequences in one model (eahmmf_hip_model_set_sequences /
# forward_seq / decode_seqs): each sequence against an oracle engine of its
# own (the reference's Engine holds one sequence), prompts of different
# lengths -- one past a 64-position split, so the batched decode step mixes
# one-split and several-split tokens -- then decode steps over every
# sequence in one batch (in shuffled order), over a ragged subset, and a
# single-sequence step; logits at 1e-4 absolute as above, greedy tokens
# exactly.

@pytest.mark.parametrize("shape", [
    dict(D=256, NH=4, NKV=2, HD=64, attn=gt.F32, lens=[37, 5, 150, 1]),
    dict(D=256, NH=16, NKV=2, HD=128, attn=gt.Q8_0, lens=[70, 3, 12, 9, 130, 2]),
], ids=["hd64-grp2-4seq", "hd128-grp8-6seq"])
def test_sequences_against_oracle(torch_dev, binding, shape):
    import oracle
    lens = shape["lens"]
    S = len(lens)
    spec = small_spec(7, shape["D"], shape["NH"], shape["NKV"], shape["HD"], 8, 2, 128, 512, 2, 200, shape["attn"])
    rng = np.random.default_rng(5)
    m = binding.DeviceModel(hp_of(spec), spec.tensors)
    try:
        m.set_sequences(S)
        orc = [oracle.OracleModel(spec) for _ in range(S)]
        last, pos = [], list(lens)
        for s, n in enumerate(lens):
            prompt = rng.integers(0, spec.n_vocab, n).astype(np.int32)
            lg, lo = m.eval(prompt, 0, 32, seq=s), orc[s].eval(prompt, 0, 32)
            np.testing.assert_allclose(lg, lo, rtol=0, atol=1e-4)
            last.append(lo)
        order = rng.permutation(S)
        subset = [int(v) for v in order[: S // 2 + 1]][::-1]
        for seqs in ([int(v) for v in order], list(range(S)), subset, [S - 1]):
            toks = [int(np.argmax(last[s])) for s in seqs]
            lg = m.decode_seqs(toks, seqs, [pos[s] for s in seqs])
            for i, s in enumerate(seqs):
                lo = orc[s].forward([toks[i]], pos[s])
                np.testing.assert_allclose(lg[i], lo, rtol=0, atol=1e-4, err_msg=f"sequence {s}")
                assert int(np.argmax(lg[i])) == int(np.argmax(lo))
                last[s] = lo
                pos[s] += 1
        # sequence 0 through the one-sequence entry points still sees its own rows
        t = int(np.argmax(last[0]))
        np.testing.assert_allclose(m.forward([t], pos[0]), orc[0].forward([t], pos[0]), rtol=0, atol=1e-4)
        # argument checks: a sequence twice, outside the set, a position past the context
        for toks, seqs, p in (([1, 2], [0, 0], [5, 6]), ([1], [S], [0]), ([1], [0], [spec.n_ctx])):
            with pytest.raises(RuntimeError):
                m.decode_seqs(toks, seqs, p)
        with pytest.raises(RuntimeError):
            m.forward([1], 0, seq=S)
        # a new set of sequences starts empty
        m.set_sequences(2)
        prompt = rng.integers(0, spec.n_vocab, 9).astype(np.int32)
        fresh = oracle.OracleModel(spec)
        np.testing.assert_allclose(m.eval(prompt, 0, 4, seq=1), fresh.eval(prompt, 0, 4), rtol=0, atol=1e-4)
    finally:
        m.close()


def test_model_from_gguf_file(tmp_path, torch_dev, binding):
    """The tiny model loaded from a GGUF file through the binding's reader
    gives the reference's baseline logits (as Engine::load + eval)."""
    spec = gt.test_tiny_spec()
    path = tmp_path / "tiny.gguf"
    gt.write_gguf(spec, str(path))
    ref = np.load(os.path.join(GOLDEN, "tiny_ref.npz"))
    m = binding.model_from_gguf(str(path), 128)
    try:
        lg = m.eval(ref["prompt"], 0, 32)
        np.testing.assert_allclose(lg, ref["logits_b32"], rtol=0, atol=1e-4)
    finally:
        m.close()
