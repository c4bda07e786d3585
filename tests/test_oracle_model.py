"""Pins the oracle's matmul, routing, MoE block and end-to-end forward (CPU).

* matmul: against the compiled reference's matmul (tests/golden/
  matmul_golden.npz) and against an fp64 brute force over dequantized rows.
* routing: against a brute-force sort with the reference's ordering rule and
  against the compiled reference's routing trace on the tiny model.
* forward: the reference's own baseline/logits.txt (2e-6, argmax 147) on the
  model drawn in tests/test_tiny.py's rng order, and the compiled
  reference's greedy tokens on the config-0 model.
"""
import os

import numpy as np
import pytest

import gguf_tools as gt
import oracle
import synth
from conftest import GOLDEN


def test_matmul_matches_compiled_reference():
    g = np.load(os.path.join(GOLDEN, "matmul_golden.npz"))
    i = 0
    while f"case{i}_meta" in g:
        t, ne0, ne1, nb = (int(v) for v in g[f"case{i}_meta"])
        y = oracle.matmul(t, g[f"case{i}_w"], ne0, g[f"case{i}_x"])
        want = g[f"case{i}_y"]
        assert y.shape == (nb, ne1)
        np.testing.assert_allclose(y, want, rtol=1e-5, atol=1e-6 * np.abs(want).max())
        i += 1
    assert i >= 6


@pytest.mark.parametrize("t,ne0", [(oracle.Q4_K, 512), (oracle.Q5_K, 256), (oracle.Q6_K, 768), (oracle.Q8_0, 96)])
def test_matmul_fp64_brute_force(t, ne0):
    rng = np.random.default_rng(7)
    w = synth.random_rows(t, 9, ne0, rng)
    x = rng.normal(0, 1, (3, ne0)).astype(np.float32)
    dq = oracle.dequant_rows(t, w, ne0).astype(np.float64)
    want = x.astype(np.float64) @ dq.T
    got = oracle.matmul(t, w, ne0, x)
    np.testing.assert_allclose(got, want, rtol=1e-5, atol=1e-5 * np.abs(want).max())


def brute_route(logits, k):
    ids, ws = [], []
    for row in logits:
        e = np.exp(row.astype(np.float64) - row.max())
        order = sorted(range(len(row)), key=lambda i: (-e[i], i))[:k]
        tot = sum(e[i] for i in order)
        ids.append(order)
        ws.append([e[i] / tot for i in order])
    return np.array(ids), np.array(ws)


def test_route_topk_brute_force():
    rng = np.random.default_rng(11)
    logits = rng.normal(0, 1, (64, 128)).astype(np.float32)
    logits[3, 10] = logits[3, 20] = logits[3].max() + 1  # exact tie -> lower index first
    logits[5, :] = 0.25  # all equal
    ids, w = oracle.route_topk(logits, 8)
    bids, bw = brute_route(logits, 8)
    assert np.array_equal(ids, bids)
    np.testing.assert_allclose(w, bw, rtol=1e-6)
    assert list(ids[3][:2]) == [10, 20]
    assert list(ids[5]) == list(range(8))


@pytest.fixture(scope="module")
def tiny():
    spec = gt.test_tiny_spec()
    ref = np.load(os.path.join(GOLDEN, "tiny_ref.npz"))
    return spec, ref


def baseline_logits():
    txt = open(os.path.join(GOLDEN, "baseline_logits.txt")).read().replace("argmax", "").split()
    vals = [float(v) for v in txt]
    return np.array(vals[:16]), int(vals[16])


def test_tiny_weights_match_fixture(tiny):
    spec, ref = tiny
    assert gt.weight_digest(spec) == bytes(ref["digest"]).decode()


def test_tiny_forward_matches_reference_baseline(tiny):
    spec, ref = tiny
    m = oracle.OracleModel(spec)
    lg = m.eval(ref["prompt"], 0, 32)
    want, am = baseline_logits()
    assert np.abs(lg[:16] - want).max() < 2e-6
    assert int(np.argmax(lg)) == am == 147
    np.testing.assert_allclose(lg, ref["logits_b32"], rtol=0, atol=2e-6)


def test_tiny_greedy_and_routing_trace(tiny):
    spec, ref = tiny
    m = oracle.OracleModel(spec)
    lg = m.eval(ref["prompt"], 0, 4)
    np.testing.assert_allclose(lg, ref["logits_b4"], rtol=0, atol=2e-6)
    gen = []
    pos = len(ref["prompt"])
    for i in range(len(ref["gen"])):
        t = int(np.argmax(lg))
        gen.append(t)
        lg = m.forward([t], pos)
        pos += 1
        np.testing.assert_allclose(lg, ref["step_logits"][i + 1], rtol=0, atol=5e-6)
    assert gen == list(ref["gen"])
    ids, w = m.trace()
    assert np.array_equal(ids, ref["trace_ids"])
    # the router logits come out of an fp32 dot product whose summation order
    # differs from the reference's omp-simd reduction, so weights agree to a
    # few ulps of the logits rather than bit for bit
    np.testing.assert_allclose(w, ref["trace_w"], rtol=5e-5, atol=0)


def test_config0_greedy_matches_reference():
    ref = np.load(os.path.join(GOLDEN, "config0_ref.npz"))
    spec = gt.config0_spec(seed=0)
    assert gt.weight_digest(spec) == bytes(ref["digest"]).decode()
    m = oracle.OracleModel(spec)
    lg = m.eval(ref["prompt"], 0, 16)
    np.testing.assert_allclose(lg, ref["step_logits"][0], rtol=0, atol=2e-6)
    pos = len(ref["prompt"])
    gen = []
    for i in range(len(ref["gen"])):
        t = int(np.argmax(lg))
        gen.append(t)
        lg = m.forward([t], pos)
        pos += 1
    assert gen == list(ref["gen"])
    ids, w = m.trace()
    assert np.array_equal(ids, ref["trace_ids"])
    # the router logits come out of an fp32 dot product whose summation order
    # differs from the reference's omp-simd reduction, so weights agree to a
    # few ulps of the logits rather than bit for bit
    np.testing.assert_allclose(w, ref["trace_w"], rtol=5e-5, atol=0)


def test_moe_hook_with_oracle_block_reproduces_forward(tiny):
    """The expert-block hook used for end-to-end checks of the HIP path: with
    the oracle's own block plugged in, logits are bit-identical."""
    spec, ref = tiny
    E = spec.n_expert
    layers = []
    for l in range(spec.n_layer):
        comps = []
        for nm in ("ffn_gate_exps", "ffn_up_exps", "ffn_down_exps"):
            t, ne, data = spec.tensors[f"blk.{l}.{nm}.weight"]
            data = np.ascontiguousarray(data).reshape(E, -1)
            comps.append((t, data))
        layers.append([[(comps[c][0], comps[c][1][e].reshape(-1)) for c in range(3)] for e in range(E)])
    a = oracle.OracleModel(spec)
    want = a.eval(ref["prompt"], 0, 32)
    b = oracle.OracleModel(spec)
    calls = []

    def hook(layer, x, ids, w):
        calls.append((layer, x.shape[0]))
        return oracle.moe_layer(layers[layer], x, ids, w)

    b.set_moe_hook(hook)
    got = b.eval(ref["prompt"], 0, 32)
    assert np.array_equal(got.view(np.uint32), want.view(np.uint32))
    assert calls == [(l, len(ref["prompt"])) for l in range(spec.n_layer)]
