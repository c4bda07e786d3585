"""Writes the golden fixtures under tests/golden/ from the compiled reference.

Run in a container that has the reference sources (oracle/_ref/libref.so is
built from them by oracle/Makefile):

    python tests/golden/make_golden.py

Every fixture holds inputs and the reference's outputs only:

  dequant_golden.npz   random blocks per format -> reference dq_* output
                       (qwen3moe.cpp:128-202)
  matmul_golden.npz    small W/x per format -> reference matmul output
                       (qwen3moe.cpp:397-419)
  tiny_ref.npz         test_tiny model (rng order of tests/test_tiny.py):
                       logits after the 15-token prompt at batch 32 and 4, 12
                       greedy tokens, the routing trace (ids and weights)
  config0_ref.npz      config-0 model (Q8_0 experts, FF 128, vocab 1024):
                       16-token seeded prompt + 32 greedy tokens, logits of
                       every step, routing trace, weight digest
  baseline_logits.txt  copy of the reference's baseline/logits.txt (data)
"""
import os
import shutil
import sys
import tempfile

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(os.path.dirname(HERE))
sys.path.insert(0, ROOT)
sys.path.insert(0, os.path.dirname(HERE))

import oracle  # noqa: E402
import gguf_tools as gt  # noqa: E402

REF_BASELINE = "/root/reference/baseline/logits.txt"
PROMPT = [5, 17, 200, 33, 99, 3, 150, 256, 42, 77, 8, 9, 10, 11, 12]


def half_bits(vals):
    return np.asarray(vals, dtype=np.float32).astype(np.float16).view(np.uint16)


def random_blocks(t, n, rng, specials=True):
    """Random block bytes with finite fp16 scale fields; with ``specials`` the
    first blocks carry edge values (zero, negative, subnormal, large)."""
    nbytes = oracle.BLOCK[t][1]
    raw = rng.integers(0, 256, (n, nbytes), dtype=np.uint8)
    edge = np.array([0.0, -0.0, 1.0, -1.0, 6.0e-8, -3.0e-6, 65504.0, 2.0 ** -14, 0.5, -2.5e-3], dtype=np.float32)
    scales = rng.uniform(-2e-2, 2e-2, n).astype(np.float32)
    mins = rng.uniform(-2e-2, 2e-2, n).astype(np.float32)
    if specials:
        scales[:len(edge)] = edge
        mins[:len(edge)] = edge[::-1]
    if t == oracle.Q6_K:
        raw[:, 208:210] = half_bits(scales).view(np.uint8).reshape(n, 2)
    else:
        raw[:, 0:2] = half_bits(scales).view(np.uint8).reshape(n, 2)
        if t in (oracle.Q4_K, oracle.Q5_K):
            raw[:, 2:4] = half_bits(mins).view(np.uint8).reshape(n, 2)
    return raw


def make_dequant(rng):
    out = {}
    for t in (oracle.Q8_0, oracle.Q4_K, oracle.Q5_K, oracle.Q6_K):
        blocks = random_blocks(t, 48, rng)
        blck = oracle.BLOCK[t][0]
        ref = oracle.ref_dequant_rows(t, blocks, blck)
        out[f"blocks_{t}"] = blocks
        out[f"values_{t}"] = ref
    np.savez(os.path.join(HERE, "dequant_golden.npz"), **out)


def make_matmul(rng):
    out = {}
    cases = [(oracle.Q8_0, 128, 5, 3), (oracle.Q8_0, 96, 3, 2), (oracle.Q4_K, 512, 6, 3), (oracle.Q5_K, 512, 5, 2),
             (oracle.Q6_K, 768, 4, 3), (oracle.Q6_K, 256, 7, 1)]
    for i, (t, ne0, ne1, nb) in enumerate(cases):
        nblk = ne0 // oracle.BLOCK[t][0]
        w = random_blocks(t, ne1 * nblk, rng, specials=False)
        # keep the scale fields well-conditioned for a tolerance check
        w = w.reshape(ne1, -1)
        x = rng.normal(0, 1, (nb, ne0)).astype(np.float32)
        y = oracle.ref_matmul(t, w, ne0, x)
        out[f"case{i}_meta"] = np.array([t, ne0, ne1, nb], dtype=np.int64)
        out[f"case{i}_w"] = w
        out[f"case{i}_x"] = x
        out[f"case{i}_y"] = y
    np.savez(os.path.join(HERE, "matmul_golden.npz"), **out)


def run_ref_engine(spec, prompt, n_gen, batch):
    R = oracle.ref()
    with tempfile.TemporaryDirectory() as td:
        path = os.path.join(td, "m.gguf")
        gt.write_gguf(spec, path)
        h = R.ref_engine_new(path.encode(), spec.n_ctx)
        V = R.ref_engine_vocab(h)
        toks = np.asarray(prompt, dtype=np.int32)
        logits = np.empty(V, dtype=np.float32)
        R.ref_engine_eval(h, toks.ctypes.data, len(toks), 0, batch, logits.ctypes.data)
        steps = [logits.copy()]
        gen = []
        pos = len(prompt)
        lg = logits.copy()
        for _ in range(n_gen):
            t = int(np.argmax(lg))
            gen.append(t)
            tt = np.array([t], dtype=np.int32)
            R.ref_engine_forward(h, tt.ctypes.data, 1, pos, lg.ctypes.data)
            pos += 1
            steps.append(lg.copy())
        cap = 1 << 16
        ids = np.empty(cap, dtype=np.int32)
        w = np.empty(cap, dtype=np.float32)
        n = R.ref_engine_trace(h, ids.ctypes.data, w.ctypes.data, cap)
        R.ref_engine_free(h)
    return np.stack(steps), np.array(gen, dtype=np.int32), ids[:n].copy(), w[:n].copy()


def make_tiny():
    spec = gt.test_tiny_spec()
    steps32, gen32, ids32, w32 = run_ref_engine(spec, PROMPT, 12, 32)
    steps4, gen4, ids4, w4 = run_ref_engine(spec, PROMPT, 12, 4)
    np.savez(os.path.join(HERE, "tiny_ref.npz"), prompt=np.array(PROMPT, dtype=np.int32),
             logits_b32=steps32[0], logits_b4=steps4[0], step_logits=steps4, gen=gen4, trace_ids=ids4,
             trace_w=w4, digest=np.frombuffer(gt.weight_digest(spec).encode(), dtype=np.uint8))
    assert np.array_equal(gen32, gen4)


def make_config0():
    spec = gt.config0_spec(seed=0)
    prompt = np.random.default_rng(1234).integers(0, spec.n_vocab, 16).astype(np.int32)
    steps, gen, ids, w = run_ref_engine(spec, prompt, 32, 16)
    np.savez(os.path.join(HERE, "config0_ref.npz"), prompt=prompt, step_logits=steps, gen=gen, trace_ids=ids,
             trace_w=w, digest=np.frombuffer(gt.weight_digest(spec).encode(), dtype=np.uint8))


def main():
    rng = np.random.default_rng(20261201)
    make_dequant(rng)
    make_matmul(rng)
    make_tiny()
    make_config0()
    shutil.copyfile(REF_BASELINE, os.path.join(HERE, "baseline_logits.txt"))
    for f in sorted(os.listdir(HERE)):
        print(f, os.path.getsize(os.path.join(HERE, f)))


if __name__ == "__main__":
    main()
