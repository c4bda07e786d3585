"""Seeded synthetic Qwen3-MoE models and a minimal GGUF v3 writer/reader.

Test infrastructure.  Two model families:

* ``test_tiny_spec()`` draws every tensor with numpy ``default_rng(0)`` in the
  same call order as the reference's tests/test_tiny.py:5-54 (random quant
  bytes with the fp16 ``d``/``dmin`` fields overwritten by uniform scales,
  fp32 norms and router).  The values, not the file layout, are what the
  reference's baseline/logits.txt pins: the engine looks tensors up by name
  (qwen3moe.cpp:366-370, 883-905).
* ``config0_spec(seed)``: 2 layers, hidden 256, 4/2 heads of dim 64, 8 experts
  top-2, expert FFN 128, vocab 1024; experts Q8_0 quantized from N(0, 0.02)
  by the library's host quantizer, everything else fp32 N(0, 0.02) (norm
  weights 1 + N(0, 0.02)).

GGUF layout follows the format the reference parses (qwen3moe.cpp:285-346):
magic, version 3, counts, key/values, tensor infos (ne0 first), 32-byte
aligned data.
"""
import struct

import numpy as np

F32, Q8_0, Q4_K, Q5_K, Q6_K = 0, 8, 12, 13, 14
BLOCK = {F32: (32, 128), Q8_0: (32, 34), Q4_K: (256, 144), Q5_K: (256, 176), Q6_K: (256, 210)}


def row_bytes(t, ne0):
    blck, nb = BLOCK[t]
    assert ne0 % blck == 0
    return ne0 // blck * nb


class ModelSpec:
    """Hyper-parameters plus ``tensors[name] = (ggml_type, ne, data)`` with ne0 first;
    data is uint8 raw bytes for quantized tensors and float32 for F32."""

    def __init__(self, **hp):
        self.__dict__.update(hp)
        self.tensors = {}
        self.order = []

    def add(self, name, t, ne, data):
        self.tensors[name] = (t, list(ne), data)
        self.order.append(name)

    def expert_bytes(self, layer, comp, e):
        t, ne, data = self.tensors[f"blk.{layer}.{comp}.weight"]
        per = row_bytes(t, ne[0]) * ne[1]
        flat = np.ascontiguousarray(data).reshape(-1)
        return t, ne[0], ne[1], flat[e * per:(e + 1) * per]


# ---------------------------------------------------------------------------
# reference tests/test_tiny.py replica (values only)

def test_tiny_spec():
    rng = np.random.default_rng(0)
    D, NH, NKV, HD, E, K, FF, NL, CTX, BASE = 256, 4, 2, 64, 8, 2, 256, 2, 128, 10000.0
    QD, KD = NH * HD, NKV * HD
    V = 256 + 4
    dscale = {Q8_0: 3e-4, Q4_K: 3e-5, Q5_K: 1.5e-5, Q6_K: 5e-6}
    spec = ModelSpec(n_layer=NL, D=D, n_head=NH, n_kv=NKV, hd=HD, n_expert=E, n_used=K, FF=FF, n_vocab=V,
                     n_ctx=CTX, ctx_train=CTX, eps=1e-6, rope_base=BASE)

    def quant(t, shape):
        blck, nbytes = BLOCK[t]
        rows = int(np.prod(shape[:-1]))
        nblk = shape[-1] // blck
        raw = rng.integers(0, 256, (rows, nblk, nbytes), dtype=np.uint8)

        def put(off, val):
            raw[:, :, off:off + 2] = val.astype(np.float16).view(np.uint8).reshape(rows, nblk, 2)

        if t == Q6_K:
            put(208, rng.uniform(.5, 1.5, (rows, nblk)) * dscale[t])
        else:
            put(0, rng.uniform(.5, 1.5, (rows, nblk)) * dscale[t])
            if t in (Q4_K, Q5_K):
                put(2, rng.uniform(.5, 1.5, (rows, nblk)) * dscale[t])
        return raw.reshape(rows, nblk * nbytes)

    def addq(name, t, shape):
        spec.add(name, t, list(reversed(shape)), quant(t, shape))

    def addf(name, arr):
        arr = np.asarray(arr).astype(np.float32)
        spec.add(name, F32, list(reversed(arr.shape)), arr)

    addq("token_embd.weight", Q8_0, (V, D))
    addq("output.weight", Q6_K, (V, D))
    addf("output_norm.weight", rng.uniform(.8, 1.2, D))
    for l in range(NL):
        p = f"blk.{l}."
        addf(p + "attn_norm.weight", rng.uniform(.8, 1.2, D))
        addf(p + "ffn_norm.weight", rng.uniform(.8, 1.2, D))
        addf(p + "attn_q_norm.weight", rng.uniform(.8, 1.2, HD))
        addf(p + "attn_k_norm.weight", rng.uniform(.8, 1.2, HD))
        addq(p + "attn_q.weight", Q5_K, (QD, D))
        addq(p + "attn_k.weight", Q8_0, (KD, D))
        addq(p + "attn_v.weight", Q6_K, (KD, D))
        addq(p + "attn_output.weight", Q4_K, (D, QD))
        addf(p + "ffn_gate_inp.weight", rng.normal(0, .3, (E, D)))
        addq(p + "ffn_gate_exps.weight", Q5_K, (E, FF, D))
        addq(p + "ffn_up_exps.weight", Q4_K, (E, FF, D))
        addq(p + "ffn_down_exps.weight", Q6_K, (E, D, FF))
    return spec


# ---------------------------------------------------------------------------
# config 0: tiny Q8_0-expert model quantized from N(0, 0.02)

def config0_spec(seed=0, quantize=None):
    """``quantize(type, fp32[rows][ne0]) -> uint8[rows][row_bytes]``; defaults to
    the library's host quantizer."""
    if quantize is None:
        import importlib.util
        import os
        pkg = os.path.join(os.path.dirname(os.path.dirname(os.path.abspath(__file__))),
                           "eahmmf_inference_prototype_v-0.1.0_amd", "eahmmf_hip.py")
        s = importlib.util.spec_from_file_location("eahmmf_hip_bind", pkg)
        mod = importlib.util.module_from_spec(s)
        s.loader.exec_module(mod)
        quantize = mod.quantize_rows
    rng = np.random.default_rng(seed)
    D, NH, NKV, HD, E, K, FF, NL, CTX, V = 256, 4, 2, 64, 8, 2, 128, 2, 64, 1024
    QD, KD = NH * HD, NKV * HD
    spec = ModelSpec(n_layer=NL, D=D, n_head=NH, n_kv=NKV, hd=HD, n_expert=E, n_used=K, FF=FF, n_vocab=V,
                     n_ctx=CTX, ctx_train=CTX, eps=1e-6, rope_base=1e6)

    def addf(name, arr):
        arr = np.asarray(arr, dtype=np.float32)
        spec.add(name, F32, list(reversed(arr.shape)), arr)

    def n(*shape):
        return rng.normal(0, 0.02, shape).astype(np.float32)

    addf("token_embd.weight", n(V, D))
    addf("output.weight", n(V, D))
    addf("output_norm.weight", 1 + n(D))
    for l in range(NL):
        p = f"blk.{l}."
        addf(p + "attn_norm.weight", 1 + n(D))
        addf(p + "ffn_norm.weight", 1 + n(D))
        addf(p + "attn_q_norm.weight", 1 + n(HD))
        addf(p + "attn_k_norm.weight", 1 + n(HD))
        addf(p + "attn_q.weight", n(QD, D))
        addf(p + "attn_k.weight", n(KD, D))
        addf(p + "attn_v.weight", n(KD, D))
        addf(p + "attn_output.weight", n(D, QD))
        addf(p + "ffn_gate_inp.weight", n(E, D))
        for nm, shape in (("ffn_gate_exps", (E, FF, D)), ("ffn_up_exps", (E, FF, D)), ("ffn_down_exps", (E, D, FF))):
            w = n(*shape).reshape(-1, shape[-1])
            q = quantize(Q8_0, w)
            spec.add(p + nm + ".weight", Q8_0, list(reversed(shape)), q)
    return spec


# ---------------------------------------------------------------------------
# GGUF v3

def _str(s):
    b = s.encode()
    return struct.pack("<Q", len(b)) + b


def write_gguf(spec, path, align=32):
    kv = [("general.architecture", 8, "qwen3moe")]
    a = "qwen3moe."
    for key, val in (("block_count", spec.n_layer), ("context_length", spec.ctx_train),
                     ("embedding_length", spec.D), ("attention.head_count", spec.n_head),
                     ("attention.head_count_kv", spec.n_kv), ("attention.key_length", spec.hd),
                     ("attention.value_length", spec.hd), ("expert_count", spec.n_expert),
                     ("expert_used_count", spec.n_used), ("expert_feed_forward_length", spec.FF)):
        kv.append((a + key, 4, int(val)))
    kv.append((a + "rope.freq_base", 6, float(spec.rope_base)))
    kv.append((a + "attention.layer_norm_rms_epsilon", 6, float(spec.eps)))
    out = bytearray(b"GGUF" + struct.pack("<IQQ", 3, len(spec.order), len(kv)))
    for key, t, val in kv:
        out += _str(key) + struct.pack("<I", t)
        if t == 8:
            out += _str(val)
        elif t == 4:
            out += struct.pack("<I", val)
        elif t == 6:
            out += struct.pack("<f", val)
    blobs, off = [], 0
    for name in spec.order:
        t, ne, data = spec.tensors[name]
        raw = np.ascontiguousarray(data).tobytes()
        off = (off + align - 1) // align * align
        out += _str(name) + struct.pack("<I", len(ne)) + b"".join(struct.pack("<Q", d) for d in ne)
        out += struct.pack("<IQ", t, off)
        blobs.append((off, raw))
        off += len(raw)
    pad = (-len(out)) % align
    out += b"\0" * pad
    base = len(out)
    body = bytearray(off)
    for o, raw in blobs:
        body[o:o + len(raw)] = raw
    with open(path, "wb") as f:
        f.write(out)
        f.write(body)
    return base


def weight_digest(spec):
    """sha256 over tensor names and bytes, in insertion order."""
    import hashlib
    h = hashlib.sha256()
    for name in spec.order:
        h.update(name.encode())
        h.update(np.ascontiguousarray(spec.tensors[name][2]).tobytes())
    return h.hexdigest()
