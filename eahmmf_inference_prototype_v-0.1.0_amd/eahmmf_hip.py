"""ctypes binding of libeahmmf_hip.so (the C ABI in include/eahmmf_hip.h).

This is the Python view of the same entry points a C++ host (the reference's
qwen3moe.cpp) binds with ``extern "C"`` declarations.  It adds nothing to the
compute path: every call goes straight to the HIP library, and importing this
module fails loudly when the library has not been built.
"""
import ctypes
import os

_HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(_HERE, "libeahmmf_hip.so")

GGML_F32, GGML_Q8_0, GGML_Q4_K, GGML_Q5_K, GGML_Q6_K = 0, 8, 12, 13, 14
BLOCK = {GGML_F32: (32, 128), GGML_Q8_0: (32, 34), GGML_Q4_K: (256, 144), GGML_Q5_K: (256, 176), GGML_Q6_K: (256, 210)}
MAX_TOPK = 16

# Every symbol declared in include/eahmmf_hip.h.
EXPORTS = (
    "eahmmf_hip_matmul", "eahmmf_hip_matmul_pair", "eahmmf_hip_moe_decode", "eahmmf_hip_moe_decode_async",
    "eahmmf_hip_moe_decode_routed_async", "eahmmf_hip_route_topk", "eahmmf_hip_route_topk_async",
    "eahmmf_hip_dequantize", "eahmmf_hip_row_bytes", "eahmmf_hip_quantize_rows", "eahmmf_hip_alloc",
    "eahmmf_hip_free", "eahmmf_hip_h2d", "eahmmf_hip_d2h", "eahmmf_hip_sync", "eahmmf_hip_mem_info",
    "eahmmf_hip_last_error", "eahmmf_hip_device_count", "eahmmf_hip_shutdown", "eahmmf_hip_moe_layer_decode_async",
    "eahmmf_hip_set_fused", "eahmmf_hip_device_flags", "eahmmf_hip_fused_exchange", "eahmmf_hip_moe_grouped",
    "eahmmf_hip_moe_grouped_async", "eahmmf_hip_set_grouped_mfma", "eahmmf_hip_stream_read_async",
    "eahmmf_hip_h2d_batch", "eahmmf_hip_fused_status_async", "eahmmf_hip_set_fault_injection",
    "eahmmf_hip_moe_layer_decode_noalloc", "eahmmf_hip_expf_ref_async", "eahmmf_hip_moe_decode_resident",
    "eahmmf_hip_model_create", "eahmmf_hip_model_forward", "eahmmf_hip_model_eval", "eahmmf_hip_model_generate_greedy",
    "eahmmf_hip_model_set_trace", "eahmmf_hip_model_trace", "eahmmf_hip_model_trace_clear", "eahmmf_hip_model_stream",
    "eahmmf_hip_model_free", "eahmmf_hip_model_set_sequences", "eahmmf_hip_model_forward_seq",
    "eahmmf_hip_model_decode_seqs", "eahmmf_hip_set_dense_mfma", "eahmmf_hip_moe_layer_decode_xn_async", "eahmmf_hip_set_grouped_wave_max",
    "eahmmf_hip_set_grouped_dot_max", "eahmmf_hip_h2d_batch_async", "eahmmf_hip_h2d_batch_wait",
    "eahmmf_hip_h2d_batch_query",
)


class Weight(ctypes.Structure):
    _fields_ = [("dev", ctypes.c_void_p), ("type", ctypes.c_int), ("ne0", ctypes.c_int), ("ne1", ctypes.c_int),
                ("row_bytes", ctypes.c_size_t)]


class Expert(ctypes.Structure):
    _fields_ = [("gate", Weight), ("up", Weight), ("down", Weight)]


class ExpertPtrs(ctypes.Structure):
    _fields_ = [("gate", ctypes.c_void_p), ("up", ctypes.c_void_p), ("down", ctypes.c_void_p)]


class Copy(ctypes.Structure):
    _fields_ = [("dev_dst", ctypes.c_void_p), ("host_src", ctypes.c_void_p), ("bytes", ctypes.c_size_t)]


class MoeShape(ctypes.Structure):
    _fields_ = [("gate_type", ctypes.c_int), ("up_type", ctypes.c_int), ("down_type", ctypes.c_int),
                ("D", ctypes.c_int), ("FF", ctypes.c_int), ("gate_row_bytes", ctypes.c_size_t),
                ("up_row_bytes", ctypes.c_size_t), ("down_row_bytes", ctypes.c_size_t)]


class Tensor(ctypes.Structure):
    _fields_ = [("data", ctypes.c_void_p), ("on_device", ctypes.c_int), ("type", ctypes.c_int),
                ("ne0", ctypes.c_int64), ("ne1", ctypes.c_int64), ("row_bytes", ctypes.c_size_t)]


class LayerDesc(ctypes.Structure):
    _fields_ = [(n, Tensor) for n in ("attn_norm", "ffn_norm", "q_norm", "k_norm", "wq", "wk", "wv", "wo", "router",
                                      "gate_exps", "up_exps", "down_exps")]


class ModelDesc(ctypes.Structure):
    _fields_ = [(n, ctypes.c_int) for n in ("n_layer", "D", "n_head", "n_kv", "hd", "n_expert", "n_used", "FF",
                                            "n_vocab", "n_ctx")] + \
               [("eps", ctypes.c_float), ("rope_base", ctypes.c_float), ("tok_embd", Tensor),
                ("output_norm", Tensor), ("output", Tensor), ("layers", ctypes.POINTER(LayerDesc))]


def row_bytes(gtype, ne0):
    blck, nbytes = BLOCK[gtype]
    if ne0 % blck:
        raise ValueError(f"row length {ne0} is not a multiple of {blck}")
    return ne0 // blck * nbytes


def _share_torch_runtime():
    """PyTorch wheels bundle their own HIP/HSA runtime.  A process must hold
    only one: two runtimes each try to own the device and the second reports
    no device.  When torch is installed it is imported first, and the
    library's libamdhip64.so.7 dependency then resolves to the runtime torch
    already loaded (same soname).  Without torch the system ROCm runtime is
    used."""
    try:
        import torch  # noqa: F401
    except ImportError:
        pass


def load(path=LIB_PATH):
    """Load the library and declare its signatures.  Raises if it is missing."""
    if not os.path.exists(path):
        raise RuntimeError(f"{path} is not built; run __graft_entry__.build() (make -C the package)")
    _share_torch_runtime()
    lib = ctypes.CDLL(path)
    c_bool, c_int, c_sz, c_i64, vp = ctypes.c_bool, ctypes.c_int, ctypes.c_size_t, ctypes.c_int64, ctypes.c_void_p
    sig = {
        "eahmmf_hip_matmul": (c_bool, [vp, c_int, c_int, c_int, c_sz, vp, c_int, c_int, vp, c_int]),
        "eahmmf_hip_matmul_pair": (c_bool, [vp, c_int, c_int, c_int, c_sz, vp, c_int, c_int, c_int, c_sz,
                                            vp, c_int, c_int, vp, c_int, vp, c_int]),
        "eahmmf_hip_moe_decode": (c_bool, [ctypes.POINTER(Expert), vp, c_int, vp, vp]),
        "eahmmf_hip_moe_decode_async": (c_int, [ctypes.POINTER(MoeShape), ctypes.POINTER(ExpertPtrs), vp, c_int,
                                                vp, vp, vp]),
        "eahmmf_hip_moe_decode_routed_async": (c_int, [ctypes.POINTER(MoeShape), vp, c_int, vp, vp, c_int, vp, vp,
                                                       vp]),
        "eahmmf_hip_moe_layer_decode_async": (c_int, [ctypes.POINTER(MoeShape), vp, c_int, vp, c_int, vp, vp, vp,
                                                      vp, vp]),
        "eahmmf_hip_moe_layer_decode_xn_async": (c_int, [ctypes.POINTER(MoeShape), vp, c_int, vp, vp, ctypes.c_float,
                                                         vp, c_int, vp, vp, vp, vp, vp, vp]),
        "eahmmf_hip_moe_layer_decode_noalloc": (c_int, [ctypes.POINTER(MoeShape), vp, c_int, vp, c_int, vp, vp, vp,
                                                        vp, vp]),
        "eahmmf_hip_set_fused": (c_int, [c_int]),
        "eahmmf_hip_device_flags": (c_int, []),
        "eahmmf_hip_fused_status_async": (c_int, [vp, vp]),
        "eahmmf_hip_set_fault_injection": (None, [ctypes.c_uint, c_int]),
        "eahmmf_hip_fused_exchange": (c_int, []),
        "eahmmf_hip_set_grouped_mfma": (c_int, [c_int]),
        "eahmmf_hip_set_grouped_wave_max": (c_int, [c_int]),
        "eahmmf_hip_set_grouped_dot_max": (c_int, [c_int]),
        "eahmmf_hip_moe_grouped": (c_bool, [ctypes.POINTER(Expert), c_int, vp, vp, vp, c_int, vp, vp]),
        "eahmmf_hip_moe_grouped_async": (c_int, [ctypes.POINTER(MoeShape), vp, c_int, vp, vp, c_int, c_int, vp, vp,
                                                 vp]),
        "eahmmf_hip_route_topk": (c_bool, [vp, c_int, c_int, c_int, vp, vp]),
        "eahmmf_hip_route_topk_async": (c_int, [vp, c_int, c_int, c_int, vp, vp, vp]),
        "eahmmf_hip_stream_read_async": (c_int, [vp, ctypes.c_size_t, vp, vp]),
        "eahmmf_hip_expf_ref_async": (c_int, [vp, vp, c_i64, vp]),
        "eahmmf_hip_moe_decode_resident": (c_bool, [ctypes.POINTER(Expert), vp, c_int, vp, vp, vp]),
        "eahmmf_hip_h2d_batch": (c_int, [ctypes.POINTER(Copy), c_int]),
        "eahmmf_hip_h2d_batch_async": (c_int, [ctypes.POINTER(Copy), c_int, ctypes.POINTER(ctypes.c_uint64)]),
        "eahmmf_hip_h2d_batch_wait": (c_int, [ctypes.c_uint64, vp]),
        "eahmmf_hip_h2d_batch_query": (c_int, [ctypes.c_uint64]),
        "eahmmf_hip_model_create": (vp, [ctypes.POINTER(ModelDesc)]),
        "eahmmf_hip_model_forward": (c_int, [vp, vp, c_int, c_int, vp]),
        "eahmmf_hip_model_eval": (c_int, [vp, vp, c_int, c_int, c_int, vp]),
        "eahmmf_hip_model_generate_greedy": (c_int, [vp, c_int, c_int, c_int, vp, vp]),
        "eahmmf_hip_model_set_trace": (c_int, [vp, c_int]),
        "eahmmf_hip_model_trace": (c_int, [vp, vp, vp, c_int]),
        "eahmmf_hip_model_trace_clear": (None, [vp]),
        "eahmmf_hip_model_stream": (vp, [vp]),
        "eahmmf_hip_model_free": (None, [vp]),
        "eahmmf_hip_model_set_sequences": (c_int, [vp, c_int]),
        "eahmmf_hip_model_forward_seq": (c_int, [vp, c_int, vp, c_int, c_int, vp]),
        "eahmmf_hip_model_decode_seqs": (c_int, [vp, c_int, vp, vp, vp, vp]),
        "eahmmf_hip_set_dense_mfma": (c_int, [c_int]),
        "eahmmf_hip_dequantize": (c_int, [vp, c_int, c_i64, c_i64, c_sz, vp, vp]),
        "eahmmf_hip_row_bytes": (c_sz, [c_int, c_i64]),
        "eahmmf_hip_quantize_rows": (c_i64, [c_int, vp, c_i64, c_i64, vp]),
        "eahmmf_hip_alloc": (c_int, [ctypes.POINTER(vp), c_sz]),
        "eahmmf_hip_free": (c_int, [vp]),
        "eahmmf_hip_h2d": (c_int, [vp, vp, c_sz]),
        "eahmmf_hip_d2h": (c_int, [vp, vp, c_sz]),
        "eahmmf_hip_sync": (c_int, []),
        "eahmmf_hip_mem_info": (c_int, [ctypes.POINTER(c_sz), ctypes.POINTER(c_sz)]),
        "eahmmf_hip_last_error": (ctypes.c_char_p, []),
        "eahmmf_hip_device_count": (c_int, []),
        "eahmmf_hip_shutdown": (None, []),
    }
    for name, (res, args) in sig.items():
        fn = getattr(lib, name)
        fn.restype = res
        fn.argtypes = args
    return lib


_lib = None


def lib():
    global _lib
    if _lib is None:
        _lib = load()
    return _lib


def last_error():
    return lib().eahmmf_hip_last_error().decode()


def quantize_rows(gtype, src):
    """fp32 [nrows][ne0] (numpy) -> uint8 [nrows][row_bytes] via the library's host quantizer."""
    import numpy as np
    src = np.ascontiguousarray(src, dtype=np.float32)
    nrows, ne0 = src.shape
    rb = row_bytes(gtype, ne0)
    out = np.empty((nrows, rb), dtype=np.uint8)
    n = lib().eahmmf_hip_quantize_rows(gtype, src.ctypes.data, nrows, ne0, out.ctypes.data)
    if n != nrows * rb:
        raise RuntimeError(f"quantize_rows failed: {last_error()}")
    return out


_HP = ("n_layer", "D", "n_head", "n_kv", "hd", "n_expert", "n_used", "FF", "n_vocab", "n_ctx")
_LAYER = (("attn_norm", "attn_norm"), ("ffn_norm", "ffn_norm"), ("q_norm", "attn_q_norm"), ("k_norm", "attn_k_norm"),
          ("wq", "attn_q"), ("wk", "attn_k"), ("wv", "attn_v"), ("wo", "attn_output"), ("router", "ffn_gate_inp"),
          ("gate_exps", "ffn_gate_exps"), ("up_exps", "ffn_up_exps"), ("down_exps", "ffn_down_exps"))


class DeviceModel:
    """A whole Qwen3-MoE model on the current device (eahmmf_hip_model_*): the
    reference's Engine (qwen3moe.cpp:859-1084) with every layer on the GPU.

    ``hp``: mapping with n_layer, D, n_head, n_kv, hd, n_expert, n_used, FF,
    n_vocab, n_ctx, eps, rope_base.  ``tensors``: GGUF tensor name ->
    (ggml type, ne with ne0 first, data), data a numpy array of the tensor's
    bytes or values (copied to the device at creation) or an int device
    address (used in place; the caller keeps it alive).  A missing
    ``output.weight`` ties the output head to ``token_embd.weight``
    (qwen3moe.cpp:881-882)."""

    def __init__(self, hp, tensors):
        import numpy as np
        self._lib = lib()
        keep = []

        def desc(name):
            t, ne, data = tensors[name]
            ne0 = int(ne[0])
            ne1 = int(np.prod([int(v) for v in ne[1:]])) if len(ne) > 1 else 1
            if isinstance(data, int):
                return Tensor(data, 1, t, ne0, ne1, row_bytes(t, ne0))
            arr = np.ascontiguousarray(data)
            keep.append(arr)
            return Tensor(arr.ctypes.data, 0, t, ne0, ne1, row_bytes(t, ne0))

        L = int(hp["n_layer"])
        layers = (LayerDesc * L)()
        for l in range(L):
            for field, nm in _LAYER:
                setattr(layers[l], field, desc(f"blk.{l}.{nm}.weight"))
        d = ModelDesc()
        for n in _HP:
            setattr(d, n, int(hp[n]))
        d.eps = float(hp["eps"])
        d.rope_base = float(hp["rope_base"])
        d.tok_embd = desc("token_embd.weight")
        d.output_norm = desc("output_norm.weight")
        d.output = desc("output.weight") if "output.weight" in tensors else Tensor()
        d.layers = layers
        self.n_vocab = int(hp["n_vocab"])
        self.n_layer, self.n_used = L, int(hp["n_used"])
        self.h = self._lib.eahmmf_hip_model_create(ctypes.byref(d))
        if not self.h:
            raise RuntimeError(f"eahmmf_hip_model_create: {last_error()}")

    def _check(self, rc, what):
        if rc != 0:
            raise RuntimeError(f"{what} ({rc}): {last_error()}")

    def forward(self, toks, p0, logits=True, seq=0):
        """Engine::forward on sequence ``seq``: tokens at p0..; the last
        token's logits (or None)."""
        import numpy as np
        t = np.ascontiguousarray(toks, dtype=np.int32)
        out = np.empty(self.n_vocab, np.float32) if logits else None
        self._check(self._lib.eahmmf_hip_model_forward_seq(self.h, int(seq), t.ctypes.data, len(t), int(p0),
                                                           out.ctypes.data if logits else None), "forward")
        return out

    def eval(self, toks, p0, n_batch, seq=0):
        """Engine::eval on sequence ``seq``: chunks of n_batch from p0; the
        last token's logits."""
        import numpy as np
        t = np.ascontiguousarray(toks, dtype=np.int32)
        out = np.empty(self.n_vocab, np.float32)
        if seq == 0:
            self._check(self._lib.eahmmf_hip_model_eval(self.h, t.ctypes.data, len(t), int(p0), int(n_batch),
                                                        out.ctypes.data), "eval")
            return out
        if not 1 <= int(n_batch) <= 64 or len(t) == 0:
            raise ValueError("n_batch outside 1..64 or empty input")
        nb = int(n_batch)
        for i in range(0, len(t), nb):
            lg = self.forward(t[i:i + nb], int(p0) + i, logits=i + nb >= len(t), seq=seq)
        return lg

    def set_sequences(self, n_seq):
        """n_seq independent sequences (KV rows of their own), all empty."""
        self._check(self._lib.eahmmf_hip_model_set_sequences(self.h, int(n_seq)), "set_sequences")

    def decode_seqs(self, toks, seqs, pos, logits=True):
        """One decode step of several sequences in one batch: token toks[i]
        at position pos[i] of sequence seqs[i]; logits [n][n_vocab] (or None)."""
        import numpy as np
        t = np.ascontiguousarray(toks, dtype=np.int32)
        s = np.ascontiguousarray(seqs, dtype=np.int32)
        p = np.ascontiguousarray(pos, dtype=np.int32)
        if not len(t) == len(s) == len(p):
            raise ValueError("toks, seqs and pos differ in length")
        out = np.empty((len(t), self.n_vocab), np.float32) if logits else None
        self._check(self._lib.eahmmf_hip_model_decode_seqs(self.h, len(t), t.ctypes.data, s.ctypes.data,
                                                           p.ctypes.data, out.ctypes.data if logits else None),
                    "decode_seqs")
        return out

    def generate_greedy(self, first, p0, n):
        """Feeds ``first`` at p0 and then each argmax, n forwards in all, with
        one host synchronisation; returns (the n argmax tokens, last logits)."""
        import numpy as np
        toks = np.empty(n, np.int32)
        lg = np.empty(self.n_vocab, np.float32)
        self._check(self._lib.eahmmf_hip_model_generate_greedy(self.h, int(first), int(p0), int(n), toks.ctypes.data,
                                                               lg.ctypes.data), "generate_greedy")
        return toks, lg

    def set_trace(self, on):
        return self._lib.eahmmf_hip_model_set_trace(self.h, 1 if on else 0)

    def trace(self):
        """(ids, weights) recorded since the last clear, per forward: layer, token, rank."""
        import numpy as np
        n = self._lib.eahmmf_hip_model_trace(self.h, None, None, 0)
        ids, w = np.empty(n, np.int32), np.empty(n, np.float32)
        self._lib.eahmmf_hip_model_trace(self.h, ids.ctypes.data, w.ctypes.data, n)
        return ids, w

    def trace_clear(self):
        self._lib.eahmmf_hip_model_trace_clear(self.h)

    @property
    def stream(self):
        return self._lib.eahmmf_hip_model_stream(self.h)

    def close(self):
        if getattr(self, "h", None):
            self._lib.eahmmf_hip_model_free(self.h)
            self.h = None

    def __del__(self):
        self.close()


# ---------------------------------------------------------------------------
# GGUF v3 reader (the file layout qwen3moe.cpp:285-346 parses): key/values,
# the tensor table and zero-copy views of the tensor bytes in a memory map.

_GGUF_SCALAR = {0: "<B", 1: "<b", 2: "<H", 3: "<h", 4: "<I", 5: "<i", 6: "<f", 7: "<?", 10: "<Q", 11: "<q", 12: "<d"}


def read_gguf(path):
    """-> (kv: dict, tensors: {name: (ggml type, ne (ne0 first), numpy view)}).
    Quantized tensors are uint8 [rows][row_bytes] views, F32 tensors float32
    [rows][ne0]; both read-only views of a memory map of the file."""
    import mmap
    import struct

    import numpy as np
    with open(path, "rb") as f:
        mm = mmap.mmap(f.fileno(), 0, access=mmap.ACCESS_READ)
    pos = 0

    def take(fmt):
        nonlocal pos
        v = struct.unpack_from(fmt, mm, pos)
        pos += struct.calcsize(fmt)
        return v[0]

    def string():
        nonlocal pos
        n = take("<Q")
        s = bytes(mm[pos:pos + n]).decode("utf-8", "replace")
        pos += n
        return s

    def value(t):
        if t in _GGUF_SCALAR:
            return take(_GGUF_SCALAR[t])
        if t == 8:
            return string()
        if t == 9:
            et, n = take("<I"), take("<Q")
            return [value(et) for _ in range(n)]
        raise ValueError(f"{path}: unknown GGUF value type {t}")

    if bytes(mm[0:4]) != b"GGUF":
        raise ValueError(f"{path}: not a GGUF file")
    pos = 4
    version, n_tensors, n_kv = take("<I"), take("<Q"), take("<Q")
    if version < 2:
        raise ValueError(f"{path}: GGUF version {version} not supported")
    kv = {}
    for _ in range(n_kv):
        key = string()
        kv[key] = value(take("<I"))
    infos = []
    for _ in range(n_tensors):
        name = string()
        nd = take("<I")
        ne = [take("<Q") for _ in range(nd)]
        t, off = take("<I"), take("<Q")
        infos.append((name, t, ne, off))
    align = int(kv.get("general.alignment", 32))
    base = (pos + align - 1) // align * align
    buf = np.frombuffer(mm, dtype=np.uint8)
    tensors = {}
    for name, t, ne, off in infos:
        if t not in BLOCK:
            raise ValueError(f"{path}: tensor {name} has unsupported type {t}")
        rb = row_bytes(t, ne[0])
        rows = int(np.prod(ne[1:])) if len(ne) > 1 else 1
        raw = buf[base + off: base + off + rb * rows].reshape(rows, rb)
        tensors[name] = (t, list(ne), raw.view(np.float32) if t == GGML_F32 else raw)
    return kv, tensors


def gguf_hparams(kv, tensors, ctx):
    """The model hyper-parameters as the reference's Engine::load reads them
    (qwen3moe.cpp:862-882): required keys, the same defaults, n_ctx =
    min(ctx, context_length), n_vocab from the output head's rows."""
    if kv.get("general.architecture") != "qwen3moe":
        raise ValueError(f"unsupported architecture {kv.get('general.architecture')!r} (need qwen3moe)")
    a = "qwen3moe."

    def need(key):
        if a + key not in kv:
            raise ValueError(f"missing GGUF key {a + key}")
        return kv[a + key]

    hp = dict(n_layer=int(need("block_count")), D=int(need("embedding_length")), n_head=int(need("attention.head_count")),
              n_kv=int(need("attention.head_count_kv")), n_expert=int(need("expert_count")),
              n_used=int(need("expert_used_count")), FF=int(need("expert_feed_forward_length")))
    hp["hd"] = int(kv.get(a + "attention.key_length", hp["D"] // hp["n_head"]))
    hp["eps"] = float(kv.get(a + "attention.layer_norm_rms_epsilon", 1e-6))
    hp["rope_base"] = float(kv.get(a + "rope.freq_base", 1e6))
    hp["n_ctx"] = min(int(ctx), int(kv.get(a + "context_length", 4096)))
    head = tensors.get("output.weight", tensors["token_embd.weight"])
    hp["n_vocab"] = int(head[1][1])
    return hp


def model_from_gguf(path, ctx):
    """A DeviceModel of a qwen3moe GGUF file (the reference's Engine::load)."""
    kv, tensors = read_gguf(path)
    return DeviceModel(gguf_hparams(kv, tensors, ctx), tensors)
