"""Python access to the CPU checker libraries (TEST INFRASTRUCTURE ONLY).

liboracle.so      our C restatement of the reference CPU path (oracle.c)
_ref/libref.so    the reference's own qwen3moe.cpp compiled in place
                  (ref_harness.cpp), present only where the reference sources
                  were available at build time

Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg import
this package, and only to check or time against it; the shipped library never
links or calls it.
"""
import ctypes
import os

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
ORACLE_SO = os.path.join(HERE, "liboracle.so")
REF_SO = os.path.join(HERE, "_ref", "libref.so")
REF_PORTABLE_SO = os.path.join(HERE, "_ref", "libref_portable.so")

F32, Q8_0, Q4_K, Q5_K, Q6_K = 0, 8, 12, 13, 14
BLOCK = {F32: (32, 128), Q8_0: (32, 34), Q4_K: (256, 144), Q5_K: (256, 176), Q6_K: (256, 210)}

vp = ctypes.c_void_p


def row_bytes(t, ne0):
    blck, nb = BLOCK[t]
    assert ne0 % blck == 0
    return ne0 // blck * nb


class View(ctypes.Structure):
    _fields_ = [("data", vp), ("type", ctypes.c_int), ("ne0", ctypes.c_int64), ("ne1", ctypes.c_int64),
                ("row_bytes", ctypes.c_size_t)]


class Experts(ctypes.Structure):
    _fields_ = [("n_expert", ctypes.c_int), ("D", ctypes.c_int), ("FF", ctypes.c_int),
                ("views", ctypes.POINTER(View))]


class Model(ctypes.Structure):
    _fields_ = [(n, ctypes.c_int) for n in ("n_layer", "D", "n_head", "n_kv", "hd", "n_expert", "n_used", "FF",
                                               "n_vocab", "n_ctx")] + [
        ("eps", ctypes.c_float), ("rope_base", ctypes.c_float), ("tok_embd", View), ("output", View),
        ("output_norm", vp), ("attn_norm", vp), ("ffn_norm", vp), ("q_norm", vp), ("k_norm", vp),
        ("wq", ctypes.POINTER(View)), ("wk", ctypes.POINTER(View)), ("wv", ctypes.POINTER(View)),
        ("wo", ctypes.POINTER(View)), ("router", ctypes.POINTER(View)), ("experts", ctypes.POINTER(View))]


def _ptr(a):
    return a.ctypes.data


_lib = None


def lib():
    global _lib
    if _lib is None:
        if not os.path.exists(ORACLE_SO):
            raise RuntimeError("oracle/liboracle.so not built (make -C oracle)")
        L = ctypes.CDLL(ORACLE_SO)
        L.orc_f16.restype = ctypes.c_float
        L.orc_f16.argtypes = [ctypes.c_uint16]
        L.orc_scale_min_k4.argtypes = [ctypes.c_int, vp, vp, vp]
        L.orc_dequant_rows.argtypes = [ctypes.c_int, vp, ctypes.c_int64, ctypes.c_int64, ctypes.c_size_t, vp]
        L.orc_matmul.argtypes = [ctypes.c_int, ctypes.c_int64, ctypes.c_int64, ctypes.c_size_t, vp, vp,
                                 ctypes.c_int, ctypes.c_int, vp, ctypes.c_int]
        L.orc_rmsnorm.argtypes = [vp, vp, vp, ctypes.c_int, ctypes.c_float]
        L.orc_route_topk.argtypes = [vp, ctypes.c_int, ctypes.c_int, ctypes.c_int, vp, vp]
        L.orc_expf_array.argtypes = [vp, vp, ctypes.c_int64]
        L.orc_moe_layer.argtypes = [ctypes.POINTER(Experts), vp, ctypes.c_int, ctypes.c_int, vp, vp, vp]
        L.orc_state_new.restype = vp
        L.orc_state_new.argtypes = [ctypes.POINTER(Model)]
        L.orc_state_free.argtypes = [vp]
        L.orc_state_trace.argtypes = [vp, vp, vp, ctypes.c_int, ctypes.POINTER(ctypes.c_int)]
        L.orc_forward.argtypes = [vp, vp, ctypes.c_int, ctypes.c_int, vp]
        L.orc_state_set_moe_hook.argtypes = [vp, vp, vp]
        L.orc_state_set_moe_hook.restype = None
        L.orc_init()
        _lib = L
    return _lib


def f16(h):
    return lib().orc_f16(int(h))


def scale_min_k4(j, q12):
    q = np.ascontiguousarray(q12, dtype=np.uint8)
    d, m = ctypes.c_uint8(), ctypes.c_uint8()
    lib().orc_scale_min_k4(j, _ptr(q), ctypes.byref(d), ctypes.byref(m))
    return d.value, m.value


def dequant_rows(t, w, ne0):
    w = np.ascontiguousarray(w, dtype=np.uint8).reshape(-1, row_bytes(t, ne0))
    out = np.empty((w.shape[0], ne0), dtype=np.float32)
    assert lib().orc_dequant_rows(t, _ptr(w), ne0, w.shape[0], w.shape[1], _ptr(out)) == 0
    return out


def matmul(t, w, ne0, x):
    """out[nb][ne1] = W[ne1][ne0] . x[nb][ne0]"""
    w = np.ascontiguousarray(w, dtype=np.uint8).reshape(-1, row_bytes(t, ne0))
    x = np.ascontiguousarray(x, dtype=np.float32).reshape(-1, ne0)
    out = np.empty((x.shape[0], w.shape[0]), dtype=np.float32)
    assert lib().orc_matmul(t, ne0, w.shape[0], w.shape[1], _ptr(w), _ptr(x), x.shape[0], ne0, _ptr(out),
                            w.shape[0]) == 0
    return out


def rmsnorm(x, w, eps):
    """x / sqrt(mean(x^2) + eps) * w per row (qwen3moe.cpp:527-532)."""
    x = np.ascontiguousarray(x, dtype=np.float32)
    w = np.ascontiguousarray(w, dtype=np.float32)
    rows = x.reshape(-1, x.shape[-1])
    out = np.empty_like(rows)
    for r in range(rows.shape[0]):
        lib().orc_rmsnorm(_ptr(rows[r]), _ptr(w), _ptr(out[r]), rows.shape[1], ctypes.c_float(eps))
    return out.reshape(x.shape)


def route_topk(logits, k):
    logits = np.ascontiguousarray(logits, dtype=np.float32)
    nb, E = logits.shape
    ids = np.empty((nb, k), dtype=np.int32)
    w = np.empty((nb, k), dtype=np.float32)
    lib().orc_route_topk(_ptr(logits), nb, E, k, _ptr(ids), _ptr(w))
    return ids, w


def expf(x):
    """Elementwise expf of float32 x with the host libm (the routing keys' exp)."""
    x = np.ascontiguousarray(x, dtype=np.float32)
    y = np.empty_like(x)
    lib().orc_expf_array(_ptr(x), _ptr(y), x.size)
    return y


def make_view(t, w, ne0):
    w = np.ascontiguousarray(w, dtype=np.uint8)
    rb = row_bytes(t, ne0)
    return View(w.ctypes.data, t, ne0, w.size // rb, rb), w


def moe_layer(experts, xn, ids, wts):
    """experts: list of ((gtype, gate_bytes), (utype, up_bytes), (dtype, down_bytes)) with
    gate/up [FF][row] over D and down [D][row] over FF; xn [nb][D]; ids/wts [nb][k]."""
    xn = np.ascontiguousarray(xn, dtype=np.float32)
    ids = np.ascontiguousarray(ids, dtype=np.int32)
    wts = np.ascontiguousarray(wts, dtype=np.float32)
    nb, D = xn.shape
    k = ids.shape[1]
    keep = []
    views = (View * (3 * len(experts)))()
    FF = None
    for e, comps in enumerate(experts):
        for c, (t, w) in enumerate(comps):
            ne0 = D if c < 2 else None
            if c == 2:
                ne0 = FF
            v, buf = make_view(t, w, ne0)
            keep.append(buf)
            views[3 * e + c] = v
            if c == 0:
                FF = v.ne1
    ex = Experts(len(experts), D, FF, views)
    out = np.empty((nb, D), dtype=np.float32)
    assert lib().orc_moe_layer(ctypes.byref(ex), _ptr(xn), nb, k, _ptr(ids), _ptr(wts), _ptr(out)) == 0
    return out


class OracleModel:
    """Wraps orc_forward over a model described by tests/gguf_tools.ModelSpec."""

    def __init__(self, spec):
        self.spec = spec
        self._keep = []
        L = spec.n_layer

        def view(name):
            t, ne, data = spec.tensors[name]
            data = np.ascontiguousarray(data)
            self._keep.append(data)
            rb = row_bytes(t, ne[0])
            nrows = int(np.prod(ne[1:]))
            return View(data.ctypes.data, t, ne[0], nrows, rb)

        def f32(name):
            t, ne, data = spec.tensors[name]
            arr = np.ascontiguousarray(np.frombuffer(np.ascontiguousarray(data).tobytes(), dtype=np.float32))
            self._keep.append(arr)
            return arr

        def arr_ptrs(fmt):
            a = (vp * L)(*[f32(fmt % l).ctypes.data for l in range(L)])
            self._keep.append(a)
            return ctypes.cast(a, vp)

        def arr_views(fmt):
            a = (View * L)(*[view(fmt % l) for l in range(L)])
            self._keep.append(a)
            return a

        E = spec.n_expert
        ex = (View * (L * E * 3))()
        for l in range(L):
            for c, nm in enumerate(("ffn_gate_exps", "ffn_up_exps", "ffn_down_exps")):
                t, ne, data = spec.tensors[f"blk.{l}.{nm}.weight"]
                data = np.ascontiguousarray(data).reshape(-1)
                self._keep.append(data)
                rb = row_bytes(t, ne[0])
                per = rb * ne[1]
                for e in range(E):
                    ex[(l * E + e) * 3 + c] = View(data.ctypes.data + e * per, t, ne[0], ne[1], rb)
        self._keep.append(ex)
        outn = f32("output_norm.weight")
        m = Model()
        for n in ("n_layer", "D", "n_head", "n_kv", "hd", "n_expert", "n_used", "FF", "n_vocab", "n_ctx"):
            setattr(m, n, getattr(spec, n))
        m.eps = spec.eps
        m.rope_base = spec.rope_base
        m.tok_embd = view("token_embd.weight")
        m.output = view("output.weight")
        m.output_norm = outn.ctypes.data
        m.attn_norm = arr_ptrs("blk.%d.attn_norm.weight")
        m.ffn_norm = arr_ptrs("blk.%d.ffn_norm.weight")
        m.q_norm = arr_ptrs("blk.%d.attn_q_norm.weight")
        m.k_norm = arr_ptrs("blk.%d.attn_k_norm.weight")
        m.wq = arr_views("blk.%d.attn_q.weight")
        m.wk = arr_views("blk.%d.attn_k.weight")
        m.wv = arr_views("blk.%d.attn_v.weight")
        m.wo = arr_views("blk.%d.attn_output.weight")
        m.router = arr_views("blk.%d.ffn_gate_inp.weight")
        m.experts = ex
        self._model = m
        self.state = lib().orc_state_new(ctypes.byref(m))

    MoeHook = ctypes.CFUNCTYPE(ctypes.c_int, vp, ctypes.c_int, ctypes.POINTER(ctypes.c_float), ctypes.c_int,
                               ctypes.c_int, ctypes.POINTER(ctypes.c_int), ctypes.POINTER(ctypes.c_float),
                               ctypes.POINTER(ctypes.c_float))

    def set_moe_hook(self, fn):
        """Replace the expert block of every layer with fn(layer, xn[nb][D],
        ids[nb][k], wts[nb][k]) -> out[nb][D] (numpy arrays); None restores the
        oracle's own block."""
        if fn is None:
            self._hook = None
            lib().orc_state_set_moe_hook(self.state, None, None)
            return
        D = self.spec.D

        def tramp(ctx, layer, xn, nb, k, ids, wts, out):
            try:
                x = np.ctypeslib.as_array(xn, shape=(nb, D)).copy()
                i = np.ctypeslib.as_array(ids, shape=(nb, k)).copy()
                w = np.ctypeslib.as_array(wts, shape=(nb, k)).copy()
                y = np.asarray(fn(layer, x, i, w), dtype=np.float32)
                np.ctypeslib.as_array(out, shape=(nb, D))[:] = y
                return 0
            except Exception:  # reported as a failed forward
                import traceback
                traceback.print_exc()
                return 1

        self._hook = self.MoeHook(tramp)
        lib().orc_state_set_moe_hook(self.state, ctypes.cast(self._hook, vp), None)

    def forward(self, toks, p0, want_logits=True):
        """One batch at positions p0.. (Engine::forward)."""
        toks = np.ascontiguousarray(toks, dtype=np.int32)
        logits = np.empty(self.spec.n_vocab, dtype=np.float32) if want_logits else None
        rc = lib().orc_forward(self.state, _ptr(toks), len(toks), p0, _ptr(logits) if want_logits else None)
        assert rc == 0
        return logits

    def eval(self, toks, p0, n_batch):
        """Chunked evaluation (Engine::eval, qwen3moe.cpp:1078-1084)."""
        logits = None
        for i in range(0, len(toks), n_batch):
            chunk = toks[i:i + n_batch]
            last = i + len(chunk) == len(toks)
            logits = self.forward(chunk, p0 + i, want_logits=last)
        return logits

    def trace(self):
        n = ctypes.c_int()
        lib().orc_state_trace(self.state, None, None, 0, ctypes.byref(n))
        ids = np.empty(n.value, dtype=np.int32)
        w = np.empty(n.value, dtype=np.float32)
        lib().orc_state_trace(self.state, _ptr(ids), _ptr(w), n.value, None)
        return ids, w

    def __del__(self):
        try:
            lib().orc_state_free(self.state)
        except Exception:
            pass


# ---------------------------------------------------------------------------
# The compiled reference (present where /root/reference existed at build time).

_ref = None


def ref_available(path=REF_SO):
    return os.path.exists(path)


def ref(path=REF_SO):
    global _ref
    if _ref is None:
        if not os.path.exists(path):
            raise RuntimeError(f"{path} not built (needs the reference sources)")
        R = ctypes.CDLL(path)
        R.ref_dequant_block.argtypes = [ctypes.c_int, vp, vp]
        R.ref_matmul.argtypes = [ctypes.c_int, ctypes.c_int64, ctypes.c_int64, ctypes.c_size_t, vp, vp, ctypes.c_int,
                                 ctypes.c_int, vp, ctypes.c_int]
        R.ref_engine_new.restype = vp
        R.ref_engine_new.argtypes = [ctypes.c_char_p, ctypes.c_int]
        R.ref_engine_free.argtypes = [vp]
        R.ref_engine_vocab.argtypes = [vp]
        R.ref_engine_eval.argtypes = [vp, vp, ctypes.c_int, ctypes.c_int, ctypes.c_int, vp]
        R.ref_engine_forward.argtypes = [vp, vp, ctypes.c_int, ctypes.c_int, vp]
        R.ref_engine_trace.argtypes = [vp, vp, vp, ctypes.c_int]
        R.ref_engine_trace_clear.argtypes = [vp]
        R.ref_init()
        _ref = R
    return _ref


def ref_dequant_rows(t, w, ne0):
    blck, nbytes = BLOCK[t]
    w = np.ascontiguousarray(w, dtype=np.uint8).reshape(-1, nbytes)
    out = np.empty((w.shape[0], blck), dtype=np.float32)
    R = ref()
    for i in range(w.shape[0]):
        assert R.ref_dequant_block(t, w[i].ctypes.data, out[i].ctypes.data) == 0
    return out.reshape(-1, ne0)


def ref_matmul(t, w, ne0, x):
    w = np.ascontiguousarray(w, dtype=np.uint8).reshape(-1, row_bytes(t, ne0))
    x = np.ascontiguousarray(x, dtype=np.float32).reshape(-1, ne0)
    out = np.empty((x.shape[0], w.shape[0]), dtype=np.float32)
    assert ref().ref_matmul(t, ne0, w.shape[0], w.shape[1], _ptr(w), _ptr(x), x.shape[0], ne0, _ptr(out),
                            w.shape[0]) == 0
    return out
