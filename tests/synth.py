"""Synthetic expert weights for parity tests (test infrastructure)."""
import numpy as np

import gguf_tools as gt

DSCALE = {gt.Q8_0: 3e-4, gt.Q4_K: 3e-5, gt.Q5_K: 1.5e-5, gt.Q6_K: 5e-6}


def random_rows(t, nrows, ne0, rng, dscale=None):
    """Random block bytes whose fp16 d (and dmin) fields are uniform(.5, 1.5) *
    dscale, the scheme of the reference's tests/test_tiny.py:18-31."""
    blck, nbytes = gt.BLOCK[t]
    nblk = ne0 // blck
    dscale = DSCALE[t] if dscale is None else dscale
    raw = rng.integers(0, 256, (nrows, nblk, nbytes), dtype=np.uint8)

    def put(off):
        raw[:, :, off:off + 2] = (rng.uniform(.5, 1.5, (nrows, nblk)) * dscale).astype(np.float16).view(
            np.uint8).reshape(nrows, nblk, 2)

    if t == gt.Q6_K:
        put(208)
    else:
        put(0)
        if t in (gt.Q4_K, gt.Q5_K):
            put(2)
    return raw.reshape(nrows, nblk * nbytes)


def quantized_rows(binding, t, nrows, ne0, rng, sigma=0.02):
    """N(0, sigma) fp32 rows quantized by the library's host quantizer."""
    w = rng.normal(0, sigma, (nrows, ne0)).astype(np.float32)
    return binding.quantize_rows(t, w)
