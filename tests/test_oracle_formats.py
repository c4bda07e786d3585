"""Pins the oracle's format decoding (CPU only).

* f16: all 65536 codes against numpy's IEEE half conversion (an independent
  implementation); NaN codes must come back as the canonical NaN with the
  input's sign, as the reference's table does (qwen3moe.cpp:55-62).
* scale_min_k4: every index j over all byte values that j reads, against a
  closed form written as a different bit formulation (6-bit fields gathered
  from a 96-bit little-endian integer layout description).
* dequant: bit-exact against the compiled reference's dq_* output on random
  blocks including edge scales (tests/golden/dequant_golden.npz).
* structural identities that a dropped term, swapped nibble or wrong bit index
  would break (Q8_0 is d*q; Q4_K with dmin = 0 is a pure scale; Q5_K equals
  Q4_K plus 16*d*sc where the high bit is set; Q6_K sign symmetry).
"""
import os

import numpy as np
import pytest

import oracle
from conftest import GOLDEN


def test_f16_exhaustive():
    codes = np.arange(65536, dtype=np.uint32)
    ours = np.array([oracle.f16(c) for c in codes], dtype=np.float32)
    ref = codes.astype(np.uint16).view(np.float16).astype(np.float32)
    nan = np.isnan(ref)
    assert np.array_equal(ours[~nan].view(np.uint32), ref[~nan].view(np.uint32))
    bits = ours[nan].view(np.uint32)
    sign = (codes[nan] >> 15) << 31
    assert np.array_equal(bits, (0x7FC00000 | sign).astype(np.uint32))


def test_scale_min_k4_exhaustive():
    # closed form: scales for j<4 are the low 6 bits of byte j, mins the low 6
    # bits of byte j+4; for j>=4 the low nibble (scale) / high nibble (min) of
    # byte j+4 extended by the top two bits of byte j-4 (scale) / byte j (min).
    vals = np.arange(256, dtype=np.int64)
    a, b = np.meshgrid(vals, vals, indexing="ij")
    for j in range(8):
        q = np.zeros((256 * 256, 12), dtype=np.uint8)
        if j < 4:
            q[:, j] = a.ravel()
            q[:, j + 4] = b.ravel()
            exp_d = a.ravel() % 64
            exp_m = b.ravel() % 64
        else:
            q[:, j + 4] = a.ravel()
            q[:, j - 4] = b.ravel()
            q[:, j] = (b.ravel() * 7 + 13) % 256
            exp_d = (a.ravel() % 16) + 16 * (b.ravel() // 64)
            exp_m = (a.ravel() // 16) + 16 * (q[:, j].astype(np.int64) // 64)
        # sample to keep the run short, but cover every value of both bytes
        idx = np.unique(np.concatenate([np.arange(0, 65536, 257), np.arange(0, 65536, 251), np.arange(255, 65536, 256)]))
        for i in idx:
            d, m = oracle.scale_min_k4(j, q[i])
            assert (d, m) == (exp_d[i], exp_m[i]), (j, i)


@pytest.mark.parametrize("t", [oracle.Q8_0, oracle.Q4_K, oracle.Q5_K, oracle.Q6_K])
def test_dequant_matches_compiled_reference(t):
    g = np.load(os.path.join(GOLDEN, "dequant_golden.npz"))
    blocks, want = g[f"blocks_{t}"], g[f"values_{t}"]
    blck = oracle.BLOCK[t][0]
    got = oracle.dequant_rows(t, blocks, blck)
    assert got.shape == want.shape
    assert np.array_equal(got.view(np.uint32), want.view(np.uint32))


def _half(v):
    return np.array([v], dtype=np.float16).view(np.uint8)


def test_q8_0_is_d_times_q():
    rng = np.random.default_rng(1)
    b = rng.integers(0, 256, (8, 34), dtype=np.uint8)
    for i, d in enumerate([0.5, -0.25, 3.0e-3, 1.0, 7.0, -1.5, 2.0 ** -20, 100.0]):
        b[i, :2] = _half(d)
    y = oracle.dequant_rows(oracle.Q8_0, b, 32)
    d = b[:, :2].copy().view(np.float16).astype(np.float32)
    q = b[:, 2:].view(np.int8).astype(np.float32)
    assert np.array_equal(y, (d * q).astype(np.float32))


def _k4_pack(sc, mn):
    q = np.zeros(12, dtype=np.uint8)
    for j in range(4):
        q[j] = (sc[j] & 63) | ((sc[j + 4] >> 4) << 6)
        q[j + 4] = (mn[j] & 63) | ((mn[j + 4] >> 4) << 6)
        q[j + 8] = (sc[j + 4] & 15) | ((mn[j + 4] & 15) << 4)
    return q


def test_q4_k_layout_identity():
    """dmin = 0 and power-of-two d: every value is exactly d*sc_j*nibble, with
    sub-block 2g in the low and 2g+1 in the high nibbles of qs[32g..32g+32)."""
    rng = np.random.default_rng(2)
    sc = rng.integers(0, 64, 8)
    mn = rng.integers(0, 64, 8)
    b = np.zeros(144, dtype=np.uint8)
    b[0:2] = _half(0.5)
    b[2:4] = _half(0.0)
    b[4:16] = _k4_pack(sc, mn)
    b[16:] = rng.integers(0, 256, 128, dtype=np.uint8)
    y = oracle.dequant_rows(oracle.Q4_K, b, 256)[0]
    for g in range(4):
        qs = b[16 + 32 * g:16 + 32 * g + 32]
        assert np.array_equal(y[64 * g:64 * g + 32], 0.5 * sc[2 * g] * (qs & 15))
        assert np.array_equal(y[64 * g + 32:64 * g + 64], 0.5 * sc[2 * g + 1] * (qs >> 4))
    # dmin > 0: the min is subtracted per sub-block
    b[2:4] = _half(0.25)
    y2 = oracle.dequant_rows(oracle.Q4_K, b, 256)[0]
    for j in range(8):
        assert np.array_equal(y2[32 * j:32 * j + 32], y[32 * j:32 * j + 32] - np.float32(0.25 * mn[j]))


def test_q5_k_high_bit_identity():
    rng = np.random.default_rng(3)
    sc = rng.integers(1, 64, 8)
    mn = rng.integers(0, 64, 8)
    b = np.zeros(176, dtype=np.uint8)
    b[0:2] = _half(0.125)
    b[2:4] = _half(0.0)
    b[4:16] = _k4_pack(sc, mn)
    b[48:] = rng.integers(0, 256, 128, dtype=np.uint8)
    base = oracle.dequant_rows(oracle.Q5_K, b, 256)[0]
    for bit in range(8):
        for l in (0, 7, 31):
            bb = b.copy()
            bb[16 + l] = 1 << bit
            y = oracle.dequant_rows(oracle.Q5_K, bb, 256)[0]
            k = 64 * (bit // 2) + 32 * (bit % 2) + l
            diff = np.nonzero(y != base)[0]
            assert list(diff) == [k]
            assert y[k] - base[k] == np.float32(0.125 * sc[bit] * 16)


def test_q6_k_bit_positions():
    """One 6-bit code at a time: value index k gets (code-32)*d*sc[k//16]."""
    b = np.zeros(210, dtype=np.uint8)
    b[192:208] = np.arange(1, 17, dtype=np.int8).view(np.uint8)
    b[208:210] = _half(0.5)
    for k in (0, 5, 31, 32, 63, 64, 100, 127, 128, 160, 200, 255):
        n, u, l = k // 128, (k % 128) // 32, k % 32
        for code in (0, 17, 33, 63):
            bb = b.copy()
            # every other value has code 32 (=> 0)
            for kk in range(256):
                nn, uu, ll = kk // 128, (kk % 128) // 32, kk % 32
                c = code if kk == k else 32
                lo = 64 * nn + ll + 32 * (uu & 1)
                bb[lo] |= (c & 15) << (0 if uu < 2 else 4)
                bb[128 + 32 * nn + ll] |= ((c >> 4) & 3) << (2 * uu)
            y = oracle.dequant_rows(oracle.Q6_K, bb, 256)[0]
            want = np.zeros(256, dtype=np.float32)
            want[k] = np.float32(np.float32(0.5 * (k // 16 + 1)) * (code - 32))
            assert np.array_equal(y, want), (k, code)
