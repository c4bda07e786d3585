"""C ABI checks that need no GPU: exports, argument validation, host helpers."""
import os
import re

import ctypes

import numpy as np
import pytest

import oracle
from conftest import ROOT


def declared_symbols():
    txt = open(os.path.join(ROOT, "include", "eahmmf_hip.h")).read()
    txt = re.sub(r"/\*.*?\*/", "", txt, flags=re.S)
    return sorted(set(re.findall(r"\b(eahmmf_hip_[a-z0-9_]+)\s*\(", txt)))


def test_every_declared_symbol_is_exported(binding, hip):
    syms = declared_symbols()
    assert len(syms) >= 19
    for s in syms:
        assert hasattr(hip, s), s
    assert set(syms) == set(binding.EXPORTS)


def test_invalid_arguments_fail_without_touching_the_device(binding, hip):
    x = np.zeros(256, dtype=np.float32)
    out = np.zeros(8, dtype=np.float32)
    # null weights, unsupported type, bad ldx, row_bytes mismatch: all rejected up front
    assert not hip.eahmmf_hip_matmul(None, 12, 256, 8, 144, x.ctypes.data, 1, 256, out.ctypes.data, 8)
    assert "null" in hip.eahmmf_hip_last_error().decode()
    fake = 4096  # never dereferenced: validation fails first
    assert not hip.eahmmf_hip_matmul(fake, 2, 256, 8, 144, x.ctypes.data, 1, 256, out.ctypes.data, 8)
    assert "type" in hip.eahmmf_hip_last_error().decode()
    assert not hip.eahmmf_hip_matmul(fake, 12, 256, 8, 144, x.ctypes.data, 1, 128, out.ctypes.data, 8)
    assert not hip.eahmmf_hip_matmul(fake, 12, 256, 8, 140, x.ctypes.data, 1, 256, out.ctypes.data, 8)  # too short
    assert not hip.eahmmf_hip_matmul(fake, 12, 256, 8, 152, x.ctypes.data, 1, 256, out.ctypes.data, 8)  # unaligned
    assert "multiple of 16" in hip.eahmmf_hip_last_error().decode()
    assert not hip.eahmmf_hip_matmul(fake, 14, 256, 8, 211, x.ctypes.data, 1, 256, out.ctypes.data, 8)
    assert not hip.eahmmf_hip_matmul(fake, 12, 200, 8, 144, x.ctypes.data, 1, 256, out.ctypes.data, 8)
    assert not hip.eahmmf_hip_matmul_pair(fake, 12, 256, 8, 144, fake, 12, 256, 4, 144, x.ctypes.data, 1, 256,
                                          out.ctypes.data, 8, out.ctypes.data, 8)
    assert "mismatch" in hip.eahmmf_hip_last_error().decode()
    ids = np.zeros(8, dtype=np.int32)
    assert not hip.eahmmf_hip_route_topk(x.ctypes.data, 1, 128, 17, ids.ctypes.data, out.ctypes.data)
    assert not hip.eahmmf_hip_route_topk(x.ctypes.data, 1, 1024, 8, ids.ctypes.data, out.ctypes.data)
    # streaming read: nothing to do for 0 bytes; null, unaligned or ragged sizes rejected up front
    assert hip.eahmmf_hip_stream_read_async(None, 0, None, None) == 0
    assert hip.eahmmf_hip_stream_read_async(None, 16, fake, None) == -1
    assert "null" in hip.eahmmf_hip_last_error().decode()
    assert hip.eahmmf_hip_stream_read_async(fake + 8, 16, fake, None) == -1
    assert hip.eahmmf_hip_stream_read_async(fake, 24, fake, None) == -1
    assert "multiple of 16" in hip.eahmmf_hip_last_error().decode()
    # bulk staging: negative counts and null copies rejected up front, an empty batch is a no-op
    assert hip.eahmmf_hip_h2d_batch(None, 0) == 0
    assert hip.eahmmf_hip_h2d_batch(None, 1) == -1
    assert hip.eahmmf_hip_h2d_batch(None, -1) == -1
    bad = (binding.Copy * 1)(binding.Copy(None, x.ctypes.data, 16))
    assert hip.eahmmf_hip_h2d_batch(bad, 1) == -1
    assert "null pointer" in hip.eahmmf_hip_last_error().decode()
    ticket = ctypes.c_uint64(0)
    assert hip.eahmmf_hip_h2d_batch_async(None, 1, ctypes.byref(ticket)) == -1
    assert hip.eahmmf_hip_h2d_batch_async(bad, 1, ctypes.byref(ticket)) == -1
    assert "null pointer" in hip.eahmmf_hip_last_error().decode()
    assert hip.eahmmf_hip_h2d_batch_async(bad, 1, None) == -1
    assert "ticket" in hip.eahmmf_hip_last_error().decode()
    # the model's sequence entry points: a null model is rejected up front
    assert hip.eahmmf_hip_model_set_sequences(None, 2) == -1
    assert hip.eahmmf_hip_model_forward_seq(None, 0, ids.ctypes.data, 1, 0, None) == -1
    assert hip.eahmmf_hip_model_decode_seqs(None, 1, ids.ctypes.data, ids.ctypes.data, ids.ctypes.data, None) == -1
    assert "null" in hip.eahmmf_hip_last_error().decode()


@pytest.mark.parametrize("t,ne0", [(0, 64), (8, 96), (12, 2048), (13, 768), (14, 768), (14, 1536)])
def test_row_bytes(hip, t, ne0):
    assert hip.eahmmf_hip_row_bytes(t, ne0) == oracle.row_bytes(t, ne0)


def test_grouped_path_knobs(hip):
    """The grouped block's kernel-path settings (host state only): the
    integer-dot path is on for blocks of at most 32 tokens by default
    (reported as 33), 0 turns it off, 1..32 also routes small groups of larger
    blocks to it; the per-wave matrix-core split is clamped to 32."""
    d0, w0, m0 = (hip.eahmmf_hip_set_grouped_dot_max(-1), hip.eahmmf_hip_set_grouped_wave_max(-1),
                  hip.eahmmf_hip_set_grouped_mfma(-1))
    try:
        assert d0 == 33 and w0 == 32 and m0 == 1
        assert hip.eahmmf_hip_set_grouped_dot_max(0) == 33
        assert hip.eahmmf_hip_set_grouped_dot_max(-1) == 0
        assert hip.eahmmf_hip_set_grouped_dot_max(4) == 0
        assert hip.eahmmf_hip_set_grouped_dot_max(-1) == 4
        assert hip.eahmmf_hip_set_grouped_dot_max(100) == 4
        assert hip.eahmmf_hip_set_grouped_dot_max(-1) == 33
        assert hip.eahmmf_hip_set_grouped_wave_max(99) == 32
        assert hip.eahmmf_hip_set_grouped_wave_max(-1) == 32
    finally:
        hip.eahmmf_hip_set_grouped_dot_max(d0)
        hip.eahmmf_hip_set_grouped_wave_max(w0)
        hip.eahmmf_hip_set_grouped_mfma(m0)


def test_dense_mfma_switch(hip):
    assert hip.eahmmf_hip_set_dense_mfma(0) == 1  # on by default
    assert hip.eahmmf_hip_set_dense_mfma(1) == 0
    assert hip.eahmmf_hip_set_dense_mfma(1) == 1


def test_row_bytes_rejects(hip):
    assert hip.eahmmf_hip_row_bytes(12, 300) == 0
    assert hip.eahmmf_hip_row_bytes(3, 256) == 0


@pytest.mark.parametrize("t,bits", [(8, 8), (12, 4), (13, 5), (14, 6)])
def test_quantizer_round_trip(binding, t, bits):
    """Quantize N(0, 0.02) rows and decode them with the oracle: the error is
    bounded by the format's step size (a broken layout gives O(1) errors)."""
    rng = np.random.default_rng(5)
    ne0 = 512
    w = rng.normal(0, 0.02, (16, ne0)).astype(np.float32)
    q = binding.quantize_rows(t, w)
    back = oracle.dequant_rows(t, q, ne0)
    err = np.abs(back - w)
    amax = np.abs(w).max()
    assert err.max() < amax * 2.0 ** (2 - bits) * 1.2
    assert err.mean() < amax * 2.0 ** (-bits)
