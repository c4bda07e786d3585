"""The device routing's exp (csrc/expf_ref.h) against the host libm's expf,
which the reference's routing keys use (qwen3moe.cpp:1013-1016).

The routing ranks by e = expf(l - max) with the lower id first on equal e, so
the device must reproduce expf bit for bit.  Pinned here on the CPU:
- the 2^(i/32) table against a 60-digit computation;
- the same header compiled for the host against libm's expf over every one
  of the 2^32 float inputs (the device build uses the same double-precision
  operations in the same order; tests/test_gpu_routing_ties.py compares the
  device build with libm on the GPU);
- that the check resolves the kind of mistake that matters: computing the
  reduction with a separate multiply and add changes 2 of the 2^32 results,
  and the sweep finds them.
"""
import os
import re
import shutil
import struct
import subprocess
from decimal import Decimal, getcontext

import pytest

from conftest import PKG_DIR, TESTS

HDR = os.path.join(PKG_DIR, "csrc", "expf_ref.h")
SRC = os.path.join(TESTS, "native", "expf_check.cpp")


def test_exp2_table_is_correctly_rounded():
    text = open(HDR).read()
    body = text[text.index("#define EAHMMF_EXP2_TAB"):]
    body = body[:body.index("}") + 1]
    tab = [int(h, 16) for h in re.findall(r"0x([0-9a-f]{16})ull", body)]
    assert len(tab) == 32
    getcontext().prec = 60
    for i, t in enumerate(tab):
        v = float(Decimal(2) ** (Decimal(i) / Decimal(32)))  # correctly rounded to double
        bits = struct.unpack("<Q", struct.pack("<d", v))[0]
        assert (bits - (i << 47)) % (1 << 64) == t, i


@pytest.fixture(scope="module")
def checker(tmp_path_factory):
    if not shutil.which("g++"):
        pytest.skip("g++ not available")
    out = str(tmp_path_factory.mktemp("expf") / "expf_check")
    base = ["g++", "-O2", "-fopenmp", "-I", os.path.dirname(HDR), SRC, "-o", out]
    r = subprocess.run(base[:2] + ["-march=native"] + base[2:], capture_output=True, text=True)
    if r.returncode != 0:
        r = subprocess.run(base, capture_output=True, text=True)
    assert r.returncode == 0, r.stderr
    return out


def run(checker, *args):
    r = subprocess.run([checker, "1", *args], capture_output=True, text=True, timeout=600)
    n, bad = (int(v) for v in r.stdout.split())
    return n, bad, r.stderr


def test_every_float_matches_libm(checker):
    n, bad, err = run(checker)
    assert n == 1 << 32
    assert bad == 0, err


def test_the_sweep_resolves_an_unfused_reduction(checker):
    n, bad, _ = run(checker, "unfused")
    assert n == 1 << 32
    assert bad > 0
