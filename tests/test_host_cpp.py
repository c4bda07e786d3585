"""C++ host side: HipDevice (the expert store's DeviceBackend over the C ABI)
and the store's calling pattern, built with g++ against include/ only.

CPU: the header compiles on its own (tests/test_store_hip.py compiles it over
the reference's own eahmmf.h).  GPU: the built checker program passes every
check.
"""
import os
import subprocess

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
PKG = os.path.join(ROOT, "eahmmf_inference_prototype_v-0.1.0_amd")
HOST = os.path.join(PKG, "host")
BIN = os.path.join(PKG, "_build", "test_hip_device")



def _gxx(args, cwd):
    return subprocess.run(["g++", "-std=c++17", "-Wall", "-Wextra", "-Werror", "-Wno-unused-parameter"] + args,
                          cwd=cwd, capture_output=True, text=True)


def test_header_compiles_standalone(tmp_path):
    r = _gxx(["-fsyntax-only", "-I", os.path.join(ROOT, "include"), "-I", HOST,
              os.path.join(HOST, "test_hip_device.cpp")], tmp_path)
    assert r.returncode == 0, r.stderr


def test_checker_program_built():
    assert os.path.exists(BIN), "build() produces the C++ checker next to libeahmmf_hip.so"


@pytest.mark.gpu
def test_hip_device_and_store_pattern_on_gpu():
    print("running", BIN, flush=True)
    r = subprocess.run([BIN], capture_output=True, text=True, timeout=120)
    assert r.returncode == 0, r.stdout + r.stderr
    assert "all checks passed" in r.stdout
