"""HipDevice inside the reference's own expert store and engine.

The reference's eahmmf.h and qwen3moe.cpp are compiled in place (never
copied) with HipDevice (host/hip_device.h over libeahmmf_hip.so) as the
store's device backend: oracle/store_harness.cpp, built by oracle/Makefile
into oracle/_ref/store_hip_check.  What the harness checks on the GPU is
listed at its top: the reference's tier matrix bitwise with HipDevice in the
loop, a residency walk with byte checks, pinned/strict service, the expert
matmul dispatch with the reference's shadow criterion, the single-call block
over leased views, and partial residency.

CPU: HipDeviceOn<eahmmf::DeviceBackend> compiles against the reference's
own eahmmf.h (skipped where the reference sources are absent).
"""
import os
import subprocess

import pytest

from conftest import PKG_DIR, ROOT

REF = "/root/reference"
HARNESS = os.path.join(ROOT, "oracle", "_ref", "store_hip_check")


@pytest.mark.skipif(not os.path.exists(os.path.join(REF, "eahmmf.h")), reason="reference sources not present")
def test_hip_device_compiles_against_the_reference_store(tmp_path):
    src = tmp_path / "over_ref.cpp"
    src.write_text('#include "eahmmf.h"\n#include "hip_device.h"\n#include "expert_dispatch.h"\n'
                   "int main() {\n"
                   "    eahmmf::Config cfg;\n"
                   "    cfg.gpu_compute = true;\n"
                   "    eahmmf::DeviceBackend* d = new eahmmf_hip::HipDeviceOn<eahmmf::DeviceBackend>();\n"
                   "    std::vector<std::array<eahmmf::TensorRef, 3>> refs;\n"
                   "    eahmmf::ExpertStore store(nullptr, 0, 0, 0, refs, cfg, d);\n"
                   "    (void)store;\n"
                   "    delete d;\n"
                   "    return 0;\n"
                   "}\n")
    r = subprocess.run(["g++", "-std=c++17", "-fsyntax-only", "-Wall", "-Wextra", "-Werror", "-Wno-unused-parameter",
                        "-I", REF, "-I", os.path.join(ROOT, "include"), "-I", os.path.join(PKG_DIR, "host"), str(src)],
                       capture_output=True, text=True)
    assert r.returncode == 0, r.stderr


@pytest.mark.skipif(not os.path.exists(os.path.join(REF, "qwen3moe.cpp")), reason="reference sources not present")
def test_store_harness_built():
    assert os.path.exists(HARNESS), "__graft_entry__.build() builds oracle/_ref/store_hip_check"


@pytest.mark.gpu
def test_reference_store_with_hip_device(tmp_path):
    import gguf_tools as gt
    if not os.path.exists(HARNESS):
        pytest.fail("oracle/_ref/store_hip_check is not built (build() in the container with the reference)")
    path = str(tmp_path / "tiny.gguf")
    gt.write_gguf(gt.test_tiny_spec(), path)
    print("running", HARNESS, flush=True)
    r = subprocess.run([HARNESS, path], capture_output=True, text=True, timeout=300)
    print(r.stderr[-4000:])
    assert r.returncode == 0, r.stdout + r.stderr[-4000:]
    assert "all" in r.stdout and "checks passed" in r.stdout
