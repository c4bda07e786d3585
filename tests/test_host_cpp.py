"""C++ host side: HipDevice (the expert store's DeviceBackend over the C ABI)
and the store's calling pattern, built with g++ against include/ only.

CPU: the header compiles on its own and over a second base class with the
reference's DeviceBackend methods (eahmmf.h:88-100), as it would inside the
reference build.  GPU: the built checker program passes every check.
"""
import os
import subprocess

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
PKG = os.path.join(ROOT, "eahmmf_inference_prototype_v-0.1.0_amd")
HOST = os.path.join(PKG, "host")
BIN = os.path.join(PKG, "_build", "test_hip_device")

OTHER_BASE = r"""
#include <stddef.h>
#include <stdint.h>
namespace eahmmf {  // a stand-in with the reference's DeviceBackend methods
struct DeviceBackend {
    virtual ~DeviceBackend() {}
    virtual const char* name() const = 0;
    virtual void* alloc(size_t bytes) = 0;
    virtual void release(void* p, size_t bytes) = 0;
    virtual bool h2d(void* dev_dst, const void* host_src, size_t n) = 0;
    virtual bool d2h(void* host_dst, const void* dev_src, size_t n) = 0;
    virtual bool sync() = 0;
    virtual bool cpu_readable() const = 0;
    virtual size_t total_memory() const { return SIZE_MAX; }
    virtual size_t free_memory() const { return SIZE_MAX; }
};
}
#include "hip_device.h"
int main() {
    eahmmf::DeviceBackend* d = new eahmmf_hip::HipDeviceOn<eahmmf::DeviceBackend>();
    int ok = d->cpu_readable() ? 1 : 0;
    delete d;
    return ok;
}
"""


def _gxx(args, cwd):
    return subprocess.run(["g++", "-std=c++17", "-Wall", "-Wextra", "-Werror", "-Wno-unused-parameter"] + args,
                          cwd=cwd, capture_output=True, text=True)


def test_header_compiles_standalone(tmp_path):
    r = _gxx(["-fsyntax-only", "-I", os.path.join(ROOT, "include"), "-I", HOST,
              os.path.join(HOST, "test_hip_device.cpp")], tmp_path)
    assert r.returncode == 0, r.stderr


def test_header_over_reference_shaped_base(tmp_path):
    src = tmp_path / "other_base.cpp"
    src.write_text(OTHER_BASE)
    r = _gxx(["-fsyntax-only", "-I", os.path.join(ROOT, "include"), "-I", HOST, str(src)], tmp_path)
    assert r.returncode == 0, r.stderr


def test_checker_program_built():
    assert os.path.exists(BIN), "build() produces the C++ checker next to libeahmmf_hip.so"


@pytest.mark.gpu
def test_hip_device_and_store_pattern_on_gpu():
    print("running", BIN, flush=True)
    r = subprocess.run([BIN], capture_output=True, text=True, timeout=120)
    assert r.returncode == 0, r.stdout + r.stderr
    assert "all checks passed" in r.stdout
