import importlib.util
import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
TESTS = os.path.dirname(os.path.abspath(__file__))
GOLDEN = os.path.join(TESTS, "golden")
PKG_DIR = os.path.join(ROOT, "eahmmf_inference_prototype_v-0.1.0_amd")
for p in (ROOT, TESTS):
    if p not in sys.path:
        sys.path.insert(0, p)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (runs through the HIP C ABI)")


def load_binding():
    """The package directory name is not a Python identifier; load its ctypes
    binding module by path."""
    name = "eahmmf_hip_binding"
    if name in sys.modules:
        return sys.modules[name]
    spec = importlib.util.spec_from_file_location(name, os.path.join(PKG_DIR, "eahmmf_hip.py"))
    mod = importlib.util.module_from_spec(spec)
    spec.loader.exec_module(mod)
    sys.modules[name] = mod
    return mod


@pytest.fixture(scope="session")
def binding():
    return load_binding()


@pytest.fixture(scope="session")
def hip(binding):
    return binding.lib()


@pytest.fixture(scope="session")
def torch_dev():
    """torch with a visible GPU (for tests marked gpu)."""
    import torch
    assert torch.cuda.is_available()
    return torch
