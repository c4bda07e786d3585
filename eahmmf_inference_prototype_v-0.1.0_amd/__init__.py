"""MI355X (gfx950) quantized MoE expert-FFN path for the EAHMMF Qwen3-MoE engine.

The product is libeahmmf_hip.so (HIP kernels + C ABI, include/eahmmf_hip.h)
and the C++ host headers under host/.  This Python package only exposes the
C ABI through ctypes (eahmmf_hip.py) for tests and benchmarks.
"""
from . import eahmmf_hip  # noqa: F401
