"""KVForge decode-attention path, MI355X-native.

The product is the HIP library libkvf_hip.so (hand-written gfx950 kernels
behind the kvf::Args / kvf_launch C-ABI in include/kvf_abi.h), the kvf
compiler (kvforge_amd/compiler) and the HIP tools (sweep, bw_probe, driver).
This Python package is a thin ctypes face of that ABI for tests and bench.py.
"""
from . import runtime  # noqa: F401

__all__ = ["runtime"]
