"""ainfer_amd: INT4 mixture-of-experts layer for AMD Instinct MI355X (gfx950).

The product is libainfer_moe.so (hand-written HIP kernels behind the C ABI in
include/ainfer_moe.h).  This package builds it, binds it with ctypes and
holds the synthetic benchmark configurations.
"""
from . import _lib
from .synthetic import CONFIGS, MoeConfig

__all__ = ["CONFIGS", "MoeConfig", "_lib"]
