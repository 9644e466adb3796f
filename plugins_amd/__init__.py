"""MI355X-native EXL3 quantized matmul (the turboexl3 plugins' hot path).

The product is the C-ABI library plugins_amd/lib/libexl3_mi355x.so (HIP
kernels for gfx950 behind include/exl3_mi355x.h); `plugins_amd.exl3` is its
Python host mirror.
"""
from . import exl3  # noqa: F401

__all__ = ["exl3"]
