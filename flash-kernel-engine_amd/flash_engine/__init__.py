"""flash_engine (MI355X build): the quantized GEMM path of flash-kernel-engine
on gfx950 HIP kernels.  Mirrors reference python/flash_engine/__init__.py for
this path; the reference's attention / normalisation ops are not part of it.
"""
from ._lib import version
from .ops import (fp8_gemm_scaled, fused_swiglu, gemm_half, print_device_info, quantize_per_token,
                  quantized_gemm_int8, w8a8_gate_up_swiglu, w8a8_gemm, w8a8_linear, w8a8_swiglu)

__version__ = "1.2.0"

__all__ = [
    "quantized_gemm_int8",
    "w8a8_gemm",
    "fp8_gemm_scaled",
    "quantize_per_token",
    "w8a8_linear",
    "w8a8_swiglu",
    "w8a8_gate_up_swiglu",
    "fused_swiglu",
    "gemm_half",
    "print_device_info",
    "version",
]
