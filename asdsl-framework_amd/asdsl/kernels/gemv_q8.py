"""8-bit (one byte per weight) fused GEMV API on the HIP library.

Mirrors the reference's asdsl/kernels/gemv_q8.py:33-141; the PyTorch fallback
there is not provided (the HIP kernel is the only path).
"""

from __future__ import annotations

from asdsl import _hip
from asdsl.kernels import _native_gemv_q8


def has_native_kernel() -> bool:
    """Reference: gemv_q8.py:33-35."""
    return _hip.exported("asdsl_gemv_q8_unpacked")


def fused_dequant_gemv(w_u8, x, scales, biases, m: int, k: int, group_size: int = 128, *,
                       cache_tiling: bool = True):
    """Reference: fused_dequant_gemv (gemv_q8.py:42-77):
    y = sum_g s*sum(w*x) + b*sum(x) per (row, group), fp32."""
    return _native_gemv_q8.fused_dequant_gemv(w_u8, x, scales, biases, m, k, group_size, cache_tiling)


def gemv_q8_unpacked(w_u8, x, scales, biases, m: int, k: int, group_size: int = 128, *,
                     cache_tiling: bool = True):
    """Reference: gemv_q8_unpacked (gemv_q8.py:80-141)."""
    return fused_dequant_gemv(w_u8, x, scales, biases, m, k, group_size, cache_tiling=cache_tiling)
