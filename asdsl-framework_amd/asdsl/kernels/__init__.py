"""HIP (gfx950) implementations of the reference's GEMV kernel API.

Mirrors asdsl/kernels/__init__.py:20-76 of the reference: the high-level
wrappers (gemv_q4*, gemv_q8_unpacked, the sparse GEMVs and bitmask) keep the
reference's names and arguments, and the pybind-module stand-ins
(``_native_gemv``, ``_native_gemv_q8``, ``_native_sparse_gemv``) keep its
function names.  Every call runs on the GPU through libasdsl_hip.so.  The
2- and 3-bit kernels and the CPU table-lookup (LUT) kernels of the reference
are not part of this package.
"""

from asdsl.kernels import _native_gemv  # noqa: F401
from asdsl.kernels.gemv_q4 import gemv_q4, gemv_q4_packed, gemv_q4_unpacked, gemv_q4km_q8, has_native_kernel
from asdsl.kernels.gemv_q8 import gemv_q8_unpacked
from asdsl.kernels.gemv_q8 import has_native_kernel as has_native_q8_kernel
from asdsl.kernels.gemv_sparse import (
    compute_activation_bitmask,
    gemv_sparse_unpacked,
    gemv_sparse_with_indices,
    has_native_sparse_kernel,
)

KERNEL_TIER = "HIP_GFX950"

__all__ = [
    "KERNEL_TIER",
    "gemv_q4",
    "gemv_q4_packed",
    "gemv_q4_unpacked",
    "gemv_q4km_q8",
    "has_native_kernel",
    "gemv_q8_unpacked",
    "has_native_q8_kernel",
    "compute_activation_bitmask",
    "gemv_sparse_unpacked",
    "gemv_sparse_with_indices",
    "has_native_sparse_kernel",
]
