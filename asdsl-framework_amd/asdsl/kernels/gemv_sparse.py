"""Activation-sparse GEMV API and bitmask utility on the HIP library.

Mirrors the reference's asdsl/kernels/gemv_sparse.py:26-130; the NumPy
fallbacks there are not provided (the HIP kernels are the only path).
"""

from __future__ import annotations

import numpy as np

from asdsl import _hip
from asdsl.kernels import _native_sparse_gemv as _native_sparse


def has_native_sparse_kernel() -> bool:
    """Reference: gemv_sparse.py:26-27."""
    return _hip.exported("asdsl_gemv_sparse_unpacked")


def compute_activation_bitmask(act, threshold: float = 0.01):
    """Reference: compute_activation_bitmask (gemv_sparse.py:50-76).

    Returns (bitmask u32[ceil(K/32)], active_indices i32 of |act| >= threshold).
    The bitmask is computed on the GPU.  The index list is host glue, as in
    the reference: numpy for numpy input, torch.nonzero for a device tensor.
    """
    flat = act.reshape(-1)
    if _hip.is_device_tensor(flat):
        flat = flat.float().contiguous()
        bitmask = _native_sparse.compute_bitmask(flat, threshold)
        import torch

        idx = torch.nonzero(flat.abs() >= threshold).reshape(-1).to(torch.int32)
        return bitmask, idx
    flat = np.ascontiguousarray(flat, dtype=np.float32)
    bitmask = np.asarray(_native_sparse.compute_bitmask(flat, threshold))
    return bitmask, np.where(np.abs(flat) >= threshold)[0].astype(np.int32)


def gemv_sparse_unpacked(w, x, scales, biases, bitmask, M: int, K: int, group_size: int):
    """Reference: gemv_sparse_unpacked (gemv_sparse.py:79-103)."""
    return _native_sparse.gemv_sparse_unpacked(w, x, scales, biases, bitmask, M, K, group_size)


def gemv_sparse_with_indices(w, x, scales, biases, active_indices, M: int, K: int, group_size: int):
    """Reference: gemv_sparse_with_indices (gemv_sparse.py:106-130)."""
    return _native_sparse.gemv_sparse_with_indices(w, x, scales, biases, active_indices, M, K, group_size)
