"""Fused 4-bit GEMV API (y = dequant(W_q4) @ x) on the HIP library.

Mirrors the reference's asdsl/kernels/gemv_q4.py:75-416 (names, arguments,
argument errors).  Every call runs on the GPU through ``_native_gemv``; there
is no NumPy fallback.  numpy inputs are uploaded and the result comes back as
numpy; device tensors stay on the device and the result is a device tensor
(asynchronous on the current stream).
"""

from __future__ import annotations

from typing import TYPE_CHECKING

import numpy as np

from asdsl import _hip
from asdsl.kernels import _native_gemv as _native
from asdsl.kernels._buffers import new_output, shape_of

if TYPE_CHECKING:
    from asdsl.quantization.core import QuantizedTensor


def has_native_kernel() -> bool:
    """Reference: gemv_q4.py:75-81.  True: the HIP library is the only path
    (importing this module fails without it)."""
    return _hip.exported("asdsl_gemv_q4_packed")


def _write_out(out, y):
    if _hip.is_device_tensor(out):
        out.copy_(y if _hip.is_device_tensor(y) else _hip.to_device(y, np.float32))
    else:
        np.copyto(out, y.cpu().numpy() if _hip.is_device_tensor(y) else y)
    return out


def gemv_q4_packed(w_packed, x, scales, biases, M: int, K: int, group_size: int, out=None,
                   use_lut: bool = False, use_q8: bool = False, lut_cache=None, bits: int = 4):
    """Reference: gemv_q4_packed (gemv_q4.py:215-324).

    x (K,) -> y (M,); x (B, K) -> y (B, M).  ``use_q8`` selects the symmetric
    Q4xQ8 integer kernel (scales only, q-8; gemv_q4.py:269-273).  ``use_lut``
    and ``lut_cache`` select the reference's CPU table-lookup kernels, which
    compute the same y; here they run the same fused kernel as the default.
    """
    del lut_cache, bits
    xs = shape_of(x)
    if out is not None and (shape_of(out)[0] != M or str(out.dtype) not in ("float32", "torch.float32")):
        raise ValueError(f"out must be float32 shape ({M},), got {shape_of(out)} {out.dtype}")
    if len(xs) == 1:
        if xs[0] != K:
            raise ValueError(f"x length {xs[0]} does not match K={K}")
    elif len(xs) == 2:
        if xs[1] != K:
            raise ValueError(f"x.shape[1]={xs[1]} does not match K={K}")
    else:
        raise ValueError("x must be 1-D (K,) or 2-D (batch, K)")

    if use_q8 and len(xs) == 1:
        y = new_output((M,), np.float32, w_packed, x)
        _native.gemv_q4_q8_avx2(w_packed, scales, x, y, M, K, group_size)
        return y if out is None else _write_out(out, y)
    del use_lut
    y = _native.gemv_q4_packed(w_packed, x, scales, biases, M, K, group_size)
    if out is not None and len(xs) == 1:
        return _write_out(out, y)
    return y


def gemv_q4_unpacked(w, x, scales, biases, M: int, K: int, group_size: int):
    """Reference: gemv_q4_unpacked (gemv_q4.py:327-363); one byte per value."""
    return _native.gemv_q4_unpacked(w, x, scales, biases, M, K, group_size)


def gemv_q4km_q8(weights_q4km, x, out_features: int, in_features: int):
    """Reference: gemv_q4km_q8 (gemv_q4.py:366-383): 144-byte superblocks."""
    n = int(np.prod(shape_of(x)))
    if n != in_features:
        raise ValueError(f"x length {n} does not match in_features={in_features}")
    y = new_output((out_features,), np.float32, weights_q4km, x)
    xv = x.reshape(-1) if hasattr(x, "reshape") else x
    _native.gemv_q4km_q8_avx2(weights_q4km.reshape(-1), xv, y, out_features, in_features)
    return y


def gemv_q4(qtensor: "QuantizedTensor", x):
    """Reference: gemv_q4 (gemv_q4.py:386-416): GEMV from a 4-bit QuantizedTensor
    (symmetric tensors get bias -7.5*scale, asymmetric -zero*scale)."""
    if qtensor.bits != 4:
        raise ValueError(f"gemv_q4 only supports 4-bit tensors, got {qtensor.bits}-bit")
    M, K = qtensor.shape
    scales = np.asarray(qtensor.scales).astype(np.float32)
    if qtensor.is_symmetric:
        biases = np.full_like(scales, -7.5) * scales
    else:
        biases = -np.asarray(qtensor.zeros).astype(np.float32) * scales
    return gemv_q4_packed(qtensor.data, x, scales, biases, M, K, qtensor.group_size)
