"""Group-wise weight quantizer and 4-bit packing (the formats the GEMVs read).

Follows the reference's asdsl/quantization/core.py:
  * compute_scale_zero (core.py:63-94): asymmetric scale = max(max-min, 1e-5)/15,
    zero = -min/scale (both fp32, then stored fp16); symmetric scale =
    max(amax, 1e-5)/7.5 (fp16).
  * quantize_weights (core.py:358-424, optimize_clips=False path):
    q = clip(rne(w / max(scale_f16, 1e-4) + zero_f16), 0, 15)   (asymmetric)
    q = clip(rne(w / max(scale_f16, 1e-4) + 7.5), 0, 15)          (symmetric)
  * _pack_bits / _unpack_bits for 4 bits (core.py:543-600): two values per
    byte, low nibble = even index.
The MSE clip search (optimize_clips=True, core.py:291-355) is a quality
feature outside the GEMV path and is not provided.
"""

from __future__ import annotations

from dataclasses import dataclass

import numpy as np


@dataclass
class QuantizedTensor:
    data: np.ndarray          # packed uint8 (2 nibbles per byte)
    scales: np.ndarray        # float16 per group
    zeros: np.ndarray | None  # float16 per group (asymmetric) or None
    bits: int
    group_size: int
    shape: tuple[int, ...]
    is_symmetric: bool = True

    @property
    def numel(self) -> int:
        n = 1
        for s in self.shape:
            n *= s
        return n


def _pack_bits(data: np.ndarray, bits: int) -> np.ndarray:
    if bits == 8:
        return np.asarray(data, dtype=np.uint8)
    if bits != 4:
        raise ValueError(f"Unsupported bit-width: {bits}")
    data = np.asarray(data, dtype=np.uint8).reshape(-1)
    if data.size % 2:
        data = np.append(data, np.uint8(0))
    return ((data[0::2] & 0x0F) | ((data[1::2] & 0x0F) << 4)).astype(np.uint8)


def _unpack_bits(packed: np.ndarray, bits: int) -> np.ndarray:
    if bits == 8:
        return np.asarray(packed, dtype=np.uint8)
    if bits != 4:
        raise ValueError(f"Unsupported bit-width: {bits}")
    packed = np.asarray(packed, dtype=np.uint8)
    return np.stack([packed & 0x0F, (packed >> 4) & 0x0F], axis=-1).reshape(-1).astype(np.uint8)


def compute_scale_zero(grouped: np.ndarray, bits: int, symmetric: bool = True):
    qmax = (1 << bits) - 1
    if symmetric:
        abs_max = np.maximum(np.abs(grouped).max(axis=-1, keepdims=True), np.float32(1e-5))
        return (abs_max / np.float32(qmax / 2)).astype(np.float16), None
    w_min = grouped.min(axis=-1, keepdims=True)
    w_max = grouped.max(axis=-1, keepdims=True)
    w_range = np.maximum(w_max - w_min, np.float32(1e-5))
    scales = w_range / np.float32(qmax)
    zeros = -w_min / scales
    return scales.astype(np.float16), zeros.astype(np.float16)


def quantize_groups(weights: np.ndarray, bits: int, group_size: int, symmetric: bool):
    """Return (q uint8 [n_groups, gs], scales f16 [n_groups], zeros f16 or None)."""
    flat = np.asarray(weights, dtype=np.float32).reshape(-1)
    rem = flat.size % group_size
    if rem:
        flat = np.concatenate([flat, np.zeros(group_size - rem, np.float32)])
    grouped = flat.reshape(-1, group_size)
    scales, zeros = compute_scale_zero(grouped, bits, symmetric)
    qmax = (1 << bits) - 1
    denom = np.maximum(scales.astype(np.float32), np.float32(1e-4))
    if symmetric:
        q = np.round(grouped / denom + np.float32(qmax / 2))
    else:
        q = np.round(grouped / denom + zeros.astype(np.float32))
    q = np.clip(q, 0, qmax).astype(np.uint8)
    return q, scales.reshape(-1), (zeros.reshape(-1) if zeros is not None else None)


def quantize_weights(weights, bits: int = 4, group_size: int = 128, symmetric: bool = True,
                     optimize_clips: bool = False) -> QuantizedTensor:
    if optimize_clips:
        raise NotImplementedError("MSE clip search is not part of the GEMV path")
    w = np.asarray(weights.detach().cpu().float().numpy() if hasattr(weights, "detach") else weights,
                   dtype=np.float32)
    q, scales, zeros = quantize_groups(w, bits, group_size, symmetric)
    return QuantizedTensor(_pack_bits(q.reshape(-1), bits), scales, zeros, bits, group_size,
                           tuple(w.shape), symmetric)


def dequantize_weights(qt: QuantizedTensor) -> np.ndarray:
    q = _unpack_bits(qt.data, qt.bits).astype(np.float32)
    q = q[: (q.size // qt.group_size) * qt.group_size].reshape(-1, qt.group_size)
    s = qt.scales.astype(np.float32)[:, None]
    if qt.is_symmetric:
        w = (q - np.float32(((1 << qt.bits) - 1) / 2)) * s
    else:
        w = (q - qt.zeros.astype(np.float32)[:, None]) * s
    return w.reshape(-1)[: qt.numel].reshape(qt.shape)


def packed_scale_bias(qt: QuantizedTensor) -> tuple[np.ndarray, np.ndarray]:
    """fp32 per-group (scale, bias = -zero*scale) as the model store keeps them
    (experiments/phi4_cpu_run.py:3130-3140) and as gemv_q4_packed consumes them."""
    n_groups = qt.numel // qt.group_size
    sc = qt.scales[:n_groups].astype(np.float32)
    if qt.is_symmetric:
        bi = (np.float32(-((1 << qt.bits) - 1) / 2) * sc).astype(np.float32)
    else:
        bi = (-qt.zeros[:n_groups].astype(np.float32) * sc).astype(np.float32)
    return sc, bi
