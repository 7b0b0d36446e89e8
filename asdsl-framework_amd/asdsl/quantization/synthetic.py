"""Seeded synthetic weights and activations for the GEMV workloads.

Weights W ~ N(0, 0.02) fp32, activations x ~ N(0, 1) fp32, quantized per K
group in the reference format (asdsl/quantization/core.py:63-94,358-424).
Seeds follow the reference's tests (default_rng(42) for weights,
tests/conftest.py:23; benchmarks/kernel_preflight.py:32).

``preq2_from_weights_torch`` restates the numpy quantizer with torch ops so
that the 600M-element lm_head can be quantized on the device in seconds; it
is bit-identical to ``repack.quantize_preq2`` (same IEEE fp32 division,
round-half-even and fp16 conversions; checked by the tests on the CPU).
"""

from __future__ import annotations

import numpy as np

from asdsl.quantization.core import packed_scale_bias, quantize_weights
from asdsl.quantization.repack import (blocks_to_flat, quantize_preq2, repack_asymmetric_to_q4_32_blocks,
                                       repack_fp32_to_q4_128_blocks)

WEIGHT_STD = 0.02


def gaussian_weights(rows: int, cols: int, seed: int = 42, std: float = WEIGHT_STD) -> np.ndarray:
    rng = np.random.default_rng(seed)
    return rng.standard_normal((rows, cols), dtype=np.float32) * np.float32(std)


def activation(k: int, seed: int = 43, batch: int | None = None) -> np.ndarray:
    rng = np.random.default_rng(seed)
    shape = (k,) if batch is None else (batch, k)
    return rng.standard_normal(shape, dtype=np.float32)


def preq_blocks(w: np.ndarray) -> np.ndarray:
    """fp32 W -> flat 20-byte preq blocks via the reference chain
    quantize_weights(asym, gs=32) -> (scale, bias) -> repack (repack_q4_32.py:63-108)."""
    rows, cols = w.shape
    qt = quantize_weights(w, bits=4, group_size=32, symmetric=False)
    sc, bi = packed_scale_bias(qt)
    return blocks_to_flat(repack_asymmetric_to_q4_32_blocks(qt.data, sc, bi, rows, cols, 32)).reshape(-1)


def preq2(w: np.ndarray, group_size: int = 32) -> tuple[np.ndarray, np.ndarray]:
    return quantize_preq2(w, group_size)


def q4_128_blocks(w: np.ndarray) -> np.ndarray:
    rows, cols = w.shape
    return blocks_to_flat(repack_fp32_to_q4_128_blocks(w, rows, cols)).reshape(-1)


# ---------------------------------------------------------------- torch mirror
def preq2_from_weights_torch(w, group_size: int = 32):
    """torch fp32 W (rows, cols) on any device -> (meta uint8 flat, quant uint8 flat)."""
    import torch

    rows, cols = w.shape
    G = cols // group_size
    g = w.reshape(rows, G, group_size).float()
    w_min = g.amin(dim=-1, keepdim=True)
    w_max = g.amax(dim=-1, keepdim=True)
    w_range = torch.clamp_min(w_max - w_min, 1e-5)
    scales = w_range / 15.0
    zeros = -w_min / scales
    s16 = scales.half()
    z16 = zeros.half()
    denom = torch.clamp_min(s16.float(), 1e-4)
    q = torch.clamp(torch.round(g / denom + z16.float()), 0, 15).to(torch.uint8)
    sc = s16.float()
    bi = -z16.float() * sc
    sc64 = torch.clamp_min(sc.double(), 1e-8)
    zero = (-bi.double() / sc64).half()
    meta = torch.stack([sc64.half().view(torch.int16), zero.view(torch.int16)], dim=-1)
    meta = meta.reshape(rows, G, 2).contiguous().view(torch.uint8).reshape(-1)
    nib = (q[..., 0::2] | (q[..., 1::2] << 4)).reshape(rows, G, group_size // 2)
    n_bands = (rows + 3) // 4
    padded = torch.zeros((n_bands * 4, G, group_size // 2), dtype=torch.uint8, device=w.device)
    padded[:rows] = nib
    quant = padded.reshape(n_bands, 4, G, group_size // 2).permute(0, 2, 1, 3).contiguous().reshape(-1)
    return meta, quant


def q4_128_from_weights_torch(w):
    """torch fp32 W (rows, cols) on any device -> flat Q4_128 66-byte blocks
    (uint8), the torch restatement of repack.q4_128_groups: scale =
    f16(amax/7), q = clip(rne(w * f32(7/amax)) + 8, 0, 15), all-zero group ->
    scale 0 and q = 8."""
    import torch

    rows, cols = w.shape
    G = cols // 128
    g = w.reshape(rows * G, 128).float()
    amax = g.abs().amax(dim=1)
    tiny = amax < 1e-12
    safe = torch.where(tiny, torch.ones_like(amax), amax).double()
    inv32 = (7.0 / safe).float()
    q = torch.clamp(torch.round(g * inv32[:, None]) + 8.0, 0, 15).to(torch.uint8)
    q[tiny] = 8
    scale = torch.where(tiny, torch.zeros_like(safe), safe / 7.0).half()
    nib = (q[:, 0::2] | (q[:, 1::2] << 4))
    blocks = torch.empty((rows * G, 66), dtype=torch.uint8, device=w.device)
    blocks[:, 0:2] = scale.view(torch.int16).reshape(-1, 1).view(torch.uint8)
    blocks[:, 2:] = nib
    return blocks.reshape(-1)
