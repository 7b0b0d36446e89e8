"""The output projection (lm_head) quantized the way the reference's engine
does it when it is handed fp16 or fp32 weights (a tied embedding, most
often): the UnifiedEngine constructor, unified_engine.cpp:320-398 at
lm_head_group_size 32 and 413-461 at 128.

Per group of `group_size` weights of a row: amax = max |w|; amax < 1e-12
gives scale 0 and every level 8; otherwise scale = amax * float32(1/7) (the
reference build turns the division by the constant into a reciprocal
multiply) stored as fp16 rounded to nearest even, inv = 7 / amax as a float32
division, level = round-half-away-from-zero(w * inv) + 8 clamped to [0, 15]
(std::round).  The zero point is the constant 8: at group size 32 the
reference stores it as fp16 8.0 in 20-byte preq blocks and copies those
into its preq2 lm_head byte for byte; at 128 it writes 66-byte Q4_128 blocks
(implicit zero 8).  Either way the preq2 operands here carry (scale, fp16
8.0) per group, so DecodeEngine runs the reference's lm_head bit for bit
(preq2 at gs 32, preq2-g128 at gs 128).

Unlike repack_q4_128.py's quantizer, ties round away from zero and the
scale is formed in float32; the two differ only at ties.
"""

from __future__ import annotations

import numpy as np


def quantize_output_projection(w, group_size: int = 128):
    """torch float16/float32 [rows][cols] on any device -> flat uint8
    (meta, quant) preq2 operands at group_size 32 or 128 (cols a multiple of
    it), on the weights' device."""
    import torch

    if group_size not in (32, 128):
        raise ValueError("quantize_output_projection: group_size must be 32 or 128")
    if w.dim() != 2 or w.shape[1] % group_size:
        raise ValueError(f"quantize_output_projection: weights [rows][cols] with cols a multiple of {group_size}")
    rows, cols = w.shape
    G = cols // group_size
    out_meta = torch.empty((rows, G, 2), dtype=torch.int16, device=w.device)
    n_bands = (rows + 3) // 4
    quant = torch.zeros((n_bands * 4, G, group_size // 2), dtype=torch.uint8, device=w.device)
    one_seventh = torch.tensor(np.float32(1.0 / 7.0), device=w.device)
    seven = torch.tensor(np.float32(7.0), device=w.device)
    step = max(1, (1 << 26) // cols)  # rows per chunk: ~64M elements of float32 temporaries
    for r0 in range(0, rows, step):
        r1 = min(rows, r0 + step)
        g = w[r0:r1].reshape(-1, G, group_size).float()
        amax = g.abs().amax(dim=2)
        tiny = amax < 1e-12
        safe = torch.where(tiny, torch.ones_like(amax), amax)
        inv = seven / safe
        v = g * inv[:, :, None]
        t = torch.trunc(v)
        r = t + torch.where((v - t).abs() >= 0.5, torch.sign(v), torch.zeros_like(v))
        q = torch.clamp(r + 8.0, 0, 15).to(torch.uint8)
        q[tiny] = 8
        s16 = torch.where(tiny, torch.zeros_like(safe), safe * one_seventh).half()
        out_meta[r0:r1, :, 0] = s16.view(torch.int16)
        quant[r0:r1] = q[..., 0::2] | (q[..., 1::2] << 4)
    out_meta[:, :, 1] = int(np.float16(8.0).view(np.int16))
    meta = out_meta.view(torch.uint8).reshape(-1)
    quant = quant.reshape(n_bands, 4, G, group_size // 2).permute(0, 2, 1, 3).contiguous().reshape(-1)
    return meta, quant
