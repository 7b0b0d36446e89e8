"""Helpers for the decode tests on the reference's C0.1 weight profile
(qkv/o preq2 g32; gate_up/down Q4_128 blocks, run here as preq2-g128; an
fp16 output projection the reference engine quantizes to Q4_128 at load).

quantize_lm_head_q4_128_torch is the torch mirror of
oracle.decode.quantize_lm_head_q4_128 (the engine's load-time rule,
unified_engine.cpp:413-461), so the 614M-element output projection can be
quantized on the device; tests/test_decode_c01_helpers.py pins it bit for
bit against the oracle on the CPU and tests/test_gpu_decode_reference.py
checks a slice of the device result the same way.
"""

from __future__ import annotations

import numpy as np


def quantize_lm_head_q4_128_torch(w):
    """torch float32/float16 [rows][cols] (any device) -> flat uint8 Q4_128
    blocks: scale = fp16(amax * f32(1/7)), inv = 7 / amax (float32),
    q = round-half-away(x * inv) + 8 clamped to [0, 15]; amax < 1e-12 ->
    scale 0, q = 8."""
    import torch

    rows, cols = w.shape
    G = cols // 128
    g = w.reshape(rows * G, 128).float()
    amax = g.abs().amax(dim=1)
    tiny = amax < 1e-12
    safe = torch.where(tiny, torch.ones_like(amax), amax)
    scale = safe * torch.tensor(np.float32(1.0 / 7.0), device=w.device)
    inv = torch.tensor(np.float32(7.0), device=w.device) / safe
    v = g * inv[:, None]
    t = torch.trunc(v)
    r = t + torch.where((v - t).abs() >= 0.5, torch.sign(v), torch.zeros_like(v))
    q = torch.clamp(r + 8.0, 0, 15).to(torch.uint8)
    q[tiny] = 8
    s16 = torch.where(tiny, torch.zeros_like(scale), scale).half()
    blocks = torch.empty((rows * G, 66), dtype=torch.uint8, device=w.device)
    blocks[:, 0:2] = s16.view(torch.int16).reshape(-1, 1).view(torch.uint8)
    blocks[:, 2:] = q[:, 0::2] | (q[:, 1::2] << 4)
    return blocks.reshape(-1)


def tie_rows_torch(rows: int, cols: int, gen, device):
    """fp16 [rows][cols] ~ N(0, 1) whose every fourth row holds, per
    128-group, one +-7 and otherwise +-(k + 0.5), k in 0..6: ties of the
    lm_head quantizer (inverse scale exactly 1)."""
    import torch

    w = torch.randn((rows, cols), generator=gen, device=device, dtype=torch.float32)
    tie = w[0::4]
    k = torch.randint(0, 7, tie.shape, generator=gen, device=device).float() + 0.5
    sgn = torch.where(torch.rand(tie.shape, generator=gen, device=device) < 0.5, -1.0, 1.0)
    t = k * sgn
    t[:, ::128] = 7.0 * sgn[:, ::128]
    w[0::4] = t
    return w.half()
