"""Helper of the decode tests on the reference's C0.1 weight profile: an
output projection whose ties exercise the engine's load-time lm_head rule
(asdsl.quantization.lm_head)."""

from __future__ import annotations

import numpy as np


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
