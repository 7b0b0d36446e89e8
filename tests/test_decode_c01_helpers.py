"""The torch mirror of the reference engine's lm_head Q4_128 quantizer
(tests/decode_c01.py) equals oracle.decode.quantize_lm_head_q4_128 byte for
byte on the CPU, ties and all-zero groups included."""

from __future__ import annotations

import numpy as np

from decode_c01 import quantize_lm_head_q4_128_torch, tie_rows_torch
from oracle import decode as od


def test_torch_lm_head_quantizer_equals_oracle():
    import torch

    gen = torch.Generator().manual_seed(3)
    w = tie_rows_torch(512, 768, gen, "cpu")
    w[5, 128:256] = 0.0  # an all-zero group: scale 0, nibbles 0x88
    got = quantize_lm_head_q4_128_torch(w).numpy()
    want = od.quantize_lm_head_q4_128(w.float().numpy())
    assert np.array_equal(got, want)
    blk = want.reshape(512, 6, 66)[5, 1]
    assert blk[0] == 0 and blk[1] == 0 and np.all(blk[2:] == 0x88)


def test_lm_head_quantizer_known_group():
    """One hand-made group: amax 7 (scale fp16(1.0), inverse 1), ties round
    half away from zero: 2.5 -> 3, -3.5 -> -4, 0.5 -> 1, -0.5 -> -1, and
    6.49 -> 6; q = r + 8."""
    x = np.zeros((1, 128), np.float32)
    x[0, :6] = [7.0, 2.5, -3.5, 0.5, -0.5, 6.49]
    b = od.quantize_lm_head_q4_128(x)
    assert b[0] == 0x00 and b[1] == 0x3C  # fp16 1.0
    q = np.empty(128, np.int64)
    q[0::2] = b[2:] & 0xF
    q[1::2] = b[2:] >> 4
    assert list(q[:6] - 8) == [7, 3, -4, 1, -1, 6]
    assert np.all(q[6:] == 8)
