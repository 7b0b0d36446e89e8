"""The output projection quantized as the reference engine does at load
(asdsl.quantization.lm_head.quantize_output_projection, run here on the
CPU) equals the oracle's restatement byte for byte at both group sizes --
oracle.decode.quantize_lm_head_q4_128 repacked to preq2-g128, and
oracle.decode.quantize_lm_head_preq_g32 repacked to preq2 -- ties and
all-zero groups included; and hand-made groups give the rule's levels."""

from __future__ import annotations

import numpy as np
import pytest

from asdsl.quantization.lm_head import quantize_output_projection
from asdsl.quantization.repack import repack_preq_blocks_to_preq2, repack_q4_128_blocks_to_preq2
from decode_c01 import tie_rows_torch
from oracle import decode as od


@pytest.mark.parametrize("gs", [32, 128])
def test_output_projection_quantizer_equals_oracle(gs):
    import torch

    gen = torch.Generator().manual_seed(3 + gs)
    w = tie_rows_torch(514, 768, gen, "cpu")  # a tail band of 2 rows
    w[5, 128:256] = 0.0  # all-zero groups: scale 0, levels 8
    meta, quant = quantize_output_projection(w, gs)
    wf = w.float().numpy()
    if gs == 128:
        want = repack_q4_128_blocks_to_preq2(od.quantize_lm_head_q4_128(wf), 514, 768)
    else:
        want = repack_preq_blocks_to_preq2(od.quantize_lm_head_preq_g32(wf), 514, 768, 32)
    assert np.array_equal(meta.numpy(), np.ravel(want[0])) and np.array_equal(quant.numpy(), np.ravel(want[1]))


def test_lm_head_quantizer_known_group():
    """One hand-made group: amax 7 (scale fp16(1.0), inverse 1), ties round
    half away from zero: 2.5 -> 3, -3.5 -> -4, 0.5 -> 1, -0.5 -> -1, and
    6.49 -> 6; level = r + 8; at group size 32 the block carries zero fp16 8.0."""
    x = np.zeros((1, 128), np.float32)
    x[0, :6] = [7.0, 2.5, -3.5, 0.5, -0.5, 6.49]
    b = od.quantize_lm_head_q4_128(x)
    assert b[0] == 0x00 and b[1] == 0x3C  # fp16 1.0
    q = np.empty(128, np.int64)
    q[0::2] = b[2:] & 0xF
    q[1::2] = b[2:] >> 4
    assert list(q[:6] - 8) == [7, 3, -4, 1, -1, 6]
    assert np.all(q[6:] == 8)
    p = od.quantize_lm_head_preq_g32(x).reshape(4, 20)
    assert list(p[0, :4]) == [0x00, 0x3C, 0x00, 0x48]  # scale 1.0, zero 8.0
    assert list(p[1, :4]) == [0x00, 0x00, 0x00, 0x48] and np.all(p[1, 4:] == 0x88)  # all-zero group
