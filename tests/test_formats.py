"""Host-side weight formats: the repackers and the torch quantizer mirrors
produce the reference's bytes (CPU only)."""

from __future__ import annotations

import numpy as np
import torch

from asdsl.quantization import synthetic as syn
from asdsl.quantization.repack import repack_preq_blocks_to_preq2


def test_q4_128_torch_mirror_matches_numpy():
    w = syn.gaussian_weights(41, 1024, 9)
    w[5, 256:384] = 0.0
    w[6, :128] = 1e-13
    assert np.array_equal(syn.q4_128_blocks(w), syn.q4_128_from_weights_torch(torch.from_numpy(w)).numpy())


def test_preq2_torch_mirror_matches_numpy():
    for gs in (32, 128):
        w = syn.gaussian_weights(37, 512, 3 + gs)
        m_np, q_np = syn.preq2(w, gs)
        m_t, q_t = syn.preq2_from_weights_torch(torch.from_numpy(w), gs)
        assert np.array_equal(m_np, m_t.numpy()) and np.array_equal(q_np, q_t.numpy())


def test_preq2_repack_is_preq_bytes():
    """meta == preq block bytes [0:4]; band slot r%4 == preq block bytes [4:20]."""
    M, K = 10, 256
    blocks = syn.preq_blocks(syn.gaussian_weights(M, K, 1)).reshape(M, K // 32, 20)
    meta, quant = repack_preq_blocks_to_preq2(blocks.reshape(-1), M, K, 32)
    assert np.array_equal(meta.reshape(M, K // 32, 4), blocks[:, :, 0:4])
    for r in range(M):
        assert np.array_equal(quant[r // 4, :, (r % 4) * 16:(r % 4) * 16 + 16], blocks[r, :, 4:20])
    assert np.all(quant[2, :, 32:] == 0)  # padded tail band


def test_q4_128_block_layout():
    w = np.zeros((1, 128), np.float32)
    w[0, 0] = 0.7
    w[0, 1] = -0.7
    b = syn.q4_128_blocks(w)
    assert b.size == 66
    assert b[:2].view(np.float16)[0] == np.float16(0.1)
    assert b[2] == (15 | (1 << 4))  # q0 = 7+8, q1 = -7+8, low nibble first
    assert np.all(b[3:] == 0x88)
