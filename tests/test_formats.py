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


def _asym(rows, cols, gs, seed):
    rng = np.random.default_rng(seed)
    q = rng.integers(0, 16, (rows, cols), dtype=np.uint8)
    packed = ((q[:, 1::2] << 4) | q[:, 0::2]).astype(np.uint8)
    sc = rng.uniform(0.01, 0.5, (rows, cols // gs)).astype(np.float32)
    bi = rng.uniform(-0.1, 0.1, (rows, cols // gs)).astype(np.float32)
    sc[0, 0], sc[0, 1] = np.float32(1e-8), 0.0
    return packed, sc, bi


def test_host_repackers_match_the_oracle():
    """The host restatements write the oracle's bytes (tail bands, edge
    scales, a zero Q4_128 group included)."""
    import oracle
    from asdsl.quantization import repack as rp

    rows = 10
    packed, sc, bi = _asym(rows, 256, 32, 1)
    assert np.array_equal(rp.repack_asymmetric_to_q4_32_blocks(packed, sc, bi, rows, 256).reshape(-1),
                          oracle.repack_asym_to_q4_32(packed, sc, bi, rows, 256))
    for gs in (32, 128):
        packed, sc, bi = _asym(rows, 512, gs, 2 + gs)
        got = rp.repack_asymmetric_to_preq2(packed, sc, bi, rows, 512, gs)
        want = oracle.repack_asym_to_preq2(packed, sc, bi, rows, 512, gs)
        assert np.array_equal(got[0], want[0]) and np.array_equal(got[1], want[1])
    packed, sc, bi = _asym(rows, 512, 128, 3)
    assert np.array_equal(rp.repack_asymmetric_to_q4_128_blocks(packed, sc, bi, rows, 512).reshape(-1),
                          oracle.repack_asym_to_q4_128(packed, sc, bi, rows, 512))
    w = syn.gaussian_weights(rows, 512, 4)
    w[2, 128:256] = 0.0
    blocks = rp.repack_fp32_to_q4_128_blocks(w, rows, 512)
    assert np.array_equal(blocks.reshape(-1), oracle.repack_fp32_to_q4_128(w, rows, 512))
    got = rp.repack_q4_128_blocks_to_preq2(blocks, rows, 512)
    want = oracle.repack_q4_128_to_preq2(blocks, rows, 512)
    assert np.array_equal(got[0], want[0]) and np.array_equal(got[1], want[1])


def test_reference_module_names():
    from asdsl.quantization import repack_preq2, repack_q4_128, repack_q4_32

    assert repack_q4_32.BLOCK_SIZE == 20 and repack_q4_128.BLOCK_SIZE == 66 and repack_q4_128.GROUP_SIZE == 128
    assert repack_preq2.preq2_flat_sizes(10, 256, 32) == (10 * 8 * 4, 3 * 8 * 64)
    assert callable(repack_q4_32.repack_asymmetric_to_q4_32_blocks)
