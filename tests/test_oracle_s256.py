"""Pins for the Q4_S256 oracle (CPU): the reference's golden vectors (its
compiled gemv_q4_s256_preq_avx2 through oracle/_ref, tests/golden/
make_golden.py), the compiled reference on random shapes where it is built,
and the float64 closed form y = sum_k (q_k - 8) s_k x8_k xs_k."""

from __future__ import annotations

import numpy as np
import pytest

import oracle
from conftest import rel_l2

GOLD = "q4_s256_reference.npz"


def _blocks(M, K, seed):
    import sys
    from pathlib import Path
    sys.path.insert(0, str(Path(__file__).resolve().parent / "golden"))
    from make_golden import s256_blocks

    return s256_blocks(M, K, seed)


def _closed_form(blocks, xq, xs, M, K):
    b = blocks.reshape(M, K // 256, 144)
    s = b[:, :, :16].copy().view(np.float16).astype(np.float64).reshape(M, K // 32)
    nib = b[:, :, 16:].reshape(M, K // 256, 8, 16)
    q = np.stack([nib & 0x0F, nib >> 4], axis=-1).reshape(M, K // 32, 32).astype(np.float64)
    w = ((q - 8.0) * s[:, :, None]).reshape(M, K)
    x = xq.astype(np.float64) * np.repeat(xs.astype(np.float64), 32)
    return w @ x


def test_golden_vectors():
    g = np.load(__import__("conftest").GOLDEN / GOLD)
    M, K = (int(v) for v in g["s256_shape"])
    got = oracle.gemv_q4_s256(g["s256_blocks"], g["s256_xq"], g["s256_xs"], M, K)
    assert rel_l2(got, g["s256_y"]) < 1e-5


@pytest.mark.parametrize("M,K", [(5, 256), (64, 3072), (9, 17920), (6, 8192)])
def test_closed_form(M, K):
    rng = np.random.default_rng(M + K)
    blocks = _blocks(M, K, M * K)
    x = rng.standard_normal(K).astype(np.float32)
    xq, xs = oracle.quantize_activation(x, 32)
    got = oracle.gemv_q4_s256(blocks, xq, xs, M, K)
    assert rel_l2(got, _closed_form(blocks, xq, xs, M, K)) < 1e-6


@pytest.mark.parametrize("M,K", [(7, 256), (130, 3072), (33, 8192)])
def test_compiled_reference(M, K):
    ref = oracle.reference_q4_s256()
    if ref is None:
        pytest.skip("oracle/_ref/libref_q4_s256.so not built (needs the reference tree)")
    blocks = _blocks(M, K, 3 * M + K)
    x = np.random.default_rng(K).standard_normal(K).astype(np.float32)
    xq, xs = oracle.quantize_activation(x, 32)
    assert rel_l2(oracle.gemv_q4_s256(blocks, xq, xs, M, K), ref(blocks, xq, xs, M, K)) < 1e-5
