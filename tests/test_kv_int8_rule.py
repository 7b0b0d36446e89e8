"""The int8 KV cache rule on the host side (no GPU): the engine's torch
quantizer (used to fill a cache with a synthetic prefix) against the
oracle's set_kv_cache restatement, with the cases the rule fixes by itself:
a zero block (scale 1e-12, codes 0), a block whose amax is exactly 127
(scale 1, codes = round-half-even(x): 2.5 -> 2, 3.5 -> 4, -0.5 -> 0), the
clamp at +-127 and the sign symmetry."""

from __future__ import annotations

import numpy as np

from oracle import decode as od


def test_torch_quantizer_matches_the_oracle():
    import torch

    from asdsl.engine import kv_quantize_int8

    rng = np.random.default_rng(7)
    rows = rng.standard_normal((3, 50, 128)).astype(np.float32) * rng.uniform(1e-3, 10, (3, 50, 1)).astype(
        np.float32)
    rows[0, 0] = 0.0                                  # all-zero row: both blocks
    rows[0, 1, :64] = 1e-13                           # amax below 1e-12
    rows[1, 0, :64] = 0.0
    rows[1, 0, 0], rows[1, 0, 1:6] = 127.0, [2.5, 3.5, -0.5, -2.5, 126.5]  # scale 1: ties to even
    q, s = kv_quantize_int8(torch.from_numpy(rows))
    want_q, want_s = od.kv_quantize_q8(rows.reshape(-1, 128))
    assert np.array_equal(q.numpy().reshape(-1, 128), want_q)
    assert np.array_equal(s.numpy().reshape(-1, 2), want_s)
    assert np.array_equal(want_q[50, :6], [127, 2, 4, 0, -2, 126])
    assert want_s[50, 0] == np.float32(127.0) * np.float32(1.0 / 127.0)
    assert np.all(want_q[0] == 0) and np.all(want_s[0] == np.float32(1e-12))
    assert np.all(want_q[1, :64] == 0) and want_s[1, 0] == np.float32(1e-12)
    assert want_q.min() >= -127 and want_q.max() <= 127
    nq, ns = od.kv_quantize_q8(-rows.reshape(-1, 128))
    assert np.array_equal(nq, -want_q) and np.array_equal(ns, want_s)


def test_dequantized_rows_within_half_a_step():
    """|float(code) * scale - x| <= scale / 2 (plus rounding) for every
    element: what the attention reads back."""
    rng = np.random.default_rng(3)
    rows = rng.standard_normal((64, 128)).astype(np.float32) * 3
    q, s = od.kv_quantize_q8(rows)
    back = od.kv_dequant_q8(q, s)
    step = np.repeat(s, 64, axis=1)
    assert np.all(np.abs(back - rows) <= step * 0.5 * (1 + 1e-5))
