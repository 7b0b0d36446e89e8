"""Pins the decode-step oracle (oracle/decode.py) with properties a wrong
restatement would break: RoPE is a rotation whose q.k depends only on the
position difference, the polynomial exp tracks exp, attention reduces to known
answers, and the reference's own tolerances for RMSNorm and SwiGLU
(tests/test_native_ops.py:17-49) hold against float64 closed forms."""

from __future__ import annotations

import math

import numpy as np
import pytest

from oracle import decode as od


def _tables(max_seq=64, rot=96):
    from asdsl.engine import rope_tables

    return rope_tables(max_seq, rot)


def test_rope_tables_known_values():
    cos, sin = _tables()
    # freq_0 = 1: angle = pos; the last pair turns by theta^(-94/96) per step
    assert cos[7, 0] == np.float32(math.cos(7.0)) and sin[7, 0] == np.float32(math.sin(7.0))
    f = 10000.0 ** (-94.0 / 96.0)
    assert sin[5, 47] == np.float32(math.sin(5 * f))
    assert np.all(cos[0] == 1.0) and np.all(sin[0] == 0.0)


def test_rope_is_relative_position_rotation():
    cos, sin = _tables()
    rng = np.random.default_rng(0)
    q = rng.standard_normal((1, 128)).astype(np.float32)
    k = rng.standard_normal((1, 128)).astype(np.float32)

    def dot(m, n):
        return float((od.rope(q, cos[m], sin[m]) @ od.rope(k, cos[n], sin[n]).T)[0, 0])

    # q.k depends only on m - n (the defining RoPE property; a wrong pairing of
    # dims or a sign error breaks it)
    assert dot(9, 4) == pytest.approx(dot(25, 20), rel=1e-5)
    assert dot(3, 3) == pytest.approx(float((q @ k.T)[0, 0]), rel=1e-5)
    # dims past the rotary part are untouched; the rotation keeps pair norms
    r = od.rope(q, cos[11], sin[11])
    assert np.array_equal(r[:, 96:], q[:, 96:])
    np.testing.assert_allclose(r[0, :48] ** 2 + r[0, 48:96] ** 2, q[0, :48] ** 2 + q[0, 48:96] ** 2, rtol=1e-5)
    # composition: rotating by a then b equals rotating by a + b
    ab = od.rope(od.rope(q, cos[6], sin[6]), cos[10], sin[10])
    np.testing.assert_allclose(ab, od.rope(q, cos[16], sin[16]), rtol=1e-5, atol=1e-5)


def test_fast_exp_tracks_exp():
    # degree-5 polynomial on [-1/2, 1/2]: ~1.4e-6 relative, plus fp32 rounding of the
    # steps (the product x*log2(e) adds up to |x|*2^-24*ln2 for large |x|)
    x = np.linspace(-80.0, 80.0, 200001, dtype=np.float32)
    rel = np.abs(od.fast_exp(x).astype(np.float64) / np.exp(x.astype(np.float64)) - 1.0)
    assert np.max(rel) < 1e-5
    assert np.max(rel[np.abs(x) <= 8]) < 5e-6
    assert od.fast_exp(np.float32([0.0]))[0] == 1.0
    assert od.fast_exp(np.float32([-1000.0]))[0] == od.fast_exp(np.float32([-87.3]))[0]


def test_swiglu_and_rmsnorm_closed_forms():
    rng = np.random.default_rng(1)
    g = rng.standard_normal(4096).astype(np.float32) * 4
    u = rng.standard_normal(4096).astype(np.float32)
    g64, u64 = g.astype(np.float64), u.astype(np.float64)
    want = g64 / (1.0 + np.exp(-g64)) * u64
    np.testing.assert_allclose(od.swiglu(g, u), want, rtol=1e-5, atol=1e-6)
    t = od.swiglu(g, u, threshold=0.5)
    assert np.all((t == 0) | (np.abs(t) >= 0.5)) and np.count_nonzero(t == 0) > 0
    x = rng.standard_normal(3072).astype(np.float32)
    w = (1 + 0.1 * rng.standard_normal(3072)).astype(np.float32)
    ref = x.astype(np.float64) / np.sqrt(np.mean(x.astype(np.float64) ** 2) + 1e-5) * w
    np.testing.assert_allclose(od.rmsnorm(x, w, 1e-5), ref, rtol=1e-5, atol=1e-6)
    # a constant vector normalizes to +-w (up to eps)
    np.testing.assert_allclose(od.rmsnorm(np.full(64, -3.0, np.float32), w[:64], 1e-5), -w[:64], rtol=1e-5)


def test_attention_known_answers():
    rng = np.random.default_rng(2)
    q = rng.standard_normal((6, 128)).astype(np.float32)
    v = rng.standard_normal((2, 9, 128)).astype(np.float32)
    # identical keys: uniform weights, output = mean of the values
    k = np.repeat(rng.standard_normal((2, 1, 128)).astype(np.float32), 9, axis=1)
    out = od.attention(q, k, v, 2)
    np.testing.assert_allclose(out[0], v[0].mean(0), rtol=1e-5, atol=1e-6)
    np.testing.assert_allclose(out[5], v[1].mean(0), rtol=1e-5, atol=1e-6)  # GQA: heads 3..5 -> kv head 1
    # one position: output = that value
    np.testing.assert_allclose(od.attention(q, k[:, :1], v[:, :1], 2)[4], v[1, 0], rtol=1e-6)
    # a key along q with a large margin takes (almost) all the weight
    k2 = rng.standard_normal((2, 9, 128)).astype(np.float32) * 0.01
    k2[0, 4] = q[1] * 10
    np.testing.assert_allclose(od.attention(q, k2, v, 2)[1], v[0, 4], rtol=1e-4, atol=1e-4)


def test_argmax_first_on_ties():
    assert od.argmax_first(np.float32([1, 5, 2, 5, 5])) == 1
