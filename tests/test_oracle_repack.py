"""Pins for the oracle's weight repackers (CPU only).

The reference's repackers are Python loops over numpy scalars
(asdsl/quantization/repack_q4_32.py, repack_preq2.py, repack_q4_128.py), so
their arithmetic is numpy's: float64 division, numpy's float16 cast of a
float64, float32 array arithmetic, round half to even.  The C oracle is
checked against those numpy operations, against byte-layout invariants, and
against what dequantization fixes (preq and preq2 decode to the same
weights; the fp16 (scale, zero) reproduce the asymmetric weights to fp16
precision; the symmetric Q4_128 levels of a known group).
"""

from __future__ import annotations

import numpy as np
import pytest

import oracle


def _asym(rows, cols, gs, seed, lo=0.01, hi=0.5):
    """Asymmetric Q4 weights as the reference's synthetic tests build them
    (benchmarks/test_preq2_correctness.py:12-21): random nibbles, scales and
    biases per group."""
    rng = np.random.default_rng(seed)
    G = cols // gs
    q = rng.integers(0, 16, (rows, cols), dtype=np.uint8)
    packed = ((q[:, 1::2] << 4) | q[:, 0::2]).astype(np.uint8)
    scales = rng.uniform(lo, hi, (rows, G)).astype(np.float32)
    biases = rng.uniform(-0.1, 0.1, (rows, G)).astype(np.float32)
    return q, packed, scales, biases


def test_double_to_half_matches_numpy_cast():
    """Random magnitudes over the whole fp16 range (normals, subnormals,
    overflow), exact ties between neighbouring fp16 values (normal and
    subnormal), the overflow threshold, signed zeros and infinities."""
    rng = np.random.default_rng(0)
    d = [rng.standard_normal(20000) * np.exp(rng.uniform(-25, 13, 20000))]
    h = np.arange(0, 0x7BFF, dtype=np.uint16).view(np.float16).astype(np.float64)
    d.append((h[:-1] + h[1:]) / 2)  # every tie, round half to even
    d.append(-(h[:-1] + h[1:]) / 2)
    d.append(np.nextafter((h[:-1] + h[1:]) / 2, np.inf))
    d.append(np.array([0.0, -0.0, 65504.0, 65519.999, 65520.0, 70000.0, -65520.0, np.inf, -np.inf, 1e-300,
                       -1e-300, 2.0 ** -24, 2.0 ** -25, 3 * 2.0 ** -26, 2.0 ** -14 - 2.0 ** -25]))
    d = np.concatenate(d)
    with np.errstate(over="ignore"):
        want = d.astype(np.float16).view(np.uint16)
    assert np.array_equal(oracle.double_to_half(d), want)


def test_asym_to_q4_32_matches_numpy_ops():
    """Block = f16(float(max(s, 1e-8))) | f16(-b / that) | packed bytes,
    with numpy's own float64 division and float16 cast; one group per edge
    scale (float32(1e-8) keeps itself, smaller scales become 1e-8)."""
    rows, cols = 7, 256
    q, packed, sc, bi = _asym(rows, cols, 32, 1)
    sc[0, 0] = np.float32(1e-8)
    sc[0, 1] = np.float32(1e-9)
    sc[0, 2] = 0.0
    bi[1, 0] = 0.0
    got = oracle.repack_asym_to_q4_32(packed, sc, bi, rows, cols).reshape(rows, cols // 32, 20)
    for r in range(rows):
        for g in range(cols // 32):
            s = max(sc[r, g], 1e-8)
            want_s = np.float16(float(s)).view(np.uint16)
            with np.errstate(over="ignore"):
                want_z = np.float16(-float(bi[r, g]) / float(s)).view(np.uint16)
            assert got[r, g, 0:2].view(np.uint16)[0] == want_s
            assert got[r, g, 2:4].view(np.uint16)[0] == want_z
            assert np.array_equal(got[r, g, 4:], packed[r, g * 16:(g + 1) * 16])


def test_asym_to_q4_32_dequant_reproduces_weights():
    """The preq block decodes (q - zero16) * scale16; against the asymmetric
    weights s*q + b it differs only by the fp16 rounding of scale and zero."""
    rows, cols = 16, 512
    q, packed, sc, bi = _asym(rows, cols, 32, 2)
    blocks = oracle.repack_asym_to_q4_32(packed, sc, bi, rows, cols)
    got = oracle.dequant_preq(blocks, rows, cols)
    want = np.repeat(sc, 32, axis=1) * q + np.repeat(bi, 32, axis=1)
    # |d(s*(q - z))| <= |q - z| * |ds| + s * |dz|, ds <= s * 2^-11, dz <= |z| * 2^-11
    z = np.repeat(-bi / sc, 32, axis=1)
    s = np.repeat(sc, 32, axis=1)
    bound = (np.abs(q - z) * s + s * np.abs(z)) * 2.0 ** -10 + 1e-7
    assert np.all(np.abs(got - want) <= bound)


def test_preq_to_preq2_bytes_and_dequant():
    """meta = block bytes 0..3, band slot r%4 = block bytes 4..19, tail slots
    zero; and preq2 decodes to exactly the preq weights (the reference's
    repack_preq2.py docstring: bit-identical dequant)."""
    rows, cols = 10, 384
    q, packed, sc, bi = _asym(rows, cols, 32, 3)
    preq = oracle.repack_asym_to_q4_32(packed, sc, bi, rows, cols)
    meta, quant = oracle.repack_preq_to_preq2(preq, rows, cols)
    G = cols // 32
    b = preq.reshape(rows, G, 20)
    assert np.array_equal(meta.reshape(rows, G, 4), b[:, :, 0:4])
    qb = quant.reshape(3, G, 64)
    for r in range(rows):
        assert np.array_equal(qb[r // 4, :, 16 * (r % 4):16 * (r % 4) + 16], b[r, :, 4:20])
    assert np.all(qb[2, :, 32:] == 0)
    assert np.array_equal(oracle.dequant_preq2(meta, quant, rows, cols, 32).view(np.uint32),
                          oracle.dequant_preq(preq, rows, cols).view(np.uint32))


@pytest.mark.parametrize("rows", [1, 4, 6, 13])
def test_asym_to_preq2_g32_is_the_composition(rows):
    cols = 256
    q, packed, sc, bi = _asym(rows, cols, 32, 4 + rows)
    want = oracle.repack_preq_to_preq2(oracle.repack_asym_to_q4_32(packed, sc, bi, rows, cols), rows, cols)
    got = oracle.repack_asym_to_preq2(packed, sc, bi, rows, cols, 32)
    assert np.array_equal(got[0], want[0]) and np.array_equal(got[1], want[1])


def test_asym_to_preq2_g128_meta_bands_and_dequant():
    """g128: meta = (f16 scale, f16 zero) as at g32; slot r%4 of a 256-byte
    (band, group) holds the row's 64 packed bytes; decodes to the weights."""
    rows, cols = 9, 512
    q, packed, sc, bi = _asym(rows, cols, 128, 5)
    meta, quant = oracle.repack_asym_to_preq2(packed, sc, bi, rows, cols, 128)
    G = cols // 128
    m = meta.reshape(rows, G, 2, 2).view(np.uint16).reshape(rows, G, 2)
    s64 = sc.astype(np.float64)
    assert np.array_equal(m[:, :, 0], s64.astype(np.float16).view(np.uint16))
    assert np.array_equal(m[:, :, 1], (-bi.astype(np.float64) / s64).astype(np.float16).view(np.uint16))
    qb = quant.reshape(3, G, 256)
    for r in range(rows):
        assert np.array_equal(qb[r // 4, :, 64 * (r % 4):64 * (r % 4) + 64], packed[r].reshape(G, 64))
    assert np.all(qb[2, :, 64:] == 0)
    got = oracle.dequant_preq2(meta, quant, rows, cols, 128)
    want = np.repeat(sc, 128, axis=1) * q + np.repeat(bi, 128, axis=1)
    assert np.max(np.abs(got - want)) < 2e-3


def test_q4_128_known_groups():
    """A group holding +amax and -amax maps them to levels 15 and 1, zeros to
    8, and exact half-steps round to even; an all-zero (or < 1e-12) group is
    scale 0 with every nibble 8 (repack_q4_128.py:24-27)."""
    w = np.zeros((3, 128), np.float32)
    w[0, 0], w[0, 1] = 7.0, -7.0  # amax 7: inv = 1, levels are w + 8
    w[0, 2], w[0, 3], w[0, 4], w[0, 5] = 0.5, 1.5, -0.5, -2.5  # ties -> 0, 2, -0, -2
    w[2, :] = 1e-13
    blocks = oracle.repack_fp32_to_q4_128(w, 3, 128).reshape(3, 66)
    assert blocks[0, 0:2].view(np.uint16)[0] == np.float16(1.0).view(np.uint16)
    q = np.stack([blocks[0, 2:] & 0x0F, blocks[0, 2:] >> 4], axis=1).reshape(-1)
    assert list(q[:6]) == [15, 1, 8, 10, 8, 6] and np.all(q[6:] == 8)
    for r in (1, 2):
        assert blocks[r, 0] == 0 and blocks[r, 1] == 0 and np.all(blocks[r, 2:] == 0x88)


def test_q4_128_matches_numpy_ops_and_bounds():
    """Random groups: the oracle's levels equal numpy's float32 expression
    clip(round(w * float32(7 / amax)) + 8, 0, 15) and its scale numpy's
    float16 of amax / 7; decoding stays within half a step of the weights."""
    rng = np.random.default_rng(6)
    rows, cols = 12, 1024
    w = (rng.standard_normal((rows, cols)) * 0.02).astype(np.float32)
    blocks = oracle.repack_fp32_to_q4_128(w, rows, cols).reshape(rows, cols // 128, 66)
    g = w.reshape(rows, cols // 128, 128)
    amax = np.abs(g).max(axis=-1)
    inv = np.array([[np.float32(7.0 / float(a)) for a in row] for row in amax], np.float32)
    want_q = np.clip(np.round(g * inv[..., None]) + np.float32(8.0), 0, 15).astype(np.uint8)
    got_q = np.stack([blocks[..., 2:] & 0x0F, blocks[..., 2:] >> 4], axis=-1).reshape(rows, cols // 128, 128)
    assert np.array_equal(got_q, want_q)
    want_s = np.array([[np.float16(float(a) / 7.0) for a in row] for row in amax]).view(np.uint16)
    assert np.array_equal(blocks[..., 0:2].copy().view(np.uint16)[..., 0], want_s)
    s16 = want_s.view(np.float16).astype(np.float32)[..., None]
    err = np.abs((got_q.astype(np.float32) - 8) * s16 - g)
    assert np.all(err <= 0.5 * s16 * (1 + 2.0 ** -9) + 1e-7 + np.abs(g) * 2.0 ** -10)


def test_asym_to_q4_128_is_requant_of_float32_dequant():
    """repack_asymmetric_to_q4_128: the group dequantized in float32 as
    (q - f32(zero)) * f32(scale), zero = -b / max(s, 1e-8) in float64, then the
    fp32 requantizer; checked against numpy's float32 arithmetic."""
    rows, cols = 5, 512
    q, packed, sc, bi = _asym(rows, cols, 128, 7)
    got = oracle.repack_asym_to_q4_128(packed, sc, bi, rows, cols)
    s64 = sc.astype(np.float64)
    zero = (-bi.astype(np.float64) / s64).astype(np.float32)
    wf = (q.astype(np.float32).reshape(rows, -1, 128) - zero[..., None]) * sc.astype(np.float32)[..., None]
    want = oracle.repack_fp32_to_q4_128(wf.reshape(rows, cols), rows, cols)
    assert np.array_equal(got, want)


def test_q4_128_to_preq2_decodes_to_the_same_weights():
    """Every weight of the converted preq2-g128 equals the Q4_128 block's
    (q - 8) * scale, decoded here straight from the block bytes."""
    rng = np.random.default_rng(8)
    rows, cols = 7, 384
    w = (rng.standard_normal((rows, cols)) * 0.02).astype(np.float32)
    w[3, 128:256] = 0.0
    blocks = oracle.repack_fp32_to_q4_128(w, rows, cols)
    meta, quant = oracle.repack_q4_128_to_preq2(blocks, rows, cols)
    b = blocks.reshape(rows, cols // 128, 66)
    s = b[..., 0:2].copy().view(np.float16).astype(np.float32)
    q = np.stack([b[..., 2:] & 0x0F, b[..., 2:] >> 4], axis=-1).reshape(rows, cols // 128, 128)
    want = ((q.astype(np.float32) - 8.0) * s).reshape(rows, cols)
    got = oracle.dequant_preq2(meta, quant, rows, cols, 128)
    assert np.array_equal(got.view(np.uint32), want.view(np.uint32))
    assert np.all(quant.reshape(2, 3, 256)[1, :, 192:] == 0)
