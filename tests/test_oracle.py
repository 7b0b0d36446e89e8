"""Pins of the CPU oracle (the parity checker for the HIP kernels).

Each oracle function is checked against
  (1) the golden fixtures written from the reference's compiled kernels,
  (2) the reference's compiled kernels themselves on fresh seeded inputs
      (oracle/_ref, only where it is built),
  (3) float64 closed forms and brute force on tiny inputs, chosen so that a
      dropped term, a sign error or a transposed index fails.
"""

from __future__ import annotations

import numpy as np
import pytest

import oracle
from asdsl.quantization import synthetic as syn
from asdsl.quantization.repack import repack_preq_blocks_to_preq2
from conftest import GOLDEN, rel_l2

REF = oracle.reference_available("_native_gemv")
needs_ref = pytest.mark.skipif(not REF, reason="oracle/_ref not built (reference tree not mounted)")


@pytest.fixture(scope="module")
def golden():
    return np.load(GOLDEN / "gemv_q4_reference.npz")


# ------------------------------------------------------------------ fp16
def test_half_to_float_all_patterns():
    bits = np.arange(65536, dtype=np.uint32).astype(np.uint16)
    want = bits.view(np.float16).astype(np.float32)
    got = np.array([oracle.half_to_float(int(b)) for b in bits[::97]], np.float32)
    w = want[::97]
    finite = np.isfinite(w)
    assert np.array_equal(got[finite], w[finite])
    assert np.all(np.isnan(got[np.isnan(w)]))


# ------------------------------------------------------------------ A1
@pytest.mark.parametrize("gs", [32, 128])
def test_quantize_activation_golden(golden, gs):
    xq, xs = oracle.quantize_activation(golden[f"qa{gs}_x"], gs)
    assert np.array_equal(xq, golden[f"qa{gs}_xq"])
    assert np.array_equal(xs.view(np.uint32), golden[f"qa{gs}_xs"].view(np.uint32))


def test_quantize_activation_closed_form():
    x = syn.activation(4096, 5)
    xq, xs = oracle.quantize_activation(x, 32)
    g = x.reshape(-1, 32)
    amax = np.abs(g).max(axis=1)
    assert np.array_equal(xs, (amax * np.float32(1.0 / 127.0)).astype(np.float32))
    inv = (np.float32(127.0) / amax).astype(np.float32)
    want = np.clip(np.rint((g * inv[:, None]).astype(np.float32)), -128, 127).astype(np.int8).reshape(-1)
    assert np.array_equal(xq, want)
    # the quantized vector reproduces x to half a step
    err = np.abs(xq.reshape(-1, 32) * xs[:, None] - g)
    assert np.all(err <= 0.5001 * xs[:, None])


@needs_ref
@pytest.mark.parametrize("gs", [32, 64, 128])
def test_quantize_activation_vs_reference(gs):
    ng = oracle.load_reference("_native_gemv")
    rng = np.random.default_rng(11)
    for trial in range(8):
        K = 2048
        x = (rng.standard_normal(K) * 10.0 ** rng.uniform(-6, 6, K // gs).repeat(gs)).astype(np.float32)
        xq_r = np.zeros(K, np.int8)
        xs_r = np.zeros(K // gs, np.float32)
        ng.quantize_activation_avx2(x, xq_r, xs_r, K, gs)
        xq, xs = oracle.quantize_activation(x, gs)
        assert np.array_equal(xq, xq_r)
        assert np.array_equal(xs.view(np.uint32), xs_r.view(np.uint32))


# ------------------------------------------------------------------ A3 preq
def _closed_form_preq(blocks, x, M, K):
    """float64 sum_k dequant(W)[r,k] * xs_g * xq[k]."""
    w = oracle.dequant_preq(blocks, M, K).astype(np.float64)
    xq, xs = oracle.quantize_activation(x, 32)
    xd = xq.astype(np.float64) * np.repeat(xs.astype(np.float64), 32)
    return w @ xd


def test_preq_golden(golden):
    M, K = map(int, golden["preq_shape"])
    y = oracle.gemv_preq_fused(golden["preq_blocks"], golden["preq_x"], M, K)
    assert rel_l2(y, golden["preq_y_fused"]) < 1e-6
    assert rel_l2(y, golden["preq_y_q8"]) < 1e-6


def test_preq_closed_form():
    M, K = 37, 640
    w = syn.gaussian_weights(M, K, 3)
    blocks = syn.preq_blocks(w)
    x = syn.activation(K, 4)
    y = oracle.gemv_preq_fused(blocks, x, M, K)
    assert rel_l2(y, _closed_form_preq(blocks, x, M, K)) < 1e-6
    # and it approximates the unquantized product (quantization noise only)
    assert rel_l2(y, w.astype(np.float64) @ x.astype(np.float64)) < 0.1


def test_preq_brute_force_tiny():
    """One row, one group: every term written out by hand."""
    blk = np.zeros(20, np.uint8)
    s, z = np.float16(0.25), np.float16(3.0)
    blk[0:2] = np.array([s]).view(np.uint8)
    blk[2:4] = np.array([z]).view(np.uint8)
    q = np.arange(32) % 16
    blk[4:] = (q[0::2] | (q[1::2] << 4)).astype(np.uint8)
    x = np.linspace(-1, 1, 32).astype(np.float32)
    xq, xs = oracle.quantize_activation(x, 32)
    want = sum((q[k] - 3.0) * 0.25 * float(xq[k]) * float(xs[0]) for k in range(32))
    y = oracle.gemv_preq(blk, xq, xs, 1, 32)
    assert abs(y[0] - want) <= 1e-6 * abs(want)


@needs_ref
def test_preq_vs_reference():
    ng = oracle.load_reference("_native_gemv")
    for (M, K, seed) in [(64, 3072, 1), (33, 8192, 2), (130, 1024, 3)]:
        blocks = syn.preq_blocks(syn.gaussian_weights(M, K, seed))
        x = syn.activation(K, seed + 100)
        y_r = np.zeros(M, np.float32)
        ng.gemv_q4_32_preq_fused_avx2(blocks, x, y_r, M, K, 32)
        assert rel_l2(oracle.gemv_preq_fused(blocks, x, M, K), y_r) < 1e-6


# ------------------------------------------------------------------ A4/A5 preq2
def test_preq2_golden(golden):
    M, K = map(int, golden["preq_shape"])
    y = oracle.gemv_preq2_fused(golden["preq2_meta"], golden["preq2_quant"], golden["preq_x"], M, K, 32)
    assert rel_l2(y, golden["preq2_y"]) < 1e-6


def test_preq2_equals_preq_and_dequant_bitexact():
    M, K = 70, 1024
    blocks = syn.preq_blocks(syn.gaussian_weights(M, K, 8))
    meta, quant = repack_preq_blocks_to_preq2(blocks, M, K, 32)
    assert np.array_equal(oracle.dequant_preq2(meta, quant, M, K, 32).view(np.uint32),
                          oracle.dequant_preq(blocks, M, K).view(np.uint32))
    x = syn.activation(K, 9)
    assert rel_l2(oracle.gemv_preq2_fused(meta, quant, x, M, K, 32), oracle.gemv_preq_fused(blocks, x, M, K)) < 1e-7


@pytest.mark.parametrize("gs", [32, 128])
def test_preq2_closed_form(gs):
    M, K = 45, 1024
    w = syn.gaussian_weights(M, K, 12)
    meta, quant = syn.preq2(w, gs)
    x = syn.activation(K, 13)
    wd = oracle.dequant_preq2(meta, quant, M, K, gs).astype(np.float64)
    xq, xs = oracle.quantize_activation(x, gs)
    want = wd @ (xq.astype(np.float64) * np.repeat(xs.astype(np.float64), gs))
    y = oracle.gemv_preq2_fused(meta, quant, x, M, K, gs)
    assert rel_l2(y, want) < 1e-6
    assert rel_l2(y, w.astype(np.float64) @ x.astype(np.float64)) < 0.15


@needs_ref
def test_preq2_vs_reference():
    ng = oracle.load_reference("_native_gemv")
    for (M, K, seed) in [(512, 3072, 42), (66, 8192, 5)]:
        blocks = syn.preq_blocks(syn.gaussian_weights(M, K, seed))
        meta, quant = repack_preq_blocks_to_preq2(blocks, M, K, 32)
        x = syn.activation(K, seed + 1)
        y_r = np.zeros(M, np.float32)
        ng.gemv_preq2_fused_avx2(meta.reshape(-1), quant.reshape(-1), x, y_r, M, K, 32)
        assert rel_l2(oracle.gemv_preq2_fused(meta, quant, x, M, K, 32), y_r) < 1e-6
