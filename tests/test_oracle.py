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


# ------------------------------------------------------------------ A6 Q4_128
def test_q4_128_golden(golden):
    M, K = map(int, golden["q128_shape"])
    y = oracle.gemv_q4_128(golden["q128_blocks"], golden["q128_xq"], golden["q128_xs"], M, K)
    assert rel_l2(y, golden["q128_y"]) < 1e-6


def test_q4_128_closed_form_and_zero_group():
    M, K = 9, 512
    w = syn.gaussian_weights(M, K, 3)
    w[2, :128] = 0.0
    blocks = syn.q4_128_blocks(w).reshape(M, K // 128, 66)
    assert blocks[2, 0, 0] == 0 and blocks[2, 0, 1] == 0 and np.all(blocks[2, 0, 2:] == 0x88)
    q = np.stack([blocks[:, :, 2:] & 15, blocks[:, :, 2:] >> 4], -1).reshape(M, K // 128, 128).astype(np.float64)
    s = blocks[:, :, 0:2].copy().view(np.float16).astype(np.float64)
    wd = ((q - 8.0) * s).reshape(M, K)
    x = syn.activation(K, 4)
    xq, xs = oracle.quantize_activation(x, 128)
    want = wd @ (xq.astype(np.float64) * np.repeat(xs.astype(np.float64), 128))
    assert rel_l2(oracle.gemv_q4_128(blocks, xq, xs, M, K), want) < 1e-6
    # sanity only: symmetric 4-bit g128 quantization noise on N(0, 0.02) weights
    assert rel_l2(wd @ x.astype(np.float64), w.astype(np.float64) @ x.astype(np.float64)) < 0.3


def test_preq2_g128_matches_the_reference_q4_128_gemv_golden(golden):
    """The reference has no preq2 kernel at group size 128, but preq2-g128
    repacked from Q4_128 blocks holds the same weights ((q - 8) * s, zero 8),
    so the preq2 oracle at gs 128 must give the reference's Q4_128 GEMV
    output (gemv_q4_128_preq_avx2, the golden vectors) on the same input."""
    M, K = map(int, golden["q128_shape"])
    meta, quant = oracle.repack_q4_128_to_preq2(golden["q128_blocks"], M, K)
    y = oracle.gemv_preq2(meta, quant, golden["q128_xq"], golden["q128_xs"], M, K, 128)
    assert rel_l2(y, golden["q128_y"]) < 1e-6


@needs_ref
@pytest.mark.parametrize("M,K", [(64, 3072), (33, 8192)])
def test_preq2_g128_fused_vs_reference_q4_128(M, K):
    """Same identity on random weights and activations against the compiled
    reference: its activation quantizer at gs 128 and its Q4_128 GEMV."""
    ng = oracle.load_reference("_native_gemv")
    rng = np.random.default_rng(M + K)
    blocks = syn.q4_128_blocks(syn.gaussian_weights(M, K, M * K))
    x = (rng.standard_normal(K) * 10.0 ** rng.uniform(-3, 3, K // 128).repeat(128)).astype(np.float32)
    xq_r = np.zeros(K, np.int8)
    xs_r = np.zeros(K // 128, np.float32)
    ng.quantize_activation_avx2(x, xq_r, xs_r, K, 128)
    y_r = np.zeros(M, np.float32)
    ng.gemv_q4_128_preq_avx2(blocks.reshape(-1), xq_r, xs_r, y_r, M, K, 128)
    meta, quant = oracle.repack_q4_128_to_preq2(blocks, M, K)
    assert rel_l2(oracle.gemv_preq2_fused(meta, quant, x, M, K, 128), y_r) < 1e-6


def test_gemm_q4_128_is_column_loop():
    M, K, B = 7, 256, 3
    blocks = syn.q4_128_blocks(syn.gaussian_weights(M, K, 5))
    X = np.random.default_rng(1).standard_normal((B, K)).astype(np.float32)
    bl = blocks.reshape(M, K // 128, 66)
    q = np.stack([bl[:, :, 2:] & 15, bl[:, :, 2:] >> 4], -1).reshape(M, K // 128, 128).astype(np.float32)
    s = bl[:, :, 0:2].copy().view(np.float16).astype(np.float32)
    wd = ((q - 8.0) * s).reshape(M, K).astype(np.float64)
    assert rel_l2(oracle.gemm_q4_128(blocks, X, M, K, B), X.astype(np.float64) @ wd.T) < 1e-6


# ------------------------------------------------------------------ A9(ii) Q4xQ8
def test_q4_q8_golden(golden):
    M, K = map(int, golden["q4q8_shape"])
    y = oracle.gemv_q4_q8(golden["q4q8_w"], golden["q4q8_s"], golden["q4q8_x"], M, K, 32)
    assert rel_l2(y, golden["q4q8_y"]) < 1e-6


@needs_ref
@pytest.mark.parametrize("gs", [32, 64, 128])
def test_q4_q8_vs_reference(gs):
    ng = oracle.load_reference("_native_gemv")
    rng = np.random.default_rng(gs)
    M, K = 33, 3072
    w = rng.integers(0, 256, M * K // 2, dtype=np.uint8)
    s = (rng.random(M * K // gs) * 0.01).astype(np.float32)
    x = syn.activation(K, 9)
    y = np.zeros(M, np.float32)
    ng.gemv_q4_q8_avx2(w, s, x, y, M, K, gs)
    assert rel_l2(oracle.gemv_q4_q8(w, s, x, M, K, gs), y) < 1e-6


# ------------------------------------------------------------------ A8 Q4_K
def test_q4km_golden(golden):
    M, K = map(int, golden["q4k_shape"])
    assert rel_l2(oracle.gemv_q4km(golden["q4k_w"], golden["q4k_x"], M, K), golden["q4k_y"]) < 1e-6


def test_q4km_closed_form():
    """Decode the 6-bit bitstream independently (bit arithmetic on a Python int)."""
    rng = np.random.default_rng(2)
    M, K = 3, 512
    w = rng.integers(0, 256, (M, K // 256, 144), dtype=np.uint8)
    w[:, :, 0:2] = np.frombuffer(np.float16(0.02).tobytes(), np.uint8)
    w[:, :, 2:4] = np.frombuffer(np.float16(0.01).tobytes(), np.uint8)
    x = syn.activation(K, 3)
    xq, xs = oracle.quantize_activation_q4k(x)
    want = np.zeros(M)
    for r in range(M):
        for b in range(K // 256):
            blk = w[r, b]
            bits = int.from_bytes(bytes(blk[4:16]), "little")
            six = [(bits >> (6 * i)) & 63 for i in range(16)]
            d, dmin = 0.02, 0.01
            for sb in range(8):
                q = np.stack([blk[16 + 16 * sb:32 + 16 * sb] & 15, blk[16 + 16 * sb:32 + 16 * sb] >> 4], -1).reshape(-1)
                xs8 = xq[b * 256 + sb * 32: b * 256 + sb * 32 + 32].astype(np.float64)
                want[r] += (float(np.float16(d)) * six[sb] * (q @ xs8)
                            - float(np.float16(dmin)) * six[sb + 8] * xs8.sum()) * xs[b * 8 + sb]
    assert rel_l2(oracle.gemv_q4km(w.reshape(-1), x, M, K), want) < 1e-6
    # quantizer: round half away from zero, clamp 127, zero group -> scale 0
    xx = np.zeros(64, np.float32)
    xx[32:] = np.linspace(-1, 1, 32)
    xx[33] = 0.5 * 2 / 31 * 1  # arbitrary
    q, s = oracle.quantize_activation_q4k(xx)
    assert s[0] == 0 and np.all(q[:32] == 0)
    assert np.array_equal(q[32:], np.clip(np.sign(xx[32:] * np.float32(127) / np.float32(1)) *
                                          np.floor(np.abs((xx[32:] * (np.float32(127.0) / np.float32(1.0))).astype(np.float32)) + 0.5), -127, 127))


@needs_ref
def test_q4km_vs_reference():
    ng = oracle.load_reference("_native_gemv")
    rng = np.random.default_rng(5)
    M, K = 40, 3072
    w = rng.integers(0, 256, (M, K // 256, 144), dtype=np.uint8)
    w[:, :, 0:2] = np.frombuffer(np.float16(0.011).tobytes(), np.uint8)
    w[:, :, 2:4] = np.frombuffer(np.float16(0.003).tobytes(), np.uint8)
    w = w.reshape(-1)
    x = syn.activation(K, 6)
    y = np.zeros(M, np.float32)
    ng.gemv_q4km_q8_avx2(w, x, y, M, K)
    assert rel_l2(oracle.gemv_q4km(w, x, M, K), y) < 1e-6


# ------------------------------------------------------------------ A10 fp32 affine
def test_affine_golden(golden):
    M, K = map(int, golden["aff_shape"])
    g = golden
    assert rel_l2(oracle.gemv_affine(g["aff_wp"], g["aff_x"], g["aff_s32"], g["aff_b32"], M, K, 32),
                  g["aff_y_packed"]) < 1e-6
    assert rel_l2(oracle.gemv_affine(g["aff_wu"], g["aff_x"], g["aff_s32"], g["aff_b32"], M, K, 32, packed=False),
                  g["aff_y_unpacked"]) < 1e-6
    assert rel_l2(oracle.gemv_q4_gs64(g["aff_wp"], g["aff_x"], g["aff_s64"], M, K), g["aff_y_gs64"]) < 1e-6
    assert rel_l2(oracle.matmul_batch_q4(g["aff_wp"], g["aff_s32"], g["aff_b32"], g["aff_X"], M, K, 3, 32),
                  g["aff_Y_batch"]) < 1e-6


def test_affine_known_answers():
    """tests/test_gemv_q4.py:150-163 (all weights 8, x=1, s=.1, b=-.75 -> 1.6) and
    asdsl/kernels/native/test_kernel.cpp:16,39 (0x77 bytes, s=1, x=1 -> 448 exactly)."""
    w = np.full(32, 0x88, np.uint8)  # 2 rows x 32 nibbles of 8
    y = oracle.gemv_affine(w, np.ones(32, np.float32), np.array([0.1, 0.1], np.float32),
                           np.array([-0.75, -0.75], np.float32), 2, 32, 32)
    np.testing.assert_allclose(y, [1.6, 1.6], rtol=1e-5)
    y = oracle.gemv_q4_gs64(np.full(32, 0x77, np.uint8), np.ones(64, np.float32), np.ones(1, np.float32), 1, 64)
    assert y[0] == 448.0


def test_affine_closed_form_and_batch_loop():
    rng = np.random.default_rng(7)
    M, K, gs = 11, 192, 64
    w = rng.integers(0, 256, M * K // 2, dtype=np.uint8)
    s = rng.random(M * K // gs).astype(np.float32)
    b = rng.standard_normal(M * K // gs).astype(np.float32)
    x = rng.standard_normal(K).astype(np.float32)
    q = np.stack([w & 15, w >> 4], -1).reshape(M, K).astype(np.float64)
    wd = q * np.repeat(s.reshape(M, -1), gs, 1) + np.repeat(b.reshape(M, -1), gs, 1)
    assert rel_l2(oracle.gemv_affine(w, x, s, b, M, K, gs), wd @ x) < 1e-6
    X = rng.standard_normal((4, K)).astype(np.float32)
    Y = oracle.matmul_batch_q4(w, s, b, X, M, K, 4, gs)
    for i in range(4):  # batch == loop (tests/test_gemv_q4_batched.py:10-64)
        assert rel_l2(Y[i], oracle.gemv_affine(w, X[i], s, b, M, K, gs)) < 1e-5


def test_q8_weight_golden(golden):
    M, K = map(int, golden["q8_shape"])
    g = golden
    assert rel_l2(oracle.gemv_affine(g["q8_w"], g["q8_x"], g["q8_s"], g["q8_b"], M, K, 128, packed=False),
                  g["q8_y"]) < 1e-6


# ------------------------------------------------------------------ A12 sparse
def test_sparse_golden(golden):
    g = golden
    M, K = map(int, g["q8_shape"])
    assert np.array_equal(oracle.compute_bitmask(g["sp_x"], 0.01), g["sp_mask"])
    assert np.array_equal(oracle.bitmask_indices(g["sp_mask"], K), g["sp_idx"])
    assert rel_l2(oracle.gemv_sparse_indices(g["q8_w"], g["sp_x"], g["q8_s"], g["q8_b"], g["sp_idx"], M, K, 128),
                  g["sp_y_idx"]) < 1e-6
    assert rel_l2(oracle.gemv_sparse_indices(g["q8_w"], g["sp_x"], g["q8_s"], g["q8_b"],
                                             oracle.bitmask_indices(g["sp_mask"], K), M, K, 128), g["sp_y_mask"]) < 1e-6
    IN, OUT = map(int, g["dT_shape"])
    assert rel_l2(oracle.sparse_down_proj_T(g["dT_w"], g["dT_s"], g["dT_b"], g["dT_x"], g["dT_rows"], IN, OUT, 32),
                  g["dT_y"]) < 1e-6


def test_sparse_equals_dense_on_zeroed_vector():
    rng = np.random.default_rng(3)
    M, K, gs = 13, 512, 128
    w = rng.integers(0, 256, M * K, dtype=np.uint8)
    s = rng.random(M * K // gs).astype(np.float32)
    b = rng.standard_normal(M * K // gs).astype(np.float32)
    x = np.maximum(0, rng.standard_normal(K) - 0.5).astype(np.float32)
    idx = np.nonzero(x)[0].astype(np.int32)
    dense = oracle.gemv_affine(w, x, s, b, M, K, gs, packed=False)
    assert rel_l2(oracle.gemv_sparse_indices(w, x, s, b, idx, M, K, gs), dense) < 1e-6


def test_sparse_down_proj_T_closed_form():
    rng = np.random.default_rng(4)
    IN, OUT = 512, 96
    wT = rng.integers(0, 256, IN * OUT // 2, dtype=np.uint8)
    sT = (rng.random(IN * OUT // 32) * 0.01).astype(np.float32)
    bT = (-8 * sT).astype(np.float32)
    x = np.maximum(0, rng.standard_normal(IN) - 0.84).astype(np.float32)
    rows = np.nonzero(x)[0].astype(np.int32)
    q = np.stack([wT & 15, wT >> 4], -1).reshape(IN, OUT).astype(np.float64)
    wd = q * np.repeat(sT.reshape(IN, -1), 32, 1) + np.repeat(bT.reshape(IN, -1), 32, 1)
    assert rel_l2(oracle.sparse_down_proj_T(wT, sT, bT, x, rows, IN, OUT, 32), x.astype(np.float64) @ wd) < 1e-6


@needs_ref
def test_sparse_down_proj_T_reference_is_racy_beyond_one_chunk():
    """Finding: the reference accumulates into per-thread buffers indexed by
    ai % nthreads inside a pool parallel_for (gemv_sparse_avx2.cpp:297-300), so
    concurrent chunks race.  With <= 4 active rows (one serial chunk) it agrees
    with the oracle; the oracle follows the intended, race-free sum."""
    sp = oracle.load_reference("_native_sparse_gemv")
    rng = np.random.default_rng(0)
    IN, OUT = 512, 64
    wT = rng.integers(0, 256, IN * OUT // 2, dtype=np.uint8)
    sT = (rng.random(IN * OUT // 32) * 0.01).astype(np.float32)
    bT = (-8 * sT).astype(np.float32)
    x = np.maximum(0, rng.standard_normal(IN) - 0.84).astype(np.float32)
    rows = np.nonzero(x)[0].astype(np.int32)
    for n in (1, 2, 3, 4):
        r = rows[:n]
        assert rel_l2(oracle.sparse_down_proj_T(wT, sT, bT, x, r, IN, OUT, 32),
                      np.asarray(sp.sparse_down_proj_T(wT, sT, bT, x, r, IN, OUT, 32))) < 1e-6
