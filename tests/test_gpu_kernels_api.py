"""The high-level asdsl.kernels API (the reference's asdsl/kernels/__init__.py:20-76)
on the GPU, in the style of the reference's tests/test_gemv_q4.py.

Bars as in the reference tests: rtol 1e-4 against a float64 scalar closed
form for the fp32-affine kernels, 1e-3 against dequantize-then-multiply for
QuantizedTensor input, exact repeatability; within 1e-4 relative L2 of the
oracle for the integer kernels.
"""

from __future__ import annotations

import numpy as np
import pytest

import oracle
from asdsl.quantization.core import _pack_bits, dequantize_weights, quantize_weights
from conftest import rel_l2

pytestmark = pytest.mark.gpu


def _scalar_reference(w_int_2d, x, scales, biases, group_size):
    """y[m] = sum_g dot(w, x)_g * s + b * sum(x_g), in float64."""
    M, K = w_int_2d.shape
    G = K // group_size
    y = np.zeros(M, np.float64)
    for m in range(M):
        for g in range(G):
            k0, k1 = g * group_size, (g + 1) * group_size
            wg, xg = w_int_2d[m, k0:k1].astype(np.float64), x[k0:k1].astype(np.float64)
            y[m] += wg @ xg * scales[m * G + g] + biases[m * G + g] * xg.sum()
    return y.astype(np.float32)


def _data(rng, M, K, gs):
    w_int = rng.integers(0, 16, size=(M, K), dtype=np.uint8)
    x = rng.standard_normal(K).astype(np.float32)
    scales = rng.uniform(0.001, 0.1, M * K // gs).astype(np.float32)
    biases = rng.uniform(-0.5, 0.5, M * K // gs).astype(np.float32)
    return w_int, _pack_bits(w_int.ravel(), 4), x, scales, biases


@pytest.mark.parametrize("M,K,gs", [(4, 32, 16), (128, 256, 32), (64, 512, 128), (1, 64, 32), (512, 1024, 32)])
def test_packed_and_unpacked_api(gpu, M, K, gs):
    from asdsl.kernels import gemv_q4_packed, gemv_q4_unpacked

    w_int, w_packed, x, s, b = _data(np.random.default_rng(M + K), M, K, gs)
    want = _scalar_reference(w_int, x, s, b, gs)
    np.testing.assert_allclose(gemv_q4_packed(w_packed, x, s, b, M, K, gs), want, rtol=1e-4, atol=1e-4)
    np.testing.assert_allclose(gemv_q4_unpacked(w_int.ravel(), x, s, b, M, K, gs), want, rtol=1e-4, atol=1e-4)


def test_known_values_zero_weights_deterministic(gpu):
    from asdsl.kernels import gemv_q4_packed

    y = gemv_q4_packed(_pack_bits(np.full(64, 8, np.uint8), 4), np.ones(32, np.float32),
                       np.array([0.1, 0.1], np.float32), np.array([-0.75, -0.75], np.float32), 2, 32, 32)
    np.testing.assert_allclose(y, [1.6, 1.6], rtol=1e-5)
    x = np.random.default_rng(77).standard_normal(64).astype(np.float32)
    s, b = np.full(8, 0.05, np.float32), np.full(8, -0.3, np.float32)
    y0 = gemv_q4_packed(_pack_bits(np.zeros(256, np.uint8), 4), x, s, b, 4, 64, 32)
    np.testing.assert_allclose(y0, _scalar_reference(np.zeros((4, 64), np.uint8), x, s, b, 32), rtol=1e-4, atol=1e-5)
    w_int, w_packed, x, s, b = _data(np.random.default_rng(100), 32, 128, 32)
    np.testing.assert_array_equal(gemv_q4_packed(w_packed, x, s, b, 32, 128, 32),
                                  gemv_q4_packed(w_packed, x, s, b, 32, 128, 32))


def test_batch_out_and_q8_paths(gpu):
    import torch
    from asdsl.kernels import gemv_q4_packed

    M, K, gs = 96, 256, 32
    w_int, w_packed, x, s, b = _data(np.random.default_rng(5), M, K, gs)
    X = np.random.default_rng(6).standard_normal((3, K)).astype(np.float32)
    Y = gemv_q4_packed(w_packed, X, s, b, M, K, gs)
    assert Y.shape == (3, M)
    for i in range(3):
        np.testing.assert_allclose(Y[i], _scalar_reference(w_int, X[i], s, b, gs), rtol=1e-4, atol=1e-4)
    out = np.empty(M, np.float32)
    r = gemv_q4_packed(w_packed, x, s, b, M, K, gs, out=out)
    assert r is out
    np.testing.assert_allclose(out, _scalar_reference(w_int, x, s, b, gs), rtol=1e-4, atol=1e-4)
    dev_out = torch.empty(M, device="cuda")
    gemv_q4_packed(torch.from_numpy(w_packed).cuda(), torch.from_numpy(x).cuda(), torch.from_numpy(s).cuda(),
                   torch.from_numpy(b).cuda(), M, K, gs, out=dev_out)
    np.testing.assert_allclose(dev_out.cpu().numpy(), out, rtol=1e-5, atol=1e-6)
    # use_q8: the symmetric Q4xQ8 kernel (scales only, q - 8), as gemv_q4.py:269-273
    yq = gemv_q4_packed(w_packed, x, s, b, M, K, gs, use_q8=True)
    assert rel_l2(yq, oracle.gemv_q4_q8(w_packed, s, x, M, K, gs)) < 1e-4
    with pytest.raises(ValueError, match="does not match K"):
        gemv_q4_packed(w_packed, x[:-2], s, b, M, K, gs)


@pytest.mark.parametrize("symmetric", [False, True])
def test_quantized_tensor_matches_dequant_matvec(gpu, symmetric):
    from asdsl.kernels import gemv_q4

    rng = np.random.default_rng(42 if not symmetric else 99)
    W = rng.standard_normal((64, 128)).astype(np.float32)
    x = rng.standard_normal(128).astype(np.float32)
    qt = quantize_weights(W, bits=4, group_size=32, symmetric=symmetric)
    np.testing.assert_allclose(gemv_q4(qt, x), dequantize_weights(qt) @ x, rtol=1e-3, atol=1e-4)
    with pytest.raises(ValueError, match="4-bit"):
        gemv_q4(quantize_weights(W, bits=8, group_size=128), x)


def test_q4km_q8_and_q8_wrappers(gpu):
    from asdsl.kernels import gemv_q4km_q8, gemv_q8_unpacked

    rng = np.random.default_rng(9)
    M, K = 64, 512
    w = rng.integers(0, 256, (M * (K // 256), 144), dtype=np.uint8)
    dd = np.stack([rng.random(M * (K // 256)) * 0.02 + 1e-3, rng.random(M * (K // 256)) * 0.01], 1)
    w[:, 0:4] = dd.astype(np.float16).view(np.uint8).reshape(-1, 4)  # finite d, dmin
    w = w.reshape(-1)
    x = rng.standard_normal(K).astype(np.float32)
    assert rel_l2(gemv_q4km_q8(w, x, M, K), oracle.gemv_q4km(w, x, M, K)) < 1e-4
    wq8 = rng.integers(0, 256, M * K, dtype=np.uint8)
    s = rng.uniform(1e-3, 1e-2, M * K // 128).astype(np.float32)
    b = rng.uniform(-0.5, 0.5, M * K // 128).astype(np.float32)
    want = oracle.gemv_affine(wq8, x, s, b, M, K, 128, packed=False)
    assert rel_l2(gemv_q8_unpacked(wq8, x, s, b, M, K), want) < 1e-4


def test_sparse_wrappers(gpu):
    import torch
    from asdsl.kernels import compute_activation_bitmask, gemv_sparse_unpacked, gemv_sparse_with_indices

    rng = np.random.default_rng(3)
    M, K, gs = 48, 320, 32
    act = rng.standard_normal(K).astype(np.float32)
    act[rng.random(K) < 0.6] = 0.0
    mask, idx = compute_activation_bitmask(act, threshold=0.01)
    assert np.array_equal(mask, oracle.compute_bitmask(act, 0.01))
    assert np.array_equal(idx, np.where(np.abs(act) >= 0.01)[0])
    dmask, didx = compute_activation_bitmask(torch.from_numpy(act).cuda(), threshold=0.01)
    assert np.array_equal(dmask.cpu().numpy().view(np.uint32), mask.view(np.uint32))
    assert np.array_equal(didx.cpu().numpy(), idx)
    w = rng.integers(0, 16, M * K, dtype=np.uint8)
    s = rng.uniform(1e-3, 1e-1, M * K // gs).astype(np.float32)
    b = rng.uniform(-0.5, 0.5, M * K // gs).astype(np.float32)
    want = oracle.gemv_sparse_indices(w, act, s, b, idx, M, K, gs)
    assert rel_l2(gemv_sparse_unpacked(w, act, s, b, mask, M, K, gs), want) < 1e-4
    assert rel_l2(gemv_sparse_with_indices(w, act, s, b, idx, M, K, gs), want) < 1e-4


def test_g4fused_entry_and_q8_call_counter(gpu):
    """gemv_q4_32_preq_g4fused_4row_avx2 computes the fused preq GEMV
    (gemv_q4_preq_restored.cpp:603-626) and gemv_q4_q8_avx2 calls are counted
    (gemv_q4_avx2.cpp:140,1442)."""
    from asdsl.kernels import _native_gemv as ng
    from asdsl.quantization import synthetic as syn

    M, K = 3072, 3072
    blocks = syn.preq_blocks(syn.gaussian_weights(M, K, 11))
    x = syn.activation(K, 12)
    y = np.full(M, np.nan, np.float32)
    ng.gemv_q4_32_preq_g4fused_4row_avx2(blocks, x, y, M, K)
    assert rel_l2(y, oracle.gemv_preq_fused(blocks, x, M, K)) < 1e-4
    before = ng.get_q8_call_count()
    w = np.random.default_rng(1).integers(0, 256, M * K // 2, dtype=np.uint8)
    s = np.full(M * K // 32, 0.01, np.float32)
    ng.gemv_q4_q8_avx2(w, s, x, np.zeros(M, np.float32), M, K, 32)
    assert ng.get_q8_call_count() == before + 1
