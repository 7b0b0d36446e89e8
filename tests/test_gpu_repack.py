"""HIP parity for the weight repackers: every output byte equal to the
oracle's (oracle/asdsl_oracle.c, pinned in tests/test_oracle_repack.py),
at small shapes with ragged 4-row bands and edge scales, and at the Phi-4
lm_head and gate_up shapes."""

from __future__ import annotations

import numpy as np
import pytest

import oracle

pytestmark = pytest.mark.gpu


def _host(t):
    return t.cpu().numpy()


def _asym_dev(rows, cols, gs, seed, edge=True):
    import torch

    g = torch.Generator(device="cuda").manual_seed(seed)
    packed = torch.randint(0, 256, (rows, cols // 2), generator=g, device="cuda", dtype=torch.int32).to(torch.uint8)
    sc = torch.rand((rows, cols // gs), generator=g, device="cuda") * 0.49 + 0.01
    bi = torch.rand((rows, cols // gs), generator=g, device="cuda") * 0.2 - 0.1
    if edge:  # scale float32(1e-8) (kept), 1e-9 and 0 (both floored to 1e-8), a zero bias,
        # and a zero point beyond the fp16 range (-> inf); on as many groups as there are
        G = sc.shape[1]
        sc[0, 0] = float(np.float32(1e-8))
        sc[0, 1 % G] = 1e-9
        sc[0, 2 % G] = 0.0
        bi[0, 1 % G] = 0.0
        sc[rows - 1, G - 1] = 1e-6
    return packed, sc, bi


@pytest.mark.parametrize("rows,cols", [(1, 64), (6, 256), (13, 3072)])
def test_asym_to_q4_32_bytes(gpu, rows, cols):
    from asdsl.quantization.repack import repack_asymmetric_to_q4_32_blocks

    packed, sc, bi = _asym_dev(rows, cols, 32, rows)
    got = repack_asymmetric_to_q4_32_blocks(packed, sc, bi, rows, cols)
    assert got.is_cuda and tuple(got.shape) == (rows, cols // 32, 20)
    want = oracle.repack_asym_to_q4_32(_host(packed), _host(sc), _host(bi), rows, cols)
    assert np.array_equal(_host(got).reshape(-1), want)


@pytest.mark.parametrize("rows,cols", [(1, 32), (7, 256), (4096 + 3, 3072)])
def test_preq_to_preq2_bytes(gpu, rows, cols):
    from asdsl.quantization.repack import repack_asymmetric_to_q4_32_blocks, repack_preq_blocks_to_preq2

    packed, sc, bi = _asym_dev(rows, cols, 32, 10 + rows)
    preq = repack_asymmetric_to_q4_32_blocks(packed, sc, bi, rows, cols).reshape(-1)
    meta, quant = repack_preq_blocks_to_preq2(preq, rows, cols)
    assert tuple(meta.shape) == (rows, cols // 32 * 4) and tuple(quant.shape) == ((rows + 3) // 4, cols // 32, 64)
    wm, wq = oracle.repack_preq_to_preq2(_host(preq), rows, cols)
    assert np.array_equal(_host(meta).reshape(-1), wm) and np.array_equal(_host(quant).reshape(-1), wq)


@pytest.mark.parametrize("gs", [32, 128])
@pytest.mark.parametrize("rows", [1, 5, 258])
def test_asym_to_preq2_bytes(gpu, gs, rows):
    from asdsl.quantization.repack import repack_asymmetric_to_preq2

    cols = 1024
    packed, sc, bi = _asym_dev(rows, cols, gs, 20 + rows + gs)
    meta, quant = repack_asymmetric_to_preq2(packed, sc, bi, rows, cols, gs)
    wm, wq = oracle.repack_asym_to_preq2(_host(packed), _host(sc), _host(bi), rows, cols, gs)
    assert np.array_equal(_host(meta), wm) and np.array_equal(_host(quant), wq)


@pytest.mark.parametrize("rows,cols", [(1, 128), (9, 640), (300, 3072)])
def test_q4_128_requantizers_bytes(gpu, rows, cols):
    """fp32 -> Q4_128 (with an all-zero and a sub-1e-12 group, and exact
    half-step ties) and asymmetric -> Q4_128."""
    import torch
    from asdsl.quantization.repack import repack_asymmetric_to_q4_128_blocks, repack_fp32_to_q4_128_blocks

    g = torch.Generator(device="cuda").manual_seed(rows)
    w = torch.randn((rows, cols), generator=g, device="cuda") * 0.02
    w[0, :128] = 0.0
    if rows > 2:
        w[1, :128] = 1e-13
        w[2, :128] = torch.arange(128, device="cuda", dtype=torch.float32) * 0.5 - 32.0  # amax 32: ties
    got = repack_fp32_to_q4_128_blocks(w, rows, cols)
    assert np.array_equal(_host(got).reshape(-1), oracle.repack_fp32_to_q4_128(_host(w), rows, cols))
    packed, sc, bi = _asym_dev(rows, cols, 128, 30 + rows)
    got = repack_asymmetric_to_q4_128_blocks(packed, sc, bi, rows, cols)
    want = oracle.repack_asym_to_q4_128(_host(packed), _host(sc), _host(bi), rows, cols)
    assert np.array_equal(_host(got).reshape(-1), want)


@pytest.mark.parametrize("rows", [3, 130])
def test_q4_128_to_preq2_bytes(gpu, rows):
    import torch
    from asdsl.quantization.repack import repack_fp32_to_q4_128_blocks, repack_q4_128_blocks_to_preq2

    cols = 768
    w = torch.randn((rows, cols), generator=torch.Generator(device="cuda").manual_seed(rows), device="cuda")
    blocks = repack_fp32_to_q4_128_blocks(w, rows, cols)
    meta, quant = repack_q4_128_blocks_to_preq2(blocks, rows, cols)
    wm, wq = oracle.repack_q4_128_to_preq2(_host(blocks), rows, cols)
    assert np.array_equal(_host(meta), wm) and np.array_equal(_host(quant), wq)


def test_lm_head_and_gate_up_shapes(gpu):
    """Full Phi-4 shapes: lm_head 200064 x 3072 (asymmetric -> preq2 g128, and
    preq -> preq2 g32) and gate_up 16384 x 3072 (asymmetric -> Q4_128)."""
    from asdsl.quantization.repack import (repack_asymmetric_to_preq2, repack_asymmetric_to_q4_128_blocks,
                                           repack_asymmetric_to_q4_32_blocks, repack_preq_blocks_to_preq2)

    M, K = 200064, 3072
    packed, sc, bi = _asym_dev(M, K, 128, 1)
    meta, quant = repack_asymmetric_to_preq2(packed, sc, bi, M, K, 128)
    wm, wq = oracle.repack_asym_to_preq2(_host(packed), _host(sc), _host(bi), M, K, 128)
    assert np.array_equal(_host(meta), wm) and np.array_equal(_host(quant), wq)
    del meta, quant, wm, wq
    packed, sc, bi = _asym_dev(M, K, 32, 2)
    preq = repack_asymmetric_to_q4_32_blocks(packed, sc, bi, M, K).reshape(-1)
    meta, quant = repack_preq_blocks_to_preq2(preq, M, K)
    wm, wq = oracle.repack_preq_to_preq2(_host(preq), M, K)
    assert np.array_equal(_host(meta).reshape(-1), wm) and np.array_equal(_host(quant).reshape(-1), wq)
    del meta, quant, wm, wq, preq
    M = 16384
    packed, sc, bi = _asym_dev(M, K, 128, 3)
    got = repack_asymmetric_to_q4_128_blocks(packed, sc, bi, M, K)
    want = oracle.repack_asym_to_q4_128(_host(packed), _host(sc), _host(bi), M, K)
    assert np.array_equal(_host(got).reshape(-1), want)


def test_argument_errors(gpu):
    import torch
    from asdsl.quantization import _device_repack as dr
    from asdsl.quantization.repack import repack_preq_blocks_to_preq2

    with pytest.raises(ValueError, match="too small"):
        repack_preq_blocks_to_preq2(torch.zeros(100, dtype=torch.uint8, device="cuda"), 4, 64)
    with pytest.raises(ValueError, match="group_size=32"):
        repack_preq_blocks_to_preq2(torch.zeros(100, dtype=torch.uint8, device="cuda"), 1, 64, 128)
    with pytest.raises(ValueError, match="multiple of 128"):
        dr.fp32_to_q4_128(torch.zeros(256, device="cuda"), 2, 100)
    with pytest.raises(ValueError, match="scales"):
        dr.asym_to_preq2(torch.zeros(64, dtype=torch.uint8, device="cuda"), torch.zeros(1, device="cuda"),
                         torch.zeros(4, device="cuda"), 4, 32, 32)
