"""The *_ws entry points (caller-owned work buffer, no allocation by the
library) give the same bits as their library-buffer forms: the sparse
down-projection at several part counts, the batched preq2 GEMV on its MFMA
form, and the batched fp32-affine GEMMs (matmul_batch_q4, gemm_q4_128,
gemv_q4_packed and gemv_q4_avx2_gs64 with a batch).  The buffers come from
the *_work_bytes queries; a buffer too small is refused."""

from __future__ import annotations

import numpy as np
import pytest

from asdsl.quantization import synthetic as syn

pytestmark = pytest.mark.gpu


def _dev(a):
    import torch

    return torch.from_numpy(np.ascontiguousarray(a)).cuda()


def _same(a, b):
    return np.array_equal(a.cpu().numpy().view(np.uint32), b.cpu().numpy().view(np.uint32))


@pytest.mark.parametrize("n_active", [3, 40, 1662, 8192])
def test_sparse_down_ws_equals_library_buffer(gpu, n_active):
    import torch
    from asdsl import _hip

    IN, OUT, gs = 8192, 3072, 32
    rng = np.random.default_rng(n_active)
    wT = _dev(rng.integers(0, 256, IN * OUT // 2, dtype=np.uint8))
    sT = _dev((rng.random(IN * OUT // gs) * 0.01 + 1e-3).astype(np.float32))
    bT = -8.0 * sT
    x = np.zeros(IN, np.float32)
    rows = np.sort(rng.choice(IN, n_active, replace=False)).astype(np.int32)
    x[rows] = rng.random(n_active).astype(np.float32) + 0.1
    dx, dr = _dev(x), _dev(rows)
    y1 = torch.empty(OUT, device="cuda")
    y2 = torch.full((OUT,), float("nan"), device="cuda")
    nbytes = _hip.LIB.asdsl_sparse_down_work_bytes(OUT)
    work = torch.empty(nbytes, dtype=torch.uint8, device="cuda")
    s, P = _hip.stream_handle(), _hip.ptr
    _hip.call("asdsl_sparse_down_proj_T", P(wT), P(sT), P(bT), P(dx), P(dr), n_active, P(y1), IN, OUT, gs, s)
    _hip.call("asdsl_sparse_down_proj_T_ws", P(wT), P(sT), P(bT), P(dx), P(dr), n_active, P(y2), IN, OUT, gs,
              P(work), nbytes, s)
    torch.cuda.synchronize()
    assert _same(y1, y2)
    with pytest.raises(ValueError, match="work buffer"):
        _hip.call("asdsl_sparse_down_proj_T_ws", P(wT), P(sT), P(bT), P(dx), P(dr), n_active, P(y2), IN, OUT, gs,
                  P(work), nbytes - 4, s)


@pytest.mark.parametrize("M,K,N", [(16384, 3072, 16), (3072, 8192, 5)])
def test_preq2_batch_ws_equals_library_buffer(gpu, M, K, N):
    import torch
    from asdsl import _hip

    g = torch.Generator(device="cuda").manual_seed(M + N)
    w = torch.randn((M, K), generator=g, device="cuda") * 0.02
    meta, quant = syn.preq2_from_weights_torch(w, 32)
    del w
    X = _dev(syn.activation(K, 9, batch=N))
    Y1 = torch.empty((N, M), device="cuda")
    Y2 = torch.full((N, M), float("nan"), device="cuda")
    nbytes = _hip.LIB.asdsl_gemv_preq2_fused_batch_work_bytes(K)
    work = torch.empty(nbytes, dtype=torch.uint8, device="cuda")
    s, P = _hip.stream_handle(), _hip.ptr
    _hip.call("asdsl_gemv_preq2_fused_batch", P(meta), P(quant), P(X), P(Y1), M, K, 32, N, s)
    _hip.call("asdsl_gemv_preq2_fused_batch_ws", P(meta), P(quant), P(X), P(Y2), M, K, 32, N, P(work), nbytes, s)
    torch.cuda.synchronize()
    assert _same(Y1, Y2)


@pytest.mark.parametrize("M,K,gs,B", [(16384, 3072, 32, 4), (3072, 8192, 128, 16), (4096, 4096, 64, 3)])
def test_affine_batch_ws_equals_library_buffer(gpu, M, K, gs, B):
    import torch
    from asdsl import _hip

    rng = np.random.default_rng(M + K + B)
    w = _dev(rng.integers(0, 256, M * K // 2, dtype=np.uint8))
    sc = _dev((rng.random(M * K // gs) * 0.01).astype(np.float32))
    bi = _dev((rng.random(M * K // gs) * 0.1 - 0.05).astype(np.float32))
    X = _dev(rng.standard_normal((B, K)).astype(np.float32))
    nbytes = _hip.LIB.asdsl_affine_batch_work_bytes(M, K, gs)
    assert nbytes > 0
    work = torch.empty(nbytes, dtype=torch.uint8, device="cuda")
    s, P = _hip.stream_handle(), _hip.ptr
    Y1 = torch.empty((B, M), device="cuda")
    Y2 = torch.full((B, M), float("nan"), device="cuda")
    _hip.call("asdsl_matmul_batch_q4", P(w), P(sc), P(bi), P(X), P(Y1), M, K, B, gs, s)
    _hip.call("asdsl_matmul_batch_q4_ws", P(w), P(sc), P(bi), P(X), P(Y2), M, K, B, gs, P(work), nbytes, s)
    torch.cuda.synchronize()
    assert _same(Y1, Y2)
    Y3 = torch.full((B, M), float("nan"), device="cuda")
    _hip.call("asdsl_gemv_q4_packed_ws", P(w), P(X), P(sc), P(bi), P(Y3), M, K, gs, B, P(work), nbytes, s)
    torch.cuda.synchronize()
    assert _same(Y1, Y3)
    if gs == 64:
        Y4 = torch.empty((B, M), device="cuda")
        Y5 = torch.full((B, M), float("nan"), device="cuda")
        _hip.call("asdsl_gemv_q4_gs64", P(w), P(X), P(sc), P(Y4), M, K, B, s)
        _hip.call("asdsl_gemv_q4_gs64_ws", P(w), P(X), P(sc), P(Y5), M, K, B, P(work), nbytes, s)
        torch.cuda.synchronize()
        assert _same(Y4, Y5)


def test_gemm_q4_128_ws_equals_library_buffer(gpu):
    import torch
    from asdsl import _hip

    M, K, B = 16384, 3072, 8
    g = torch.Generator(device="cuda").manual_seed(5)
    w = torch.randn((M, K), generator=g, device="cuda") * 0.02
    blocks = syn.q4_128_from_weights_torch(w)
    del w
    X = _dev(syn.activation(K, 10, batch=B))
    nbytes = _hip.LIB.asdsl_affine_batch_work_bytes(M, K, 128)
    work = torch.empty(nbytes, dtype=torch.uint8, device="cuda")
    s, P = _hip.stream_handle(), _hip.ptr
    Y1 = torch.empty((B, M), device="cuda")
    Y2 = torch.full((B, M), float("nan"), device="cuda")
    _hip.call("asdsl_gemm_q4_128", P(blocks), P(X), P(Y1), M, K, 128, B, s)
    _hip.call("asdsl_gemm_q4_128_ws", P(blocks), P(X), P(Y2), M, K, 128, B, P(work), nbytes, s)
    torch.cuda.synchronize()
    assert _same(Y1, Y2)
