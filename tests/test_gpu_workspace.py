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


_RESERVE_CHILD = r'''
import sys
import numpy as np
import torch
from asdsl import _hip

s, P = _hip.stream_handle(), _hip.ptr
LIB = _hip.LIB


def case(IN, OUT, gs, n_active, seed):
    rng = np.random.default_rng(seed)
    dev = lambda a: torch.from_numpy(np.ascontiguousarray(a)).cuda()  # noqa: E731
    wT = dev(rng.integers(0, 256, IN * OUT // 2, dtype=np.uint8))
    sT = dev((rng.random(IN * OUT // gs) * 0.01 + 1e-3).astype(np.float32))
    bT = -8.0 * sT
    x = np.zeros(IN, np.float32)
    rows = np.sort(rng.choice(IN, n_active, replace=False)).astype(np.int32)
    x[rows] = rng.random(n_active).astype(np.float32) + 0.1
    return wT, sT, bT, dev(x), dev(rows)


def plain(args, n_active, y, IN, OUT, gs, stream=None):
    wT, sT, bT, x, rows = args
    return LIB.asdsl_sparse_down_proj_T(P(wT), P(sT), P(bT), P(x), P(rows), n_active, P(y), IN, OUT, gs,
                                        s if stream is None else stream)


def same(a, b):
    return np.array_equal(a.cpu().numpy().view(np.uint32), b.cpu().numpy().view(np.uint32))


small = (2048, 1024, 32, 1500)
big = (2048, 16384, 32, 2048)
need_small = LIB.asdsl_sparse_down_work_bytes(small[1])
assert LIB.asdsl_reserve_workspace(need_small) == 0, _hip.last_error()

# within the reservation: the plain form runs and gives the _ws form's bits
a = case(*small, seed=1)
y1 = torch.empty(small[1], device="cuda")
y2 = torch.full((small[1],), float("nan"), device="cuda")
work = torch.empty(need_small, dtype=torch.uint8, device="cuda")
assert plain(a, small[3], y1, *small[:3]) == 0, _hip.last_error()
wT, sT, bT, x, rows = a
assert LIB.asdsl_sparse_down_proj_T_ws(P(wT), P(sT), P(bT), P(x), P(rows), small[3], P(y2), small[0], small[1],
                                       small[2], P(work), need_small, s) == 0
torch.cuda.synchronize()
assert same(y1, y2)

# and under graph capture, replayed three times with eager work between
yg = torch.full((small[1],), float("nan"), device="cuda")
g = torch.cuda.CUDAGraph()
with torch.cuda.graph(g):
    st = plain(a, small[3], yg, *small[:3], stream=int(torch.cuda.current_stream().cuda_stream))
assert st == 0, _hip.last_error()
for _ in range(3):
    yg.fill_(float("nan"))
    torch.cuda.synchronize()
    g.replay()
    torch.cuda.synchronize()
    assert same(yg, y1)

# beyond it: refused, nothing allocated
b = case(*big, seed=2)
yb = torch.empty(big[1], device="cuda")
st = plain(b, big[3], yb, *big[:3])
assert st == _hip.ASDSL_ERR_INVALID_ARGUMENT, st
assert "reserved" in _hip.last_error(), _hip.last_error()

# 0 returns to growth on demand
assert LIB.asdsl_reserve_workspace(0) == 0
assert plain(b, big[3], yb, *big[:3]) == 0, _hip.last_error()
torch.cuda.synchronize()
print("RESERVE_OK")
'''


def test_reserved_workspace_never_grows(gpu):
    """asdsl_reserve_workspace, in a fresh process (the library buffer is
    per process and earlier tests grow it): after reserving the sparse
    down-projection's need at 1024 outputs, the plain form runs within it
    with the _ws form's bits, also captured in a graph and replayed; the
    same call at 16384 outputs, which needs more, is refused with
    ASDSL_ERR_INVALID_ARGUMENT instead of allocating; reserving 0 returns to
    growth on demand."""
    import os
    import subprocess
    import sys

    from conftest import REPO

    env = dict(os.environ, PYTHONPATH=os.pathsep.join([str(REPO), str(REPO / "asdsl-framework_amd")]))
    r = subprocess.run([sys.executable, "-c", _RESERVE_CHILD], capture_output=True, text=True, timeout=240, env=env)
    assert r.returncode == 0 and "RESERVE_OK" in r.stdout, (r.stdout[-2000:], r.stderr[-4000:])
