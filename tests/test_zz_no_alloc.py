"""asdsl_sparse_down_proj_T_noalloc, the entry point that allocates nothing
(its partial rows live in the library's static device array), through the C
ABI: the same bits as asdsl_sparse_down_proj_T on two calls in a row, the
second smaller (fewer listed rows and fewer outputs) than the first, both
with enough rows that the partial rows are used; and sizes beyond the array
refused."""

from __future__ import annotations

import numpy as np
import pytest

pytestmark = pytest.mark.gpu


def _dev(a):
    import torch

    return torch.from_numpy(np.ascontiguousarray(a)).cuda()


def _case(IN, OUT, gs, n_active, seed):
    rng = np.random.default_rng(seed)
    wT = rng.integers(0, 256, IN * OUT // 2, dtype=np.uint8)
    sT = (rng.random(IN * OUT // gs) * 0.01 + 1e-3).astype(np.float32)
    bT = (-8.0 * sT).astype(np.float32)
    x = np.zeros(IN, np.float32)
    rows = np.sort(rng.choice(IN, n_active, replace=False)).astype(np.int32)
    x[rows] = (rng.random(n_active) + 0.1).astype(np.float32)
    return [_dev(a) for a in (wT, sT, bT, x, rows)]


def test_noalloc_matches_allocating_entry_twice_then_smaller(gpu):
    import torch
    from asdsl import _hip

    s, P = _hip.stream_handle(), _hip.ptr
    for IN, OUT, gs, n_active, seed in [(8192, 3072, 32, 1662, 1), (2048, 1024, 64, 200, 2)]:
        wT, sT, bT, x, rows = _case(IN, OUT, gs, n_active, seed)
        want = torch.empty(OUT, device="cuda")
        got = torch.full((OUT,), float("nan"), device="cuda")
        _hip.call("asdsl_sparse_down_proj_T", P(wT), P(sT), P(bT), P(x), P(rows), n_active, P(want), IN, OUT, gs, s)
        _hip.call("asdsl_sparse_down_proj_T_noalloc", P(wT), P(sT), P(bT), P(x), P(rows), n_active, P(got), IN, OUT,
                  gs, s)
        torch.cuda.synchronize()
        assert np.array_equal(got.cpu().numpy().view(np.uint32), want.cpu().numpy().view(np.uint32)), (OUT, n_active)


def test_noalloc_refuses_outputs_beyond_its_array(gpu):
    from asdsl import _hip

    one = 256
    st = _hip.LIB.asdsl_sparse_down_proj_T_noalloc(one, one, one, one, one, 4, one, 8, 16384 + 32, 32, None)
    assert st == _hip.ASDSL_ERR_INVALID_ARGUMENT
    assert "exceeds" in _hip.last_error()
