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
    """Real device buffers sized for the refused shape, so that the refusal
    does not depend on the order of the argument checks."""
    import torch
    from asdsl import _hip

    IN, OUT, gs, n = 8, 16384 + 32, 32, 4
    wT = torch.zeros(IN * OUT // 2, dtype=torch.uint8, device="cuda")
    sT = torch.ones(IN * OUT // gs, device="cuda")
    bT = torch.zeros(IN * OUT // gs, device="cuda")
    x = torch.ones(IN, device="cuda")
    rows = torch.arange(n, dtype=torch.int32, device="cuda")
    y = torch.empty(OUT, device="cuda")
    P = _hip.ptr
    st = _hip.LIB.asdsl_sparse_down_proj_T_noalloc(P(wT), P(sT), P(bT), P(x), P(rows), n, P(y), IN, OUT, gs,
                                                   _hip.stream_handle())
    assert st == _hip.ASDSL_ERR_INVALID_ARGUMENT
    assert "exceeds" in _hip.last_error()


def test_noalloc_under_graph_capture(gpu):
    """The entry point inside a captured graph with more than one part (its
    partial rows in the static array): three replays, with eager work and
    synchronizations between them, each bit for bit the eager result.  An
    entry point that allocated on first use could not be captured fresh."""
    import torch
    from asdsl import _hip

    s, P = _hip.stream_handle(), _hip.ptr
    IN, OUT, gs, n_active = 8192, 3072, 32, 1662
    wT, sT, bT, x, rows = _case(IN, OUT, gs, n_active, 3)
    want = torch.empty(OUT, device="cuda")
    _hip.call("asdsl_sparse_down_proj_T_noalloc", P(wT), P(sT), P(bT), P(x), P(rows), n_active, P(want), IN, OUT,
              gs, s)
    torch.cuda.synchronize()
    got = torch.full((OUT,), float("nan"), device="cuda")
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        st = _hip.LIB.asdsl_sparse_down_proj_T_noalloc(P(wT), P(sT), P(bT), P(x), P(rows), n_active, P(got), IN,
                                                       OUT, gs, int(torch.cuda.current_stream().cuda_stream))
    assert st == 0, _hip.last_error()
    for i in range(3):
        got.fill_(float("nan"))
        (x * 2.0).sum()  # eager work between replays
        torch.cuda.synchronize()
        g.replay()
        torch.cuda.synchronize()
        assert np.array_equal(got.cpu().numpy().view(np.uint32), want.cpu().numpy().view(np.uint32)), i
