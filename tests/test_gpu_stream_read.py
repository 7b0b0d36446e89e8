"""The calibration read kernel (asdsl_stream_read): it reads without writing
(the sink keeps its value unless the loaded words fold to the sentinel) and
validates its arguments like every other entry point."""

from __future__ import annotations

import pytest

pytestmark = pytest.mark.gpu


def test_reads_without_writing_and_validates(gpu):
    import torch
    from asdsl import _hip

    buf = torch.arange(1 << 20, dtype=torch.int32, device="cuda")  # 4 MiB
    sink = torch.full((1,), 7, dtype=torch.int32, device="cuda")
    for grid in (0, 3, 1024):
        _hip.call("asdsl_stream_read", _hip.ptr(buf), buf.numel() * 4, _hip.ptr(sink), grid, _hip.stream_handle())
    torch.cuda.synchronize()
    assert int(sink.item()) == 7  # the words fold to a value other than the sentinel
    with pytest.raises(ValueError, match="multiple of 16"):
        _hip.call("asdsl_stream_read", _hip.ptr(buf), 20, _hip.ptr(sink), 0, _hip.stream_handle())
    with pytest.raises(ValueError, match="null pointer"):
        _hip.call("asdsl_stream_read", None, 64, _hip.ptr(sink), 0, _hip.stream_handle())
