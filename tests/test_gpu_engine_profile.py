"""Per-stage timing of the decode step: the stage recorder of the C ABI
(asdsl_profile_stages_begin/_end) and the engine's ASDSL_ENGINE_PROFILE
report, the counterpart of the reference's
(asdsl/kernels/native/unified_engine.cpp:58-95, 1668-1687)."""

from __future__ import annotations

import ctypes
import subprocess
import sys

import pytest

from asdsl import _hip
from conftest import REPO


def test_stage_recorder_argument_errors():
    """Checked before any HIP call, so these run without a device."""
    labels = (ctypes.c_char_p * 4)()
    ms = (ctypes.c_float * 4)()
    count, span = ctypes.c_int(0), ctypes.c_float(0.0)
    st = _hip.LIB.asdsl_profile_stages_end(4, labels, ms, ctypes.byref(count), ctypes.byref(span))
    assert st == _hip.ASDSL_ERR_INVALID_ARGUMENT and "not armed" in _hip.last_error()
    for bad in (0, -1, 65537):
        assert _hip.LIB.asdsl_profile_stages_begin(bad) == _hip.ASDSL_ERR_INVALID_ARGUMENT
        assert "max_launches" in _hip.last_error()


def _engine(ctx, monkeypatch, token):
    from asdsl.engine import DecodeConfig, DecodeEngine

    monkeypatch.setenv("ASDSL_ENGINE_PROFILE", "1")
    monkeypatch.setenv("ASDSL_ENGINE_PROFILE_TOKEN", str(token))
    eng = DecodeEngine.synthetic(DecodeConfig(n_layers=2, vocab=4096, max_seq=1024), seed=4)
    eng.prefill_kv_random(ctx, seed=5)
    return eng


@pytest.mark.gpu
@pytest.mark.parametrize("ctx,per_layer", [(100, 5), (600, 6)])
def test_profiled_step_keeps_the_replayed_bits(gpu, monkeypatch, capsys, ctx, per_layer):
    """Four greedy steps from ctx with the third profiled (run eagerly with
    its launches timed) against the same four steps replayed from a graph:
    bitwise equal logits and tokens.  The profile holds every stage of the
    step's form (the combine from 512 positions on), one launch per stage
    and layer, positive durations, and a span no shorter than the kernels it
    covers, which run one after another on the stream."""
    import torch

    eng = _engine(ctx, monkeypatch, token=3)
    snap = [(L["k_cache"].clone(), L["v_cache"].clone()) for L in eng.layers]
    runs = []
    for profiled in (True, False):
        for L, (k, v) in zip(eng.layers, snap):
            L["k_cache"].copy_(k)
            L["v_cache"].copy_(v)
        eng.token.fill_(21)
        eng.pos.fill_(ctx)
        eng._host_pos = ctx
        eng._decode_idx = 0
        if not profiled:
            eng._profile_token = None
        out = []
        for _ in range(4):
            eng.step()
            torch.cuda.synchronize()
            out.append((eng.logits.clone(), eng.next_token()))
        runs.append(out)
        assert int(eng.pos.item()) == ctx + 4 and eng._host_pos == ctx + 4
    for (la, ta), (lb, tb) in zip(*runs):
        assert torch.equal(la, lb) and ta == tb

    prof = eng.last_profile
    assert prof["token"] == 3
    want = {"qkv", "attention", "o_proj", "gate_up", "down", "lm_head", "finalize"}
    if per_layer == 6:
        want.add("attention_combine")
    st = prof["stages_ms"]
    assert set(st) == want
    assert prof["launches"] == per_layer * 2 + 2
    assert all(v > 0.0 for v in st.values())
    assert prof["span_ms"] >= sum(st.values()) * (1 - 1e-3)
    err = capsys.readouterr().err
    assert "[ASDSL_ENGINE_PROFILE] decode token 3 (ms, 2 layers):" in err
    for key in ("gate_up_gemv", "down_gemv", "qkv_gemv", "o_gemv", "activation_q8", "prep_fused", "lm_head",
                "other", "total"):
        assert f"\n  {key} " in err


@pytest.mark.gpu
def test_forward_token_profiled_and_launch_limit(gpu, monkeypatch, capsys):
    """forward_token counts toward the target token like step(); a recorder
    armed for fewer launches than a step makes reports that from end."""
    eng = _engine(50, monkeypatch, token=1)
    eng.forward_token(7, 50)
    assert eng.last_profile["token"] == 1 and eng.last_profile["launches"] == 12
    assert "decode token 1" in capsys.readouterr().err
    with pytest.raises(ValueError, match="12 launches, 3 recorded"):
        _hip.profile_stages(lambda: eng._queue_step(_hip.stream_handle(), 256), max_launches=3)


_LOAD_ORDER = """
import sys
sys.path.insert(0, {pkg!r})
from asdsl import _hip          # the library first, torch after it
import torch
x = torch.ones(4, device="cuda")
assert _hip.cu_count() > 0
print("ok")
"""


@pytest.mark.gpu
def test_library_imported_before_torch(gpu):
    """Importing the library before torch leaves one HIP runtime in the
    process: the library's device calls work beside torch's tensors."""
    res = subprocess.run([sys.executable, "-c", _LOAD_ORDER.format(pkg=str(REPO / "asdsl-framework_amd"))],
                         capture_output=True, text=True, timeout=300)
    assert res.returncode == 0 and res.stdout.strip().endswith("ok"), res.stderr[-2000:]


@pytest.mark.gpu
def test_explicit_launch_events_while_recording_are_reported(gpu, monkeypatch):
    """A launch that takes the pair armed by asdsl_profile_next_launch is
    not recorded by the stage recorder; end says so instead of returning a
    partial profile, and the explicit events still time that launch."""
    import torch

    eng = _engine(50, monkeypatch, token=0)
    start, stop = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    start.record()  # torch creates the HIP events at their first record
    stop.record()
    torch.cuda.synchronize()
    assert start.cuda_event and stop.cuda_event

    def run():
        _hip.check(_hip.LIB.asdsl_profile_next_launch(ctypes.c_void_p(start.cuda_event),
                                                      ctypes.c_void_p(stop.cuda_event)), "next_launch")
        eng._queue_step(_hip.stream_handle(), 256)

    with pytest.raises(ValueError, match="asdsl_profile_next_launch"):
        _hip.profile_stages(run, max_launches=64)
    torch.cuda.synchronize()
    assert start.elapsed_time(stop) > 0.0
