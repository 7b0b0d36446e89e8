"""The timing build (lib/libasdsl_hip_timeline.so, -DASDSL_WG_TIMELINE): it
exports the product's entry points plus the timeline hook, the product build
does not export the hook, and on a GPU its per-workgroup stamps describe the
decode step's kernels in launch order."""

from __future__ import annotations

import ctypes
import json
import os
import subprocess
import sys

import pytest

from conftest import REPO
from test_abi import declared_entry_points

TIMELINE_LIB = REPO / "asdsl-framework_amd" / "lib" / "libasdsl_hip_timeline.so"

needs_timing_build = pytest.mark.skipif(not TIMELINE_LIB.exists(), reason="timing build not built")


@needs_timing_build
def test_timing_build_exports_the_product_api_and_the_hook():
    lib = ctypes.CDLL(str(TIMELINE_LIB))
    missing = [n for n in declared_entry_points() if not hasattr(lib, n)]
    assert not missing, f"timing build lacks: {missing}"
    assert hasattr(lib, "asdsl_timeline_set_buffer")


def test_product_build_has_no_timeline_hook():
    from asdsl import _hip

    assert not _hip.exported("asdsl_timeline_set_buffer")


def _timeline(contexts, layers=2):
    env = dict(os.environ, ASDSL_HIP_LIB=str(TIMELINE_LIB))
    cmd = [sys.executable, str(REPO / "bench.py"), "--decode-timeline", *map(str, contexts),
           "--timeline-layers", str(layers)]
    res = subprocess.run(cmd, env=env, capture_output=True, text=True, timeout=300, cwd=REPO)
    assert res.returncode == 0, res.stderr[-2000:]
    return [json.loads(line)["decode_timeline"] for line in res.stdout.splitlines() if "decode_timeline" in line]


@pytest.mark.gpu
@needs_timing_build
def test_timeline_orders_the_layer_kernels():
    """ctx 100: the short form (qkv, attention, o_proj merging the splits,
    gate_up, down); ctx 600: the long form, whose combine runs before a plain
    o_proj.  Kernels follow each other without overlap, every phase is
    non-negative, and the workgroup counts are the launches' (Phi-4 shape)."""
    short, long_ = _timeline([100, 600])
    assert [k["kernel"] for k in short["kernels"]] == [
        "qkv (norm)", "attention", "o_proj (split merge)", "gate_up (SwiGLU)", "down"]
    assert [k["kernel"] for k in long_["kernels"]] == [
        "qkv (norm)", "attention", "attention combine", "o_proj", "gate_up (SwiGLU)", "down"]
    for tl in (short, long_):
        ks = tl["kernels"]
        assert ks[0]["first_start_us"] == 0.0
        for prev, k in zip(ks, ks[1:]):
            assert k["gap_us"] >= 0.0 and k["first_start_us"] >= prev["last_end_us"]
        for k in ks:
            assert k["last_end_us"] > k["first_start_us"]
            for name, v in k.items():
                if name.endswith("_us") and isinstance(v, list):
                    assert 0.0 <= v[0] <= v[1], (k["kernel"], name, v)
    wgs = {k["kernel"]: k["workgroups"] for k in short["kernels"]}
    assert wgs["qkv (norm)"] == 160 and wgs["gate_up (SwiGLU)"] == 256 and wgs["down"] == 256
    assert wgs["attention"] == 2 * 8  # position 108: two splits of 64, eight KV heads
    wgs = {k["kernel"]: k["workgroups"] for k in long_["kernels"]}
    assert wgs["attention"] == 10 * 8 and wgs["attention combine"] == 24  # position 608: ten splits
