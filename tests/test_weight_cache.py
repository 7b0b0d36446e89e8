"""The reference's weight-cache files (CPU): the preq block cache
(``phi4_preq_blocks_v1``, experiments/phi4_cpu_run.py:627-780) and the
lm_head preq2 cache (``phi4_lmhead_preq2_v1``,
asdsl/quantization/lmhead_preq2_cache.py).  Round trips restore the same
bytes; every field the reference validates rejects a mismatching file, as the
reference's round-trip test expects (benchmarks/test_preq_cache_roundtrip.py)."""

from __future__ import annotations

import json
from types import SimpleNamespace

import numpy as np
import pytest

from asdsl.quantization import lmhead_preq2_cache as lc
from asdsl.quantization import preq_cache as pc
from asdsl.quantization.repack import repack_asymmetric_to_q4_32_blocks


def _store(gs=32):
    rng = np.random.default_rng(gs)
    st = pc.PreqStore(group_size=gs)
    shapes = {(0, "gate_up_proj"): (64, 3072), (0, "o_proj"): (8, 256), (1, "qkv_proj"): (12, 512)}
    st._quant_shapes = dict(shapes)
    bs = pc.block_size_for(gs)
    for k, (r, c) in shapes.items():
        st._preq_blocks_np[k] = rng.integers(0, 256, r * (c // gs) * bs, dtype=np.uint8)
    return st


@pytest.mark.parametrize("gs", [32, 128])
def test_preq_cache_round_trip(tmp_path, gs):
    st = _store(gs)
    path = tmp_path / "preq.safetensors"
    pc.save_preq_cache(st, path)
    st2 = pc.PreqStore(group_size=gs, _quant_shapes=dict(st._quant_shapes))
    assert pc.try_restore_preq_cache(st2, path)
    assert st2._preq_built and set(st2._preq_blocks_np) == set(st._preq_blocks_np)
    for k, v in st._preq_blocks_np.items():
        assert np.array_equal(st2._preq_blocks_np[k], v)


def test_preq_cache_metadata_is_the_reference_layout(tmp_path):
    """format, block_size and the quantization config as strings; the shape
    map a JSON object of "layer|name": [rows, cols] with sorted keys."""
    from safetensors import safe_open

    st = _store(32)
    path = tmp_path / "preq.safetensors"
    pc.save_preq_cache(st, path)
    with safe_open(str(path), framework="np") as f:
        md = f.metadata()
        keys = sorted(f.keys())
    assert md["format"] == "phi4_preq_blocks_v1" and md["block_size"] == "20"
    assert md["bits"] == "4" and md["group_size"] == "32" and md["symmetric"] == "False"
    assert md["sparsity_threshold"] == "0.01" and md["enable_qcsd"] == "False"
    assert json.loads(md["quant_shapes"]) == {"0|gate_up_proj": [64, 3072], "0|o_proj": [8, 256],
                                              "1|qkv_proj": [12, 512]}
    assert list(json.loads(md["quant_shapes"])) == sorted(json.loads(md["quant_shapes"]))
    assert keys == ["L0_gate_up_proj", "L0_o_proj", "L1_qkv_proj"]


def test_preq_cache_rejects_mismatches(tmp_path):
    st = _store(32)
    path = tmp_path / "preq.safetensors"
    pc.save_preq_cache(st, path)
    fresh = lambda **kw: pc.PreqStore(**{"group_size": 32, "_quant_shapes": dict(st._quant_shapes), **kw})  # noqa: E731
    assert not pc.try_restore_preq_cache(fresh(), tmp_path / "missing.safetensors")
    assert not pc.try_restore_preq_cache(fresh(group_size=128), path)           # block size / group size
    assert not pc.try_restore_preq_cache(fresh(bits=3), path)                   # quant config
    assert not pc.try_restore_preq_cache(fresh(_symmetric=True), path)
    assert not pc.try_restore_preq_cache(fresh(_sparsity_threshold=0.02), path)
    other = dict(st._quant_shapes)
    other[(2, "down_proj")] = (4, 256)
    assert not pc.try_restore_preq_cache(fresh(_quant_shapes=other), path)      # projection set
    # a tensor whose byte count does not match its recorded shape
    bad = _store(32)
    bad._preq_blocks_np[(0, "o_proj")] = bad._preq_blocks_np[(0, "o_proj")][:-20]
    pc.save_preq_cache(bad, tmp_path / "bad.safetensors")
    st3 = fresh()
    assert not pc.try_restore_preq_cache(st3, tmp_path / "bad.safetensors") and not st3._preq_blocks_np
    # another format tag
    import safetensors.numpy as st_np

    st_np.save_file({"L0_o_proj": np.zeros(8, np.uint8)}, str(tmp_path / "x.safetensors"),
                    metadata={"format": "phi4_cpu_weights_v1", "block_size": "20"})
    assert not pc.try_restore_preq_cache(fresh(), tmp_path / "x.safetensors")


def test_preq_cache_of_repacked_weights(tmp_path):
    """The reference's round-trip case: 64 x 3072 gate_up weights quantized
    and repacked to preq blocks, saved and restored byte for byte."""
    rows, cols = 64, 3072
    rng = np.random.default_rng(0)
    q = rng.integers(0, 16, (rows, cols), dtype=np.uint8)
    packed = ((q[:, 1::2] << 4) | q[:, 0::2]).astype(np.uint8)
    sc = rng.uniform(0.001, 0.01, (rows, cols // 32)).astype(np.float32)
    bi = rng.uniform(-0.05, 0.0, (rows, cols // 32)).astype(np.float32)
    blocks = repack_asymmetric_to_q4_32_blocks(packed, sc, bi, rows, cols).reshape(-1)
    st = pc.PreqStore(_quant_shapes={(0, "gate_up_proj"): (rows, cols)})
    st._preq_blocks_np[(0, "gate_up_proj")] = blocks
    pc.save_preq_cache(st, tmp_path / "p.safetensors")
    st2 = pc.PreqStore(_quant_shapes=dict(st._quant_shapes))
    assert pc.try_restore_preq_cache(st2, tmp_path / "p.safetensors")
    assert np.array_equal(st2._preq_blocks_np[(0, "gate_up_proj")], blocks)


def test_lmhead_cache_round_trip_and_rejects(tmp_path, monkeypatch):
    monkeypatch.delenv("ASDSL_LMHEAD_GS", raising=False)
    monkeypatch.delenv("PHI4_NO_LMHEAD_PREQ2_CACHE", raising=False)
    store = SimpleNamespace(group_size=32, lm_head=np.zeros((10, 256), np.float32))
    _, _, _, mb, qb = lc._expected_sizes(store)
    assert (mb, qb) == (10 * 8 * 4, 3 * 8 * 64)
    rng = np.random.default_rng(1)
    meta, quant = rng.integers(0, 256, mb, dtype=np.uint8), rng.integers(0, 256, qb, dtype=np.uint8)
    path = tmp_path / "lm.safetensors"
    lc.save_lmhead_preq2_cache(store, path, meta, quant)
    got = lc.try_restore_lmhead_preq2_cache(store, path)
    assert got is not None and np.array_equal(got[0], meta) and np.array_equal(got[1], quant)
    # vocab, hidden and group size are each checked
    assert lc.try_restore_lmhead_preq2_cache(SimpleNamespace(group_size=32, lm_head=np.zeros((11, 256))), path) is None
    assert lc.try_restore_lmhead_preq2_cache(SimpleNamespace(group_size=32, lm_head=np.zeros((10, 512))), path) is None
    monkeypatch.setenv("ASDSL_LMHEAD_GS", "128")
    assert lc.try_restore_lmhead_preq2_cache(store, path) is None
    monkeypatch.delenv("ASDSL_LMHEAD_GS")
    monkeypatch.setenv("PHI4_NO_LMHEAD_PREQ2_CACHE", "1")
    assert lc.try_restore_lmhead_preq2_cache(store, path) is None
    monkeypatch.delenv("PHI4_NO_LMHEAD_PREQ2_CACHE")
    with pytest.raises(ValueError, match="size mismatch"):
        lc.save_lmhead_preq2_cache(store, path, meta[:-1], quant)


def test_lmhead_cache_g128_sizes(monkeypatch):
    """At group size 128 the blobs are preq2-g128: 256 bytes per band and group."""
    monkeypatch.setenv("ASDSL_LMHEAD_GS", "128")
    store = SimpleNamespace(group_size=32, lm_head=None)
    assert lc._expected_sizes(store) == (200064, 3072, 128, 200064 * 24 * 4, 50016 * 24 * 256)
