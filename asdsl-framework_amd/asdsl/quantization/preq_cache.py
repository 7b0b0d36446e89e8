"""The preq block cache file (format ``phi4_preq_blocks_v1``), read and
written as the reference does (experiments/phi4_cpu_run.py: format and
projection names 627-628, _preq_tensor_key 711-719, the quantization-config
metadata 666-708, try_restore_preq_cache 722-764, save_preq_cache 767-780):
one safetensors file with a uint8 tensor ``L{layer}_{projection}`` of preq
blocks per projection (20-byte Q4_32 blocks at group size 32, 66-byte
Q4_128 blocks at 128), metadata ``format``, ``block_size`` and the store's
quantization config, all checked before the blocks are used.

The store is duck-typed like the reference's WeightStore: ``group_size``,
``bits``, ``_quant_shapes`` {(layer, name): (rows, cols)} and the optional
config attributes; restored blocks land in ``_preq_blocks_np`` (host) or,
with ``device=``, in ``_preq_blocks_dev`` as device tensors, read from the
file once and copied to the GPU with no host-side repack.
:func:`preq2_from_preq_blocks` then builds the preq2 / preq2-g128 operands
of the decode GEMVs on the device.
"""

from __future__ import annotations

import json
import math
from dataclasses import dataclass, field
from pathlib import Path
from typing import Any

import numpy as np

PREQ_CACHE_FORMAT = "phi4_preq_blocks_v1"
PROJ_NAMES = ("qkv_proj", "o_proj", "gate_up_proj", "down_proj")
_BLOCK_SIZE = {32: 20, 128: 66}


@dataclass
class PreqStore:
    """The fields of the reference's WeightStore that the preq cache reads."""

    bits: int = 4
    group_size: int = 32
    _quant_shapes: dict = field(default_factory=dict)
    _preq_blocks_np: dict = field(default_factory=dict)
    _preq_blocks_dev: dict = field(default_factory=dict)
    _preq_built: bool = False
    _enable_qcsd: bool = False
    _draft_bits: int = 2
    _draft_group_size: int = 32
    _enable_sparse: bool = False
    _sparsity_threshold: float = 0.01
    _symmetric: bool = False
    _optimize_clips: bool = False


def block_size_for(group_size: int) -> int:
    try:
        return _BLOCK_SIZE[group_size]
    except KeyError:
        raise ValueError(f"preq cache: group_size must be 32 or 128, got {group_size}") from None


def _preq_tensor_key(layer: int, name: str) -> str:
    return f"L{layer}_{name}"


def _parse_preq_tensor_key(key: str) -> tuple[int, str]:
    if not key.startswith("L"):
        raise ValueError(f"invalid preq cache key: {key!r}")
    layer_s, _, name = key[1:].partition("_")
    return int(layer_s), name


def _shape_map_to_json(shapes: dict) -> str:
    """{(layer, name): (rows, cols)} as the JSON object the reference writes:
    keys "layer|name", values [rows, cols], keys sorted (phi4_cpu_run.py:373-375)."""
    return json.dumps({f"{li}|{nm}": [int(r), int(c)] for (li, nm), (r, c) in shapes.items()}, sort_keys=True)


def _shape_map_from_json(text: str) -> dict:
    out = {}
    for k, v in json.loads(text).items():
        li, nm = k.split("|", 1)
        out[(int(li), nm)] = (int(v[0]), int(v[1]))
    return out


def _quantize_config_meta(store: Any) -> dict[str, str]:
    return {
        "bits": str(store.bits),
        "group_size": str(store.group_size),
        "enable_qcsd": str(getattr(store, "_enable_qcsd", False)),
        "draft_bits": str(getattr(store, "_draft_bits", 2)),
        "draft_group_size": str(getattr(store, "_draft_group_size", 32)),
        "enable_sparse": str(getattr(store, "_enable_sparse", False)),
        "sparsity_threshold": json.dumps(getattr(store, "_sparsity_threshold", 0.01)),
        "symmetric": str(getattr(store, "_symmetric", False)),
        "optimize_clips": str(getattr(store, "_optimize_clips", False)),
        "quant_shapes": _shape_map_to_json(store._quant_shapes),
    }


def _meta_sparsity_value(text: str) -> float:
    try:
        return float(json.loads(text))
    except (json.JSONDecodeError, TypeError, ValueError):
        return float(text)


def _quantize_config_matches(store: Any, md: dict | None) -> bool:
    if not md or "quant_shapes" not in md:
        return False
    try:
        if _shape_map_from_json(md["quant_shapes"]) != dict(store._quant_shapes):
            return False
        return all([
            int(md["bits"]) == store.bits,
            int(md["group_size"]) == store.group_size,
            md.get("enable_qcsd", "False") == str(getattr(store, "_enable_qcsd", False)),
            int(md.get("draft_bits", "2")) == getattr(store, "_draft_bits", 2),
            int(md.get("draft_group_size", "32")) == getattr(store, "_draft_group_size", 32),
            md.get("enable_sparse", "False") == str(getattr(store, "_enable_sparse", False)),
            math.isclose(_meta_sparsity_value(md.get("sparsity_threshold", "0.01")),
                         float(getattr(store, "_sparsity_threshold", 0.01)), rel_tol=0.0, abs_tol=1e-9),
            md.get("symmetric", str(getattr(store, "_symmetric", False))) == str(getattr(store, "_symmetric", False)),
            md.get("optimize_clips", str(getattr(store, "_optimize_clips", False)))
            == str(getattr(store, "_optimize_clips", False)),
        ])
    except (KeyError, TypeError, ValueError):
        return False


def try_restore_preq_cache(store: Any, path, *, device=None) -> bool:
    """Restore every projection's preq blocks from `path` into the store;
    False (store untouched) unless the format, block size, quantization
    config, projection set and every tensor's byte count match."""
    path = Path(path)
    if not path.is_file():
        return False
    bs = block_size_for(store.group_size)
    from safetensors import safe_open

    with safe_open(str(path), framework="np") as f:
        md = f.metadata() or {}
        keys = list(f.keys())
    if md.get("format") != PREQ_CACHE_FORMAT or md.get("block_size") != str(bs):
        return False
    if not _quantize_config_matches(store, md):
        return False
    try:
        parsed = {_parse_preq_tensor_key(k): k for k in keys}
    except ValueError:
        return False
    expected = {(li, nm) for (li, nm) in store._quant_shapes if nm in PROJ_NAMES}
    if set(parsed) != expected:
        return False
    if device is not None:
        import safetensors.torch as st_t

        loaded = st_t.load_file(str(path), device=str(device))
    else:
        import safetensors.numpy as st_np

        loaded = st_np.load_file(str(path))
    out = {}
    for (li, nm), key in parsed.items():
        rows, cols = store._quant_shapes[(li, nm)]
        t = loaded[key]
        n = int(t.numel()) if device is not None else int(t.size)
        if n != rows * (cols // store.group_size) * bs or str(t.dtype).split(".")[-1] != "uint8":
            return False
        out[(li, nm)] = t.reshape(-1).contiguous() if device is not None else np.ascontiguousarray(t).reshape(-1)
    if device is not None:
        store._preq_blocks_dev = out
    else:
        store._preq_blocks_np = out
    store._preq_built = True
    return True


def save_preq_cache(store: Any, path) -> None:
    """Write the store's preq blocks (host arrays or device tensors) to one
    safetensors file with the format's metadata."""
    import safetensors.numpy as st_np

    blocks = store._preq_blocks_np or getattr(store, "_preq_blocks_dev", {})
    tensors = {}
    for (li, nm), b in blocks.items():
        if type(b).__module__.startswith("torch"):
            b = b.detach().cpu().numpy()
        tensors[_preq_tensor_key(li, nm)] = np.ascontiguousarray(b, dtype=np.uint8)
    meta = {"format": PREQ_CACHE_FORMAT, "block_size": str(block_size_for(store.group_size))}
    meta.update(_quantize_config_meta(store))
    path = Path(path)
    path.parent.mkdir(parents=True, exist_ok=True)
    st_np.save_file(tensors, str(path), metadata=meta)


def preq2_from_preq_blocks(blocks, rows: int, cols: int, group_size: int):
    """Flat (meta, quant) preq2 operands from one projection's preq blocks:
    at group size 32 the reference's preq -> preq2 repack, at 128 the
    Q4_128 -> preq2-g128 conversion (scale s, zero 8).  Device tensors in,
    device tensors out (HIP kernels on the current stream)."""
    from asdsl.quantization import repack as rp

    if group_size == 32:
        meta, quant = rp.repack_preq_blocks_to_preq2(blocks, rows, cols, 32)
        return rp.meta_to_flat(meta), rp.quant_to_flat(quant)
    if group_size == 128:
        return rp.repack_q4_128_blocks_to_preq2(blocks, rows, cols)
    raise ValueError(f"preq2_from_preq_blocks: group_size must be 32 or 128, got {group_size}")
