"""GGUF tensor reader and K-quant decoding for the GPU framework.

Mirrors the reference's asdsl/io/gguf_loader.py (type table, GGUF name map,
``read_gguf_tensors``, ``logical_shape``, ``row_bytes_for_type``,
``dequant_tensor``, ``k_blocks_rowmajor`` / ``q4k_blocks_rowmajor``,
``summarize_tensors``) without the ``gguf`` package, which is not installed
here: the file is parsed directly from a read-only memory map following the
GGUF layout (magic "GGUF", version 2 or 3, tensor and metadata counts,
typed key/value metadata, tensor infos, a data section aligned to
``general.alignment``, default 32).  Tensor payloads are views of the map,
never copies.

Block-quantized tensors decode on the GPU (``asdsl_dequant_gguf_q2k``,
``_q3k``, ``_q4k``, ``_q5k``, ``_q6k``, ``_q4_0``, ``_q4_1``, ``_q5_0``,
``_q5_1``, ``_q8_0``); there is no CPU decode path, and other types (Q8_1,
Q8_K and the IQ types) are refused.  Deviations from the reference,
each a fix:

* ``data`` is the tensor's raw bytes for every type.  The reference converts
  the gguf reader's arrays with ``np.ascontiguousarray(..., dtype=np.uint8)``
  (gguf_loader.py:97-101), which casts float tensors value by value, so its
  F32/F16 tensors do not decode.
* ``GGML_TYPE_NAMES`` follows ggml.h from id 24 on (I8, I16, I32, I64, F64,
  IQ1_M = 29, BF16 = 30); the reference's table names 24 "iq1_m" and 25
  "bf16" (gguf_loader.py:35-36).
"""

from __future__ import annotations

from pathlib import Path
from typing import Any

import numpy as np

GGUF_MAGIC = b"GGUF"
GGUF_DEFAULT_ALIGNMENT = 32

# ggml type ids (ggml.h)
GGML_TYPE_NAMES: dict[int, str] = {
    0: "f32", 1: "f16", 2: "q4_0", 3: "q4_1", 6: "q5_0", 7: "q5_1", 8: "q8_0", 9: "q8_1",
    10: "q2_k", 11: "q3_k", 12: "q4_k", 13: "q5_k", 14: "q6_k", 15: "q8_k",
    16: "iq2_xxs", 17: "iq2_xs", 18: "iq3_xxs", 19: "iq1_s", 20: "iq4_nl", 21: "iq3_s", 22: "iq2_s",
    23: "iq4_xs", 24: "i8", 25: "i16", 26: "i32", 27: "i64", 28: "f64", 29: "iq1_m", 30: "bf16",
}

# (weights per block, bytes per block) of each type
GGML_BLOCK: dict[str, tuple[int, int]] = {
    "f32": (1, 4), "f16": (1, 2), "bf16": (1, 2), "f64": (1, 8), "i8": (1, 1), "i16": (1, 2), "i32": (1, 4),
    "i64": (1, 8), "q4_0": (32, 18), "q4_1": (32, 20), "q5_0": (32, 22), "q5_1": (32, 24), "q8_0": (32, 34),
    "q8_1": (32, 36), "q2_k": (256, 84), "q3_k": (256, 110), "q4_k": (256, 144), "q5_k": (256, 176),
    "q6_k": (256, 210), "q8_k": (256, 292), "iq2_xxs": (256, 66), "iq2_xs": (256, 74), "iq3_xxs": (256, 98),
    "iq1_s": (256, 50), "iq4_nl": (32, 18), "iq3_s": (256, 110), "iq2_s": (256, 82), "iq4_xs": (256, 136),
    "iq1_m": (256, 56),
}

# K-quant block sizes (bytes per 256 weights along the input axis)
_K_BLOCK_BYTES: dict[str, int] = {t: GGML_BLOCK[t][1] for t in ("q2_k", "q3_k", "q4_k", "q5_k", "q6_k", "q8_k")}
# legacy 32-weight block types whose rows are whole blocks
_ROW_BLOCK_TYPES = ("q4_0", "q4_1", "q5_0", "q5_1", "q8_0", "q8_1")
# types decoded on the GPU: ggml type -> C-ABI decoder
_DEVICE_DECODERS = {"q2_k": "asdsl_dequant_gguf_q2k", "q3_k": "asdsl_dequant_gguf_q3k",
                    "q4_k": "asdsl_dequant_gguf_q4k", "q5_k": "asdsl_dequant_gguf_q5k",
                    "q6_k": "asdsl_dequant_gguf_q6k", "q4_0": "asdsl_dequant_gguf_q4_0",
                    "q4_1": "asdsl_dequant_gguf_q4_1", "q5_0": "asdsl_dequant_gguf_q5_0",
                    "q5_1": "asdsl_dequant_gguf_q5_1", "q8_0": "asdsl_dequant_gguf_q8_0"}

# GGUF tensor suffix -> (ASDSL projection, module), the reference's map
GGUF_TO_ASDSL: dict[str, tuple[str, str]] = {
    "attn_qkv.weight": ("qkv_proj", "attn"),
    "attn_output.weight": ("o_proj", "attn"),
    "ffn_gate_up.weight": ("gate_up_proj", "ffn"),
    "ffn_gate.weight": ("gate_proj", "ffn"),
    "ffn_up.weight": ("up_proj", "ffn"),
    "ffn_down.weight": ("down_proj", "ffn"),
    "attn_norm.weight": ("attn_norm", "norm"),
    "ffn_norm.weight": ("ffn_norm", "norm"),
    "token_embd.weight": ("token_embd", "embed"),
    "output_norm.weight": ("output_norm", "norm"),
    "output.weight": ("lm_head", "output"),
}

# metadata value types
_VALUE_DTYPES = {0: "<u1", 1: "<i1", 2: "<u2", 3: "<i2", 4: "<u4", 5: "<i4", 6: "<f4", 7: "<u1", 10: "<u8",
                 11: "<i8", 12: "<f8"}
_STRING, _ARRAY, _BOOL = 8, 9, 7


def ggml_type_name(type_id: int) -> str:
    return GGML_TYPE_NAMES.get(type_id, f"unknown_{type_id}")


def row_bytes_for_type(type_name: str, in_features: int) -> int:
    """Size in bytes of one stored row of `in_features` weights (one output
    feature) of a block-quantized ggml type: whole blocks of the type's
    weights-per-block."""
    t = type_name.lower()
    if t in _K_BLOCK_BYTES:
        return (in_features // 256) * _K_BLOCK_BYTES[t]
    if t in _ROW_BLOCK_TYPES:
        per, nbytes = GGML_BLOCK[t]
        return (in_features // per) * nbytes
    raise ValueError(f"no stored-row size for ggml type {type_name!r}")


def logical_shape(file_shape: tuple[int, ...], type_name: str) -> tuple[int, int]:
    """A GGUF weight's dims as stored (ne0, the contiguous input axis, first)
    turned into the (out_features, in_features) of W in y = W x."""
    if len(file_shape) != 2:
        raise ValueError(f"logical_shape: a weight has two dims, this one {tuple(file_shape)}")
    return int(file_shape[1]), int(file_shape[0])


class _Cursor:
    """Little-endian reads over a uint8 memory map."""

    def __init__(self, buf: np.ndarray):
        self.buf, self.pos = buf, 0

    def take(self, n: int) -> np.ndarray:
        if self.pos + n > self.buf.size:
            raise ValueError("GGUF: truncated file")
        out = self.buf[self.pos:self.pos + n]
        self.pos += n
        return out

    def scalar(self, dtype: str):
        return np.frombuffer(self.take(np.dtype(dtype).itemsize), dtype=dtype)[0].item()

    def string(self) -> str:
        n = self.scalar("<u8")
        return bytes(self.take(n)).decode("utf-8", errors="replace")

    def value(self, vtype: int):
        if vtype == _STRING:
            return self.string()
        if vtype == _ARRAY:
            etype, count = self.scalar("<u4"), self.scalar("<u8")
            if etype in _VALUE_DTYPES:
                dt = np.dtype(_VALUE_DTYPES[etype])
                arr = np.frombuffer(self.take(count * dt.itemsize), dtype=dt).copy()
                return arr.astype(bool) if etype == _BOOL else arr
            return [self.value(etype) for _ in range(count)]
        if vtype in _VALUE_DTYPES:
            v = self.scalar(_VALUE_DTYPES[vtype])
            return bool(v) if vtype == _BOOL else v
        raise ValueError(f"GGUF: unknown metadata value type {vtype}")


class GGUFFile:
    """A parsed GGUF file: ``version``, ``metadata`` (key -> value),
    ``alignment``, ``data_offset`` and ``tensors`` (name -> (ggml type id,
    file dims, byte offset in the file, byte count)).  Payloads are views of
    the read-only memory map."""

    def __init__(self, path: str | Path):
        self.path = str(path)
        self._map = np.memmap(self.path, dtype=np.uint8, mode="r")
        cur = _Cursor(self._map)
        if bytes(cur.take(4)) != GGUF_MAGIC:
            raise ValueError(f"{self.path}: not a GGUF file")
        self.version = cur.scalar("<u4")
        if self.version not in (2, 3):
            raise ValueError(f"{self.path}: GGUF version {self.version} is not supported (2 or 3)")
        n_tensors, n_kv = cur.scalar("<u8"), cur.scalar("<u8")
        self.metadata: dict[str, Any] = {}
        for _ in range(n_kv):
            key = cur.string()
            self.metadata[key] = cur.value(cur.scalar("<u4"))
        infos = []
        for _ in range(n_tensors):
            name = cur.string()
            n_dims = cur.scalar("<u4")
            dims = tuple(cur.scalar("<u8") for _ in range(n_dims))
            infos.append((name, cur.scalar("<u4"), dims, cur.scalar("<u8")))
        self.alignment = int(self.metadata.get("general.alignment", GGUF_DEFAULT_ALIGNMENT))
        if self.alignment <= 0 or self.alignment & (self.alignment - 1):
            raise ValueError(f"{self.path}: general.alignment {self.alignment} is not a power of two")
        self.data_offset = -(-cur.pos // self.alignment) * self.alignment
        self.tensors: dict[str, tuple[int, tuple[int, ...], int, int]] = {}
        for name, type_id, dims, offset in infos:
            tname = ggml_type_name(type_id)
            if tname not in GGML_BLOCK:
                raise ValueError(f"{self.path}: tensor {name} has unsupported ggml type {type_id}")
            per, nbytes = GGML_BLOCK[tname]
            n = int(np.prod(dims, dtype=np.int64)) if dims else 1
            if dims and dims[0] % per:
                raise ValueError(f"{self.path}: tensor {name}: ne0={dims[0]} not a multiple of {per} ({tname})")
            size = n // per * nbytes
            start = self.data_offset + offset
            if offset % self.alignment or start + size > self._map.size:
                raise ValueError(f"{self.path}: tensor {name} lies outside the data section")
            self.tensors[name] = (type_id, dims, start, size)

    def tensor_bytes(self, name: str) -> np.ndarray:
        _, _, start, size = self.tensors[name]
        return self._map[start:start + size]


def read_gguf_metadata(path: str | Path) -> dict[str, Any]:
    return GGUFFile(path).metadata


def read_gguf_tensors(path: str | Path, *, name_filter: str | None = None) -> dict[str, dict[str, Any]]:
    """Every tensor of a GGUF file (those whose name contains name_filter).

    Returns name -> {type, type_id, shape, file_shape, data (raw bytes, a
    uint8 view of the file), n_bytes, and for rank-2 tensors logical_shape
    (out, in) and, for block-quantized types, row_bytes}."""
    f = GGUFFile(path)
    out: dict[str, dict[str, Any]] = {}
    for name, (type_id, dims, _, size) in f.tensors.items():
        if name_filter and name_filter not in name:
            continue
        tname = ggml_type_name(type_id)
        info: dict[str, Any] = {"type": tname, "type_id": type_id, "shape": dims, "file_shape": dims,
                                "data": f.tensor_bytes(name), "n_bytes": size}
        if len(dims) == 2:
            info["logical_shape"] = logical_shape(dims, tname)
            if tname in _K_BLOCK_BYTES or tname in _ROW_BLOCK_TYPES:
                info["row_bytes"] = row_bytes_for_type(tname, info["logical_shape"][1])
        out[name] = info
    return out


def _blocks_rowmajor(info: dict[str, Any], tname: str, fn: str) -> np.ndarray:
    """The tensor's raw bytes, checked to be exactly rows x row_bytes: GGUF
    stores a weight one output row after another, each a run of blocks."""
    rows, cols = info["logical_shape"]
    flat = np.asarray(info["data"], dtype=np.uint8).reshape(-1)
    want = rows * row_bytes_for_type(tname, cols)
    if flat.size != want:
        raise ValueError(f"{fn}: {rows} x {cols} {tname} weights take {want} bytes, the tensor has {flat.size}")
    return flat


def k_blocks_rowmajor(info: dict[str, Any], type_name: str | None = None) -> np.ndarray:
    """A K-quant weight's bytes: per output row, in_features/256 blocks."""
    tname = (type_name or str(info.get("type", ""))).lower()
    if tname not in _K_BLOCK_BYTES:
        raise ValueError(f"k_blocks_rowmajor: {tname!r} is not a K-quant type")
    return _blocks_rowmajor(info, tname, "k_blocks_rowmajor")


def q4k_blocks_rowmajor(info: dict[str, Any]) -> np.ndarray:
    """A ggml Q4_K weight's bytes, 144 per 256 weights of a row -- what the
    reference gives its Q4_K GEMV.  ``q4km_from_gguf`` rearranges them into
    the ASDSL Q4_K variant that GEMV decodes."""
    return k_blocks_rowmajor(info, "q4_k")


def q5k_blocks_rowmajor(info: dict[str, Any]) -> np.ndarray:
    """A ggml Q5_K weight's bytes, 176 per 256 weights of a row."""
    return k_blocks_rowmajor(info, "q5_k")


def q6k_blocks_rowmajor(info: dict[str, Any]) -> np.ndarray:
    """A ggml Q6_K weight's bytes, 210 per 256 weights of a row."""
    return k_blocks_rowmajor(info, "q6_k")


def _dense(info: dict[str, Any]) -> np.ndarray:
    raw = np.asarray(info["data"], dtype=np.uint8)
    t = info["type"]
    if t == "f32":
        arr = raw.view("<f4").astype(np.float32)
    elif t == "f16":
        arr = raw.view("<f2").astype(np.float32)
    else:  # bf16: the top half of a float32
        arr = (raw.view("<u2").astype(np.uint32) << 16).view(np.float32)
    return arr


def dequant_tensor_device(info: dict[str, Any]):
    """A tensor decoded to float32 on the GPU: shape (out, in) for rank-2
    tensors (1-D otherwise).  Q2_K..Q6_K, Q4_0, Q4_1, Q5_0, Q5_1 and Q8_0
    decode in the HIP kernels; F32/F16/BF16 are converted from their bytes
    and uploaded."""
    from asdsl import _hip

    torch = _hip._torch()
    t = str(info["type"]).lower()
    dims = tuple(info["shape"])
    shape = info.get("logical_shape", dims if len(dims) != 1 else (dims[0],))
    if t in ("f32", "f16", "bf16"):
        return torch.from_numpy(np.ascontiguousarray(_dense(info)).reshape(shape)).to(_hip.device())
    fn = _DEVICE_DECODERS.get(t)
    if fn is None or len(dims) != 2:
        raise ValueError(f"dequant_tensor: type {info.get('type')} (rank {len(dims)}) is not decoded here "
                         f"({', '.join(k.upper() for k in _DEVICE_DECODERS)}, F32, F16, BF16)")
    rows, cols = shape
    blocks = _hip.to_device(_blocks_rowmajor(info, t, "dequant_tensor"), np.uint8)
    out = torch.empty((rows, cols), dtype=torch.float32, device=_hip.device())
    _hip.call(fn, _hip.ptr(blocks), _hip.ptr(out), rows, cols, _hip.stream_handle())
    return out


def dequant_tensor(info: dict[str, Any]) -> np.ndarray:
    """Decode one tensor to float32 with shape (out_features, in_features)
    (1-D tensors stay 1-D), as the reference's dequant_tensor returns it."""
    t = str(info["type"]).lower()
    if t in ("f32", "f16", "bf16"):
        dims = tuple(info["shape"])
        return np.ascontiguousarray(_dense(info).reshape(info.get("logical_shape", dims if len(dims) != 1
                                                                   else (dims[0],))))
    return dequant_tensor_device(info).cpu().numpy()


def q4km_from_gguf(info: dict[str, Any]):
    """A ggml Q4_K tensor as ASDSL Q4_K variant blocks on the GPU (uint8
    [rows x cols/256 x 144]), for asdsl_gemv_q4km / gemv_q4km_q8_avx2."""
    from asdsl import _hip

    rows, cols = info["logical_shape"]
    src = _hip.to_device(q4k_blocks_rowmajor(info), np.uint8)
    out = _hip.empty_device((rows * (cols // 256) * 144,), np.uint8)
    _hip.call("asdsl_repack_gguf_q4k_to_q4km", _hip.ptr(src), _hip.ptr(out), rows, cols, _hip.stream_handle())
    return out


def summarize_tensors(path: str | Path, limit: int = 10) -> list[dict[str, Any]]:
    """JSON-serializable summary of the first ``limit`` tensors by name."""
    tensors = read_gguf_tensors(path)
    rows: list[dict[str, Any]] = []
    for name in sorted(tensors):
        info = tensors[name]
        row = {"name": name, "type": info["type"], "type_id": info.get("type_id"), "shape": list(info["shape"])}
        if "logical_shape" in info:
            row["logical_shape"] = list(info["logical_shape"])
        rows.append(row)
        if len(rows) >= limit:
            break
    return rows
