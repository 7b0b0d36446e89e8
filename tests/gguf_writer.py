"""A minimal GGUF (version 3, or 2: the same layout) writer for test fixtures: typed metadata and
tensors given as raw bytes, laid out as the format defines it (magic,
version, tensor and key/value counts, metadata, tensor infos with offsets
relative to the data section, the data section aligned to
``general.alignment``, each tensor's offset a multiple of it)."""

from __future__ import annotations

import struct

import numpy as np

# metadata value type codes
UINT8, INT8, UINT16, INT16, UINT32, INT32, FLOAT32, BOOL, STRING, ARRAY, UINT64, INT64, FLOAT64 = range(13)
_FMT = {UINT8: "<B", INT8: "<b", UINT16: "<H", INT16: "<h", UINT32: "<I", INT32: "<i", FLOAT32: "<f", BOOL: "<?",
        UINT64: "<Q", INT64: "<q", FLOAT64: "<d"}


def _string(s: str) -> bytes:
    b = s.encode("utf-8")
    return struct.pack("<Q", len(b)) + b


def _value(vtype: int, v) -> bytes:
    if vtype == STRING:
        return _string(v)
    if vtype == ARRAY:
        etype, items = v
        out = struct.pack("<IQ", etype, len(items))
        return out + b"".join(_value(etype, x) for x in items)
    return struct.pack(_FMT[vtype], v)


def write_gguf(path, tensors: list, metadata: list | None = None, alignment: int = 32, version: int = 3) -> None:
    """tensors: [(name, ggml type id, dims (ne0 first), raw bytes)];
    metadata: [(key, value type, value)] (ARRAY values as (element type,
    items)).  A ``general.alignment`` entry is added when alignment != 32."""
    meta = list(metadata or [])
    if alignment != 32:
        meta.append(("general.alignment", UINT32, alignment))
    head = b"GGUF" + struct.pack("<IQQ", version, len(tensors), len(meta))
    head += b"".join(_string(k) + struct.pack("<I", t) + _value(t, v) for k, t, v in meta)
    offset, infos, blobs = 0, b"", []
    for name, type_id, dims, raw in tensors:
        infos += _string(name) + struct.pack("<I", len(dims)) + b"".join(struct.pack("<Q", d) for d in dims)
        infos += struct.pack("<IQ", type_id, offset)
        raw = bytes(np.asarray(raw, dtype=np.uint8).reshape(-1))
        pad = -len(raw) % alignment
        blobs.append(raw + b"\0" * pad)
        offset += len(raw) + pad
    body = head + infos
    body += b"\0" * (-len(body) % alignment)
    with open(path, "wb") as f:
        f.write(body + b"".join(blobs))
