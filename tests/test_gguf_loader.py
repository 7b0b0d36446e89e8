"""The GGUF reader (asdsl.io.gguf_loader) on the CPU: files assembled byte by
byte from the format's layout, files from tests/gguf_writer.py with every
metadata type, alignment and tensor type, the reference loader's API
(logical shapes, row bytes, K-block flattening; asdsl/io/gguf_loader.py:
81-218) and its error paths."""

from __future__ import annotations

import struct

import numpy as np
import pytest

from asdsl.io import gguf_loader as gl
from gguf_writer import (ARRAY, BOOL, FLOAT32, FLOAT64, INT8, INT16, INT32, INT64, STRING, UINT8, UINT16, UINT32,
                         UINT64, write_gguf)


def test_hand_assembled_file(tmp_path):
    """Version 3, one metadata string, two tensors: an F32 vector and a
    2 x 256 Q4_K matrix (ne0 = 256 in, ne1 = 2 out), default alignment 32."""
    name = b"general.name"
    kv = struct.pack("<Q", len(name)) + name + struct.pack("<I", 8) + struct.pack("<Q", 3) + b"abc"
    vec = np.arange(5, dtype="<f4").tobytes()  # 20 bytes, padded to 32
    q4k = (np.arange(2 * 144) % 251).astype(np.uint8).tobytes()
    t1 = struct.pack("<Q", 3) + b"vec" + struct.pack("<I", 1) + struct.pack("<Q", 5) + struct.pack("<IQ", 0, 0)
    t2 = struct.pack("<Q", 3) + b"mat" + struct.pack("<I", 2) + struct.pack("<QQ", 256, 2) + struct.pack("<IQ", 12, 32)
    head = b"GGUF" + struct.pack("<IQQ", 3, 2, 1) + kv + t1 + t2
    head += b"\0" * (-len(head) % 32)
    path = tmp_path / "hand.gguf"
    path.write_bytes(head + vec + b"\0" * 12 + q4k)

    f = gl.GGUFFile(path)
    assert f.version == 3 and f.metadata == {"general.name": "abc"} and f.data_offset == len(head)
    t = gl.read_gguf_tensors(path)
    assert t["vec"]["type"] == "f32" and t["vec"]["shape"] == (5,) and t["vec"]["n_bytes"] == 20
    assert np.array_equal(gl.dequant_tensor(t["vec"]), np.arange(5, dtype=np.float32))
    m = t["mat"]
    assert m["type"] == "q4_k" and m["type_id"] == 12 and m["file_shape"] == (256, 2)
    assert m["logical_shape"] == (2, 256) and m["row_bytes"] == 144 and m["n_bytes"] == 288
    assert bytes(gl.q4k_blocks_rowmajor(m)) == q4k
    assert gl.read_gguf_tensors(path, name_filter="ma").keys() == {"mat"}


def test_writer_round_trip_every_metadata_type(tmp_path):
    meta = [("u8", UINT8, 200), ("i8", INT8, -5), ("u16", UINT16, 60000), ("i16", INT16, -300),
            ("u32", UINT32, 4_000_000_000), ("i32", INT32, -70000), ("f32", FLOAT32, 1.5), ("b", BOOL, True),
            ("s", STRING, "phi3 é"), ("u64", UINT64, 2**40), ("i64", INT64, -(2**40)), ("f64", FLOAT64, 0.1),
            ("ai", ARRAY, (INT32, [1, -2, 3])), ("as", ARRAY, (STRING, ["a", "bc", ""])),
            ("ab", ARRAY, (BOOL, [True, False])), ("aa", ARRAY, (ARRAY, [(UINT8, [1, 2]), (UINT8, [])]))]
    path = tmp_path / "m.gguf"
    write_gguf(path, [("x", 0, (4,), np.zeros(16, np.uint8))], meta)
    md = gl.read_gguf_metadata(path)
    for k, _, v in meta[:12]:
        assert md[k] == pytest.approx(v) if isinstance(v, float) else md[k] == v, k
    assert md["ai"].tolist() == [1, -2, 3] and md["as"] == ["a", "bc", ""] and md["ab"].tolist() == [True, False]
    assert [a.tolist() for a in md["aa"]] == [[1, 2], []]


@pytest.mark.parametrize("alignment", [32, 64, 256])
def test_tensor_types_and_alignment(tmp_path, alignment):
    rng = np.random.default_rng(alignment)
    f16 = rng.standard_normal((3, 8)).astype(np.float16)
    f32 = rng.standard_normal((2, 4)).astype(np.float32)
    bf = rng.standard_normal(6).astype(np.float32)
    bf16 = (bf.view(np.uint32) >> 16).astype(np.uint16)
    q6k = rng.integers(0, 256, 3 * 2 * 210, dtype=np.uint8)
    q80 = rng.integers(0, 256, 4 * 34, dtype=np.uint8)
    path = tmp_path / "t.gguf"
    write_gguf(path, [("a", 1, (8, 3), f16.view(np.uint8)), ("b", 0, (4, 2), f32.view(np.uint8)),
                      ("c", 30, (6,), bf16.view(np.uint8)), ("d", 14, (512, 3), q6k), ("e", 8, (128,), q80)],
               alignment=alignment)
    f = gl.GGUFFile(path)
    assert f.alignment == alignment and f.data_offset % alignment == 0
    assert all((start - f.data_offset) % alignment == 0 for _, _, start, _ in f.tensors.values())
    t = gl.read_gguf_tensors(path)
    assert np.array_equal(gl.dequant_tensor(t["a"]), f16.astype(np.float32))
    assert np.array_equal(gl.dequant_tensor(t["b"]), f32)
    assert np.array_equal(gl.dequant_tensor(t["c"]), (bf16.astype(np.uint32) << 16).view(np.float32))
    assert t["d"]["logical_shape"] == (3, 512) and t["d"]["row_bytes"] == 420
    assert np.array_equal(gl.q6k_blocks_rowmajor(t["d"]), q6k)
    assert t["e"]["type"] == "q8_0" and t["e"]["n_bytes"] == 4 * 34
    rows = gl.summarize_tensors(path, limit=2)
    assert [r["name"] for r in rows] == ["a", "b"] and rows[0]["logical_shape"] == [3, 8]


def test_reference_helpers():
    assert gl.row_bytes_for_type("Q4_K", 3072) == 12 * 144 and gl.row_bytes_for_type("q6_k", 8192) == 32 * 210
    assert gl.row_bytes_for_type("q5_k", 512) == 2 * 176 and gl.row_bytes_for_type("Q8_0", 256) == 8 * 34
    with pytest.raises(ValueError):
        gl.row_bytes_for_type("iq2_xs", 256)
    assert gl.logical_shape((3072, 5120), "q4_k") == (5120, 3072) == gl.logical_shape((3072, 5120), "f16")
    with pytest.raises(ValueError):
        gl.logical_shape((4,), "f32")
    assert gl.ggml_type_name(12) == "q4_k" and gl.ggml_type_name(30) == "bf16" and gl.ggml_type_name(99) == "unknown_99"
    info = {"type": "q4_k", "logical_shape": (2, 256), "data": np.zeros(200, np.uint8)}
    with pytest.raises(ValueError, match="take 288 bytes, the tensor has 200"):
        gl.q4k_blocks_rowmajor(info)
    with pytest.raises(ValueError):
        gl.k_blocks_rowmajor({"type": "f32", "logical_shape": (1, 1), "data": np.zeros(4, np.uint8)})


def test_rejects_malformed_files(tmp_path):
    good = tmp_path / "g.gguf"
    write_gguf(good, [("x", 0, (4,), np.zeros(16, np.uint8))])
    raw = good.read_bytes()
    cases = {"magic": b"GGUX" + raw[4:], "version": raw[:4] + struct.pack("<I", 1) + raw[8:],
             "truncated": raw[:30], "past_end": raw[:-20]}
    for what, data in cases.items():
        p = tmp_path / f"{what}.gguf"
        p.write_bytes(data)
        with pytest.raises(ValueError):
            gl.GGUFFile(p)
    p = tmp_path / "type.gguf"
    write_gguf(p, [("x", 77, (4,), np.zeros(16, np.uint8))])
    with pytest.raises(ValueError, match="unsupported ggml type"):
        gl.GGUFFile(p)
    p = tmp_path / "ne0.gguf"
    write_gguf(p, [("x", 12, (128, 2), np.zeros(144, np.uint8))])
    with pytest.raises(ValueError, match="not a multiple of 256"):
        gl.GGUFFile(p)


def test_no_cpu_decode_of_k_quants(tmp_path):
    """K-quant tensors decode only on the GPU: without a device the call
    fails instead of falling back to a CPU path."""
    import torch

    if torch.cuda.is_available():
        pytest.skip("a device is present")
    info = {"type": "q4_k", "shape": (256, 1), "logical_shape": (1, 256), "data": np.zeros(144, np.uint8)}
    with pytest.raises(Exception):
        gl.dequant_tensor(info)


def test_version_2_reads_like_version_3(tmp_path):
    """Versions 2 and 3 share the layout (64-bit counts and lengths); 3
    only adds big-endian files, which the reader does not take."""
    raw = np.arange(32, dtype=np.float32)
    for version in (2, 3):
        path = tmp_path / f"v{version}.gguf"
        write_gguf(path, [("t", 0, (8, 4), raw.view(np.uint8))], [("k", STRING, "v")], version=version)
        f = gl.GGUFFile(path)
        assert f.version == version and f.metadata == {"k": "v"}
        t = gl.read_gguf_tensors(path)["t"]
        assert t["logical_shape"] == (4, 8)
        assert np.array_equal(gl.dequant_tensor(t), raw.reshape(4, 8))


def test_config_from_gguf_caps_the_kv_length():
    """A file's trained context sizes the KV cache only up to 4096 positions
    unless max_seq is passed; every other field comes from the metadata."""
    from asdsl.engine import GGUF_DEFAULT_MAX_SEQ, config_from_gguf

    meta = {"general.architecture": "phi3", "phi3.embedding_length": 3072, "phi3.feed_forward_length": 8192,
            "phi3.block_count": 32, "phi3.attention.head_count": 24, "phi3.attention.head_count_kv": 8,
            "phi3.rope.dimension_count": 96, "phi3.context_length": 131072,
            "phi3.attention.layer_norm_rms_epsilon": 1e-5, "phi3.rope.freq_base": 10000.0,
            "tokenizer.ggml.tokens": [f"t{i}" for i in range(200064)]}
    c = config_from_gguf(meta)
    assert GGUF_DEFAULT_MAX_SEQ == 4096 and c.max_seq == 4096
    assert (c.hidden, c.ffn, c.n_layers, c.n_heads, c.n_kv_heads, c.rotary_dim, c.vocab) == \
        (3072, 8192, 32, 24, 8, 96, 200064)
    assert config_from_gguf(meta, max_seq=131072).max_seq == 131072
    assert config_from_gguf({**meta, "phi3.context_length": 512}).max_seq == 512
