"""The C-ABI library: loads, exports every declared entry point, and rejects
bad arguments before touching HIP (so these run without a GPU)."""

from __future__ import annotations

import ctypes
import re

import numpy as np
import pytest

from conftest import REPO

HEADER = REPO / "include" / "asdsl_hip.h"


def declared_entry_points() -> list[str]:
    text = HEADER.read_text()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(asdsl_[a-z0-9_]+)\s*\(", text)))


def test_header_declares_entry_points():
    names = declared_entry_points()
    assert "asdsl_gemv_preq2_fused" in names and len(names) >= 8


def test_library_exports_every_declared_symbol():
    from asdsl import _hip

    missing = [n for n in declared_entry_points() if not _hip.exported(n)]
    assert not missing, f"declared but not exported: {missing}"
    assert _hip.LIB.asdsl_abi_version() == 3


def test_python_signatures_cover_header():
    from asdsl import _hip

    assert set(declared_entry_points()) <= set(_hip.SIGNATURES)


def test_invalid_arguments_rejected_without_gpu():
    from asdsl import _hip

    lib = _hip.LIB
    one = ctypes.c_void_p(16)
    # null pointers
    assert lib.asdsl_gemv_preq2_fused(None, None, None, None, 4, 64, 32, None) == _hip.ASDSL_ERR_INVALID_ARGUMENT
    assert "null" in _hip.last_error()
    # group size / divisibility / size limits, as the reference checks
    assert lib.asdsl_gemv_preq2_fused(one, one, one, one, 4, 64, 64, None) == _hip.ASDSL_ERR_INVALID_ARGUMENT
    assert "group_size" in _hip.last_error()
    assert lib.asdsl_gemv_preq2_fused(one, one, one, one, 4, 48, 32, None) == _hip.ASDSL_ERR_INVALID_ARGUMENT
    assert lib.asdsl_gemv_preq2_fused(one, one, one, one, 4, 32 * 641, 32, None) == _hip.ASDSL_ERR_INVALID_ARGUMENT
    assert "exceeds" in _hip.last_error()
    assert lib.asdsl_gemv_q4_32_preq_fused(one, one, one, 0, 64, 32, None) == _hip.ASDSL_ERR_INVALID_ARGUMENT
    assert lib.asdsl_quantize_activation(one, one, one, 100, 32, None) == _hip.ASDSL_ERR_INVALID_ARGUMENT
    # the calibration read's launch shapes
    u32 = ctypes.c_void_p(16)
    for grid, threads, inflight, slab in ((1, 1024, 4, 2), (1, 256, 5, 2), (1, 256, 2, 0), (1, 256, 4, 3),
                                          (0, 256, 4, 0)):
        assert lib.asdsl_stream_read_ex(one, 4096, u32, grid, threads, inflight, slab, None) == \
            _hip.ASDSL_ERR_INVALID_ARGUMENT, (grid, threads, inflight, slab)


def test_python_wrapper_validates_sizes():
    from asdsl.kernels import _native_gemv as ng

    with pytest.raises(ValueError, match="meta"):
        ng.gemv_preq2_fused_avx2(np.zeros(10, np.uint8), np.zeros(1 << 12, np.uint8),
                                 np.zeros(64, np.float32), np.zeros(4, np.float32), 4, 64, 32)
    with pytest.raises(ValueError, match="group_size"):
        ng.gemv_q4_32_preq_fused_avx2(np.zeros(1 << 12, np.uint8), np.zeros(64, np.float32),
                                      np.zeros(4, np.float32), 4, 64, 16)
    with pytest.raises(ValueError, match="y"):
        ng.gemv_preq2_fused_avx2(np.zeros(32, np.uint8), np.zeros(1 << 12, np.uint8),
                                 np.zeros(64, np.float32), np.zeros(3, np.float32), 4, 64, 32)


def test_no_cpu_fallback():
    """Valid arguments on a machine without a GPU must fail loudly, not compute."""
    import torch

    if torch.cuda.is_available():
        pytest.skip("a GPU is present")
    from asdsl import _hip

    one = ctypes.c_void_p(16)
    assert _hip.LIB.asdsl_gemv_preq2_fused(one, one, one, one, 4, 64, 32, None) == _hip.ASDSL_ERR_HIP
    from asdsl.kernels import _native_gemv as ng

    with pytest.raises(RuntimeError):
        ng.gemv_preq2_fused_avx2(np.zeros(32, np.uint8), np.zeros(128, np.uint8),
                                 np.zeros(64, np.float32), np.zeros(4, np.float32), 4, 64, 32)


def test_work_buffer_queries_and_checks_without_gpu():
    """The *_work_bytes queries need no device; a caller buffer below the
    queried size is an argument error raised before any HIP call."""
    from asdsl import _hip

    lib = _hip.LIB
    one = ctypes.c_void_p(256)
    assert lib.asdsl_sparse_down_work_bytes(3072) == 32 * 3072 * 4
    assert lib.asdsl_sparse_down_work_bytes(0) == 0
    # per 32-element slice and column: 32 int8 codes, a (scale, sum) pair, a slice sum
    assert lib.asdsl_gemv_preq2_fused_batch_work_bytes(3072) == 96 * 16 * 44
    assert lib.asdsl_gemv_preq2_fused_batch_work_bytes(100) == 0
    # gate_up 16384 x 3072 at group 32: 96 units, one K slab (8 waves x 12 units): image + sums only
    assert lib.asdsl_affine_batch_work_bytes(16384, 3072, 32) == 96 * 2 * 64 * 16 + 96 * 16 * 4 + 16 * 4
    assert lib.asdsl_affine_batch_work_bytes(16384, 3000, 32) == 0
    assert lib.asdsl_sparse_down_proj_T_ws(one, one, one, one, one, 8, one, 64, 3072, 64, one, 1024,
                                           None) == _hip.ASDSL_ERR_INVALID_ARGUMENT
    assert "work buffer" in _hip.last_error()
    assert lib.asdsl_gemv_preq2_fused_batch_ws(one, one, one, one, 64, 3072, 32, 4, one, 100,
                                               None) == _hip.ASDSL_ERR_INVALID_ARGUMENT
    assert "work buffer" in _hip.last_error()


def test_decode_structs_match_the_header(tmp_path):
    """The engine's ctypes mirrors of asdsl_decode_layer / asdsl_decode_model
    have the header's field offsets and sizes (a C program built with gcc
    from the header prints them)."""
    import shutil
    import subprocess

    from asdsl.engine import _Layer, _Model

    if shutil.which("gcc") is None:
        pytest.skip("gcc not available")
    fields = {"asdsl_decode_layer": [n for n, _ in _Layer._fields_],
              "asdsl_decode_model": [n for n, _ in _Model._fields_]}
    lines = ["#include <stdio.h>", "#include <stddef.h>", '#include "asdsl_hip.h"', "int main(void) {"]
    for st, names in fields.items():
        lines.append(f'printf("{st} %zu\\n", sizeof({st}));')
        for n in names:
            lines.append(f'printf("{st}.{n} %zu\\n", offsetof({st}, {n}));')
    lines += ["return 0;", "}"]
    src = tmp_path / "layout.c"
    src.write_text("\n".join(lines) + "\n")
    exe = tmp_path / "layout"
    subprocess.run(["gcc", "-x", "c", f"-I{REPO / 'include'}", str(src), "-o", str(exe)], check=True)
    got = dict(line.split() for line in subprocess.run([str(exe)], check=True, capture_output=True,
                                                       text=True).stdout.splitlines())
    for st, cls in (("asdsl_decode_layer", _Layer), ("asdsl_decode_model", _Model)):
        assert int(got[st]) == ctypes.sizeof(cls), st
        for n in fields[st]:
            assert int(got[f"{st}.{n}"]) == getattr(cls, n).offset, (st, n)
