"""Device side of the repackers: the HIP kernels behind the functions of
``asdsl.quantization.repack`` when their inputs are device tensors.

Outputs are new device tensors shaped as the host functions shape theirs;
the calls are queued on the current stream.  Buffer sizes are checked here
before anything is launched (the kernels trust them).
"""

from __future__ import annotations

import numpy as np

from asdsl import _hip


def _numel(a) -> int:
    return int(a.numel()) if hasattr(a, "numel") else int(np.asarray(a).size)


def _need(a, n: int, what: str, fn: str) -> None:
    if _numel(a) < n:
        raise ValueError(f"{fn}: {what} holds {_numel(a)} elements, needs {n}")


def _check_dims(fn: str, rows: int, cols: int, gs: int) -> None:
    if rows <= 0 or cols <= 0 or cols % gs:
        raise ValueError(f"{fn}: rows must be positive and cols a positive multiple of {gs}")


def _asym_inputs(fn, packed, scales, biases, rows, cols, gs):
    _check_dims(fn, rows, cols, gs)
    G = cols // gs
    _need(packed, rows * cols // 2, "packed", fn)
    _need(scales, rows * G, "scales", fn)
    _need(biases, rows * G, "biases", fn)
    return (_hip.to_device(packed, np.uint8).reshape(-1), _hip.to_device(scales, np.float32).reshape(-1),
            _hip.to_device(biases, np.float32).reshape(-1))


def asym_to_q4_32(packed, scales, biases, rows: int, cols: int):
    fn = "repack_asymmetric_to_q4_32_blocks"
    p, s, b = _asym_inputs(fn, packed, scales, biases, rows, cols, 32)
    out = _hip.empty_device((rows, cols // 32, 20), np.uint8)
    _hip.call("asdsl_repack_asym_to_q4_32", _hip.ptr(p), _hip.ptr(s), _hip.ptr(b), _hip.ptr(out), rows, cols, 32,
              _hip.stream_handle())
    return out


def preq_to_preq2(flat_preq, rows: int, cols: int):
    fn = "repack_preq_blocks_to_preq2"
    _check_dims(fn, rows, cols, 32)
    G = cols // 32
    if _numel(flat_preq) < rows * G * 20:
        raise ValueError("flat_preq too small for shape")
    pq = _hip.to_device(flat_preq, np.uint8).reshape(-1)
    meta = _hip.empty_device((rows, G * 4), np.uint8)
    quant = _hip.empty_device(((rows + 3) // 4, G, 64), np.uint8)
    _hip.call("asdsl_repack_preq_to_preq2", _hip.ptr(pq), _hip.ptr(meta), _hip.ptr(quant), rows, cols, 32,
              _hip.stream_handle())
    return meta, quant


def asym_to_preq2(packed, scales, biases, rows: int, cols: int, group_size: int):
    fn = "repack_asymmetric_to_preq2"
    if group_size not in (32, 128):
        raise ValueError(f"{fn}: group_size must be 32 or 128")
    p, s, b = _asym_inputs(fn, packed, scales, biases, rows, cols, group_size)
    G = cols // group_size
    meta = _hip.empty_device((rows * G * 4,), np.uint8)
    quant = _hip.empty_device(((rows + 3) // 4 * G * 2 * group_size,), np.uint8)
    _hip.call("asdsl_repack_asym_to_preq2", _hip.ptr(p), _hip.ptr(s), _hip.ptr(b), _hip.ptr(meta), _hip.ptr(quant),
              rows, cols, group_size, _hip.stream_handle())
    return meta, quant


def fp32_to_q4_128(weights, rows: int, cols: int):
    fn = "repack_fp32_to_q4_128_blocks"
    _check_dims(fn, rows, cols, 128)
    _need(weights, rows * cols, "weights", fn)
    w = _hip.to_device(weights, np.float32).reshape(-1)
    out = _hip.empty_device((rows, cols // 128, 66), np.uint8)
    _hip.call("asdsl_repack_fp32_to_q4_128", _hip.ptr(w), _hip.ptr(out), rows, cols, 128, _hip.stream_handle())
    return out


def asym_to_q4_128(packed, scales, biases, rows: int, cols: int):
    fn = "repack_asymmetric_to_q4_128_blocks"
    p, s, b = _asym_inputs(fn, packed, scales, biases, rows, cols, 128)
    out = _hip.empty_device((rows, cols // 128, 66), np.uint8)
    _hip.call("asdsl_repack_asym_to_q4_128", _hip.ptr(p), _hip.ptr(s), _hip.ptr(b), _hip.ptr(out), rows, cols, 128,
              _hip.stream_handle())
    return out


def q4_128_to_preq2(blocks, rows: int, cols: int):
    fn = "repack_q4_128_blocks_to_preq2"
    _check_dims(fn, rows, cols, 128)
    G = cols // 128
    _need(blocks, rows * G * 66, "blocks", fn)
    b = _hip.to_device(blocks, np.uint8).reshape(-1)
    meta = _hip.empty_device((rows * G * 4,), np.uint8)
    quant = _hip.empty_device(((rows + 3) // 4 * G * 256,), np.uint8)
    _hip.call("asdsl_repack_q4_128_to_preq2", _hip.ptr(b), _hip.ptr(meta), _hip.ptr(quant), rows, cols,
              _hip.stream_handle())
    return meta, quant
