"""Drop-in for the reference's ``_native_gemv`` pybind11 module, running on HIP.

Function names, argument order, defaults and out-parameter conventions follow
the reference bindings (asdsl/kernels/native/gemv_q4_avx2.cpp:1162-1506).
Arrays may be numpy arrays (uploaded, result copied back into the caller's
``y`` exactly like the pybind forcecast path) or device ``torch`` tensors
(zero-copy, asynchronous on the current stream).  Unlike the reference's
preq/preq2 bindings, which do not check sizes, every buffer is validated
against the shape before anything is launched (ValueError otherwise).
"""

from __future__ import annotations

import numpy as np

from asdsl import _hip
from asdsl.kernels._buffers import DeviceCall

has_q4km_gemv = False  # set True once the Q4_K kernel is linked (see bottom)


def _preq2_quant_bytes(M: int, K: int, gs: int) -> int:
    return ((M + 3) // 4) * (K // gs) * 4 * (gs // 2)


def _check_gs(gs: int, allowed, fn: str) -> None:
    if gs not in allowed:
        raise ValueError(f"{fn}: group_size must be {' or '.join(map(str, allowed))}")


def _check_dims(M: int, K: int, gs: int, fn: str) -> None:
    if M <= 0 or K <= 0:
        raise ValueError(f"{fn}: invalid dimensions")
    if K % gs:
        raise ValueError(f"{fn}: in_features must be divisible by group_size")


# ------------------------------------------------------------ activation Q8
def quantize_activation_avx2(x, x_q8, x_scales, in_features: int, group_size: int = 32) -> None:
    """Reference: quantize_activation_avx2 (gemv_q4_preq_restored.cpp:505-549)."""
    fn = "quantize_activation_avx2"
    _check_gs(group_size, (32, 64, 128), fn)
    _check_dims(1, in_features, group_size, fn)
    c = DeviceCall(fn)
    px = c.input(x, np.float32, in_features, "x")
    pq = c.output(x_q8, np.int8, in_features, "x_q8")
    ps = c.output(x_scales, np.float32, in_features // group_size, "x_scales")
    c.run("asdsl_quantize_activation", px, pq, ps, in_features, group_size)


# ------------------------------------------------------------ preq (20 B)
def gemv_q4_32_preq_avx2(blocks, x_q8, x_scales, y, out_features: int, in_features: int,
                         group_size: int = 32) -> None:
    """Reference: gemv_q4_32_preq_avx2 (gemv_q4_preq_restored.cpp:551-573)."""
    fn = "gemv_q4_32_preq_avx2"
    _check_gs(group_size, (32,), fn)
    _check_dims(out_features, in_features, group_size, fn)
    G = in_features // 32
    c = DeviceCall(fn)
    pb = c.input(blocks, np.uint8, out_features * G * 20, "blocks")
    pq = c.input(x_q8, np.int8, in_features, "x_q8")
    ps = c.input(x_scales, np.float32, G, "x_scales")
    py = c.output(y, np.float32, out_features, "y")
    c.run("asdsl_gemv_q4_32_preq", pb, pq, ps, py, out_features, in_features, group_size)


def _preq_fused(fn: str, blocks, x_fp32, y, out_features: int, in_features: int, group_size: int) -> None:
    _check_gs(group_size, (32,), fn)
    _check_dims(out_features, in_features, group_size, fn)
    G = in_features // 32
    c = DeviceCall(fn)
    pb = c.input(blocks, np.uint8, out_features * G * 20, "blocks")
    px = c.input(x_fp32, np.float32, in_features, "x_fp32")
    py = c.output(y, np.float32, out_features, "y")
    c.run("asdsl_gemv_q4_32_preq_fused", pb, px, py, out_features, in_features, group_size)


def gemv_q4_32_preq_fused_avx2(blocks, x_fp32, y, out_features: int, in_features: int, group_size: int = 32):
    """Reference: gemv_q4_32_preq_fused_avx2 (gemv_q4_preq_restored.cpp:652-669)."""
    _preq_fused("gemv_q4_32_preq_fused_avx2", blocks, x_fp32, y, out_features, in_features, group_size)


def gemv_q4_32_preq_4row_avx2(blocks, x_fp32, y, out_features: int, in_features: int, group_size: int = 32):
    """Reference: gemv_q4_32_preq_4row_avx2 (gemv_q4_preq_restored.cpp:575-597); same math as fused."""
    _preq_fused("gemv_q4_32_preq_4row_avx2", blocks, x_fp32, y, out_features, in_features, group_size)


def gemv_q4_32_preq_8row_avx2(blocks, x_fp32, y, out_features: int, in_features: int, group_size: int = 32):
    """Reference: gemv_q4_32_preq_8row_avx2 (gemv_q4_preq_restored.cpp:628-650); same math as fused."""
    _preq_fused("gemv_q4_32_preq_8row_avx2", blocks, x_fp32, y, out_features, in_features, group_size)


# ------------------------------------------------------------ preq2
def gemv_preq2_fused_avx2(meta, quant, x_fp32, y, out_features: int, in_features: int,
                          group_size: int = 32) -> None:
    """Reference: gemv_preq2_fused_avx2 (gemv_preq2_avx2.cpp:301-319).
    group_size=128 selects the asymmetric preq2-g128 layout (no reference counterpart)."""
    fn = "gemv_preq2_fused_avx2"
    _check_gs(group_size, (32, 128), fn)
    _check_dims(out_features, in_features, group_size, fn)
    G = in_features // group_size
    c = DeviceCall(fn)
    pm = c.input(meta, np.uint8, out_features * G * 4, "meta")
    pq = c.input(quant, np.uint8, _preq2_quant_bytes(out_features, in_features, group_size), "quant")
    px = c.input(x_fp32, np.float32, in_features, "x_fp32")
    py = c.output(y, np.float32, out_features, "y")
    c.run("asdsl_gemv_preq2_fused", pm, pq, px, py, out_features, in_features, group_size)


def gemv_preq2_avx2(meta, quant, x_q8, x_scales, y, out_features: int, in_features: int,
                    group_size: int = 32) -> None:
    """Reference: gemv_preq2_avx2 (gemv_preq2_avx2.cpp:321-337), pre-quantized activation."""
    fn = "gemv_preq2_avx2"
    _check_gs(group_size, (32, 128), fn)
    _check_dims(out_features, in_features, group_size, fn)
    G = in_features // group_size
    c = DeviceCall(fn)
    pm = c.input(meta, np.uint8, out_features * G * 4, "meta")
    pq = c.input(quant, np.uint8, _preq2_quant_bytes(out_features, in_features, group_size), "quant")
    pxq = c.input(x_q8, np.int8, in_features, "x_q8")
    pxs = c.input(x_scales, np.float32, G, "x_scales")
    py = c.output(y, np.float32, out_features, "y")
    c.run("asdsl_gemv_preq2", pm, pq, pxq, pxs, py, out_features, in_features, group_size)


# ------------------------------------------------------------ Q4_128
def gemv_q4_128_preq_avx2(blocks, x_q8, x_scales, y, out_features: int, in_features: int,
                          group_size: int = 128) -> None:
    """Reference: gemv_q4_128_preq_avx2 (gemv_q4_128.cpp:94-257), symmetric
    66-byte g128 blocks, activation pre-quantized per 128."""
    fn = "gemv_q4_128_preq_avx2"
    _check_gs(group_size, (128,), fn)
    _check_dims(out_features, in_features, group_size, fn)
    G = in_features // 128
    c = DeviceCall(fn)
    pb = c.input(blocks, np.uint8, out_features * G * 66, "blocks")
    pq = c.input(x_q8, np.int8, in_features, "x_q8")
    ps = c.input(x_scales, np.float32, G, "x_scales")
    py = c.output(y, np.float32, out_features, "y")
    c.run("asdsl_gemv_q4_128_preq", pb, pq, ps, py, out_features, in_features, group_size)


def gemv_q4_128_fused(blocks, x_fp32, y, out_features: int, in_features: int, group_size: int = 128) -> None:
    """Q4_128 GEMV that quantizes the fp32 activation per 128 inside the call
    (the engine's quantize + gemv_q4_128_preq_avx2 pair, unified_engine.cpp:1646-1653)."""
    fn = "gemv_q4_128_fused"
    _check_gs(group_size, (128,), fn)
    _check_dims(out_features, in_features, group_size, fn)
    G = in_features // 128
    c = DeviceCall(fn)
    pb = c.input(blocks, np.uint8, out_features * G * 66, "blocks")
    px = c.input(x_fp32, np.float32, in_features, "x_fp32")
    py = c.output(y, np.float32, out_features, "y")
    c.run("asdsl_gemv_q4_128_fused", pb, px, py, out_features, in_features, group_size)


def dequant_preq2(meta, quant, out_features: int, in_features: int, group_size: int = 32):
    """Dequantized fp32 W[M, K] = (q - z) * s of a preq2 matrix (debug/validation)."""
    fn = "dequant_preq2"
    _check_gs(group_size, (32, 128), fn)
    _check_dims(out_features, in_features, group_size, fn)
    G = in_features // group_size
    c = DeviceCall(fn)
    pm = c.input(meta, np.uint8, out_features * G * 4, "meta")
    pq = c.input(quant, np.uint8, _preq2_quant_bytes(out_features, in_features, group_size), "quant")
    w = np.empty((out_features, in_features), np.float32) if not _hip.is_device_tensor(meta) else \
        _hip.empty_device((out_features, in_features), np.float32)
    pw = c.output(w, np.float32, out_features * in_features, "w")
    c.run("asdsl_dequant_preq2", pm, pq, pw, out_features, in_features, group_size)
    return w


def check_avx2() -> bool:
    """The reference probes the CPU; here the compute device is the GPU."""
    return False


def check_fma() -> bool:
    return False


def check_avx512() -> bool:
    return False
