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
from asdsl.kernels._buffers import DeviceCall, new_output, shape_of

has_q4km_gemv = True


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


# ------------------------------------------------------------ diagnostic counters
# The reference counts gemv_q4_q8_avx2 calls (gemv_q4_avx2.cpp:129,140) and the
# preq GEMV's per-(row, group) single-group accumulations
# (gemv_q4_preq_restored.cpp:22-23,305,325): every group of every row goes
# through the classic accumulate unless the 4-group inner loop runs
# (ASDSL_PREQ_G4FUSED=1, or ASDSL_PREQ_G4GATE_UP_ONLY=1 with >= 8192 rows, or
# the g4fused entry point; gemv_q4_preq_restored.cpp:47-82,350-352), which
# leaves only the groups past the last multiple of 4.  The x-preloaded
# accumulate is never called there.  The same counts are kept here per call,
# so scripts that read them see the reference's values.
_q8_calls = 0
_preq_classic = 0
_preq_xloaded = 0


def _g4_inner(out_features: int, forced: bool) -> bool:
    import os

    if forced:
        return True
    if os.environ.get("ASDSL_PREQ_G4GATE_UP_ONLY", "")[:1] == "1":
        return out_features >= 8192
    v = os.environ.get("ASDSL_PREQ_G4FUSED", "")
    return bool(v) and v[0] != "0"


def _count_preq_groups(out_features: int, n_groups: int, g4_forced: bool) -> None:
    global _preq_classic
    use_g4 = n_groups >= 4 and n_groups % 4 == 0 and _g4_inner(out_features, g4_forced)
    _preq_classic += out_features * (n_groups - (n_groups // 4) * 4 if use_g4 else n_groups)


def get_q8_call_count() -> int:
    """Calls of gemv_q4_q8_avx2 so far (gemv_q4_avx2.cpp:1442)."""
    return _q8_calls


def get_preq_classic_accum_calls() -> int:
    """Single-group accumulations of the preq GEMVs since the last reset (gemv_q4_avx2.cpp:1445)."""
    return _preq_classic


def get_preq_xloaded_accum_calls() -> int:
    """x-preloaded single-group accumulations since the last reset (gemv_q4_avx2.cpp:1448)."""
    return _preq_xloaded


def reset_preq_accum_call_counts() -> None:
    """Reference: reset_preq_accum_call_counts (gemv_q4_avx2.cpp:1451)."""
    global _preq_classic, _preq_xloaded
    _preq_classic = 0
    _preq_xloaded = 0


def _affine_work(c: DeviceCall, M: int, K: int, group_size: int, batch: int):
    """A caller-owned work buffer (a device temporary of this call) for the
    batched fp32-affine GEMMs, or (None, 0) when the call runs per column."""
    nbytes = int(_hip.LIB.asdsl_affine_batch_work_bytes(M, K, group_size)) if batch > 1 else 0
    return (c.scratch(nbytes, np.uint8), nbytes) if nbytes else (None, 0)


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
    _count_preq_groups(out_features, G, False)


def _preq_fused(fn: str, blocks, x_fp32, y, out_features: int, in_features: int, group_size: int,
                g4: bool = False) -> None:
    _check_gs(group_size, (32,), fn)
    _check_dims(out_features, in_features, group_size, fn)
    G = in_features // 32
    c = DeviceCall(fn)
    pb = c.input(blocks, np.uint8, out_features * G * 20, "blocks")
    px = c.input(x_fp32, np.float32, in_features, "x_fp32")
    py = c.output(y, np.float32, out_features, "y")
    c.run("asdsl_gemv_q4_32_preq_fused", pb, px, py, out_features, in_features, group_size)
    _count_preq_groups(out_features, G, g4)


def gemv_q4_32_preq_fused_avx2(blocks, x_fp32, y, out_features: int, in_features: int, group_size: int = 32):
    """Reference: gemv_q4_32_preq_fused_avx2 (gemv_q4_preq_restored.cpp:652-669)."""
    _preq_fused("gemv_q4_32_preq_fused_avx2", blocks, x_fp32, y, out_features, in_features, group_size)


def gemv_q4_32_preq_4row_avx2(blocks, x_fp32, y, out_features: int, in_features: int, group_size: int = 32):
    """Reference: gemv_q4_32_preq_4row_avx2 (gemv_q4_preq_restored.cpp:575-597); same math as fused."""
    _preq_fused("gemv_q4_32_preq_4row_avx2", blocks, x_fp32, y, out_features, in_features, group_size)


def gemv_q4_32_preq_8row_avx2(blocks, x_fp32, y, out_features: int, in_features: int, group_size: int = 32):
    """Reference: gemv_q4_32_preq_8row_avx2 (gemv_q4_preq_restored.cpp:628-650); same math as fused."""
    _preq_fused("gemv_q4_32_preq_8row_avx2", blocks, x_fp32, y, out_features, in_features, group_size)


def gemv_q4_32_preq_g4fused_4row_avx2(blocks, x_fp32, y, out_features: int, in_features: int,
                                      group_size: int = 32):
    """Reference: gemv_q4_32_preq_g4fused_4row_avx2 (gemv_q4_preq_restored.cpp:603-626): the
    4-group inner loop forced on, same math as fused; the group count must be a
    multiple of 4 (and at most 640), as the reference requires."""
    fn = "gemv_q4_32_preq_g4fused_4row_avx2"
    _check_gs(group_size, (32,), fn)
    if out_features <= 0 or in_features <= 0:
        raise ValueError(f"{fn}: invalid dimensions")
    n_groups = in_features // group_size
    if n_groups > 640 or n_groups % 4:
        raise ValueError(f"{fn}: n_groups must be <= 640 and divisible by 4")
    _preq_fused(fn, blocks, x_fp32, y, out_features, in_features, group_size, g4=True)


# ------------------------------------------------------------ preq2
def gemv_preq2_fused_avx2(meta, quant, x_fp32, y, out_features: int, in_features: int,
                          group_size: int = 32) -> None:
    """Reference: gemv_preq2_fused_avx2 (gemv_preq2_avx2.cpp:301-319).
    group_size=128 selects the asymmetric preq2-g128 layout (no reference counterpart).
    A 2-D x_fp32 of shape (N, K) with y of shape (N, M) runs the batched
    verification kernel: every row of x is quantized on its own, so y[n]
    equals the 1-D call on x[n]."""
    fn = "gemv_preq2_fused_avx2"
    _check_gs(group_size, (32, 128), fn)
    _check_dims(out_features, in_features, group_size, fn)
    G = in_features // group_size
    xs = shape_of(x_fp32)
    n_cols = xs[0] if len(xs) == 2 else 1
    if len(xs) == 2 and xs[1] != in_features:
        raise ValueError(f"{fn}: x_fp32 must be (N, in_features)")
    c = DeviceCall(fn)
    pm = c.input(meta, np.uint8, out_features * G * 4, "meta")
    pq = c.input(quant, np.uint8, _preq2_quant_bytes(out_features, in_features, group_size), "quant")
    px = c.input(x_fp32, np.float32, n_cols * in_features, "x_fp32")
    py = c.output(y, np.float32, n_cols * out_features, "y")
    if len(xs) == 2:
        nbytes = int(_hip.LIB.asdsl_gemv_preq2_fused_batch_work_bytes(in_features))
        c.run("asdsl_gemv_preq2_fused_batch_ws", pm, pq, px, py, out_features, in_features, group_size, n_cols,
              c.scratch(nbytes, np.uint8), nbytes)
    else:
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


def _check_s256(out_features: int, in_features: int, fn: str) -> None:
    if out_features <= 0 or in_features <= 0:
        raise ValueError(f"{fn}: invalid dimensions")
    if in_features % 256:
        raise ValueError("gemv_q4_s256: in_features must be divisible by 256")


def gemv_q4_s256_preq_avx2(blocks, x_q8, x_scales, y, out_features: int, in_features: int,
                           group_size: int = 32) -> None:
    """Reference: gemv_q4_s256_preq_avx2 (gemv_q4_s256.cpp:79-209): 144-byte
    superblocks of 8 fp16 sub-scales + 128 nibble bytes, activation
    pre-quantized per 32 (group_size is the activation group, must be 32).
    The reference exposes it to its engine only (unified_engine.h:127)."""
    fn = "gemv_q4_s256_preq_avx2"
    _check_gs(group_size, (32,), fn)
    _check_s256(out_features, in_features, fn)
    c = DeviceCall(fn)
    pb = c.input(blocks, np.uint8, out_features * (in_features // 256) * 144, "blocks")
    pq = c.input(x_q8, np.int8, in_features, "x_q8")
    ps = c.input(x_scales, np.float32, in_features // 32, "x_scales")
    py = c.output(y, np.float32, out_features, "y")
    c.run("asdsl_gemv_q4_s256", pb, pq, ps, py, out_features, in_features, group_size)


def gemv_q4_s256_fused(blocks, x_fp32, y, out_features: int, in_features: int) -> None:
    """Q4_S256 GEMV that quantizes the fp32 activation per 32 (A1 rule) inside
    the call (the engine's quantize + gemv_q4_s256_preq_avx2 pair,
    unified_engine.cpp:1414-1416)."""
    fn = "gemv_q4_s256_fused"
    _check_s256(out_features, in_features, fn)
    c = DeviceCall(fn)
    pb = c.input(blocks, np.uint8, out_features * (in_features // 256) * 144, "blocks")
    px = c.input(x_fp32, np.float32, in_features, "x_fp32")
    py = c.output(y, np.float32, out_features, "y")
    c.run("asdsl_gemv_q4_s256_fused", pb, px, py, out_features, in_features)


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


# ------------------------------------------------------------ fp32 affine
def _numel(a) -> int:
    n = 1
    for d in shape_of(a):
        n *= d
    return n


def _validate_gemv_args(w, x, scales, biases, M: int, K: int, group_size: int, expected_w: int) -> int:
    """validate_gemv_args (gemv_q4_avx2.cpp:901-929) + assert_x_gemv_layout
    (1065-1082): same checks, same messages; returns the batch size."""
    if M <= 0 or K <= 0 or group_size <= 0:
        raise ValueError("M, K, group_size must be positive")
    xs = shape_of(x)
    if len(xs) == 1:
        batch = 1
        if xs[0] != K:
            raise ValueError("x length must equal K")
    elif len(xs) == 2:
        batch = xs[0]
        if xs[1] != K:
            raise ValueError("x shape must be (batch, K) matching arguments")
    else:
        raise ValueError("x must be 1-D (K,) or 2-D (batch, K)")
    if batch < 1:
        raise ValueError("batch must be >= 1")
    if K % 2 != 0:
        raise ValueError("K must be even for 4-bit packing")
    if K % group_size != 0:
        raise ValueError("K must be divisible by group_size")
    if group_size % 8 != 0:
        raise ValueError("group_size must be a multiple of 8 for AVX2 vectorization")
    if _numel(w) != expected_w:
        raise ValueError("weight buffer size mismatch")
    groups = M * (K // group_size)
    if _numel(scales) != groups:
        raise ValueError("scales size mismatch")
    if biases is not None and _numel(biases) != groups:
        raise ValueError("biases size mismatch")
    return batch


def gemv_q4_packed(w_packed, x, scales, biases, M: int, K: int, group_size: int):
    """Reference: gemv_q4_packed (gemv_q4_avx2.cpp:665-749, pybind 1084-1126).
    x (K,) -> y (M,); x (B, K) -> y (B, M)."""
    batch = _validate_gemv_args(w_packed, x, scales, biases, M, K, group_size, M * K // 2)
    if group_size % 16 != 0:
        raise ValueError("group_size must be a multiple of 16 for packed weights")
    y = new_output((M,) if len(shape_of(x)) == 1 else (batch, M), np.float32, w_packed, x)
    c = DeviceCall("gemv_q4_packed")
    work, nbytes = _affine_work(c, M, K, group_size, batch)
    c.run("asdsl_gemv_q4_packed_ws", c.input(w_packed, np.uint8, M * K // 2, "w_packed"),
          c.input(x, np.float32, batch * K, "x"), c.input(scales, np.float32, M * (K // group_size), "scales"),
          c.input(biases, np.float32, M * (K // group_size), "biases"), c.output(y, np.float32, batch * M, "y"),
          M, K, group_size, batch, work, nbytes)
    return y


def gemv_q4_unpacked(w, x, scales, biases, M: int, K: int, group_size: int):
    """Reference: gemv_q4_unpacked (gemv_q4_avx2.cpp:755-806, pybind 1128-1160);
    one byte per value, used as is."""
    _validate_gemv_args(w, x, scales, biases, M, K, group_size, M * K)
    if len(shape_of(x)) != 1:
        raise ValueError("x size must equal batch * K")
    y = new_output((M,), np.float32, w, x)
    c = DeviceCall("gemv_q4_unpacked")
    c.run("asdsl_gemv_q4_unpacked", c.input(w, np.uint8, M * K, "w"), c.input(x, np.float32, K, "x"),
          c.input(scales, np.float32, M * (K // group_size), "scales"),
          c.input(biases, np.float32, M * (K // group_size), "biases"), c.output(y, np.float32, M, "y"),
          M, K, group_size)
    return y


def gemv_q4_avx2_gs64(w_packed, x, scales, rows: int, cols: int):
    """Reference: gemv_q4_avx2_gs64 (gemv_q4_avx2.cpp:1211-1268 -> gemv_q4_kernel.cpp:96-122)."""
    if cols <= 0 or rows <= 0 or cols % 64 != 0 or cols % 2 != 0:
        raise ValueError("cols must be positive, even, and divisible by 64")
    if _numel(w_packed) != rows * (cols // 2):
        raise ValueError("w_packed size must be rows * (cols/2)")
    if _numel(scales) != rows * (cols // 64):
        raise ValueError("scales length must be rows * (cols/64)")
    xs = shape_of(x)
    batch = 1 if len(xs) == 1 else xs[0]
    if len(xs) not in (1, 2) or xs[-1] != cols or _numel(x) != batch * cols:
        raise ValueError("x size must equal batch * cols")
    y = new_output((rows,) if len(xs) == 1 else (batch, rows), np.float32, w_packed, x)
    c = DeviceCall("gemv_q4_avx2_gs64")
    work, nbytes = _affine_work(c, rows, cols, 64, batch)
    c.run("asdsl_gemv_q4_gs64_ws", c.input(w_packed, np.uint8, rows * cols // 2, "w_packed"),
          c.input(x, np.float32, batch * cols, "x"), c.input(scales, np.float32, rows * (cols // 64), "scales"),
          c.output(y, np.float32, batch * rows, "y"), rows, cols, batch, work, nbytes)
    return y


def gemv_q4_q8_avx2(weights_packed, scales, x, y, out_features: int, in_features: int,
                    group_size: int = 32) -> None:
    """Reference: gemv_q4_q8_avx2 (gemv_q4_avx2.cpp:131-253): symmetric packed Q4
    with fp32 scales, x quantized per group inside; y is an out-parameter."""
    fn = "gemv_q4_q8_avx2"
    _check_gs(group_size, (32, 64, 128), fn)
    _check_dims(out_features, in_features, group_size, fn)
    G = in_features // group_size
    c = DeviceCall(fn)
    c.run("asdsl_gemv_q4_q8", c.input(weights_packed, np.uint8, out_features * in_features // 2, "weights_packed"),
          c.input(scales, np.float32, out_features * G, "scales"), c.input(x, np.float32, in_features, "x"),
          c.output(y, np.float32, out_features, "y"), out_features, in_features, group_size)
    global _q8_calls
    _q8_calls += 1


def gemv_q4km_q8_avx2(weights_q4km, x, y, out_features: int, in_features: int) -> None:
    """Reference: gemv_q4km_q8_avx2 (gemv_q4_avx2.cpp:283-420, pybind 1318-1348)."""
    fn = "gemv_q4km_q8_avx2"
    if in_features <= 0 or out_features <= 0 or in_features % 256:
        raise ValueError("in_features must be divisible by 256 for Q4_K_M")
    expected = out_features * (in_features // 256) * 144
    if _numel(weights_q4km) != expected:
        raise ValueError("Q4_K_M weight size mismatch")
    if _numel(x) != in_features or _numel(y) != out_features:
        raise ValueError("x/y size mismatch for out_features/in_features")
    c = DeviceCall(fn)
    c.run("asdsl_gemv_q4km_q8", c.input(weights_q4km, np.uint8, expected, "weights_q4km"),
          c.input(x, np.float32, in_features, "x"), c.output(y, np.float32, out_features, "y"),
          out_features, in_features)


def matmul_batch_q4(w_packed, scales, biases, X_batch, Y_batch, M: int, K: int, B: int, group_size: int = 32) -> None:
    """Reference: matmul_batch_q4 (gemv_q4_avx2.cpp:950-1059): Y_batch (B, M) out-parameter,
    overwritten.  B <= 64 (beyond it the reference overruns its accumulators)."""
    xs, ys = shape_of(X_batch), shape_of(Y_batch)
    if len(xs) != 2 or xs[0] != B or xs[1] != K:
        raise ValueError("X_batch must be shape (B, K)")
    if len(ys) != 2 or ys[0] != B or ys[1] != M:
        raise ValueError("Y_batch must be shape (B, M), caller zero-init")
    if _numel(w_packed) != M * (K // 2):
        raise ValueError("w_packed size must equal M * K/2")
    if group_size <= 0 or K % group_size or _numel(scales) != M * (K // group_size):
        raise ValueError("scales size must equal M * n_groups")
    if _numel(biases) != M * (K // group_size):
        raise ValueError("biases size must equal M * n_groups")
    if B < 1 or B > 64:
        raise ValueError("B must be in [1, 64]")
    G = K // group_size
    c = DeviceCall("matmul_batch_q4")
    work, nbytes = _affine_work(c, M, K, group_size, B)
    c.run("asdsl_matmul_batch_q4_ws", c.input(w_packed, np.uint8, M * K // 2, "w_packed"),
          c.input(scales, np.float32, M * G, "scales"), c.input(biases, np.float32, M * G, "biases"),
          c.input(X_batch, np.float32, B * K, "X_batch"), c.output(Y_batch, np.float32, B * M, "Y_batch"),
          M, K, B, group_size, work, nbytes)


def gemm_q4_128_q8_avx2(blocks, x_batch, y_batch, out_features: int, in_features: int, group_size: int,
                        batch_size: int) -> None:
    """Reference: gemm_q4_128_q8_avx2 (gemv_q4_128.cpp:262-306), the engine's
    batched g128 GEMM: fp32 x (not quantized), y_batch (B, M) overwritten."""
    fn = "gemm_q4_128_q8_avx2"
    _check_gs(group_size, (128,), fn)
    _check_dims(out_features, in_features, group_size, fn)
    if batch_size < 1 or batch_size > 64:
        raise ValueError(f"{fn}: batch_size must be in [1, 64]")
    G = in_features // 128
    c = DeviceCall(fn)
    work, nbytes = _affine_work(c, out_features, in_features, 128, batch_size)
    c.run("asdsl_gemm_q4_128_ws", c.input(blocks, np.uint8, out_features * G * 66, "blocks"),
          c.input(x_batch, np.float32, batch_size * in_features, "x_batch"),
          c.output(y_batch, np.float32, batch_size * out_features, "y_batch"),
          out_features, in_features, group_size, batch_size, work, nbytes)


has_openmp = False


def get_num_threads() -> int:
    """The reference reports its CPU thread count; here the GPU's compute units."""
    return _hip.cu_count()


def set_num_threads(n: int) -> None:
    """No-op, as in the reference's own binding (gemv_q4_avx2.cpp:1496-1497)."""


def check_avx2() -> bool:
    """The reference probes the CPU; here the compute device is the GPU."""
    return False


def check_fma() -> bool:
    return False


def check_avx512() -> bool:
    return False


def check_vnni() -> bool:
    """The reference's VNNI probe (gemv_q4_avx2.cpp:1461); the integer dot
    products here run on the GPU's dot4 and MFMA instructions instead."""
    return False


def check_avx_vnni() -> bool:
    return False


def check_avx512_vnni() -> bool:
    return False


def get_cpu_topology() -> dict:
    """Reference: get_cpu_topology (gemv_q4_avx2.cpp:1470-1493).  Same keys and
    the values its non-Windows build returns; the compute device is the GPU."""
    return {"physical_logical_ids": [], "physical_core_count": 0, "pcore_count": 0,
            "avx_vnni": False, "avx512_vnni": False}
