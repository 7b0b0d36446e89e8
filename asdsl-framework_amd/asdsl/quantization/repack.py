"""Repackers into the byte layouts the GEMV kernels read.

Given device tensors, every function here runs its HIP kernel on the current
stream and returns device tensors (``asdsl.quantization._device_repack``);
given numpy arrays it runs the host restatement below.  Both produce the
reference's bytes.  Vectorized restatements of the reference's per-row
Python loops:
  * preq   20-byte blocks  — asdsl/quantization/repack_q4_32.py:63-108
  * preq2  meta + bands    — asdsl/quantization/repack_preq2.py:22-62
  * Q4_128 66-byte blocks  — asdsl/quantization/repack_q4_128.py:22-97
and the asymmetric preq2-g128 layout (no reference counterpart; same band
structure as preq2 with 64 nibble bytes per row slot and group):
  meta[M][K/128][4] (fp16 scale, fp16 zero) + quant[ceil(M/4)][K/128][256].
"""

from __future__ import annotations

import numpy as np

from asdsl.quantization.core import _unpack_bits, quantize_groups

PREQ_BLOCK_SIZE = 20
PREQ2_META_BYTES = 4
PREQ2_ROW_BAND = 4
Q4_128_BLOCK_SIZE = 66


def _f16_bits(a) -> np.ndarray:
    with np.errstate(over="ignore"):  # out-of-range zero points become inf, as numpy casts them
        return np.asarray(a, dtype=np.float16).view(np.uint16)


def _on_device(*arrays) -> bool:
    return any(type(a).__module__.startswith("torch") and getattr(a, "is_cuda", False) for a in arrays)


def _dev():
    from asdsl.quantization import _device_repack

    return _device_repack


def _floor_scale(scales) -> np.ndarray:
    """float(max(s, 1e-8)) per float32 scale s, as the reference forms it
    (repack_q4_32.py:87): Python's max keeps s unless 1e-8 > s, which numpy
    compares in float32; the result is the float64 1e-8 or s."""
    s = np.asarray(scales, np.float32)
    return np.where(np.float32(1e-8) > s, 1e-8, s.astype(np.float64))


def _nibbles(q: np.ndarray) -> np.ndarray:
    """q uint8 [..., n] (n even) -> packed [..., n/2], low nibble = even index."""
    return ((q[..., 0::2] & 0x0F) | ((q[..., 1::2] & 0x0F) << 4)).astype(np.uint8)


# ---------------------------------------------------------------- preq g32
def repack_asymmetric_to_q4_32_blocks(packed, scales, biases, rows: int, cols: int, group_size: int = 32,
                                      *, bits: int = 4) -> np.ndarray:
    """Packed Q4 + fp32 (scale, bias=-zero*scale) -> (rows, G, 20) preq blocks.

    zero = -bias/max(scale, 1e-8) is formed in float64 and rounded to fp16, as
    the reference does with Python floats (repack_q4_32.py:84-97)."""
    if group_size != 32:
        raise ValueError("repack_asymmetric_to_q4_32_blocks requires group_size=32")
    if _on_device(packed, scales, biases):
        return _dev().asym_to_q4_32(packed, scales, biases, rows, cols)
    G = cols // group_size
    q = _unpack_bits(np.asarray(packed, np.uint8).reshape(rows, cols // 2), bits).reshape(rows, G, 32)
    sc = _floor_scale(np.asarray(scales, np.float32).reshape(rows, G))
    bi = np.asarray(biases, np.float32).reshape(rows, G).astype(np.float64)
    zero = -bi / sc
    blocks = np.empty((rows, G, PREQ_BLOCK_SIZE), np.uint8)
    blocks[:, :, 0:2] = _f16_bits(sc).reshape(rows, G, 1).view(np.uint8).reshape(rows, G, 2)
    blocks[:, :, 2:4] = _f16_bits(zero).reshape(rows, G, 1).view(np.uint8).reshape(rows, G, 2)
    blocks[:, :, 4:] = _nibbles(q)
    return np.ascontiguousarray(blocks)


def blocks_to_flat(blocks):
    rows, n_groups, bs = blocks.shape
    if _on_device(blocks):
        return blocks.reshape(rows, n_groups * bs).contiguous()
    return np.ascontiguousarray(blocks.reshape(rows, n_groups * bs))


# ---------------------------------------------------------------- preq2
def repack_preq_blocks_to_preq2(flat_preq, rows: int, cols: int, group_size: int = 32):
    """20-byte preq rows -> (meta (rows, G*4), quant (n_bands, G, 64))."""
    if group_size != 32:
        raise ValueError("preq2 repack requires group_size=32")
    if _on_device(flat_preq):
        return _dev().preq_to_preq2(flat_preq, rows, cols)
    G = cols // group_size
    flat = np.ravel(np.asarray(flat_preq, np.uint8))
    if flat.size < rows * G * PREQ_BLOCK_SIZE:
        raise ValueError("flat_preq too small for shape")
    blocks = flat[: rows * G * PREQ_BLOCK_SIZE].reshape(rows, G, PREQ_BLOCK_SIZE)
    meta = np.ascontiguousarray(blocks[:, :, 0:4].reshape(rows, G * PREQ2_META_BYTES))
    return meta, _bands(blocks[:, :, 4:20], rows, G, 16)


def _bands(nib: np.ndarray, rows: int, G: int, nbytes: int) -> np.ndarray:
    """nib (rows, G, nbytes) -> (n_bands, G, 4*nbytes), zero-padded tail band."""
    n_bands = (rows + PREQ2_ROW_BAND - 1) // PREQ2_ROW_BAND
    padded = np.zeros((n_bands * PREQ2_ROW_BAND, G, nbytes), np.uint8)
    padded[:rows] = nib
    return np.ascontiguousarray(
        padded.reshape(n_bands, PREQ2_ROW_BAND, G, nbytes).transpose(0, 2, 1, 3).reshape(n_bands, G, 4 * nbytes))


def preq2_flat_sizes(rows: int, cols: int, group_size: int = 32) -> tuple[int, int]:
    G = cols // group_size
    n_bands = (rows + PREQ2_ROW_BAND - 1) // PREQ2_ROW_BAND
    return rows * G * PREQ2_META_BYTES, n_bands * G * 4 * (group_size // 2)


def meta_to_flat(meta):
    if _on_device(meta):
        return meta.reshape(-1).contiguous()
    return np.ascontiguousarray(meta.reshape(-1))


def quant_to_flat(quant):
    if _on_device(quant):
        return quant.reshape(-1).contiguous()
    return np.ascontiguousarray(quant.reshape(-1))


def repack_asymmetric_to_preq2(packed, scales, biases, rows: int, cols: int, group_size: int = 32):
    """Packed Q4 + fp32 (scale, bias) -> flat preq2 (meta, quant) at group
    size 32 (byte for byte repack_asymmetric_to_q4_32_blocks then
    repack_preq_blocks_to_preq2) or 128 (the same fp16 pair per group, 4-row
    bands of 64-byte row slots)."""
    if group_size not in (32, 128):
        raise ValueError("repack_asymmetric_to_preq2: group_size must be 32 or 128")
    if _on_device(packed, scales, biases):
        return _dev().asym_to_preq2(packed, scales, biases, rows, cols, group_size)
    G = cols // group_size
    sc = _floor_scale(np.asarray(scales, np.float32).reshape(rows, G))
    zero = -np.asarray(biases, np.float32).reshape(rows, G).astype(np.float64) / sc
    meta = np.empty((rows, G, 2), np.uint16)
    meta[:, :, 0] = _f16_bits(sc)
    meta[:, :, 1] = _f16_bits(zero)
    nib = np.asarray(packed, np.uint8).reshape(rows, G, group_size // 2)
    return meta.view(np.uint8).reshape(-1), _bands(nib, rows, G, group_size // 2).reshape(-1)


def repack_q4_128_blocks_to_preq2(blocks, rows: int, cols: int) -> tuple:
    """Q4_128 blocks (rows, cols/128, 66) -> flat preq2-g128 (meta, quant):
    the symmetric group as scale s, zero 8 (no reference counterpart; lets
    g128 preq caches feed the preq2-g128 GEMVs)."""
    if _on_device(blocks):
        return _dev().q4_128_to_preq2(blocks, rows, cols)
    G = cols // 128
    b = np.asarray(blocks, np.uint8).reshape(rows, G, Q4_128_BLOCK_SIZE)
    meta = np.empty((rows, G, 2), np.uint16)
    meta[:, :, 0] = b[:, :, 0:2].copy().view(np.uint16)[:, :, 0]
    meta[:, :, 1] = _f16_bits(8.0)
    return meta.view(np.uint8).reshape(-1), _bands(b[:, :, 2:], rows, G, 64).reshape(-1)


def pack_preq2(q: np.ndarray, scale_f16: np.ndarray, zero_f16: np.ndarray, rows: int, cols: int,
               group_size: int) -> tuple[np.ndarray, np.ndarray]:
    """Quantized values q (rows, cols) in 0..15 with fp16 (scale, zero) per
    (row, group) -> flat (meta, quant) in the preq2 / preq2-g128 layout."""
    G = cols // group_size
    meta = np.empty((rows, G, 2), np.uint16)
    meta[:, :, 0] = _f16_bits(scale_f16).reshape(rows, G)
    meta[:, :, 1] = _f16_bits(zero_f16).reshape(rows, G)
    nib = _nibbles(np.asarray(q, np.uint8).reshape(rows, G, group_size))
    return meta.view(np.uint8).reshape(-1), _bands(nib, rows, G, group_size // 2).reshape(-1)


def quantize_preq2(weights: np.ndarray, group_size: int = 32) -> tuple[np.ndarray, np.ndarray]:
    """fp32 W (rows, cols) -> flat preq2 (gs=32) or preq2-g128 (gs=128) buffers.

    Follows the reference chain quantize_weights -> store bias -> preq repack
    (core.py:358-424; phi4_cpu_run.py:3130-3140; repack_q4_32.py:84-97), so the
    zero written is f16(-f32(-zero*scale)/scale)."""
    w = np.asarray(weights, np.float32)
    rows, cols = w.shape
    if cols % group_size:
        raise ValueError("cols must be a multiple of group_size")
    q, s16, z16 = quantize_groups(w, 4, group_size, symmetric=False)
    sc = s16.astype(np.float32)
    bi = (-z16.astype(np.float32) * sc).astype(np.float32)
    sc64 = _floor_scale(sc)
    zero = -bi.astype(np.float64) / sc64
    return pack_preq2(q.reshape(rows, cols), sc64.astype(np.float16), zero.astype(np.float16),
                      rows, cols, group_size)


# ---------------------------------------------------------------- Q4_128
def q4_128_groups(wg: np.ndarray) -> tuple[np.ndarray, np.ndarray]:
    """Symmetric g128 quantizer (repack_q4_128.py:22-31) over groups wg (n, 128):
    scale = f16(amax/7) (float64), q = clip(rne(w*f32(7/amax)) + 8, 0, 15);
    an all-zero group (amax < 1e-12) gets scale 0 and q = 8."""
    wg = np.asarray(wg, np.float32)
    amax = np.abs(wg).max(axis=1).astype(np.float64)
    tiny = amax < 1e-12
    safe = np.where(tiny, 1.0, amax)
    inv32 = (7.0 / safe).astype(np.float32)
    q = np.clip(np.round(wg * inv32[:, None]) + np.float32(8.0), 0, 15).astype(np.uint8)
    q[tiny] = 8
    scale = np.where(tiny, 0.0, amax / 7.0)
    return q, scale.astype(np.float16)


def repack_fp32_to_q4_128_blocks(weights, rows: int, cols: int, group_size: int = 128) -> np.ndarray:
    if group_size != 128:
        raise ValueError("repack_fp32_to_q4_128_blocks requires group_size=128")
    if _on_device(weights):
        return _dev().fp32_to_q4_128(weights, rows, cols)
    G = cols // 128
    q, s16 = q4_128_groups(np.asarray(weights, np.float32).reshape(rows * G, 128))
    blocks = np.empty((rows, G, Q4_128_BLOCK_SIZE), np.uint8)
    blocks[:, :, 0:2] = _f16_bits(s16).reshape(rows, G, 1).view(np.uint8).reshape(rows, G, 2)
    blocks[:, :, 2:] = _nibbles(q).reshape(rows, G, 64)
    return np.ascontiguousarray(blocks)


def repack_asymmetric_to_q4_128_blocks(packed, scales, biases, rows: int, cols: int, group_size: int = 128,
                                       *, bits: int = 4) -> np.ndarray:
    """Asymmetric packed (gs=128 scale/bias) -> symmetric Q4_128 blocks
    (repack_q4_128.py:34-68): dequantize with zero=-bias/scale (float64), then
    requantize symmetric per group."""
    if group_size != 128:
        raise ValueError("repack_asymmetric_to_q4_128_blocks requires group_size=128")
    if _on_device(packed, scales, biases):
        return _dev().asym_to_q4_128(packed, scales, biases, rows, cols)
    G = cols // 128
    q = _unpack_bits(np.asarray(packed, np.uint8).reshape(rows, cols // 2), bits).reshape(rows * G, 128)
    sc = _floor_scale(np.asarray(scales, np.float32).reshape(-1))
    zero = -np.asarray(biases, np.float32).reshape(-1).astype(np.float64) / sc
    # (q - zero) * scale with q float32 and Python-float operands -> float32 result
    w_f = ((q.astype(np.float32) - zero.astype(np.float32)[:, None]) * sc.astype(np.float32)[:, None])
    qq, s16 = q4_128_groups(w_f)
    blocks = np.empty((rows, G, Q4_128_BLOCK_SIZE), np.uint8)
    blocks[:, :, 0:2] = _f16_bits(s16).reshape(rows, G, 1).view(np.uint8).reshape(rows, G, 2)
    blocks[:, :, 2:] = _nibbles(qq).reshape(rows, G, 64)
    return np.ascontiguousarray(blocks)
