"""CPU oracle for the Q4 GEMV hot path — TEST INFRASTRUCTURE ONLY.

Only ``tests/``, ``__graft_entry__.smoke()`` and ``bench.py``'s cpu_baseline leg
may import this package.  It is the parity checker, never the thing measured
or shipped: the product path (``asdsl`` under ``asdsl-framework_amd/``) never
imports it and fails loudly when its HIP library is missing.

Two checkers live here:

* ``liboracle.so`` — a scalar C restatement of the reference formulas
  (``asdsl_oracle.c``), wrapped below with numpy in/out.
* ``_ref/`` — the reference's own AVX2 kernels compiled unchanged from its
  sources by ``make -C oracle ref`` (only where the reference tree is mounted;
  the built modules travel with the repository).  :func:`load_reference`
  imports them as the pybind11 modules the reference exposes.
"""

from __future__ import annotations

import ctypes
import importlib.machinery
import importlib.util
import os
import subprocess
from pathlib import Path

import numpy as np

ORACLE_DIR = Path(__file__).resolve().parent
# ASDSL_ORACLE_LIB names another build of asdsl_oracle.c (the sanitized one).
LIB_PATH = Path(os.environ.get("ASDSL_ORACLE_LIB") or ORACLE_DIR / "lib" / "liboracle.so")
REF_DIR = ORACLE_DIR / "_ref"
REFERENCE_TREE = Path("/root/reference")

_lib = None
_c_f32p = ctypes.POINTER(ctypes.c_float)
_c_i8p = ctypes.POINTER(ctypes.c_int8)
_c_u8p = ctypes.POINTER(ctypes.c_uint8)


def build(with_reference: bool | None = None) -> None:
    """Compile liboracle.so and, when the reference tree is present, oracle/_ref."""
    subprocess.run(["make", "-s", "-C", str(ORACLE_DIR)], check=True)
    if with_reference is None:
        with_reference = REFERENCE_TREE.is_dir()
    if with_reference:
        subprocess.run(["make", "-s", "-C", str(ORACLE_DIR), "ref"], check=True)


def lib() -> ctypes.CDLL:
    global _lib
    if _lib is None:
        if not LIB_PATH.exists():
            build(with_reference=False)
        _lib = ctypes.CDLL(str(LIB_PATH))
    return _lib


def _p(a: np.ndarray, ctype):
    return a.ctypes.data_as(ctype)


def _u8(a) -> np.ndarray:
    return np.ascontiguousarray(a, dtype=np.uint8).reshape(-1)


def _f32(a) -> np.ndarray:
    return np.ascontiguousarray(a, dtype=np.float32)


def _i8(a) -> np.ndarray:
    return np.ascontiguousarray(a, dtype=np.int8).reshape(-1)


# --------------------------------------------------------------- restatement
def quantize_activation(x, group_size: int = 32) -> tuple[np.ndarray, np.ndarray]:
    x = _f32(x).reshape(-1)
    K = x.shape[0]
    xq = np.empty(K, np.int8)
    xs = np.empty(K // group_size, np.float32)
    lib().oracle_quantize_activation(_p(x, _c_f32p), _p(xq, _c_i8p), _p(xs, _c_f32p), K, group_size)
    return xq, xs


def gemv_preq(blocks, x_q8, x_scales, M: int, K: int) -> np.ndarray:
    blocks, xq, xs = _u8(blocks), _i8(x_q8), _f32(x_scales)
    y = np.empty(M, np.float32)
    lib().oracle_gemv_preq(_p(blocks, _c_u8p), _p(xq, _c_i8p), _p(xs, _c_f32p), _p(y, _c_f32p), M, K)
    return y


def gemv_preq_fused(blocks, x, M: int, K: int) -> np.ndarray:
    xq, xs = quantize_activation(x, 32)
    return gemv_preq(blocks, xq, xs, M, K)


def gemv_preq2(meta, quant, x_q8, x_scales, M: int, K: int, group_size: int = 32) -> np.ndarray:
    meta, quant, xq, xs = _u8(meta), _u8(quant), _i8(x_q8), _f32(x_scales)
    y = np.empty(M, np.float32)
    lib().oracle_gemv_preq2(_p(meta, _c_u8p), _p(quant, _c_u8p), _p(xq, _c_i8p), _p(xs, _c_f32p),
                            _p(y, _c_f32p), M, K, group_size)
    return y


def gemv_preq2_f32sum(meta, quant, x_q8, x_scales, M: int, K: int, group_size: int = 32) -> np.ndarray:
    """gemv_preq2 with the group terms summed in float32 in group order (a
    second restatement that differs from gemv_preq2 only in that rounding)."""
    meta, quant, xq, xs = _u8(meta), _u8(quant), _i8(x_q8), _f32(x_scales)
    y = np.empty(M, np.float32)
    lib().oracle_gemv_preq2_f32sum(_p(meta, _c_u8p), _p(quant, _c_u8p), _p(xq, _c_i8p), _p(xs, _c_f32p),
                                   _p(y, _c_f32p), M, K, group_size)
    return y


def gemv_preq2_fused_f32sum(meta, quant, x, M: int, K: int, group_size: int = 32) -> np.ndarray:
    xq, xs = quantize_activation(x, group_size)
    return gemv_preq2_f32sum(meta, quant, xq, xs, M, K, group_size)


def gemv_preq2_fused(meta, quant, x, M: int, K: int, group_size: int = 32) -> np.ndarray:
    xq, xs = quantize_activation(x, group_size)
    return gemv_preq2(meta, quant, xq, xs, M, K, group_size)


def dequant_preq2(meta, quant, M: int, K: int, group_size: int = 32) -> np.ndarray:
    meta, quant = _u8(meta), _u8(quant)
    w = np.empty((M, K), np.float32)
    lib().oracle_dequant_preq2(_p(meta, _c_u8p), _p(quant, _c_u8p), _p(w, _c_f32p), M, K, group_size)
    return w


def dequant_preq(blocks, M: int, K: int) -> np.ndarray:
    blocks = _u8(blocks)
    w = np.empty((M, K), np.float32)
    lib().oracle_dequant_preq(_p(blocks, _c_u8p), _p(w, _c_f32p), M, K)
    return w


def half_to_float(bits: int) -> float:
    f = lib().oracle_half_to_float
    f.restype = ctypes.c_float
    f.argtypes = [ctypes.c_uint16]
    return float(f(bits))


# ------------------------------------------------------ compiled reference
_ref_modules: dict[str, object] = {}


def reference_available(name: str = "_native_gemv") -> bool:
    return (REF_DIR / f"{name}.so").exists()


def load_reference(name: str = "_native_gemv"):
    """Import one of the reference's pybind11 modules built under oracle/_ref."""
    if name in _ref_modules:
        return _ref_modules[name]
    path = REF_DIR / f"{name}.so"
    if not path.exists():
        raise FileNotFoundError(f"{path} not built (make -C oracle ref needs the reference tree)")
    loader = importlib.machinery.ExtensionFileLoader(name, str(path))
    spec = importlib.util.spec_from_file_location(name, str(path), loader=loader)
    mod = importlib.util.module_from_spec(spec)
    loader.exec_module(mod)
    _ref_modules[name] = mod
    return mod


# ----------------------------------------------------------- more restatements
def gemv_q4_128(blocks, x_q8, x_scales, M: int, K: int) -> np.ndarray:
    blocks, xq, xs = _u8(blocks), _i8(x_q8), _f32(x_scales)
    y = np.empty(M, np.float32)
    lib().oracle_gemv_q4_128(_p(blocks, _c_u8p), _p(xq, _c_i8p), _p(xs, _c_f32p), _p(y, _c_f32p), M, K)
    return y


def gemm_q4_128(blocks, X, M: int, K: int, B: int) -> np.ndarray:
    blocks, X = _u8(blocks), _f32(X)
    Y = np.zeros((B, M), np.float32)
    lib().oracle_gemm_q4_128(_p(blocks, _c_u8p), _p(X, _c_f32p), _p(Y, _c_f32p), M, K, B)
    return Y


def gemv_q4_q8(w_packed, scales, x, M: int, K: int, group_size: int = 32) -> np.ndarray:
    w, s, x = _u8(w_packed), _f32(scales), _f32(x).reshape(-1)
    y = np.empty(M, np.float32)
    sq = np.empty(K, np.int8)
    ss = np.empty(K // group_size, np.float32)
    lib().oracle_gemv_q4_q8(_p(w, _c_u8p), _p(s, _c_f32p), _p(x, _c_f32p), _p(y, _c_f32p), M, K, group_size,
                            _p(sq, _c_i8p), _p(ss, _c_f32p))
    return y


def quantize_activation_q4k(x) -> tuple[np.ndarray, np.ndarray]:
    x = _f32(x).reshape(-1)
    K = x.shape[0]
    xq = np.empty(K, np.int8)
    xs = np.empty(K // 32, np.float32)
    lib().oracle_quantize_activation_q4k(_p(x, _c_f32p), _p(xq, _c_i8p), _p(xs, _c_f32p), K)
    return xq, xs


def gemv_q4km(w, x, M: int, K: int) -> np.ndarray:
    w, x = _u8(w), _f32(x).reshape(-1)
    y = np.empty(M, np.float32)
    sq = np.empty(K, np.int8)
    ss = np.empty(K // 32, np.float32)
    lib().oracle_gemv_q4km(_p(w, _c_u8p), _p(x, _c_f32p), _p(y, _c_f32p), M, K, _p(sq, _c_i8p), _p(ss, _c_f32p))
    return y


def gemv_affine(w, x, scales, biases, M: int, K: int, group_size: int, packed: bool = True) -> np.ndarray:
    w, x, s = _u8(w), _f32(x).reshape(-1), _f32(scales)
    b = None if biases is None else _f32(biases)
    y = np.empty(M, np.float32)
    lib().oracle_gemv_affine(_p(w, _c_u8p), int(packed), _p(x, _c_f32p), _p(s, _c_f32p),
                             None if b is None else _p(b, _c_f32p), _p(y, _c_f32p), M, K, group_size)
    return y


def gemv_q4_gs64(w, x, scales, M: int, K: int) -> np.ndarray:
    return gemv_affine(w, x, scales, None, M, K, 64, packed=True)


def matmul_batch_q4(w, scales, biases, X, M: int, K: int, B: int, group_size: int = 32) -> np.ndarray:
    w, s, b, X = _u8(w), _f32(scales), _f32(biases), _f32(X)
    Y = np.zeros((B, M), np.float32)
    lib().oracle_matmul_batch_q4(_p(w, _c_u8p), _p(s, _c_f32p), _p(b, _c_f32p), _p(X, _c_f32p), _p(Y, _c_f32p),
                                 M, K, B, group_size)
    return Y


def compute_bitmask(x, threshold: float) -> np.ndarray:
    x = _f32(x).reshape(-1)
    K = x.shape[0]
    m = np.zeros((K + 31) // 32, np.uint32)
    f = lib().oracle_compute_bitmask
    f.argtypes = [_c_f32p, ctypes.POINTER(ctypes.c_uint32), ctypes.c_int, ctypes.c_float]
    f(_p(x, _c_f32p), m.ctypes.data_as(ctypes.POINTER(ctypes.c_uint32)), K, float(threshold))
    return m


def gemv_sparse_indices(w, x, scales, biases, idx, M: int, K: int, group_size: int) -> np.ndarray:
    w, x, s, b = _u8(w), _f32(x).reshape(-1), _f32(scales), _f32(biases)
    idx = np.ascontiguousarray(idx, np.int32).reshape(-1)
    y = np.empty(M, np.float32)
    lib().oracle_gemv_sparse_indices(_p(w, _c_u8p), _p(x, _c_f32p), _p(s, _c_f32p), _p(b, _c_f32p),
                                     idx.ctypes.data_as(ctypes.POINTER(ctypes.c_int32)), idx.size,
                                     _p(y, _c_f32p), M, K, group_size)
    return y


def bitmask_indices(mask, K: int) -> np.ndarray:
    bits = np.unpackbits(np.ascontiguousarray(mask, np.uint32).view(np.uint8), bitorder="little")[:K]
    return np.nonzero(bits)[0].astype(np.int32)


def sparse_down_proj_T(wT, sT, bT, x, rows, in_dim: int, out_dim: int, group_size: int) -> np.ndarray:
    wT, sT, bT, x = _u8(wT), _f32(sT), _f32(bT), _f32(x).reshape(-1)
    rows = np.ascontiguousarray(rows, np.int32).reshape(-1)
    y = np.empty(out_dim, np.float32)
    lib().oracle_sparse_down_proj_T(_p(wT, _c_u8p), _p(sT, _c_f32p), _p(bT, _c_f32p), _p(x, _c_f32p),
                                    rows.ctypes.data_as(ctypes.POINTER(ctypes.c_int32)), rows.size,
                                    _p(y, _c_f32p), in_dim, out_dim, group_size)
    return y


# -------------------------------------------------------------------- repack
_c_u16p = ctypes.POINTER(ctypes.c_uint16)
_c_f64p = ctypes.POINTER(ctypes.c_double)


def double_to_half(d) -> np.ndarray:
    """float64 -> fp16 bits (uint16), round to nearest even."""
    d = np.ascontiguousarray(d, dtype=np.float64).reshape(-1)
    out = np.empty(d.size, np.uint16)
    lib().oracle_double_to_half(_p(d, _c_f64p), _p(out, _c_u16p), d.size)
    return out


def repack_asym_to_q4_32(packed, scales, biases, rows: int, cols: int) -> np.ndarray:
    """repack_q4_32.py:63-102 -> flat 20-byte preq blocks (rows * cols/32 * 20)."""
    pk, sc, bi = _u8(packed), _f32(scales).reshape(-1), _f32(biases).reshape(-1)
    out = np.empty(rows * (cols // 32) * 20, np.uint8)
    lib().oracle_repack_asym_to_q4_32(_p(pk, _c_u8p), _p(sc, _c_f32p), _p(bi, _c_f32p), _p(out, _c_u8p), rows, cols)
    return out


def _preq2_sizes(rows: int, cols: int, gs: int) -> tuple[int, int]:
    G = cols // gs
    return rows * G * 4, (rows + 3) // 4 * G * 2 * gs


def repack_preq_to_preq2(preq, rows: int, cols: int) -> tuple[np.ndarray, np.ndarray]:
    """repack_preq2.py:22-49 -> flat (meta, quant)."""
    pq = _u8(preq)
    mb, qb = _preq2_sizes(rows, cols, 32)
    meta, quant = np.empty(mb, np.uint8), np.empty(qb, np.uint8)
    lib().oracle_repack_preq_to_preq2(_p(pq, _c_u8p), _p(meta, _c_u8p), _p(quant, _c_u8p), rows, cols)
    return meta, quant


def repack_asym_to_preq2(packed, scales, biases, rows: int, cols: int, group_size: int = 32):
    """Asymmetric packed Q4 -> flat preq2 (meta, quant) at group size 32 or 128."""
    pk, sc, bi = _u8(packed), _f32(scales).reshape(-1), _f32(biases).reshape(-1)
    mb, qb = _preq2_sizes(rows, cols, group_size)
    meta, quant = np.empty(mb, np.uint8), np.empty(qb, np.uint8)
    lib().oracle_repack_asym_to_preq2(_p(pk, _c_u8p), _p(sc, _c_f32p), _p(bi, _c_f32p), _p(meta, _c_u8p),
                                      _p(quant, _c_u8p), rows, cols, group_size)
    return meta, quant


def repack_fp32_to_q4_128(w, rows: int, cols: int) -> np.ndarray:
    """repack_q4_128.py:72-92 -> flat 66-byte Q4_128 blocks."""
    wf = _f32(w).reshape(-1)
    out = np.empty(rows * (cols // 128) * 66, np.uint8)
    lib().oracle_repack_fp32_to_q4_128(_p(wf, _c_f32p), _p(out, _c_u8p), rows, cols)
    return out


def repack_asym_to_q4_128(packed, scales, biases, rows: int, cols: int) -> np.ndarray:
    """repack_q4_128.py:34-69 -> flat 66-byte Q4_128 blocks."""
    pk, sc, bi = _u8(packed), _f32(scales).reshape(-1), _f32(biases).reshape(-1)
    out = np.empty(rows * (cols // 128) * 66, np.uint8)
    lib().oracle_repack_asym_to_q4_128(_p(pk, _c_u8p), _p(sc, _c_f32p), _p(bi, _c_f32p), _p(out, _c_u8p), rows,
                                       cols)
    return out


def repack_q4_128_to_preq2(blocks, rows: int, cols: int) -> tuple[np.ndarray, np.ndarray]:
    """Q4_128 blocks -> flat preq2-g128 (meta, quant) with zero 8."""
    b = _u8(blocks)
    mb, qb = _preq2_sizes(rows, cols, 128)
    meta, quant = np.empty(mb, np.uint8), np.empty(qb, np.uint8)
    lib().oracle_repack_q4_128_to_preq2(_p(b, _c_u8p), _p(meta, _c_u8p), _p(quant, _c_u8p), rows, cols)
    return meta, quant


def gemv_q4_s256(blocks, x_q8, x_scales, M: int, K: int) -> np.ndarray:
    """gemv_q4_s256_preq_avx2 restated (activation groups of 32)."""
    b, xq, xs = _u8(blocks), _i8(x_q8), _f32(x_scales).reshape(-1)
    y = np.empty(M, np.float32)
    lib().oracle_gemv_q4_s256(_p(b, _c_u8p), _p(xq, _c_i8p), _p(xs, _c_f32p), _p(y, _c_f32p), M, K)
    return y


def reference_q4_s256():
    """The reference's own Q4_S256 kernel (oracle/_ref/libref_q4_s256.so) as
    f(blocks, x_q8, x_scales, M, K) -> y, or None when it is not built."""
    path = REF_DIR / "libref_q4_s256.so"
    if not path.exists():
        return None
    so = ctypes.CDLL(str(path))

    def run(blocks, x_q8, x_scales, M: int, K: int) -> np.ndarray:
        b, xq, xs = _u8(blocks), _i8(x_q8), _f32(x_scales).reshape(-1)
        y = np.empty(M, np.float32)
        so.ref_gemv_q4_s256(_p(b, _c_u8p), _p(xq, _c_i8p), _p(xs, _c_f32p), _p(y, _c_f32p), ctypes.c_int(M),
                            ctypes.c_int(K))
        return y
    return run


# ------------------------------------------------------------------ GGUF
def _blocks_in(blocks, n_blocks: int, block_bytes: int) -> np.ndarray:
    """The block bytes as uint8, refusing a buffer shorter than n_blocks blocks
    (the C routines read n_blocks * block_bytes bytes)."""
    b = _u8(blocks)
    if n_blocks < 0 or b.size < n_blocks * block_bytes:
        raise ValueError(f"{n_blocks} blocks of {block_bytes} bytes need {n_blocks * block_bytes} bytes, got {b.size}")
    return b


def dequant_gguf_q4k(blocks, n_blocks: int) -> np.ndarray:
    """ggml Q4_K blocks (144 bytes per 256 weights) -> float32 weights."""
    b = _blocks_in(blocks, n_blocks, 144)
    w = np.empty(n_blocks * 256, np.float32)
    lib().oracle_dequant_gguf_q4k(_p(b, _c_u8p), _p(w, _c_f32p), ctypes.c_size_t(n_blocks))
    return w


def dequant_gguf_q6k(blocks, n_blocks: int) -> np.ndarray:
    """ggml Q6_K blocks (210 bytes per 256 weights) -> float32 weights."""
    b = _blocks_in(blocks, n_blocks, 210)
    w = np.empty(n_blocks * 256, np.float32)
    lib().oracle_dequant_gguf_q6k(_p(b, _c_u8p), _p(w, _c_f32p), ctypes.c_size_t(n_blocks))
    return w


def dequant_gguf_q5k(blocks, n_blocks: int) -> np.ndarray:
    """ggml Q5_K blocks (176 bytes per 256 weights) -> float32 weights."""
    b = _blocks_in(blocks, n_blocks, 176)
    w = np.empty(n_blocks * 256, np.float32)
    lib().oracle_dequant_gguf_q5k(_p(b, _c_u8p), _p(w, _c_f32p), ctypes.c_size_t(n_blocks))
    return w


def dequant_gguf_q8_0(blocks, n_blocks: int) -> np.ndarray:
    """ggml Q8_0 blocks (34 bytes per 32 weights) -> float32 weights."""
    b = _blocks_in(blocks, n_blocks, 34)
    w = np.empty(n_blocks * 32, np.float32)
    lib().oracle_dequant_gguf_q8_0(_p(b, _c_u8p), _p(w, _c_f32p), ctypes.c_size_t(n_blocks))
    return w


# bytes per 32-weight block of ggml's legacy types
LEGACY_BLOCK_BYTES = {"q4_0": 18, "q4_1": 20, "q5_0": 22, "q5_1": 24}


def dequant_gguf_legacy(kind: str, blocks, n_blocks: int) -> np.ndarray:
    """ggml Q4_0 / Q4_1 / Q5_0 / Q5_1 blocks (32 weights each) -> float32 weights."""
    nb = LEGACY_BLOCK_BYTES[kind]
    b = _blocks_in(blocks, n_blocks, nb)
    w = np.empty(n_blocks * 32, np.float32)
    lib().oracle_dequant_gguf_legacy(_p(b, _c_u8p), ctypes.c_int(nb), _p(w, _c_f32p), ctypes.c_size_t(n_blocks))
    return w


def dequant_gguf_q2k(blocks, n_blocks: int) -> np.ndarray:
    """ggml Q2_K blocks (84 bytes per 256 weights) -> float32 weights."""
    b = _blocks_in(blocks, n_blocks, 84)
    w = np.empty(n_blocks * 256, np.float32)
    lib().oracle_dequant_gguf_q2k(_p(b, _c_u8p), _p(w, _c_f32p), ctypes.c_size_t(n_blocks))
    return w


def dequant_gguf_q3k(blocks, n_blocks: int) -> np.ndarray:
    """ggml Q3_K blocks (110 bytes per 256 weights) -> float32 weights."""
    b = _blocks_in(blocks, n_blocks, 110)
    w = np.empty(n_blocks * 256, np.float32)
    lib().oracle_dequant_gguf_q3k(_p(b, _c_u8p), _p(w, _c_f32p), ctypes.c_size_t(n_blocks))
    return w


def repack_gguf_q4k_to_q4km(blocks, n_blocks: int) -> np.ndarray:
    """ggml Q4_K blocks -> the ASDSL Q4_K variant blocks gemv_q4km reads."""
    b = _blocks_in(blocks, n_blocks, 144)
    out = np.empty(n_blocks * 144, np.uint8)
    lib().oracle_repack_gguf_q4k_to_q4km(_p(b, _c_u8p), _p(out, _c_u8p), ctypes.c_size_t(n_blocks))
    return out


def quantize_q4_symmetric(w, group_size: int) -> tuple[np.ndarray, np.ndarray, np.ndarray]:
    """float32 weights (flat, a multiple of group_size) -> (packed codes,
    f32 scales, f32 biases = -7.5 * scale): quantize_weights(bits=4,
    symmetric=True) as the reference's GGUF requantization uses it."""
    x = _f32(w).reshape(-1)
    groups = x.size // group_size
    packed = np.empty(x.size // 2, np.uint8)
    scales = np.empty(groups, np.float32)
    biases = np.empty(groups, np.float32)
    lib().oracle_quantize_q4_symmetric(_p(x, _c_f32p), _p(packed, _c_u8p), _p(scales, _c_f32p),
                                       _p(biases, _c_f32p), ctypes.c_size_t(groups), group_size)
    return packed, scales, biases
