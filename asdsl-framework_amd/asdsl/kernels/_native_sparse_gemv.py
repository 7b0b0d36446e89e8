"""Drop-in for the reference's ``_native_sparse_gemv`` pybind11 module, running on HIP.

Reference: asdsl/kernels/native/gemv_sparse_avx2.cpp:421-472.  Weights are
uint8 (one per byte) with fp32 per-group scale and bias; only active columns
of the fp32 activation count:
    y[m] = sum_g scales[m,g] * sum_{k in g, active} w[m,k] x[k] + biases[m,g] * sum_{k in g, active} x[k].
"""

from __future__ import annotations

import numpy as np

from asdsl import _hip
from asdsl.kernels._buffers import DeviceCall, new_output, shape_of

has_openmp = False


def _numel(a) -> int:
    n = 1
    for d in shape_of(a):
        n *= d
    return n


def _check(w, x, scales, biases, M, K, gs, fn):
    if M <= 0 or K <= 0 or gs <= 0 or K % gs != 0:
        raise ValueError(f"{fn}: K must be a positive multiple of group_size")
    G = K // gs
    for a, n, name in ((w, M * K, "w"), (x, K, "x"), (scales, M * G, "scales"), (biases, M * G, "biases")):
        if _numel(a) < n:
            raise ValueError(f"{fn}: {name} is too small for M={M}, K={K}, group_size={gs}")


def compute_bitmask(x, threshold: float):
    """bitmask u32[(K+31)/32]: bit k set iff |x[k]| >= threshold
    (gemv_sparse_avx2.cpp:144-179)."""
    K = _numel(x)
    if K == 0:  # the reference returns an empty mask
        return new_output((0,), np.uint32, x)
    mask = new_output(((K + 31) // 32,), np.uint32, x)
    c = DeviceCall("compute_bitmask")
    c.run("asdsl_compute_bitmask", c.input(x, np.float32, K, "x"), c.output(mask, np.uint32, (K + 31) // 32, "bitmask"),
          K, float(threshold))
    return mask


def gemv_sparse_unpacked(w, x, scales, biases, bitmask, M: int, K: int, group_size: int):
    """gemv_sparse_avx2.cpp:66-139 (bitmask path)."""
    fn = "gemv_sparse_unpacked"
    _check(w, x, scales, biases, M, K, group_size, fn)
    if _numel(bitmask) < (K + 31) // 32:
        raise ValueError(f"{fn}: bitmask must have (K+31)/32 words")
    G = K // group_size
    y = new_output((M,), np.float32, w, x)
    c = DeviceCall(fn)
    c.run("asdsl_gemv_sparse_unpacked", c.input(w, np.uint8, M * K, "w"), c.input(x, np.float32, K, "x"),
          c.input(scales, np.float32, M * G, "scales"), c.input(biases, np.float32, M * G, "biases"),
          c.input(bitmask, np.uint32, (K + 31) // 32, "bitmask"), c.output(y, np.float32, M, "y"), M, K, group_size)
    return y


def gemv_sparse_with_indices(w, x, scales, biases, active_indices, M: int, K: int, group_size: int):
    """gemv_sparse_avx2.cpp:66-110 (index path).  A column listed c times
    counts c times; indices outside [0, K) are ignored.  An empty list gives
    y = 0 (the reference falls through to its bitmask path with a null mask)."""
    fn = "gemv_sparse_with_indices"
    _check(w, x, scales, biases, M, K, group_size, fn)
    G = K // group_size
    n = _numel(active_indices)
    y = new_output((M,), np.float32, w, x)
    c = DeviceCall(fn)
    c.run("asdsl_gemv_sparse_with_indices", c.input(w, np.uint8, M * K, "w"), c.input(x, np.float32, K, "x"),
          c.input(scales, np.float32, M * G, "scales"), c.input(biases, np.float32, M * G, "biases"),
          c.input(active_indices if n else np.zeros(1, np.int32), np.int32, max(n, 1), "active_indices"), n,
          c.output(y, np.float32, M, "y"), M, K, group_size,
          c.scratch((K + 31) // 32, np.uint32), c.scratch(K, np.float32))
    return y


def sparse_down_proj_T(w_T_packed, scales_T, biases_T, sparse_x, active_rows, in_dim: int, out_dim: int,
                       group_size: int):
    """gemv_sparse_avx2.cpp:273-418: y[out_dim] = sum over listed rows r with
    x[r] != 0 of x[r] * dequant(w_T[r, :]), per element fma(q, s*x, b*x)."""
    if in_dim <= 0 or out_dim <= 0 or group_size <= 0:
        raise ValueError("in_dim, out_dim, group_size must be positive")
    if out_dim % group_size != 0:
        raise ValueError("out_dim must be divisible by group_size")
    G = out_dim // group_size
    for a, n, name in ((w_T_packed, in_dim * out_dim // 2, "w_T_packed"), (scales_T, in_dim * G, "scales_T"),
                       (biases_T, in_dim * G, "biases_T"), (sparse_x, in_dim, "sparse_x")):
        if _numel(a) < n:
            raise ValueError(f"sparse_down_proj_T: {name} is too small for in_dim={in_dim}, out_dim={out_dim}")
    n = _numel(active_rows)
    y = new_output((out_dim,), np.float32, w_T_packed, sparse_x)
    c = DeviceCall("sparse_down_proj_T")
    nbytes = int(_hip.LIB.asdsl_sparse_down_work_bytes(out_dim))
    c.run("asdsl_sparse_down_proj_T_ws", c.input(w_T_packed, np.uint8, in_dim * out_dim // 2, "w_T_packed"),
          c.input(scales_T, np.float32, in_dim * G, "scales_T"), c.input(biases_T, np.float32, in_dim * G, "biases_T"),
          c.input(sparse_x, np.float32, in_dim, "sparse_x"),
          c.input(active_rows if n else np.zeros(1, np.int32), np.int32, max(n, 1), "active_rows"), n,
          c.output(y, np.float32, out_dim, "y"), in_dim, out_dim, group_size, c.scratch(nbytes, np.uint8), nbytes)
    return y
