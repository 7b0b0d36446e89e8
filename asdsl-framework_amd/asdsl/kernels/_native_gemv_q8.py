"""Drop-in for the reference's ``_native_gemv_q8`` pybind11 module, running on HIP.

Reference: asdsl/kernels/native/gemv_q8_avx2.cpp:159-261.  uint8 weights (one
per byte), fp32 per-group scale and bias, fp32 activation:
    y[m] = sum_g scales[m,g] * (sum_k w[m,k] x[k]) + biases[m,g] * (sum_k x[k]).
``cache_tiling`` only changes the reference's loop blocking and is accepted and
ignored.
"""

from __future__ import annotations

import numpy as np

from asdsl.kernels._buffers import DeviceCall, new_output, shape_of

has_openmp = False
# The reference probes the host CPU for AVX2 (gemv_q8_avx2.cpp:208-220,255);
# the kernels here run on the GPU.
has_avx2 = False


def set_pin_openmp_pcores(enabled: bool = True) -> None:
    """Reference: set_pin_openmp_pcores (gemv_q8_avx2.cpp:248-252), CPU thread
    pinning; there are no host threads to pin here."""


def detected_pcore_count() -> int:
    """Reference: detected_pcore_count (gemv_q8_avx2.cpp:204-206,253), the host's
    physical cores its kernels run on; here the GPU's compute units, as
    _native_gemv.get_num_threads reports."""
    from asdsl import _hip

    return _hip.cu_count()


def _numel(a) -> int:
    n = 1
    for d in shape_of(a):
        n *= d
    return n


def gemv_q8_unpacked(w_u8, x, scales, biases, m: int, k: int, group_size: int = 128, cache_tiling: bool = True):
    if group_size <= 0 or k % group_size != 0:
        raise ValueError("K must be a multiple of group_size")
    if m <= 0 or k <= 0:
        raise ValueError("M and K must be positive")
    G = k // group_size
    for a, n, name in ((w_u8, m * k, "w"), (x, k, "x"), (scales, m * G, "scales"), (biases, m * G, "biases")):
        if _numel(a) < n:
            raise ValueError(f"{name} is too small for M={m}, K={k}, group_size={group_size}")
    y = new_output((m,), np.float32, w_u8, x)
    c = DeviceCall("gemv_q8_unpacked")
    c.run("asdsl_gemv_q8_unpacked", c.input(w_u8, np.uint8, m * k, "w"), c.input(x, np.float32, k, "x"),
          c.input(scales, np.float32, m * G, "scales"), c.input(biases, np.float32, m * G, "biases"),
          c.output(y, np.float32, m, "y"), m, k, group_size)
    return y


def fused_dequant_gemv(w_u8, x, scales, biases, m: int, k: int, group_size: int = 128, cache_tiling: bool = True):
    return gemv_q8_unpacked(w_u8, x, scales, biases, m, k, group_size, cache_tiling)
