"""CPU checks of the high-level asdsl.kernels API: the names the reference
exports (asdsl/kernels/__init__.py:58-77, minus the 2/3-bit and LUT kernels)
and its argument errors, raised before any device work."""

from __future__ import annotations

import numpy as np
import pytest

import asdsl.kernels as K
from asdsl.quantization.core import quantize_weights

EXPECTED = ["gemv_q4", "gemv_q4_packed", "gemv_q4_unpacked", "gemv_q4km_q8", "has_native_kernel",
            "gemv_q8_unpacked", "has_native_q8_kernel", "compute_activation_bitmask", "gemv_sparse_unpacked",
            "gemv_sparse_with_indices", "has_native_sparse_kernel", "KERNEL_TIER"]


def test_exports():
    for name in EXPECTED:
        assert hasattr(K, name), name
    assert set(EXPECTED) <= set(K.__all__)
    for probe in (K.has_native_kernel, K.has_native_q8_kernel, K.has_native_sparse_kernel):
        assert probe() is True


def test_argument_errors_before_device_work():
    w = np.zeros(64, np.uint8)
    s = np.ones(4, np.float32)
    with pytest.raises(ValueError, match="does not match K"):
        K.gemv_q4_packed(w, np.ones(30, np.float32), s, s, 4, 32, 32)
    with pytest.raises(ValueError, match="1-D"):
        K.gemv_q4_packed(w, np.ones((1, 2, 32), np.float32), s, s, 4, 32, 32)
    with pytest.raises(ValueError, match="out must be float32"):
        K.gemv_q4_packed(w, np.ones(32, np.float32), s, s, 4, 32, 32, out=np.empty(3, np.float32))
    with pytest.raises(ValueError, match="in_features"):
        K.gemv_q4km_q8(np.zeros(144, np.uint8), np.ones(200, np.float32), 1, 256)
    qt = quantize_weights(np.ones((4, 128), np.float32), bits=8, group_size=128)
    with pytest.raises(ValueError, match="4-bit"):
        K.gemv_q4(qt, np.ones(128, np.float32))
