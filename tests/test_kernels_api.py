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


def test_native_modules_export_every_reference_name():
    """Each drop-in module exports every name the reference's pybind11 module
    defines (m.def / m.attr; list written from the reference sources by
    tests/golden/make_module_names.py)."""
    import importlib
    import json

    from conftest import GOLDEN

    names = json.loads((GOLDEN / "reference_module_names.json").read_text())
    assert set(names) == {"_native_gemv", "_native_gemv_q8", "_native_sparse_gemv"}
    for mod, expected in names.items():
        m = importlib.import_module(f"asdsl.kernels.{mod}")
        missing = [n for n in expected if not hasattr(m, n)]
        assert not missing, (mod, missing)


def test_capability_probes_and_topology():
    from asdsl.kernels import _native_gemv as ng
    from asdsl.kernels import _native_gemv_q8 as nq

    for probe in (ng.check_avx2, ng.check_fma, ng.check_avx512, ng.check_vnni, ng.check_avx_vnni,
                  ng.check_avx512_vnni):
        assert probe() is False
    topo = ng.get_cpu_topology()
    assert set(topo) == {"physical_logical_ids", "physical_core_count", "pcore_count", "avx_vnni", "avx512_vnni"}
    assert nq.has_avx2 is False and nq.has_openmp is False
    assert nq.set_pin_openmp_pcores(True) is None


def test_preq_accumulate_counters_follow_the_reference(monkeypatch):
    """Per preq call the reference's classic counter grows by rows x groups,
    or by rows x (groups mod 4) when its 4-group loop runs
    (gemv_q4_preq_restored.cpp:350-352,404-416); the x-preloaded one never moves."""
    from asdsl.kernels import _native_gemv as ng

    monkeypatch.delenv("ASDSL_PREQ_G4FUSED", raising=False)
    monkeypatch.delenv("ASDSL_PREQ_G4GATE_UP_ONLY", raising=False)
    ng.reset_preq_accum_call_counts()
    assert ng.get_preq_classic_accum_calls() == 0 and ng.get_preq_xloaded_accum_calls() == 0
    ng._count_preq_groups(3072, 96, False)
    assert ng.get_preq_classic_accum_calls() == 3072 * 96
    ng._count_preq_groups(3072, 96, True)  # g4fused entry: 96 % 4 == 0, nothing left over
    assert ng.get_preq_classic_accum_calls() == 3072 * 96
    monkeypatch.setenv("ASDSL_PREQ_G4GATE_UP_ONLY", "1")
    ng._count_preq_groups(4096, 8, False)   # below 8192 rows: classic
    ng._count_preq_groups(16384, 8, False)  # gate_up sized: 4-group loop
    assert ng.get_preq_classic_accum_calls() == 3072 * 96 + 4096 * 8
    ng._count_preq_groups(100, 6, False)    # 6 groups: not a multiple of 4, classic
    assert ng.get_preq_classic_accum_calls() == 3072 * 96 + 4096 * 8 + 600
    ng.reset_preq_accum_call_counts()
    assert ng.get_preq_classic_accum_calls() == 0
    assert ng.get_preq_xloaded_accum_calls() == 0


def test_g4fused_rejects_group_counts_off_a_multiple_of_four():
    from asdsl.kernels import _native_gemv as ng

    with pytest.raises(ValueError, match="divisible by 4"):
        ng.gemv_q4_32_preq_g4fused_4row_avx2(np.zeros(4 * 6 * 20, np.uint8), np.zeros(192, np.float32),
                                             np.zeros(4, np.float32), 4, 192)
    with pytest.raises(ValueError, match="group_size must be 32"):
        ng.gemv_q4_32_preq_g4fused_4row_avx2(np.zeros(4 * 4 * 20, np.uint8), np.zeros(128, np.float32),
                                             np.zeros(4, np.float32), 4, 128, 64)
