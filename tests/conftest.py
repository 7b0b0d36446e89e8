"""Shared test setup.

Markers: ``gpu`` tests need a HIP device and call the kernels through the C
ABI; everything else runs on the CPU (oracle, formats, host logic, ABI
surface).  The repository root (for ``oracle``) and ``asdsl-framework_amd``
(for the ``asdsl`` package) are put on sys.path.
"""

from __future__ import annotations

import sys
from pathlib import Path

import numpy as np
import pytest

REPO = Path(__file__).resolve().parent.parent
for p in (REPO, REPO / "asdsl-framework_amd"):
    if str(p) not in sys.path:
        sys.path.insert(0, str(p))

GOLDEN = REPO / "tests" / "golden"


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs a HIP device (MI355X); calls the HIP kernels")


@pytest.fixture
def rng():
    return np.random.default_rng(42)


def rel_l2(a, b) -> float:
    a = np.asarray(a, np.float64).ravel()
    b = np.asarray(b, np.float64).ravel()
    den = np.linalg.norm(b)
    return float(np.linalg.norm(a - b) / (den if den > 0 else 1.0))


@pytest.fixture(scope="session")
def gpu():
    """Skip-free GPU guard: a gpu-marked test on a machine without a device is
    an error, not a skip, so a missing device can never look like a pass."""
    import torch

    if not torch.cuda.is_available():
        pytest.fail("gpu test selected but no HIP device is visible")
    from asdsl import _hip

    return _hip
