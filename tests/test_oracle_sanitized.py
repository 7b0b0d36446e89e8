"""The C oracle under AddressSanitizer and UBSan.

``make -C oracle sanitize`` builds ``asdsl_oracle.c`` with
``-fsanitize=address,undefined -fno-sanitize-recover=all``.  The oracle's own
CPU tests then run in a child Python with libasan preloaded and that build
selected through ``ASDSL_ORACLE_LIB``: every oracle function they reach
(quantizers, GEMVs, dequantizers, repackers, the decode composition) is
checked for out-of-bounds accesses and undefined operations on the tests'
exact-size numpy buffers.  A planted overflow (a buffer one group short)
shows the sanitizer is armed."""

from __future__ import annotations

import os
import subprocess
import sys
from pathlib import Path

import pytest

from conftest import REPO

SAN_LIB = REPO / "oracle" / "lib" / "liboracle_san.so"
ORACLE_TESTS = ["test_oracle.py", "test_oracle_repack.py", "test_oracle_s256.py", "test_oracle_decode.py",
                "test_oracle_decode_engine.py", "test_kv_int8_rule.py"]


def _libasan() -> str | None:
    res = subprocess.run(["gcc", "-print-file-name=libasan.so"], capture_output=True, text=True)
    path = res.stdout.strip()
    return path if res.returncode == 0 and os.path.isabs(path) and Path(path).exists() else None


@pytest.fixture(scope="module")
def san_env():
    asan = _libasan()
    if asan is None:
        pytest.skip("gcc's libasan is not installed")
    subprocess.run(["make", "-s", "-C", str(REPO / "oracle"), "sanitize"], check=True)
    return dict(os.environ, LD_PRELOAD=asan, ASDSL_ORACLE_LIB=str(SAN_LIB),
                ASAN_OPTIONS="detect_leaks=0", UBSAN_OPTIONS="halt_on_error=1:print_stacktrace=1")


PLANTED = """
import ctypes, sys
import numpy as np
sys.path.insert(0, {repo!r})
import oracle
x = np.ones(64, np.float32)
xq = np.zeros(32, np.int8)            # one group of 32 short for K = 64
xs = np.zeros(2, np.float32)
v = ctypes.c_void_p
oracle.lib().oracle_quantize_activation(v(x.ctypes.data), v(xq.ctypes.data), v(xs.ctypes.data), 64, 32)
print("not caught")
"""


def test_sanitizer_catches_a_planted_overflow(san_env):
    res = subprocess.run([sys.executable, "-c", PLANTED.format(repo=str(REPO))], env=san_env,
                         capture_output=True, text=True, timeout=120)
    assert res.returncode != 0 and "not caught" not in res.stdout
    assert "heap-buffer-overflow" in res.stderr and "oracle_quantize_activation" in res.stderr


def test_oracle_tests_pass_under_sanitizers(san_env):
    files = [str(REPO / "tests" / f) for f in ORACLE_TESTS if (REPO / "tests" / f).exists()]
    res = subprocess.run([sys.executable, "-m", "pytest", "-q", "-m", "not gpu", "-p", "no:cacheprovider", *files],
                         env=san_env, capture_output=True, text=True, timeout=600, cwd=REPO)
    out = res.stdout + res.stderr
    assert "ERROR: AddressSanitizer" not in out and "runtime error:" not in out, out[-4000:]
    assert res.returncode == 0, out[-4000:]
    assert " passed" in res.stdout
