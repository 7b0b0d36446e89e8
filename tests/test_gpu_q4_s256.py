"""HIP parity for the Q4_S256 superblock GEMV (asdsl_gemv_q4_s256 and its
fused-activation form) against the oracle (tests/test_oracle_s256.py pins it
to the reference's compiled kernel): 1e-4 relative L2, the golden vectors
of the reference kernel included."""

from __future__ import annotations

import numpy as np
import pytest

import oracle
from conftest import GOLDEN, rel_l2
from test_oracle_s256 import _blocks

pytestmark = pytest.mark.gpu
TOL = 1e-4


def test_golden_vectors(gpu):
    from asdsl.kernels import _native_gemv as ng

    g = np.load(GOLDEN / "q4_s256_reference.npz")
    M, K = (int(v) for v in g["s256_shape"])
    y = np.zeros(M, np.float32)
    ng.gemv_q4_s256_preq_avx2(g["s256_blocks"], g["s256_xq"], g["s256_xs"], y, M, K, 32)
    assert rel_l2(y, g["s256_y"]) < TOL


@pytest.mark.parametrize("M,K", [(70, 256), (5120, 3072), (16384, 3072), (3072, 8192), (129, 17920)])
def test_preq_and_fused_match_oracle(gpu, M, K):
    import torch
    from asdsl.kernels import _native_gemv as ng

    blocks = _blocks(M, K, M + K)
    x = np.random.default_rng(K).standard_normal(K).astype(np.float32)
    x[:32] = 0.0  # an all-zero activation group
    xq, xs = oracle.quantize_activation(x, 32)
    want = oracle.gemv_q4_s256(blocks, xq, xs, M, K)
    bd = torch.from_numpy(blocks).cuda()
    y = torch.empty(M, device="cuda")
    ng.gemv_q4_s256_preq_avx2(bd, torch.from_numpy(xq).cuda(), torch.from_numpy(xs).cuda(), y, M, K, 32)
    y2 = torch.empty(M, device="cuda")
    ng.gemv_q4_s256_fused(bd, torch.from_numpy(x).cuda(), y2, M, K)
    torch.cuda.synchronize()
    assert rel_l2(y.cpu().numpy(), want) < TOL
    assert rel_l2(y2.cpu().numpy(), want) < TOL


def test_argument_errors(gpu):
    from asdsl.kernels import _native_gemv as ng

    with pytest.raises(ValueError, match="divisible by 256"):
        ng.gemv_q4_s256_fused(np.zeros(144, np.uint8), np.zeros(128, np.float32), np.zeros(1, np.float32), 1, 128)
    with pytest.raises(ValueError):
        ng.gemv_q4_s256_preq_avx2(np.zeros(144, np.uint8), np.zeros(256, np.int8), np.zeros(8, np.float32),
                                  np.zeros(1, np.float32), 1, 256, 128)
    with pytest.raises(ValueError, match="blocks"):
        ng.gemv_q4_s256_preq_avx2(np.zeros(100, np.uint8), np.zeros(256, np.int8), np.zeros(8, np.float32),
                                  np.zeros(1, np.float32), 1, 256, 32)
