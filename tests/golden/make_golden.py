"""Write the golden fixtures from the reference's own kernels.

Run in a container where the reference tree is mounted and oracle/_ref is
built (``make -C oracle ref``):  ``python tests/golden/make_golden.py``.
Each fixture holds seeded inputs and the outputs of the reference's compiled
AVX2 functions (called through their own pybind11 interface), so tests can
pin the oracle and the HIP kernels on machines without the reference.
"""

from __future__ import annotations

import sys
from pathlib import Path

import numpy as np

HERE = Path(__file__).resolve().parent
REPO = HERE.parent.parent
sys.path[:0] = [str(REPO), str(REPO / "asdsl-framework_amd")]

import oracle  # noqa: E402
from asdsl.quantization import synthetic as syn  # noqa: E402
from asdsl.quantization.repack import repack_preq_blocks_to_preq2  # noqa: E402


def tricky_activation(K: int, seed: int) -> np.ndarray:
    """N(0,1) with groups that exercise the quantizer's edge cases."""
    x = syn.activation(K, seed)
    x[0:32] = 0.0                                         # all-zero group -> scale 1, q 0
    x[32:64] *= 1e-10                                     # amax < 1e-9 -> zero group
    t = np.arange(32, dtype=np.float32) - 15.5            # half-integer ties at amax=127
    t[0] = 127.0
    x[64:96] = t
    x[96:128] = np.float32(3.0e38) * np.sign(x[96:128])  # huge magnitudes
    x[128:160] = np.float32(1e-30) * (x[128:160] + 1)    # tiny but nonzero
    return x


def main() -> None:
    ng = oracle.load_reference("_native_gemv")
    out = {}

    # A1: quantize_activation_avx2, gs 32 and 128
    for gs in (32, 128):
        x = tricky_activation(1024, 7)
        xq = np.zeros(1024, np.int8)
        xs = np.zeros(1024 // gs, np.float32)
        ng.quantize_activation_avx2(x, xq, xs, 1024, gs)
        out[f"qa{gs}_x"], out[f"qa{gs}_xq"], out[f"qa{gs}_xs"] = x, xq, xs

    # A3: preq g32, fused and pre-quantized, M with a non-multiple-of-4 tail
    M, K = 70, 512
    w = syn.gaussian_weights(M, K, 42)
    blocks = syn.preq_blocks(w)
    x = syn.activation(K, 43)
    y = np.zeros(M, np.float32)
    ng.gemv_q4_32_preq_fused_avx2(blocks, x, y, M, K, 32)
    xq = np.zeros(K, np.int8)
    xs = np.zeros(K // 32, np.float32)
    ng.quantize_activation_avx2(x, xq, xs, K, 32)
    y2 = np.zeros(M, np.float32)
    ng.gemv_q4_32_preq_avx2(blocks, xq, xs, y2, M, K, 32)
    out.update(preq_blocks=blocks, preq_x=x, preq_y_fused=y, preq_y_q8=y2, preq_shape=np.array([M, K]))

    # A4/A5: preq2 g32 repacked from the same blocks
    meta, quant = repack_preq_blocks_to_preq2(blocks, M, K, 32)
    y3 = np.zeros(M, np.float32)
    ng.gemv_preq2_fused_avx2(meta.reshape(-1), quant.reshape(-1), x, y3, M, K, 32)
    out.update(preq2_meta=meta.reshape(-1), preq2_quant=quant.reshape(-1), preq2_y=y3)

    np.savez_compressed(HERE / "gemv_q4_reference.npz", **out)
    total = sum(v.nbytes for v in out.values())
    print(f"wrote {HERE / 'gemv_q4_reference.npz'} ({len(out)} arrays, {total} raw bytes)")


if __name__ == "__main__":
    main()
