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

    # A6: Q4_128 (pre-quantized per 128) and its batched fp32 GEMM
    M, K = 24, 512
    w = syn.gaussian_weights(M, K, 21)
    w[3, 128:256] = 0.0                                  # all-zero group -> scale 0, nibbles 0x88
    b128 = syn.q4_128_blocks(w)
    x = syn.activation(K, 22)
    xq = np.zeros(K, np.int8)
    xs = np.zeros(K // 128, np.float32)
    ng.quantize_activation_avx2(x, xq, xs, K, 128)
    y = np.zeros(M, np.float32)
    ng.gemv_q4_128_preq_avx2(b128, xq, xs, y, M, K, 128)
    out.update(q128_blocks=b128, q128_x=x, q128_xq=xq, q128_xs=xs, q128_y=y, q128_shape=np.array([M, K]))

    rng = np.random.default_rng(31)
    # A9(ii): gemv_q4_q8 (symmetric packed + fp32 scales), gs 32
    M, K = 20, 512
    wp = rng.integers(0, 256, M * K // 2, dtype=np.uint8)
    sc = (rng.random(M * K // 32) * 0.01 + 1e-3).astype(np.float32)
    x = syn.activation(K, 32)
    y = np.zeros(M, np.float32)
    ng.gemv_q4_q8_avx2(wp, sc, x, y, M, K, 32)
    out.update(q4q8_w=wp, q4q8_s=sc, q4q8_x=x, q4q8_y=y, q4q8_shape=np.array([M, K]))

    # A8: Q4_K (ASDSL variant), random superblocks with small fp16 d/dmin
    M, K = 12, 512
    wk = rng.integers(0, 256, (M, K // 256, 144), dtype=np.uint8)
    wk[:, :, 0:2] = np.frombuffer(np.float16(0.0123).tobytes(), np.uint8)
    wk[:, :, 2:4] = np.frombuffer(np.float16(0.0041).tobytes(), np.uint8)
    wk = wk.reshape(-1)
    x = syn.activation(K, 33)
    x[32:64] = 0.0                                       # amax < 1e-12 -> scale 0
    y = np.zeros(M, np.float32)
    ng.gemv_q4km_q8_avx2(wk, x, y, M, K)
    out.update(q4k_w=wk, q4k_x=x, q4k_y=y, q4k_shape=np.array([M, K]))

    # A10: packed / unpacked affine fp32 GEMV, gs64, matmul_batch_q4
    M, K = 16, 256
    wp = rng.integers(0, 256, M * K // 2, dtype=np.uint8)
    wu = rng.integers(0, 16, M * K, dtype=np.uint8)
    s32 = (rng.random(M * K // 32) * 0.01).astype(np.float32)
    b32 = (rng.standard_normal(M * K // 32) * 0.01).astype(np.float32)
    s64 = (rng.random(M * K // 64) * 0.01).astype(np.float32)
    x = syn.activation(K, 34)
    X = rng.standard_normal((3, K)).astype(np.float32)
    Y = np.zeros((3, M), np.float32)
    ng.matmul_batch_q4(wp, s32, b32, X, Y, M, K, 3, 32)
    out.update(aff_wp=wp, aff_wu=wu, aff_s32=s32, aff_b32=b32, aff_s64=s64, aff_x=x, aff_X=X,
               aff_y_packed=np.asarray(ng.gemv_q4_packed(wp, x, s32, b32, M, K, 32)),
               aff_y_unpacked=np.asarray(ng.gemv_q4_unpacked(wu, x, s32, b32, M, K, 32)),
               aff_y_gs64=np.asarray(ng.gemv_q4_avx2_gs64(wp, x, s64, M, K)),
               aff_Y_batch=Y, aff_shape=np.array([M, K]))

    # A9(i): Q8 weight GEMV (gemv_q8_unpacked / fused_dequant_gemv), gs 128
    q8 = oracle.load_reference("_native_gemv_q8")
    M, K = 16, 512
    w8 = rng.integers(0, 256, M * K, dtype=np.uint8)
    s8 = (rng.random(M * K // 128) * 0.01).astype(np.float32)
    b8 = (rng.standard_normal(M * K // 128) * 0.01).astype(np.float32)
    x = syn.activation(K, 35)
    out.update(q8_w=w8, q8_s=s8, q8_b=b8, q8_x=x, q8_shape=np.array([M, K]),
               q8_y=np.asarray(q8.gemv_q8_unpacked(w8, x, s8, b8, M, K, 128, True)))

    # A12: bitmask, sparse GEMVs, sparse_down_proj_T (4 active rows: the
    # reference runs them as one serial chunk, see tests/test_oracle.py)
    sp = oracle.load_reference("_native_sparse_gemv")
    xs_ = np.maximum(0.0, syn.activation(K, 36) - np.float32(0.841621)).astype(np.float32)
    mask = np.asarray(sp.compute_bitmask(xs_, 0.01))
    idx = np.nonzero(np.abs(xs_) >= 0.01)[0].astype(np.int32)
    out.update(sp_x=xs_, sp_mask=mask, sp_idx=idx,
               sp_y_idx=np.asarray(sp.gemv_sparse_with_indices(w8, xs_, s8, b8, idx, M, K, 128)),
               sp_y_mask=np.asarray(sp.gemv_sparse_unpacked(w8, xs_, s8, b8, mask, M, K, 128)))
    IN, OUT = 64, 96
    wT = rng.integers(0, 256, IN * OUT // 2, dtype=np.uint8)
    sT = (rng.random(IN * OUT // 32) * 0.01).astype(np.float32)
    bT = (-8.0 * sT).astype(np.float32)
    xT = np.maximum(0.0, syn.activation(IN, 37)).astype(np.float32)
    rows = np.nonzero(xT)[0][:4].astype(np.int32)
    out.update(dT_w=wT, dT_s=sT, dT_b=bT, dT_x=xT, dT_rows=rows, dT_shape=np.array([IN, OUT]),
               dT_y=np.asarray(sp.sparse_down_proj_T(wT, sT, bT, xT, rows, IN, OUT, 32)))

    np.savez_compressed(HERE / "gemv_q4_reference.npz", **out)
    total = sum(v.nbytes for v in out.values())
    print(f"wrote {HERE / 'gemv_q4_reference.npz'} ({len(out)} arrays, {total} raw bytes)")
    s256_fixture()


def s256_blocks(M: int, K: int, seed: int) -> np.ndarray:
    """Random Q4_S256 superblocks: 8 fp16 sub-scales (both signs, one zero)
    then 128 random nibble bytes per 256 weights."""
    rng = np.random.default_rng(seed)
    nsb = M * (K // 256)
    scales = (rng.uniform(0.001, 0.05, (nsb, 8)) * rng.choice([-1.0, 1.0], (nsb, 8))).astype(np.float16)
    scales[0, 3] = 0.0
    blocks = np.empty((nsb, 144), np.uint8)
    blocks[:, :16] = scales.view(np.uint8).reshape(nsb, 16)
    blocks[:, 16:] = rng.integers(0, 256, (nsb, 128), dtype=np.uint8)
    return blocks.reshape(-1)


def s256_fixture() -> None:
    """Q4_S256 (gemv_q4_s256.cpp, no Python binding in the reference): the
    compiled reference kernel through oracle/_ref/libref_q4_s256.so, on 37
    rows (a tail row past the 4-row loop) x 512, activation quantized by the
    reference's quantize_activation_avx2."""
    ng = oracle.load_reference("_native_gemv")
    ref = oracle.reference_q4_s256()
    M, K = 37, 512
    blocks = s256_blocks(M, K, 41)
    x = tricky_activation(K, 42)
    x[96:128] = syn.activation(32, 43) * np.float32(1e4)  # large but finite: fp32 sums stay finite
    xq, xs = np.zeros(K, np.int8), np.zeros(K // 32, np.float32)
    ng.quantize_activation_avx2(x, xq, xs, K, 32)
    out = {"s256_blocks": blocks, "s256_xq": xq, "s256_xs": xs, "s256_shape": np.array([M, K]),
           "s256_y": ref(blocks, xq, xs, M, K)}
    np.savez_compressed(HERE / "q4_s256_reference.npz", **out)
    print(f"wrote {HERE / 'q4_s256_reference.npz'}")


if __name__ == "__main__":
    s256_fixture() if sys.argv[1:] == ["s256"] else main()
