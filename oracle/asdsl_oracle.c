/*
 * asdsl_oracle.c — CPU restatement of the reference's Q4 GEMV hot path.
 *
 * TEST INFRASTRUCTURE ONLY.  This file is the parity checker for the HIP
 * kernels: only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline
 * leg may load it.  The product path never calls it.
 *
 * Every function restates one reference routine in plain scalar C (no SIMD).
 * The preq/preq2 GEMVs spread their rows over OpenMP threads (each row's
 * arithmetic is the same whatever thread runs it), so that a full-size
 * decode step can be checked in a test.  Integer parts (nibble decode, int8 activation quantization,
 * integer dots) are exact and match the reference bit for bit.  Floating
 * point per-group terms are formed in fp32 in the reference's operand order;
 * the sum over groups is accumulated in double so that the oracle sits at
 * the centre of the fp32 reordering noise of both the reference (AVX2 lane
 * order) and the GPU (wave order).
 *
 * Parity pins (see tests/test_oracle_*.py):
 *   - against the reference's own C++ compiled from its sources (oracle/_ref),
 *     when that build exists (this container);
 *   - against golden fixtures under tests/golden/ produced from oracle/_ref;
 *   - against the reference's known answers (1.6: tests/test_gemv_q4.py:150-163;
 *     448.0: asdsl/kernels/native/test_kernel.cpp:16,39);
 *   - against float64 closed forms (dequant(W) . dequant(Q8(x))).
 */
#include <math.h>
#include <stdint.h>
#include <string.h>

#define EXPORT __attribute__((visibility("default")))

/* fp16 bits -> float, exact (IEEE binary16, subnormals included), as
 * _mm_cvtph_ps does (asdsl/kernels/native/gemv_preq2_avx2.cpp:35-37). */
static float half_to_float(uint16_t h) {
    const uint32_t sign = (uint32_t)(h & 0x8000u) << 16;
    const uint32_t exp = (h >> 10) & 0x1Fu;
    const uint32_t mant = h & 0x3FFu;
    float f;
    if (exp == 0) {
        f = ldexpf((float)mant, -24); /* subnormal or zero: mant * 2^-24, exact */
        return sign ? -f : f;
    }
    uint32_t bits;
    if (exp == 0x1Fu) bits = sign | 0x7F800000u | (mant << 13);
    else bits = sign | ((exp + 112u) << 23) | (mant << 13);
    memcpy(&f, &bits, 4);
    return f;
}

EXPORT float oracle_half_to_float(uint16_t h) { return half_to_float(h); }

static uint16_t rd16(const uint8_t* p) { return (uint16_t)(p[0] | (p[1] << 8)); }

/* Nibble k of a packed group: byte k/2, low nibble for even k
 * (asdsl/quantization/core.py:556-563). */
static int nib(const uint8_t* packed, int k) {
    const uint8_t b = packed[k >> 1];
    return (k & 1) ? (b >> 4) : (b & 0x0F);
}

static int sat8(int v) { return v > 127 ? 127 : (v < -128 ? -128 : v); }

/* ------------------------------------------------------------------ A1
 * quantize_activation_avx2 (asdsl/kernels/native/gemv_q4_preq_restored.cpp:505-549),
 * as compiled with setup.py's -O3 -ffast-math: amax/127.0f becomes
 * amax*(1.0f/127.0f) (reciprocal-math), 127.0f/amax stays a division,
 * cvtps_epi32 rounds half to even, packs saturate. */
EXPORT void oracle_quantize_activation(const float* x, int8_t* xq, float* xs, int K, int gs) {
    const float r127 = 1.0f / 127.0f;
    for (int g = 0; g < K / gs; ++g) {
        const float* xg = x + (size_t)g * gs;
        float amax = 0.0f;
        for (int j = 0; j < gs; ++j) {
            const float a = fabsf(xg[j]);
            amax = a > amax ? a : amax;
        }
        if (amax < 1e-9f) {
            for (int j = 0; j < gs; ++j) xq[(size_t)g * gs + j] = 0;
            xs[g] = 1.0f;
            continue;
        }
        xs[g] = amax * r127;
        const float inv = 127.0f / amax;
        for (int j = 0; j < gs; ++j) {
            volatile float p = xg[j] * inv; /* one fp32 rounding, no contraction */
            xq[(size_t)g * gs + j] = (int8_t)sat8((int)nearbyintf(p));
        }
    }
}

/* Exact integer dot of `n` nibbles (starting at element 0 of `packed`)
 * with int8 activations, and the activation sum. */
static void nib_dot(const uint8_t* packed, const int8_t* xq, int n, int32_t* d, int32_t* xsum) {
    int32_t dd = 0, ss = 0;
    for (int k = 0; k < n; ++k) {
        dd += nib(packed, k) * (int32_t)xq[k];
        ss += xq[k];
    }
    *d = dd;
    *xsum = ss;
}

/* ------------------------------------------------------------------ A3
 * preq g32 GEMV on 20-byte blocks (asdsl/kernels/native/gemv_q4_preq_restored.cpp:281-336,
 * 551-573): per group term = D*(s*xs), correction = ((z*X)*s)*xs, y = sum - corr. */
EXPORT void oracle_gemv_preq(const uint8_t* blocks, const int8_t* xq, const float* xs, float* y, int M, int K) {
    const int G = K / 32;
#pragma omp parallel for schedule(static)
    for (int r = 0; r < M; ++r) {
        double acc = 0.0, corr = 0.0;
        for (int g = 0; g < G; ++g) {
            const uint8_t* b = blocks + ((size_t)r * G + g) * 20;
            const float s = half_to_float(rd16(b));
            const float z = half_to_float(rd16(b + 2));
            int32_t d, xsum;
            nib_dot(b + 4, xq + (size_t)g * 32, 32, &d, &xsum);
            acc += (double)((float)d * (s * xs[g]));
            corr += (double)(((z * (float)xsum) * s) * xs[g]);
        }
        y[r] = (float)(acc - corr);
    }
}

EXPORT void oracle_gemv_preq_fused(const uint8_t* blocks, const float* x, float* y, int M, int K,
                                   int8_t* scratch_q, float* scratch_s) {
    oracle_quantize_activation(x, scratch_q, scratch_s, K, 32);
    oracle_gemv_preq(blocks, scratch_q, scratch_s, y, M, K);
}

/* ------------------------------------------------------------------ A4/A5/A7
 * preq2 (asdsl/kernels/native/gemv_preq2_avx2.cpp:70-93,196-297; layout
 * asdsl/quantization/repack_preq2.py:22-62): meta[M][G][4], quant bands of 4
 * rows, per (band, group) 4*(gs/2) bytes with row slot r%4 at slot*(gs/2).
 * gs=32 is the reference layout; gs=128 is the asymmetric g128 extension
 * with the same structure.  Term = D*(s*xs), correction = (z*s)*(X*xs). */
EXPORT void oracle_gemv_preq2(const uint8_t* meta, const uint8_t* quant, const int8_t* xq, const float* xs,
                              float* y, int M, int K, int gs) {
    const int G = K / gs;
    const size_t gbytes = (size_t)gs / 2;
#pragma omp parallel for schedule(static)
    for (int r = 0; r < M; ++r) {
        const int band = r / 4, slot = r % 4;
        double acc = 0.0;
        for (int g = 0; g < G; ++g) {
            const uint8_t* m = meta + ((size_t)r * G + g) * 4;
            const float s = half_to_float(rd16(m));
            const float z = half_to_float(rd16(m + 2));
            const uint8_t* q = quant + ((size_t)band * G + g) * 4 * gbytes + slot * gbytes;
            int32_t d, xsum;
            nib_dot(q, xq + (size_t)g * gs, gs, &d, &xsum);
            const float xsum_scaled = (float)xsum * xs[g];
            acc += (double)((float)d * (s * xs[g])) - (double)((z * s) * xsum_scaled);
        }
        y[r] = (float)acc;
    }
}

/* The same GEMV with the per-group terms summed in float32, in group order,
 * as a plain scalar CPU loop would (the reference sums float32 AVX2 lanes,
 * gemv_preq2_avx2.cpp:168-194).  A second restatement that differs from
 * oracle_gemv_preq2 only in the rounding of the sum: the decode tests use
 * it to measure how far rounding alone moves a deep model's logits. */
EXPORT void oracle_gemv_preq2_f32sum(const uint8_t* meta, const uint8_t* quant, const int8_t* xq, const float* xs,
                                     float* y, int M, int K, int gs) {
    const int G = K / gs;
    const size_t gbytes = (size_t)gs / 2;
#pragma omp parallel for schedule(static)
    for (int r = 0; r < M; ++r) {
        const int band = r / 4, slot = r % 4;
        float acc = 0.0f;
        for (int g = 0; g < G; ++g) {
            const uint8_t* m = meta + ((size_t)r * G + g) * 4;
            const float s = half_to_float(rd16(m));
            const float z = half_to_float(rd16(m + 2));
            const uint8_t* q = quant + ((size_t)band * G + g) * 4 * gbytes + slot * gbytes;
            int32_t d, xsum;
            nib_dot(q, xq + (size_t)g * gs, gs, &d, &xsum);
            const float xsum_scaled = (float)xsum * xs[g];
            const float term = (float)d * (s * xs[g]);
            acc = acc + term;
            acc = acc - (z * s) * xsum_scaled;
        }
        y[r] = acc;
    }
}

EXPORT void oracle_gemv_preq2_fused(const uint8_t* meta, const uint8_t* quant, const float* x, float* y, int M,
                                    int K, int gs, int8_t* scratch_q, float* scratch_s) {
    oracle_quantize_activation(x, scratch_q, scratch_s, K, gs);
    oracle_gemv_preq2(meta, quant, scratch_q, scratch_s, y, M, K, gs);
}

/* Dequantization w = (q - z) * s (experiments/phi4_cpu_run.py:3450-3467):
 * q - z is exact in fp32, one rounding in the product. */
EXPORT void oracle_dequant_preq2(const uint8_t* meta, const uint8_t* quant, float* w, int M, int K, int gs) {
    const int G = K / gs;
    const size_t gbytes = (size_t)gs / 2;
#pragma omp parallel for schedule(static)
    for (int r = 0; r < M; ++r) {
        const int band = r / 4, slot = r % 4;
        for (int g = 0; g < G; ++g) {
            const uint8_t* m = meta + ((size_t)r * G + g) * 4;
            const float s = half_to_float(rd16(m));
            const float z = half_to_float(rd16(m + 2));
            const uint8_t* q = quant + ((size_t)band * G + g) * 4 * gbytes + slot * gbytes;
            for (int k = 0; k < gs; ++k) {
                volatile float qz = (float)nib(q, k) - z;
                w[(size_t)r * K + (size_t)g * gs + k] = qz * s;
            }
        }
    }
}

EXPORT void oracle_dequant_preq(const uint8_t* blocks, float* w, int M, int K) {
    const int G = K / 32;
    for (int r = 0; r < M; ++r) {
        for (int g = 0; g < G; ++g) {
            const uint8_t* b = blocks + ((size_t)r * G + g) * 20;
            const float s = half_to_float(rd16(b));
            const float z = half_to_float(rd16(b + 2));
            for (int k = 0; k < 32; ++k) {
                volatile float qz = (float)nib(b + 4, k) - z;
                w[(size_t)r * K + (size_t)g * 32 + k] = qz * s;
            }
        }
    }
}

/* ------------------------------------------------------------------ A6
 * Q4_128 symmetric GEMV on 66-byte blocks (asdsl/kernels/native/gemv_q4_128.cpp:94-257):
 * x pre-quantized per 128; per group term D*(ws*xs), correction (8*X*xs)*ws
 * (process_r8 form, gemv_q4_128.cpp:174-217). */
EXPORT void oracle_gemv_q4_128(const uint8_t* blocks, const int8_t* xq, const float* xs, float* y, int M, int K) {
    const int G = K / 128;
    for (int r = 0; r < M; ++r) {
        double acc = 0.0, corr = 0.0;
        for (int g = 0; g < G; ++g) {
            const uint8_t* b = blocks + ((size_t)r * G + g) * 66;
            const float ws = half_to_float(rd16(b));
            int32_t d, xsum;
            nib_dot(b + 2, xq + (size_t)g * 128, 128, &d, &xsum);
            acc += (double)((float)d * (ws * xs[g]));
            corr += (double)((8.0f * (float)xsum * xs[g]) * ws);
        }
        y[r] = (float)(acc - corr);
    }
}

/* Batched Q4_128 with an fp32 activation, no quantization
 * (gemm_q4_128_q8_avx2, asdsl/kernels/native/gemv_q4_128.cpp:262-306):
 * w = (q-8)*ws in fp32, Y[b][r] = sum_k w*X[b][k] (b < 64). */
EXPORT void oracle_gemm_q4_128(const uint8_t* blocks, const float* X, float* Y, int M, int K, int B) {
    const int G = K / 128;
    for (int r = 0; r < M; ++r) {
        for (int bb = 0; bb < B && bb < 64; ++bb) {
            double acc = 0.0;
            for (int g = 0; g < G; ++g) {
                const uint8_t* b = blocks + ((size_t)r * G + g) * 66;
                const float ws = half_to_float(rd16(b));
                for (int k = 0; k < 128; ++k) {
                    const float w = (float)(nib(b + 2, k) - 8) * ws;
                    acc += (double)w * (double)X[(size_t)bb * K + (size_t)g * 128 + k];
                }
            }
            Y[(size_t)bb * M + r] = (float)acc;
        }
    }
}

/* ------------------------------------------------------------------ A9(ii)
 * gemv_q4_q8_avx2 (asdsl/kernels/native/gemv_q4_avx2.cpp:131-253): symmetric
 * packed Q4 with fp32 scales; x quantized per group_size with the A1 rule;
 * y = sum_g ((float)sum (q-8)*xq * ws) * xs. */
EXPORT void oracle_gemv_q4_q8(const uint8_t* w, const float* scales, const float* x, float* y, int M, int K, int gs,
                              int8_t* scratch_q, float* scratch_s) {
    const int G = K / gs;
    oracle_quantize_activation(x, scratch_q, scratch_s, K, gs);
    for (int r = 0; r < M; ++r) {
        double acc = 0.0;
        const uint8_t* row = w + (size_t)r * (K / 2);
        for (int g = 0; g < G; ++g) {
            int32_t d = 0;
            for (int k = 0; k < gs; ++k) d += (nib(row, g * gs + k) - 8) * (int32_t)scratch_q[(size_t)g * gs + k];
            acc += (double)(((float)d * scales[(size_t)r * G + g]) * scratch_s[g]);
        }
        y[r] = (float)acc;
    }
}

/* ------------------------------------------------------------------ A8
 * Q4_K (ASDSL variant) superblock GEMV (asdsl/kernels/native/gemv_q4_avx2.cpp:78-120,283-420):
 * 144-byte block per 256 weights: fp16 d, fp16 dmin, 12 bytes of a linear
 * LSB-first 6-bit bitstream (entries 0-7 scales, 8-15 mins), 8 x 16 bytes of
 * nibbles.  x quantized per 32: scale = amax/127 (0 if amax < 1e-12),
 * q = clamp(round_half_away(x*127/amax), -127, 127).
 * y = sum_sb (d*sc*D - dmin*m*X) * xs. */
static int get6(const uint8_t* bytes, int idx) {
    const int bit = idx * 6, byte = bit / 8, off = bit % 8;
    int v = bytes[byte] >> off;
    if (off > 2) v |= bytes[byte + 1] << (8 - off);
    return v & 0x3F;
}

EXPORT void oracle_quantize_activation_q4k(const float* x, int8_t* xq, float* xs, int K) {
    const float r127 = 1.0f / 127.0f;
    for (int g = 0; g < K / 32; ++g) {
        float amax = 0.0f;
        for (int i = 0; i < 32; ++i) {
            const float a = fabsf(x[g * 32 + i]);
            if (a > amax) amax = a;
        }
        if (amax < 1e-12f) {
            xs[g] = 0.0f;
            for (int i = 0; i < 32; ++i) xq[g * 32 + i] = 0;
            continue;
        }
        const float inv = 127.0f / amax;
        xs[g] = amax * r127;
        for (int i = 0; i < 32; ++i) {
            volatile float p = x[g * 32 + i] * inv;
            int q = (int)roundf(p);
            q = q > 127 ? 127 : (q < -127 ? -127 : q);
            xq[g * 32 + i] = (int8_t)q;
        }
    }
}

EXPORT void oracle_gemv_q4km(const uint8_t* w, const float* x, float* y, int M, int K, int8_t* scratch_q,
                             float* scratch_s) {
    const int nb = K / 256;
    oracle_quantize_activation_q4k(x, scratch_q, scratch_s, K);
    for (int r = 0; r < M; ++r) {
        double acc = 0.0;
        for (int b = 0; b < nb; ++b) {
            const uint8_t* blk = w + ((size_t)r * nb + b) * 144;
            const float d = half_to_float(rd16(blk));
            const float dmin = half_to_float(rd16(blk + 2));
            for (int sb = 0; sb < 8; ++sb) {
                const float sub_scale = d * (float)get6(blk + 4, sb);
                const float sub_min = dmin * (float)get6(blk + 4, sb + 8);
                const int8_t* q8 = scratch_q + (size_t)b * 256 + sb * 32;
                int32_t dot, xsum;
                nib_dot(blk + 16 + sb * 16, q8, 32, &dot, &xsum);
                acc += (double)((sub_scale * (float)dot - sub_min * (float)xsum) * scratch_s[b * 8 + sb]);
            }
        }
        y[r] = (float)acc;
    }
}

/* ------------------------------------------------------------------ A10
 * fp32 affine Q4 GEMVs (asdsl/kernels/native/gemv_q4_avx2.cpp:665-806):
 * y = sum_g (sum_k q*x)*s + b*sum_k x.  `packed` = 2 nibbles per byte (low =
 * even); unpacked = one raw byte per element (the byte value is used as is). */
EXPORT void oracle_gemv_affine(const uint8_t* w, int packed, const float* x, const float* s, const float* bias,
                               float* y, int M, int K, int gs) {
    const int G = K / gs;
    for (int r = 0; r < M; ++r) {
        double acc = 0.0;
        for (int g = 0; g < G; ++g) {
            double dot = 0.0, sx = 0.0;
            for (int k = g * gs; k < (g + 1) * gs; ++k) {
                const int q = packed ? nib(w + (size_t)r * (K / 2), k) : w[(size_t)r * K + k];
                dot += (double)q * x[k];
                sx += x[k];
            }
            acc += dot * s[(size_t)r * G + g] + (bias ? (double)bias[(size_t)r * G + g] * sx : 0.0);
        }
        y[r] = (float)acc;
    }
}

/* gemv_q4_avx2 gs64 (asdsl/kernels/native/gemv_q4_kernel.cpp:96-122): scales only. */
EXPORT void oracle_gemv_q4_gs64(const uint8_t* w, const float* x, const float* s, float* y, int M, int K) {
    oracle_gemv_affine(w, 1, x, s, NULL, y, M, K, 64);
}

/* matmul_batch_q4 (asdsl/kernels/native/gemv_q4_avx2.cpp:950-1021): each weight
 * dequantized once as fma(q, s, b) in fp32, then dotted with every batch row. */
EXPORT void oracle_matmul_batch_q4(const uint8_t* w, const float* s, const float* bias, const float* X, float* Y,
                                   int M, int K, int B, int gs) {
    const int G = K / gs;
    for (int r = 0; r < M; ++r) {
        for (int bb = 0; bb < B; ++bb) {
            double acc = 0.0;
            for (int k = 0; k < K; ++k) {
                const int g = k / gs;
                const float wf = fmaf((float)nib(w + (size_t)r * (K / 2), k), s[(size_t)r * G + g],
                                      bias[(size_t)r * G + g]);
                acc += (double)wf * X[(size_t)bb * K + k];
            }
            Y[(size_t)bb * M + r] = (float)acc;
        }
    }
}

/* ------------------------------------------------------------------ A12
 * compute_bitmask (asdsl/kernels/native/gemv_sparse_avx2.cpp:144-179): bit k
 * set iff |x[k]| >= threshold (ordered compares: NaN is inactive). */
EXPORT void oracle_compute_bitmask(const float* x, uint32_t* mask, int K, float thr) {
    for (int w = 0; w < (K + 31) / 32; ++w) mask[w] = 0;
    for (int k = 0; k < K; ++k)
        if (x[k] >= thr || x[k] <= -thr) mask[k / 32] |= 1u << (k % 32);
}

/* gemv_sparse_with_indices / gemv_sparse_unpacked
 * (asdsl/kernels/native/gemv_sparse_avx2.cpp:66-139): over the listed columns
 * only, y = sum_g s*sum w*x + b*sum x (raw bytes; repeats count again;
 * indices outside [0,K) are ignored here, the reference reads them unchecked). */
EXPORT void oracle_gemv_sparse_indices(const uint8_t* w, const float* x, const float* s, const float* b,
                                       const int32_t* idx, int n, float* y, int M, int K, int gs) {
    const int G = K / gs;
    for (int r = 0; r < M; ++r) {
        double acc = 0.0;
        for (int i = 0; i < n; ++i) {
            const int k = idx[i];
            if (k < 0 || k >= K) continue;
            const int g = k / gs;
            acc += (double)s[(size_t)r * G + g] * w[(size_t)r * K + k] * x[k] + (double)b[(size_t)r * G + g] * x[k];
        }
        y[r] = (float)acc;
    }
}

/* sparse_down_proj_T (asdsl/kernels/native/gemv_sparse_avx2.cpp:273-382):
 * K-major packed Q4 w_T[in_dim][out_dim/2]; for every listed row r with
 * x[r] != 0: y[o] += fma(q, s*x_r, b*x_r) with s, b the fp32 scale/bias of
 * (r, o/gs).  Out-of-range rows are skipped (as the reference does). */
EXPORT void oracle_sparse_down_proj_T(const uint8_t* wT, const float* sT, const float* bT, const float* x,
                                      const int32_t* rows, int n, float* y, int in_dim, int out_dim, int gs) {
    const int G = out_dim / gs;
    for (int o = 0; o < out_dim; ++o) {
        double a = 0.0;
        for (int i = 0; i < n; ++i) {
            const int r = rows[i];
            if (r < 0 || r >= in_dim) continue;
            const float xv = x[r];
            if (xv == 0.0f) continue;
            const int g = o / gs;
            const float sv = sT[(size_t)r * G + g] * xv;
            const float bv = bT[(size_t)r * G + g] * xv;
            a += (double)fmaf((float)nib(wT + (size_t)r * (out_dim / 2), o), sv, bv);
        }
        y[o] = (float)a;
    }
}

/* ------------------------------------------------------------------ repack */

/* float64 -> IEEE binary16 bits, round to nearest even: subnormals, overflow
 * to inf at |d| >= 65520 (the tie above 65504 goes to the even 65536).  This
 * is numpy's float16 cast of a Python float, which the reference's repackers
 * apply to fp32 scales and to float64 zero points
 * (asdsl/quantization/repack_q4_32.py:19-20; repack_q4_128.py:18-19). */
static uint16_t double_to_half(double d) {
    const uint16_t sign = signbit(d) ? 0x8000u : 0u;
    if (isnan(d)) return (uint16_t)(sign | 0x7E00u);
    const double a = fabs(d);
    if (a >= 65520.0) return (uint16_t)(sign | 0x7C00u);
    if (a < ldexp(1.0, -14)) {                          /* subnormal: units of 2^-24 */
        const double m = nearbyint(ldexp(a, 24));       /* exact scaling, ties to even */
        return (uint16_t)(sign | (uint16_t)m);          /* m == 1024 is the smallest normal */
    }
    int ex;
    frexp(a, &ex);                                      /* a = f * 2^ex, f in [0.5, 1) */
    int e = ex - 1;                                     /* a in [2^e, 2^(e+1)) */
    double m = nearbyint((ldexp(a, -e) - 1.0) * 1024.0);  /* every step exact in double */
    if (m == 1024.0) {
        m = 0.0;
        ++e;
    }
    return (uint16_t)(sign | (uint16_t)((e + 15) << 10) | (uint16_t)m);
}

EXPORT void oracle_double_to_half(const double* d, uint16_t* out, int n) {
    for (int i = 0; i < n; ++i) out[i] = double_to_half(d[i]);
}

static void wr16(uint8_t* p, uint16_t v) {
    p[0] = (uint8_t)(v & 0xFF);
    p[1] = (uint8_t)(v >> 8);
}

/* float(max(s, 1e-8)) with s a numpy float32 (repack_q4_32.py:87): Python's
 * max keeps s unless 1e-8 > s, a comparison numpy makes in float32; the
 * result is the float64 1e-8 or s. */
static double floor_scale(float s) { return (float)1e-8 > s ? 1e-8 : (double)s; }

/* repack_asymmetric_to_q4_32_blocks (asdsl/quantization/repack_q4_32.py:63-102):
 * per (row, group of 32) a 20-byte block: fp16(max(s, 1e-8)), fp16(-b / max(s, 1e-8))
 * with the division in float64, then the group's 16 packed bytes unchanged
 * (unpack low-nibble-first, repack (q[1::2] << 4) | q[0::2]: the same bytes). */
EXPORT void oracle_repack_asym_to_q4_32(const uint8_t* packed, const float* scales, const float* biases,
                                        uint8_t* blocks, int rows, int cols) {
    const int G = cols / 32;
    for (int r = 0; r < rows; ++r)
        for (int g = 0; g < G; ++g) {
            const size_t gi = (size_t)r * G + g;
            const double sc = floor_scale(scales[gi]);
            const double zero = -(double)biases[gi] / sc;
            uint8_t* blk = blocks + gi * 20;
            wr16(blk, double_to_half(sc));
            wr16(blk + 2, double_to_half(zero));
            memcpy(blk + 4, packed + (size_t)r * (cols / 2) + (size_t)g * 16, 16);
        }
}

/* repack_preq_blocks_to_preq2 (asdsl/quantization/repack_preq2.py:22-49):
 * meta[row][g] = block bytes 0..3; quant[row/4][g][16*(row%4) ..+16] = block
 * bytes 4..19; the slots of rows past `rows` in the last band are zero. */
EXPORT void oracle_repack_preq_to_preq2(const uint8_t* preq, uint8_t* meta, uint8_t* quant, int rows, int cols) {
    const int G = cols / 32;
    const int bands = (rows + 3) / 4;
    memset(quant, 0, (size_t)bands * G * 64);
    for (int r = 0; r < rows; ++r)
        for (int g = 0; g < G; ++g) {
            const uint8_t* blk = preq + ((size_t)r * G + g) * 20;
            memcpy(meta + ((size_t)r * G + g) * 4, blk, 4);
            memcpy(quant + ((size_t)(r / 4) * G + g) * 64 + 16 * (r % 4), blk + 4, 16);
        }
}

/* The asymmetric packed weights straight into the preq2 layout at group size
 * gs (32: the composition repack_q4_32 -> repack_preq2, byte for byte; 128:
 * the same per-group fp16 (scale, zero) and 4-row bands of 64-byte slots). */
EXPORT void oracle_repack_asym_to_preq2(const uint8_t* packed, const float* scales, const float* biases,
                                        uint8_t* meta, uint8_t* quant, int rows, int cols, int gs) {
    const int G = cols / gs;
    const int nb = gs / 2;
    const int bands = (rows + 3) / 4;
    memset(quant, 0, (size_t)bands * G * 4 * nb);
    for (int r = 0; r < rows; ++r)
        for (int g = 0; g < G; ++g) {
            const size_t gi = (size_t)r * G + g;
            const double sc = floor_scale(scales[gi]);
            wr16(meta + gi * 4, double_to_half(sc));
            wr16(meta + gi * 4 + 2, double_to_half(-(double)biases[gi] / sc));
            memcpy(quant + ((size_t)(r / 4) * G + g) * 4 * nb + (size_t)nb * (r % 4),
                   packed + (size_t)r * (cols / 2) + (size_t)g * nb, nb);
        }
}

/* _symmetric_quantize_group (asdsl/quantization/repack_q4_128.py:22-31) on
 * 128 float32 weights: amax = max|w|; below 1e-12 the block is scale 0 and
 * nibbles 0x88; else scale = amax / 7 and inv = 7 / amax in float64, and
 * q = clip(round(w * f32(inv)) + 8, 0, 15) in float32 (numpy rounds half to
 * even); the block is fp16(scale) then the 64 packed nibble bytes. */
static void q4_128_group(const float* w, uint8_t* blk) {
    float amax = 0.0f;
    for (int i = 0; i < 128; ++i) amax = fabsf(w[i]) > amax ? fabsf(w[i]) : amax;
    if ((double)amax < 1e-12) {
        wr16(blk, 0);
        memset(blk + 2, 0x88, 64);
        return;
    }
    const double scale = (double)amax / 7.0;
    const float inv = (float)(7.0 / (double)amax);
    uint8_t q[128];
    for (int i = 0; i < 128; ++i) {
        float v = nearbyintf(w[i] * inv) + 8.0f;
        v = v < 0.0f ? 0.0f : (v > 15.0f ? 15.0f : v);
        q[i] = (uint8_t)v;
    }
    wr16(blk, double_to_half(scale));
    for (int i = 0; i < 64; ++i) blk[2 + i] = (uint8_t)((q[2 * i + 1] << 4) | q[2 * i]);
}

/* repack_fp32_to_q4_128_blocks (asdsl/quantization/repack_q4_128.py:72-92). */
EXPORT void oracle_repack_fp32_to_q4_128(const float* w, uint8_t* blocks, int rows, int cols) {
    const int G = cols / 128;
    for (int r = 0; r < rows; ++r)
        for (int g = 0; g < G; ++g)
            q4_128_group(w + (size_t)r * cols + (size_t)g * 128, blocks + ((size_t)r * G + g) * 66);
}

/* repack_asymmetric_to_q4_128_blocks (asdsl/quantization/repack_q4_128.py:34-69):
 * the asymmetric group dequantized as float32 (q - f32(zero)) * f32(scale),
 * zero = -b / max(s, 1e-8) in float64, then requantized symmetrically. */
EXPORT void oracle_repack_asym_to_q4_128(const uint8_t* packed, const float* scales, const float* biases,
                                         uint8_t* blocks, int rows, int cols) {
    const int G = cols / 128;
    float wf[128];
    for (int r = 0; r < rows; ++r)
        for (int g = 0; g < G; ++g) {
            const size_t gi = (size_t)r * G + g;
            const double sc = floor_scale(scales[gi]);
            const float zero32 = (float)(-(double)biases[gi] / sc);
            const float sc32 = (float)sc;
            const uint8_t* pg = packed + (size_t)r * (cols / 2) + (size_t)g * 64;
            for (int i = 0; i < 128; ++i) wf[i] = ((float)nib(pg, i) - zero32) * sc32;
            q4_128_group(wf, blocks + gi * 66);
        }
}

/* Q4_128 blocks -> preq2-g128 (no reference counterpart): meta = block
 * scale | fp16 8.0, the 64 nibble bytes into the row's band slot; slots of
 * rows past `rows` in the last band are zero. */
EXPORT void oracle_repack_q4_128_to_preq2(const uint8_t* blocks, uint8_t* meta, uint8_t* quant, int rows, int cols) {
    const int G = cols / 128;
    const int bands = (rows + 3) / 4;
    memset(quant, 0, (size_t)bands * G * 256);
    for (int r = 0; r < rows; ++r)
        for (int g = 0; g < G; ++g) {
            const uint8_t* blk = blocks + ((size_t)r * G + g) * 66;
            uint8_t* m = meta + ((size_t)r * G + g) * 4;
            m[0] = blk[0];
            m[1] = blk[1];
            wr16(m + 2, 0x4800u);
            memcpy(quant + ((size_t)(r / 4) * G + g) * 256 + 64 * (r % 4), blk + 2, 64);
        }
}

/* gemv_q4_s256_preq_avx2 (asdsl/kernels/native/gemv_q4_s256.cpp:79-209):
 * per row, 144-byte superblocks of 8 fp16 sub-scales then 128 nibble bytes
 * (low nibble = even weight); per 32-weight sub-block k with activation
 * group g: sc = ws * xs[g] (fp32), y += dot(q, x8) * sc - 8 * sum(x8) * sc.
 * The sum over sub-blocks is accumulated in double. */
EXPORT void oracle_gemv_q4_s256(const uint8_t* blocks, const int8_t* xq, const float* xs, float* y, int M, int K) {
    const int NS = K / 256;
    for (int r = 0; r < M; ++r) {
        double acc = 0.0;
        for (int sb = 0; sb < NS; ++sb) {
            const uint8_t* blk = blocks + ((size_t)r * NS + sb) * 144;
            for (int k = 0; k < 8; ++k) {
                const int g = sb * 8 + k;
                const float sc = half_to_float(rd16(blk + 2 * k)) * xs[g];
                const int8_t* x = xq + (size_t)g * 32;
                int dot = 0, xsum = 0;
                for (int i = 0; i < 32; ++i) {
                    dot += nib(blk + 16 + 16 * k, i) * x[i];
                    xsum += x[i];
                }
                acc += (double)dot * sc - 8.0 * (double)xsum * sc;
            }
        }
        y[r] = (float)acc;
    }
}

/* ------------------------------------------------------------------ GGUF
 * ggml's Q4_K and Q6_K block decoders (Q5_K and Q8_0 below), as the reference reaches them through
 * the gguf package (asdsl/io/gguf_loader.py:150-181, gguf.quants.dequantize;
 * gguf-py from llama.cpp, no version pinned by the reference and absent
 * here).  Restated from ggml's published block layouts; the float32 products
 * and differences are formed in numpy's order, one rounding each.
 * PARITY UNPINNED against the gguf package itself: the tests pin these by
 * the layouts' invariants (each 6-bit field and nibble moves exactly the
 * weights the layout assigns it) and by the lossless Q4_K -> ASDSL Q4_K
 * rearrangement, whose decode through the pinned ASDSL GEMV must agree. */
static void q4k_scale_min(const uint8_t* s, int j, int* sc, int* m) {
    if (j < 4) {
        *sc = s[j] & 63;
        *m = s[j + 4] & 63;
    } else {
        *sc = (s[j + 4] & 0x0F) | ((s[j - 4] >> 6) << 4);
        *m = (s[j + 4] >> 4) | ((s[j] >> 6) << 4);
    }
}

EXPORT void oracle_dequant_gguf_q4k(const uint8_t* blocks, float* w, size_t n_blocks) {
    for (size_t b = 0; b < n_blocks; ++b) {
        const uint8_t* blk = blocks + b * 144;
        const float d = half_to_float(rd16(blk));
        const float dmin = half_to_float(rd16(blk + 2));
        for (int j = 0; j < 8; ++j) {
            int sc, m;
            q4k_scale_min(blk + 4, j, &sc, &m);
            volatile float d1 = d * (float)sc;
            volatile float m1 = dmin * (float)m;
            for (int l = 0; l < 32; ++l) {
                const uint8_t byte = blk[16 + 32 * (j / 2) + l];
                const int q = (j & 1) ? (byte >> 4) : (byte & 0x0F);
                volatile float p = d1 * (float)q;
                w[b * 256 + 32 * j + l] = p - m1;
            }
        }
    }
}

EXPORT void oracle_dequant_gguf_q6k(const uint8_t* blocks, float* w, size_t n_blocks) {
    for (size_t b = 0; b < n_blocks; ++b) {
        const uint8_t* blk = blocks + b * 210;
        const float d = half_to_float(rd16(blk + 208));
        for (int h = 0; h < 2; ++h) {
            const uint8_t* ql = blk + 64 * h;
            const uint8_t* qh = blk + 128 + 32 * h;
            const int8_t* sc = (const int8_t*)(blk + 192 + 8 * h);
            for (int k = 0; k < 4; ++k) {
                for (int l = 0; l < 32; ++l) {
                    const uint8_t lb = ql[l + 32 * (k & 1)];
                    const int lo = k < 2 ? (lb & 0x0F) : (lb >> 4);
                    const int hi = (qh[l] >> (2 * k)) & 3;
                    volatile float ds = d * (float)sc[l / 16 + 2 * k];
                    w[b * 256 + 128 * h + 32 * k + l] = ds * (float)((lo | (hi << 4)) - 32);
                }
            }
        }
    }
}

/* ggml Q5_K (176 bytes per 256 weights: fp16 d, fp16 dmin, Q4_K's 12-byte
 * scale/min field, 32 high-bit bytes qh, 128 low-nibble bytes qs): weight
 * 32j + l of sub-block j takes nibble (j & 1) of qs[32*(j/2) + l] and bit j
 * of qh[l] as its fifth bit, w = (d*sc_j)*q - (dmin*m_j) (ggml's
 * dequantize_row_q5_K; gguf-py's Q5_K.dequantize_blocks forms the same
 * float32 products).  Same parity status as the Q4_K/Q6_K decoders above. */
EXPORT void oracle_dequant_gguf_q5k(const uint8_t* blocks, float* w, size_t n_blocks) {
    for (size_t b = 0; b < n_blocks; ++b) {
        const uint8_t* blk = blocks + b * 176;
        const float d = half_to_float(rd16(blk));
        const float dmin = half_to_float(rd16(blk + 2));
        const uint8_t* qh = blk + 16;
        const uint8_t* qs = blk + 48;
        for (int j = 0; j < 8; ++j) {
            int sc, m;
            q4k_scale_min(blk + 4, j, &sc, &m);
            volatile float d1 = d * (float)sc;
            volatile float m1 = dmin * (float)m;
            for (int l = 0; l < 32; ++l) {
                const uint8_t byte = qs[32 * (j / 2) + l];
                const int q = ((j & 1) ? (byte >> 4) : (byte & 0x0F)) | (((qh[l] >> j) & 1) << 4);
                volatile float p = d1 * (float)q;
                w[b * 256 + 32 * j + l] = p - m1;
            }
        }
    }
}

/* ggml Q8_0 (34 bytes per 32 weights: fp16 d, 32 int8 codes): w = code * d
 * (dequantize_row_q8_0; gguf-py's Q8_0.dequantize_blocks, x * d in float32). */
EXPORT void oracle_dequant_gguf_q8_0(const uint8_t* blocks, float* w, size_t n_blocks) {
    for (size_t b = 0; b < n_blocks; ++b) {
        const uint8_t* blk = blocks + b * 34;
        const float d = half_to_float(rd16(blk));
        for (int l = 0; l < 32; ++l) w[b * 32 + l] = (float)(int8_t)blk[2 + l] * d;
    }
}

/* The legacy 32-weight blocks (ggml's block_q4_0 / q4_1 / q5_0 / q5_1 and
 * dequantize_row_q4_0 .. q5_1; gguf-py's Q4_0 .. Q5_1 dequantize_blocks).
 * Byte j of the 16 nibble bytes holds weight j (low nibble) and weight
 * j + 16 (high nibble); Q5 blocks add a little-endian 32-bit word whose bit
 * i is weight i's fifth bit.  Q4_0: (q - 8) * d; Q5_0: (q - 16) * d; Q4_1
 * and Q5_1: d * q + m with the product rounded before the sum (numpy's
 * order).  Same parity status as the K-quant decoders above.
 *   Q4_0: fp16 d | 16 B nibbles                 (18 bytes)
 *   Q4_1: fp16 d | fp16 m | 16 B nibbles        (20 bytes)
 *   Q5_0: fp16 d | 4 B high bits | 16 B nibbles (22 bytes)
 *   Q5_1: fp16 d | fp16 m | 4 B high bits | 16 B nibbles (24 bytes) */
static void legacy_block(const uint8_t* blk, int bytes, float* w) {
    const float d = half_to_float(rd16(blk));
    const int has_m = bytes == 20 || bytes == 24;
    const int has_h = bytes == 22 || bytes == 24;
    const float m = has_m ? half_to_float(rd16(blk + 2)) : 0.0f;
    const uint8_t* hb = blk + (has_m ? 4 : 2);
    const uint32_t qh = has_h ? (uint32_t)hb[0] | ((uint32_t)hb[1] << 8) | ((uint32_t)hb[2] << 16) |
                                    ((uint32_t)hb[3] << 24)
                              : 0u;
    const uint8_t* qs = blk + (has_m ? 4 : 2) + (has_h ? 4 : 0);
    for (int i = 0; i < 32; ++i) {
        const int nib = i < 16 ? (qs[i] & 0x0F) : (qs[i - 16] >> 4);
        const int q = nib | (int)(((qh >> i) & 1u) << 4);
        if (has_m) {
            volatile float p = d * (float)q;
            w[i] = p + m;
        } else {
            w[i] = (float)(q - (has_h ? 16 : 8)) * d;
        }
    }
}

EXPORT void oracle_dequant_gguf_legacy(const uint8_t* blocks, int block_bytes, float* w, size_t n_blocks) {
    for (size_t b = 0; b < n_blocks; ++b) legacy_block(blocks + b * block_bytes, block_bytes, w + b * 32);
}

/* ggml Q2_K (84 bytes per 256 weights: 16 scale bytes, 64 code bytes qs,
 * fp16 d, fp16 dmin) and Q3_K (110 bytes: 32 high-mask bytes hmask, 64 code
 * bytes qs, 12 bytes of sixteen 6-bit scales, fp16 d); ggml's
 * dequantize_row_q2_K / q3_K, gguf-py's Q2_K / Q3_K dequantize_blocks.  Both
 * place weight 128n + 32j + 16h + l (n, h in 0..1, j in 0..3, l in 0..15) in
 * bits 2j..2j+1 of qs[32n + 16h + l] under scale 8n + 2j + h.
 *   Q2_K: scale byte s: w = (d * (s & 15)) * q - dmin * (s >> 4).
 *   Q3_K: q -= 4 unless bit 4n + j of hmask[16h + l] is set; scale k takes
 *     its low 4 bits from byte k (k < 8, low nibble) or byte k - 8 (high
 *     nibble) and its top 2 bits from bits 2(k/4).. of byte 8 + k % 4;
 *     w = (d * (scale - 32)) * q.
 * Same parity status as the other K-quant decoders. */
EXPORT void oracle_dequant_gguf_q2k(const uint8_t* blocks, float* w, size_t n_blocks) {
    for (size_t b = 0; b < n_blocks; ++b) {
        const uint8_t* blk = blocks + b * 84;
        const uint8_t* sc = blk;
        const uint8_t* qs = blk + 16;
        const float d = half_to_float(rd16(blk + 80));
        const float dmin = half_to_float(rd16(blk + 82));
        for (int wi = 0; wi < 256; ++wi) {
            const int n = wi / 128, j = (wi % 128) / 32, h = (wi % 32) / 16, l = wi % 16;
            const uint8_t s = sc[8 * n + 2 * j + h];
            const int q = (qs[32 * n + 16 * h + l] >> (2 * j)) & 3;
            volatile float dl = d * (float)(s & 15);
            volatile float ml = dmin * (float)(s >> 4);
            volatile float p = dl * (float)q;
            w[b * 256 + wi] = p - ml;
        }
    }
}

EXPORT void oracle_dequant_gguf_q3k(const uint8_t* blocks, float* w, size_t n_blocks) {
    for (size_t b = 0; b < n_blocks; ++b) {
        const uint8_t* blk = blocks + b * 110;
        const uint8_t* hm = blk;
        const uint8_t* qs = blk + 32;
        const uint8_t* sc = blk + 96;
        const float d = half_to_float(rd16(blk + 108));
        for (int wi = 0; wi < 256; ++wi) {
            const int n = wi / 128, j = (wi % 128) / 32, h = (wi % 32) / 16, l = wi % 16;
            const int k = 8 * n + 2 * j + h;
            const int lo = k < 8 ? (sc[k] & 15) : (sc[k - 8] >> 4);
            const int hi = (sc[8 + k % 4] >> (2 * (k / 4))) & 3;
            const int scale = (lo | (hi << 4)) - 32;
            const int q = ((qs[32 * n + 16 * h + l] >> (2 * j)) & 3) - (((hm[16 * h + l] >> (4 * n + j)) & 1) ? 0 : 4);
            volatile float dl = d * (float)scale;
            w[b * 256 + wi] = dl * (float)q;
        }
    }
}

/* ggml Q4_K -> the ASDSL Q4_K variant read by oracle_gemv_q4km: the same d,
 * dmin, 6-bit fields (linear LSB-first stream, scales then mins) and codes
 * (sub-block j's 32 codes in bytes 16+16j.., low nibble first). */
EXPORT void oracle_repack_gguf_q4k_to_q4km(const uint8_t* src, uint8_t* dst, size_t n_blocks) {
    for (size_t b = 0; b < n_blocks; ++b) {
        const uint8_t* in = src + b * 144;
        uint8_t* out = dst + b * 144;
        memset(out, 0, 144);
        memcpy(out, in, 4);
        for (int idx = 0; idx < 16; ++idx) {
            int sc, m;
            q4k_scale_min(in + 4, idx % 8, &sc, &m);
            const int v = idx < 8 ? sc : m;
            for (int bit = 0; bit < 6; ++bit)
                if (v & (1 << bit)) out[4 + (6 * idx + bit) / 8] |= (uint8_t)(1u << ((6 * idx + bit) % 8));
        }
        for (int j = 0; j < 8; ++j)
            for (int k = 0; k < 32; ++k) {
                const uint8_t byte = in[16 + 32 * (j / 2) + k];
                const int q = (j & 1) ? (byte >> 4) : (byte & 0x0F);
                out[16 + 16 * j + k / 2] |= (uint8_t)(q << (4 * (k & 1)));
            }
    }
}

/* Symmetric group-wise Q4 of fp32 weights (asdsl/quantization/core.py:358-420
 * with symmetric=True, bits=4, compute_scale_zero at :63-86), as the
 * reference requantizes GGUF projections (experiments/phi4_cpu_run.py:1444-1459):
 * scale = f16(max(amax, 1e-5f) / 7.5), q = clip(rne(w / max(f32(scale),
 * 1e-4f) + 7.5), 0, 15), packed low nibble first; scales out as f32(scale),
 * biases as -7.5 * f32(scale). */
EXPORT void oracle_quantize_q4_symmetric(const float* w, uint8_t* packed, float* scales, float* biases,
                                         size_t groups, int gs) {
    for (size_t g = 0; g < groups; ++g) {
        const float* x = w + g * gs;
        float amax = 0.0f;
        for (int i = 0; i < gs; ++i) amax = fabsf(x[i]) > amax ? fabsf(x[i]) : amax;
        if (amax < 1e-5f) amax = 1e-5f;
        volatile float scale = amax / 7.5f;
        double tmp = scale;
        uint16_t bits;
        oracle_double_to_half(&tmp, &bits, 1);
        const float sf = half_to_float(bits);
        const float denom = sf > 1e-4f ? sf : 1e-4f;
        for (int i = 0; i < gs; i += 2) {
            int q[2];
            for (int e = 0; e < 2; ++e) {
                volatile float r = x[i + e] / denom;
                volatile float a = r + 7.5f;
                float v = nearbyintf(a);
                v = v < 0.0f ? 0.0f : (v > 15.0f ? 15.0f : v);
                q[e] = (int)v;
            }
            packed[(g * gs + i) / 2] = (uint8_t)(q[0] | (q[1] << 4));
        }
        scales[g] = sf;
        biases[g] = -7.5f * sf;
    }
}

