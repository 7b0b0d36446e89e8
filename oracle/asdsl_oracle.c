/*
 * asdsl_oracle.c — CPU restatement of the reference's Q4 GEMV hot path.
 *
 * TEST INFRASTRUCTURE ONLY.  This file is the parity checker for the HIP
 * kernels: only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline
 * leg may load it.  The product path never calls it.
 *
 * Every function restates one reference routine in plain scalar C (no SIMD,
 * no threads).  Integer parts (nibble decode, int8 activation quantization,
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
