// Device helpers shared by the gfx950 GEMV kernels.
//
// Conventions used throughout:
//  * "unit" = 32 consecutive K elements = 16 bytes of packed nibbles.  Every
//    Q4 layout of the reference decomposes into units, so one inner routine
//    (unit_dot) serves preq, preq2 (g32 and g128) and Q4_128.
//  * The activation is staged in LDS as int8 in "split" order: each 8-element
//    chunk is stored as two dwords, even elements (0,2,4,6) then odd (1,3,5,7).
//    A packed weight dword w holds elements 0..7 of a chunk as nibbles
//    (low nibble = even element, asdsl/quantization/core.py:556-563), so
//    (w & 0x0F0F0F0F) lines up with the even dword and ((w >> 4) & 0x0F0F0F0F)
//    with the odd dword: two v_dot4_i32_i8 per weight dword, no byte shuffles.
//    Nibbles are 0..15, so they are valid non-negative signed bytes.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace asdsl {

constexpr int kWave = 64;

typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

// 16-byte streaming load with the non-temporal hint: weight bytes are read
// exactly once per call, so they should not displace the activation or the
// output in L2/MALL.
__device__ __forceinline__ uint4 load_stream16(const uint4* p) {
    const u32x4 v = __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(p));
    return make_uint4(v.x, v.y, v.z, v.w);
}

__device__ __forceinline__ float half_bits_to_float(uint32_t bits16) {
    const _Float16 h = __builtin_bit_cast(_Float16, static_cast<uint16_t>(bits16 & 0xFFFFu));
    return static_cast<float>(h);
}

// Exact int32 dot of one unit: 16 packed bytes (uint4) against 32 int8
// activations in split order (8 dwords: even/odd pairs per 8-element chunk).
__device__ __forceinline__ int unit_dot(const uint4 w, const uint32_t* __restrict__ xs8) {
    int d = 0;
    const uint32_t wv[4] = {w.x, w.y, w.z, w.w};
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const uint32_t lo = wv[i] & 0x0F0F0F0Fu;
        const uint32_t hi = (wv[i] >> 4) & 0x0F0F0F0Fu;
        d = __builtin_amdgcn_sdot4(static_cast<int>(lo), static_cast<int>(xs8[2 * i]), d, false);
        d = __builtin_amdgcn_sdot4(static_cast<int>(hi), static_cast<int>(xs8[2 * i + 1]), d, false);
    }
    return d;
}

// Same dot with weights centred at 8 ((q-8)*x), used by the symmetric
// kernels whose reference sums (q-8)*xq directly.  Computed as D - 8*X by the
// caller instead; kept here only as documentation of the identity.

// Round-to-nearest-even float -> int, saturated to int8 (cvtps_epi32 +
// packs_epi32 + packs_epi16 in the reference: both packs saturate).
__device__ __forceinline__ int sat_rne_i8(float v) {
    int r = static_cast<int>(__builtin_rintf(v));
    r = r > 127 ? 127 : r;
    r = r < -128 ? -128 : r;
    return r;
}

__device__ __forceinline__ uint32_t pack4_i8(int a, int b, int c, int d) {
    return (static_cast<uint32_t>(a) & 0xFFu) | ((static_cast<uint32_t>(b) & 0xFFu) << 8) |
           ((static_cast<uint32_t>(c) & 0xFFu) << 16) | ((static_cast<uint32_t>(d) & 0xFFu) << 24);
}

// Sum of the four signed bytes of a dword.
__device__ __forceinline__ int sum4_i8(uint32_t v) {
    return __builtin_amdgcn_sdot4(static_cast<int>(v), 0x01010101, 0, false);
}

template <int kLanes>
__device__ __forceinline__ float group_max(float v) {
#pragma unroll
    for (int m = 1; m < kLanes; m <<= 1) v = fmaxf(v, __shfl_xor(v, m, kWave));
    return v;
}

template <int kLanes>
__device__ __forceinline__ int group_sum_i(int v) {
#pragma unroll
    for (int m = 1; m < kLanes; m <<= 1) v += __shfl_xor(v, m, kWave);
    return v;
}

// Activation quantizer of the reference (quantize_activation_avx2,
// asdsl/kernels/native/gemv_q4_preq_restored.cpp:505-549) as built with
// -O3 -ffast-math (setup.py:56-65): the compiler turns amax/127.0f into
// amax*(1/127.0f); 127.0f/amax stays a true division; cvtps_epi32 rounds
// half to even.  Each thread owns one 8-element chunk; the GS/8 threads of a
// group are consecutive lanes of one wave.
//
// Writes, for the whole vector:
//   xq_split[K/4]  int8 in split order (dwords, see file header)
//   xscale[K/GS]   per-group scale
//   xsum_sc[K/32]  per-unit (float)sum(xq) * scale
//   xq_nat         optional natural-order int8 copy (global, may be null)
//   xscale_out     optional copy of the scales (global, may be null)
template <int GS>
__device__ __forceinline__ void quantize_chunk_q8(const float* __restrict__ x, int chunk, bool active,
                                                  uint32_t* __restrict__ xq_split,
                                                  float* __restrict__ xscale,
                                                  float* __restrict__ xsum_sc,
                                                  int8_t* __restrict__ xq_nat,
                                                  float* __restrict__ xscale_out) {
    static_assert(GS % 32 == 0 || GS == 64, "group size");
    constexpr int kLanes = GS / 8;
    float v[8];
    if (active) {
        const float4 a = reinterpret_cast<const float4*>(x)[2 * chunk];
        const float4 b = reinterpret_cast<const float4*>(x)[2 * chunk + 1];
        v[0] = a.x; v[1] = a.y; v[2] = a.z; v[3] = a.w;
        v[4] = b.x; v[5] = b.y; v[6] = b.z; v[7] = b.w;
    } else {
#pragma unroll
        for (int i = 0; i < 8; ++i) v[i] = 0.0f;
    }
    float m = 0.0f;
#pragma unroll
    for (int i = 0; i < 8; ++i) m = fmaxf(m, fabsf(v[i]));
    const float amax = group_max<kLanes>(m);

    int q[8];
    float scale;
    if (amax < 1e-9f) {
#pragma unroll
        for (int i = 0; i < 8; ++i) q[i] = 0;
        scale = 1.0f;
    } else {
        scale = amax * (1.0f / 127.0f);
        const float inv = 127.0f / amax;
#pragma unroll
        for (int i = 0; i < 8; ++i) q[i] = sat_rne_i8(v[i] * inv);
    }
    const uint32_t even = pack4_i8(q[0], q[2], q[4], q[6]);
    const uint32_t odd = pack4_i8(q[1], q[3], q[5], q[7]);
    // unit (32 elements) sum: 4 consecutive chunks
    const int usum = group_sum_i<4>(sum4_i8(even) + sum4_i8(odd));
    if (active) {
        xq_split[2 * chunk] = even;
        xq_split[2 * chunk + 1] = odd;
        if (xq_nat) {
            reinterpret_cast<uint2*>(xq_nat)[chunk] =
                make_uint2(pack4_i8(q[0], q[1], q[2], q[3]), pack4_i8(q[4], q[5], q[6], q[7]));
        }
        if ((chunk & (kLanes - 1)) == 0) {
            xscale[chunk / kLanes] = scale;
            if (xscale_out) xscale_out[chunk / kLanes] = scale;
        }
        if ((chunk & 3) == 0) xsum_sc[chunk >> 2] = static_cast<float>(usum) * scale;
    }
}

// Loads a caller-quantized activation (natural int8 order + per-group scales)
// into the split-order LDS image.  Same outputs as quantize_chunk_q8.
template <int GS>
__device__ __forceinline__ void load_chunk_q8(const int8_t* __restrict__ xq, const float* __restrict__ xsc_in,
                                              int chunk, bool active,
                                              uint32_t* __restrict__ xq_split,
                                              float* __restrict__ xscale,
                                              float* __restrict__ xsum_sc) {
    constexpr int kLanes = GS / 8;
    uint2 n = make_uint2(0u, 0u);
    if (active) n = reinterpret_cast<const uint2*>(xq)[chunk];
    // natural bytes b0..b7 -> even (b0,b2,b4,b6), odd (b1,b3,b5,b7)
    const uint32_t even = __builtin_amdgcn_perm(n.y, n.x, 0x06040200u);
    const uint32_t odd = __builtin_amdgcn_perm(n.y, n.x, 0x07050301u);
    const int usum = group_sum_i<4>(sum4_i8(even) + sum4_i8(odd));
    if (active) {
        const float scale = xsc_in[chunk / kLanes];
        xq_split[2 * chunk] = even;
        xq_split[2 * chunk + 1] = odd;
        if ((chunk & (kLanes - 1)) == 0) xscale[chunk / kLanes] = scale;
        if ((chunk & 3) == 0) xsum_sc[chunk >> 2] = static_cast<float>(usum) * scale;
    }
}

}  // namespace asdsl
