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

// ------------------------------------------------------------ lane exchange
// DPP controls (GCN/CDNA encoding): quad permutes, and row (16-lane) mirrors
// and rotations.
constexpr int kDppQuadXor1 = 0xB1;      // quad_perm [1,0,3,2]
constexpr int kDppQuadXor2 = 0x4E;      // quad_perm [2,3,0,1]
constexpr int kDppRowHalfMirror = 0x141;
constexpr int kDppRowMirror = 0x140;
constexpr int kDppRowRor4 = 0x124;
constexpr int kDppRowRor8 = 0x128;
// ds_swizzle bit mode: and_mask 0x1F, xor_mask 0x10 -> lane ^ 16 within 32.
constexpr int kSwizzleXor16 = 0x401F;

template <int CTRL>
__device__ __forceinline__ float dpp(float v) {
    return __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), CTRL, 0xF, 0xF, false));
}

template <int CTRL>
__device__ __forceinline__ int dpp(int v) {
    return __builtin_amdgcn_update_dpp(0, v, CTRL, 0xF, 0xF, false);
}

__device__ __forceinline__ float swz_xor16(float v) {
    return __builtin_bit_cast(float, __builtin_amdgcn_ds_swizzle(__builtin_bit_cast(int, v), kSwizzleXor16));
}

// max over aligned groups of kLanes consecutive lanes (kLanes in {1,2,4,8,16}),
// result in every lane of the group.
template <int kLanes>
__device__ __forceinline__ float group_max(float v) {
    if (kLanes >= 2) v = fmaxf(v, dpp<kDppQuadXor1>(v));
    if (kLanes >= 4) v = fmaxf(v, dpp<kDppQuadXor2>(v));
    if (kLanes >= 8) v = fmaxf(v, dpp<kDppRowHalfMirror>(v));
    if (kLanes >= 16) v = fmaxf(v, dpp<kDppRowMirror>(v));
    return v;
}

template <int kLanes, typename T>
__device__ __forceinline__ T group_sum(T v) {
    if (kLanes >= 2) v += dpp<kDppQuadXor1>(v);
    if (kLanes >= 4) v += dpp<kDppQuadXor2>(v);
    if (kLanes >= 8) v += dpp<kDppRowHalfMirror>(v);
    if (kLanes >= 16) v += dpp<kDppRowMirror>(v);
    return v;
}

// Sum over all lanes that agree with this lane in the two "slot" bits
// [SB, SB+2) of the lane index; every lane gets the sum for its slot.
template <int SB>
__device__ __forceinline__ float slot_sum(float v) {
    static_assert(SB == 0 || SB == 2, "slot bits at 0 or 2");
    if (SB == 0) {               // reduce lane bits 2,3 (in-row), 4, 5
        v += dpp<kDppRowRor4>(v);
        v += dpp<kDppRowRor8>(v);
    } else {                     // reduce lane bits 0,1 (quad), 4, 5
        v += dpp<kDppQuadXor1>(v);
        v += dpp<kDppQuadXor2>(v);
    }
    v += swz_xor16(v);
    v += __shfl_xor(v, 32, kWave);
    return v;
}

// ------------------------------------------------------------ int8 helpers
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

// ------------------------------------------------------------ activation
// LDS image of the int8 activation: split-order int8 (K/4 dwords), per-group
// scale (K/GS floats), per-unit (float)sum(xq)*scale (K/32 floats).
struct XImage {
    uint32_t* xq;
    float* scale;
    float* usum;
};

__device__ __forceinline__ XImage x_image(uint32_t* lds, int K, int gs) {
    XImage im;
    im.xq = lds;
    im.scale = reinterpret_cast<float*>(lds + (K >> 2));
    im.usum = im.scale + K / gs;
    return im;
}

__host__ __device__ inline size_t x_image_bytes(int K, int gs) {
    return static_cast<size_t>(K) + static_cast<size_t>(K / gs) * 4 + static_cast<size_t>(K / 32) * 4;
}

// Activation quantization rules of the reference.
//  kRne: quantize_activation_avx2 (asdsl/kernels/native/gemv_q4_preq_restored.cpp:505-549)
//    as built with -O3 -ffast-math (setup.py:56-65): amax/127.0f becomes
//    amax*(1/127.0f); 127.0f/amax stays a true division; cvtps_epi32 rounds half
//    to even; packs saturate to [-128, 127]; amax < 1e-9 -> q = 0, scale 1.
//  kRoundAway: the Q4_K path (asdsl/kernels/native/gemv_q4_avx2.cpp:377-400):
//    std::round (half away from zero), clamp to [-127, 127]; amax < 1e-12 ->
//    q = 0, scale 0.
enum class QRule { kRne, kRoundAway };

// One 8-element chunk quantized: split-order int8 (even = elements 0,2,4,6;
// odd = 1,3,5,7), the group scale, and the integer sum of its 32-element unit.
struct QChunk {
    uint32_t even, odd;
    float scale;
    int usum;
    int q[8];
};

// One thread owns one 8-element chunk; the GS/8 threads of a group are
// consecutive, aligned lanes of one wave (all of them must call this).
template <int GS, QRule R = QRule::kRne>
__device__ __forceinline__ QChunk quantize8(const float (&v)[8]) {
    constexpr int kLanes = GS / 8;
    QChunk c;
    float m = 0.0f;
#pragma unroll
    for (int i = 0; i < 8; ++i) m = fmaxf(m, fabsf(v[i]));
    const float amax = group_max<kLanes>(m);
    if (amax < (R == QRule::kRne ? 1e-9f : 1e-12f)) {
#pragma unroll
        for (int i = 0; i < 8; ++i) c.q[i] = 0;
        c.scale = R == QRule::kRne ? 1.0f : 0.0f;
    } else {
        c.scale = amax * (1.0f / 127.0f);
        const float inv = 127.0f / amax;
#pragma unroll
        for (int i = 0; i < 8; ++i) {
            if (R == QRule::kRne) {
                c.q[i] = sat_rne_i8(v[i] * inv);
            } else {
                int r = static_cast<int>(__builtin_roundf(v[i] * inv));
                c.q[i] = r > 127 ? 127 : (r < -127 ? -127 : r);
            }
        }
    }
    c.even = pack4_i8(c.q[0], c.q[2], c.q[4], c.q[6]);
    c.odd = pack4_i8(c.q[1], c.q[3], c.q[5], c.q[7]);
    c.usum = group_sum<4>(sum4_i8(c.even) + sum4_i8(c.odd));  // 4 chunks = 1 unit
    return c;
}

template <int GS, QRule R = QRule::kRne>
__device__ __forceinline__ void quantize_chunk(const float (&v)[8], int chunk, bool active, XImage im,
                                               int8_t* __restrict__ xq_nat, float* __restrict__ xscale_out) {
    constexpr int kLanes = GS / 8;
    const QChunk c = quantize8<GS, R>(v);
    if (active) {
        reinterpret_cast<uint2*>(im.xq)[chunk] = make_uint2(c.even, c.odd);
        if (xq_nat) {
            reinterpret_cast<uint2*>(xq_nat)[chunk] =
                make_uint2(pack4_i8(c.q[0], c.q[1], c.q[2], c.q[3]), pack4_i8(c.q[4], c.q[5], c.q[6], c.q[7]));
        }
        if ((chunk & (kLanes - 1)) == 0) {
            im.scale[chunk / kLanes] = c.scale;
            if (xscale_out) xscale_out[chunk / kLanes] = c.scale;
        }
        if ((chunk & 3) == 0) im.usum[chunk >> 2] = static_cast<float>(c.usum) * c.scale;
    }
}

// Caller-quantized activation (natural int8 order + per-group scales).
template <int GS>
__device__ __forceinline__ void load_q8_chunk(uint2 n, float scale, int chunk, bool active, XImage im) {
    constexpr int kLanes = GS / 8;
    // natural bytes b0..b7 -> even (b0,b2,b4,b6), odd (b1,b3,b5,b7)
    const uint32_t even = __builtin_amdgcn_perm(n.y, n.x, 0x06040200u);
    const uint32_t odd = __builtin_amdgcn_perm(n.y, n.x, 0x07050301u);
    const int usum = group_sum<4>(sum4_i8(even) + sum4_i8(odd));
    if (active) {
        reinterpret_cast<uint2*>(im.xq)[chunk] = make_uint2(even, odd);
        if ((chunk & (kLanes - 1)) == 0) im.scale[chunk / kLanes] = scale;
        if ((chunk & 3) == 0) im.usum[chunk >> 2] = static_cast<float>(usum) * scale;
    }
}

// Activation staging in two phases so that its global loads can be issued
// BEFORE the weight loads: vmcnt retires in order, so a load issued after the
// weights could only be consumed once every weight load had landed.
//   ActStage::load()    issues this thread's NCH chunk loads (clamped, in bounds)
//   ActStage::process() quantizes them into the LDS image (no global loads)
// One workgroup of NT threads covers K <= 8*NT*NCH; lanes past the end form
// whole groups of their own and never store.
template <int GS, int NT, int NCH, bool Q8, QRule R = QRule::kRne>
struct ActStage {
    float v[Q8 ? 1 : NCH][8];
    uint2 n[Q8 ? NCH : 1];
    float s[Q8 ? NCH : 1];

    __device__ __forceinline__ void load(const float* __restrict__ x, const int8_t* __restrict__ xq8,
                                         const float* __restrict__ xsc, int K) {
        const int nchunk = K >> 3;
        const int tid = static_cast<int>(threadIdx.x);
#pragma unroll
        for (int i = 0; i < NCH; ++i) {
            const int c = min(i * NT + tid, nchunk - 1);
            if constexpr (Q8) {
                n[i] = reinterpret_cast<const uint2*>(xq8)[c];
                s[i] = xsc[c / (GS / 8)];
            } else {
                const float4 a = reinterpret_cast<const float4*>(x)[2 * c];
                const float4 b = reinterpret_cast<const float4*>(x)[2 * c + 1];
                v[i][0] = a.x; v[i][1] = a.y; v[i][2] = a.z; v[i][3] = a.w;
                v[i][4] = b.x; v[i][5] = b.y; v[i][6] = b.z; v[i][7] = b.w;
            }
        }
    }

    __device__ __forceinline__ void process(int K, XImage im) {
        const int nchunk = K >> 3;
        const int tid = static_cast<int>(threadIdx.x);
#pragma unroll
        for (int i = 0; i < NCH; ++i) {
            const int c = i * NT + tid;
            if constexpr (Q8) load_q8_chunk<GS>(n[i], s[i], c, c < nchunk, im);
            else quantize_chunk<GS, R>(v[i], c, c < nchunk, im, nullptr, nullptr);
        }
    }
};

// The int8 activation image of the MFMA batched GEMV (16 columns): chunk c
// (8 elements) of column n as split-order int8 at img[((c / 4) * 16 + n) * 4 +
// c % 4], and per GS-group of column n (scale, integer sum * scale) at
// fac[(c / (GS / 8)) * 16 + n]; with `us`, per 32-element slice of column n
// (integer sum * scale, the single-column GEMV's usum of that slice) at
// us[(c / 4) * 16 + n].  The GS/8 lanes of a group are consecutive lanes of
// one wave and all call this; `active` gates the stores.
constexpr int kImageCols = 16;
template <int GS>
__device__ __forceinline__ void image_store8(const float (&v)[8], int c, int n, bool active, uint2* __restrict__ img,
                                             float2* __restrict__ fac, float* __restrict__ us = nullptr) {
    constexpr int kLanes = GS / 8;
    const QChunk q = quantize8<GS>(v);
    const int gsum = kLanes == 4 ? q.usum : group_sum<kLanes>(sum4_i8(q.even) + sum4_i8(q.odd));
    if (active) {
        img[(static_cast<size_t>(c >> 2) * kImageCols + n) * 4 + (c & 3)] = make_uint2(q.even, q.odd);
        if ((c & (kLanes - 1)) == 0)
            fac[static_cast<size_t>(c / kLanes) * kImageCols + n] = make_float2(q.scale, static_cast<float>(gsum) * q.scale);
        if (us && (c & 3) == 0) us[static_cast<size_t>(c >> 2) * kImageCols + n] = static_cast<float>(q.usum) * q.scale;
    }
}

// Byte offsets of an image's parts for in_features K: img at 0 (K * 16 B),
// fac at K * 16 (room for group size 32: K / 32 * 16 pairs), us at K * 20
// (K / 32 * 16 floats); K * 22 bytes in all.
__host__ __device__ constexpr size_t image_fac_offset(int K) { return static_cast<size_t>(K) * 16; }
__host__ __device__ constexpr size_t image_us_offset(int K) { return static_cast<size_t>(K) * 20; }
__host__ __device__ constexpr size_t image_bytes(int K) { return static_cast<size_t>(K) * 22; }

// Decode-step elementwise helpers shared by the fused GEMV prologues and the
// batched verify pass, so both compute identical values.

// The reference's exp polynomial (fast_exp_avx2, unified_engine.cpp:803-825)
// in two parts, exp(x) = p * 2^i: clamp to [-87.3, 87.3], t = x*log2(e)
// rounded to fp32, i = round-to-nearest-even(t), f = t - i, p = the degree-5
// polynomial in f by fused multiply-adds, 2^i by exponent bits.  Contraction
// is off here, so the compiler cannot fuse t into f = t - i (the reference
// rounds t); the fused steps are the explicit fmaf calls.
__device__ __forceinline__ float fast_exp_poly(float x, float& two_i) {
#pragma clang fp contract(off)
    x = fmaxf(x, -87.3f);
    x = fminf(x, 87.3f);
    const float t = x * 1.4426950408889634f;
    const float fi = __builtin_rintf(t);
    const int i = static_cast<int>(fi);
    const float f = t - fi;
    float p = fmaf(0.001333838100523091f, f, 0.009618129107628477f);
    p = fmaf(p, f, 0.05550410866482158f);
    p = fmaf(p, f, 0.2402265069591007f);
    p = fmaf(p, f, 0.6931471805599453f);
    p = fmaf(p, f, 1.0f);
    two_i = __builtin_bit_cast(float, (i + 127) << 23);
    return p;
}

// swiglu_inplace (unified_engine.cpp:827-857) as the reference's build
// evaluates it: the denominator 1 + p*2^i as one fused multiply-add, the
// quotient correctly rounded (the reference build forms it with a reciprocal
// estimate and one Newton step, which differs in the last bits and depends on
// the CPU's estimate table), then (g * sigmoid) * u; zeroed where |v| < thr
// when thr > 0 (FATReLU).
__device__ __forceinline__ float swiglu_ref(float g, float u, float thr) {
#pragma clang fp contract(off)
    float two_i;
    const float p = fast_exp_poly(0.0f - g, two_i);
    const float sigmoid = 1.0f / fmaf(p, two_i, 1.0f);
    float v = (g * sigmoid) * u;
    if (thr > 0.0f && !(fabsf(v) >= thr)) v = 0.0f;
    return v;
}

__device__ __forceinline__ unsigned long long argmax_key(float v, int row) {
    const uint32_t b = __builtin_bit_cast(uint32_t, v);
    const uint32_t k = (b & 0x80000000u) ? ~b : (b | 0x80000000u);
    return (static_cast<unsigned long long>(k) << 32) | (0xFFFFFFFFu - static_cast<uint32_t>(row));
}

// Workgroup timeline of the decode step's kernels, compiled in only by the
// timing build (-DASDSL_WG_TIMELINE, lib/libasdsl_hip_timeline.so): thread 0
// of workgroup wg stores the 100 MHz wall clock at fixed point k of its kernel
// to tl[(slot * kTimelineWgs + wg) * 8 + k] of the buffer set with
// asdsl_timeline_set_buffer.  Slots: 0 o_proj with the split merge, 1 gate_up
// with SwiGLU, 2 norm-fed GEMV (qkv), 3 plain 16-wave GEMV (down), 4 the
// step's attention, 6 attention combine, 7 plain 8-wave GEMV (o_proj beyond
// 512 positions), 5 the sparse down-projection's partial kernel.
constexpr int kTimelineSlots = 8;
constexpr int kTimelineWgs = 1024;
#ifdef ASDSL_WG_TIMELINE
#define ASDSL_TIMELINE_BUFFER __device__ unsigned long long* g_timeline;
#define ASDSL_TIMELINE_STAMP(slot, wg, k)                                                                  \
    do {                                                                                                   \
        if ((slot) >= 0 && g_timeline && (wg) < kTimelineWgs && threadIdx.x == 0)                          \
            g_timeline[(static_cast<size_t>(slot) * kTimelineWgs + (wg)) * 8 + (k)] =                      \
                static_cast<unsigned long long>(wall_clock64());                                           \
    } while (0)
#else
#define ASDSL_TIMELINE_BUFFER
#define ASDSL_TIMELINE_STAMP(slot, wg, k) \
    do {                                  \
        (void)(slot);                     \
        (void)(wg);                       \
    } while (0)
#endif

}  // namespace asdsl
