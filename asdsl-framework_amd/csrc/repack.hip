// Weight repackers on the GPU: the asymmetric Q4 weights of the quantized
// store into the byte layouts the GEMVs read, and preq blocks into preq2.
// The reference runs these as per-group Python loops at load time
// (asdsl/quantization/repack_q4_32.py, repack_preq2.py, repack_q4_128.py;
// ~80 s for the 128 projection tensors of a Phi-4 model).  Every output byte
// is the reference's: its arithmetic is numpy's (float64 division and the
// float16 cast of a float64 for the fp16 scale and zero; float32 array
// arithmetic and round-half-to-even for the Q4_128 requantization), restated
// here operation for operation.
//
// These kernels are byte movers bound by HBM: each thread owns one output
// unit (a 4-row band of one group, one block, or 8 weights of a Q4_128
// group), reads its inputs with 4- or 16-byte loads and writes whole slots.
#include <hip/hip_fp16.h>

#include "abi_util.hpp"
#include "device_common.hpp"

namespace asdsl {
namespace {

constexpr int kRepackThreads = 256;

// float64 -> fp16 bits, round to nearest even (numpy's float16 cast): round
// to odd into float32 (a 24-bit significand, more than the 11 + 2 bits that
// makes the second rounding exact), then float32 -> fp16 to nearest even.
__device__ __forceinline__ uint16_t f64_to_f16(double d) {
    if (isnan(d)) return static_cast<uint16_t>((signbit(d) ? 0x8000u : 0u) | 0x7E00u);
    float f = __double2float_rz(d);
    if (static_cast<double>(f) != d) f = __uint_as_float(__float_as_uint(f) | 1u);
    return __half_as_ushort(__float2half_rn(f));
}

// float(max(s, 1e-8)) for a float32 scale s (repack_q4_32.py:87): Python's
// max keeps s unless 1e-8 > s, compared in float32; float64 1e-8 or s.
__device__ __forceinline__ double floor_scale(float s) { return 1e-8f > s ? 1e-8 : static_cast<double>(s); }

// fp16 scale | fp16 zero << 16 of one asymmetric group (zero = -b / scale).
__device__ __forceinline__ uint32_t meta_word(float s, float b) {
    const double sc = floor_scale(s);
    return static_cast<uint32_t>(f64_to_f16(sc)) | (static_cast<uint32_t>(f64_to_f16(-static_cast<double>(b) / sc)) << 16);
}

// preq (20-byte blocks, row-major) -> preq2: one thread per (band, group)
// writes meta[row][g] for the band's rows and the group's 64-byte slot;
// rows past `rows` leave their slots zero (repack_preq2.py:22-49).
__global__ __launch_bounds__(kRepackThreads) void preq_to_preq2_kernel(const uint8_t* __restrict__ preq,
                                                                       uint32_t* __restrict__ meta,
                                                                       uint4* __restrict__ quant, int rows, int G,
                                                                       size_t units) {
    const size_t u = static_cast<size_t>(blockIdx.x) * kRepackThreads + threadIdx.x;
    if (u >= units) return;
    const size_t band = u / G;
    const int g = static_cast<int>(u - band * G);
#pragma unroll
    for (int r4 = 0; r4 < 4; ++r4) {
        const size_t row = band * 4 + r4;
        uint4 slot = make_uint4(0u, 0u, 0u, 0u);
        if (row < static_cast<size_t>(rows)) {
            const uint32_t* b = reinterpret_cast<const uint32_t*>(preq + (row * G + g) * 20);
            meta[row * G + g] = b[0];
            slot = make_uint4(b[1], b[2], b[3], b[4]);
        }
        quant[u * 4 + r4] = slot;
    }
}

// asymmetric packed Q4 (gs 32) -> 20-byte preq blocks: one thread per
// (row, group) (repack_q4_32.py:63-102).
__global__ __launch_bounds__(kRepackThreads) void asym_to_q4_32_kernel(const uint4* __restrict__ packed,
                                                                       const float* __restrict__ scales,
                                                                       const float* __restrict__ biases,
                                                                       uint32_t* __restrict__ blocks, size_t units) {
    const size_t u = static_cast<size_t>(blockIdx.x) * kRepackThreads + threadIdx.x;
    if (u >= units) return;
    const uint4 q = packed[u];  // row-major packed rows of 16 bytes per group
    uint32_t* b = blocks + u * 5;
    b[0] = meta_word(scales[u], biases[u]);
    b[1] = q.x;
    b[2] = q.y;
    b[3] = q.z;
    b[4] = q.w;
}

// asymmetric packed Q4 -> preq2 at group size GS (32: the composition of the
// two repackers above; 128: the same band structure with 64-byte row slots).
// One thread per (band, group).
template <int GS>
__global__ __launch_bounds__(kRepackThreads) void asym_to_preq2_kernel(const uint4* __restrict__ packed,
                                                                       const float* __restrict__ scales,
                                                                       const float* __restrict__ biases,
                                                                       uint32_t* __restrict__ meta,
                                                                       uint4* __restrict__ quant, int rows, int G,
                                                                       size_t units) {
    constexpr int kVec = GS / 32;  // 16-byte pieces per row slot
    const size_t u = static_cast<size_t>(blockIdx.x) * kRepackThreads + threadIdx.x;
    if (u >= units) return;
    const size_t band = u / G;
    const int g = static_cast<int>(u - band * G);
#pragma unroll
    for (int r4 = 0; r4 < 4; ++r4) {
        const size_t row = band * 4 + r4;
        const bool live = row < static_cast<size_t>(rows);
        uint4 v[kVec];
#pragma unroll
        for (int i = 0; i < kVec; ++i)
            v[i] = live ? packed[(row * G + g) * kVec + i] : make_uint4(0u, 0u, 0u, 0u);
        if (live) meta[row * G + g] = meta_word(scales[row * G + g], biases[row * G + g]);
#pragma unroll
        for (int i = 0; i < kVec; ++i) quant[(u * 4 + r4) * kVec + i] = v[i];
    }
}

// Symmetric Q4_128 requantization (repack_q4_128.py:22-31), 16 lanes per
// group, 8 weights per lane: amax over the group; below 1e-12 the block is
// scale 0 and nibbles 0x88; else fp16(amax / 7) (float64) and levels
// clip(rint(w * f32(7 / amax)) + 8, 0, 15) in float32.  Writes the 66-byte
// block: lane 0 the scale, lane j nibble bytes 4j..4j+3 (2-byte aligned).
__device__ __forceinline__ void q4_128_store(const float (&w)[8], uint8_t* __restrict__ blk, int j) {
    float amax = 0.0f;
#pragma unroll
    for (int i = 0; i < 8; ++i) amax = fmaxf(amax, fabsf(w[i]));
#pragma unroll
    for (int o = 1; o < 16; o <<= 1) amax = fmaxf(amax, __shfl_xor(amax, o, kWave));
    uint32_t nib = 0x88888888u;
    uint16_t s16 = 0;
    if (static_cast<double>(amax) >= 1e-12) {
        s16 = f64_to_f16(static_cast<double>(amax) / 7.0);
        const float inv = static_cast<float>(7.0 / static_cast<double>(amax));
        nib = 0u;
#pragma unroll
        for (int i = 0; i < 8; ++i) {
            const float prod = w[i] * inv;
            const float lv = fminf(fmaxf(rintf(prod) + 8.0f, 0.0f), 15.0f);
            nib |= static_cast<uint32_t>(lv) << (4 * i);
        }
    }
    uint16_t* out = reinterpret_cast<uint16_t*>(blk);
    if (j == 0) out[0] = s16;
    out[1 + 2 * j] = static_cast<uint16_t>(nib & 0xFFFFu);
    out[2 + 2 * j] = static_cast<uint16_t>(nib >> 16);
}

// fp32 weights -> Q4_128 blocks (repack_q4_128.py:72-92).
__global__ __launch_bounds__(kRepackThreads) void fp32_to_q4_128_kernel(const float4* __restrict__ w,
                                                                        uint8_t* __restrict__ blocks, size_t groups) {
    const size_t t = static_cast<size_t>(blockIdx.x) * kRepackThreads + threadIdx.x;
    const size_t grp = t / 16;  // uniform over the 16 lanes of a group; groups*16 threads fill whole waves' groups
    const int j = static_cast<int>(t % 16);
    if (grp >= groups) return;
    const float4 a = w[grp * 32 + 2 * j];
    const float4 b = w[grp * 32 + 2 * j + 1];
    const float v[8] = {a.x, a.y, a.z, a.w, b.x, b.y, b.z, b.w};
    q4_128_store(v, blocks + grp * 66, j);
}

// asymmetric packed Q4 (gs 128) -> Q4_128 blocks (repack_q4_128.py:34-69):
// the group decoded in float32 as (q - f32(zero)) * f32(max(s, 1e-8)), zero
// = -b / max(s, 1e-8) in float64, then requantized.
__global__ __launch_bounds__(kRepackThreads) void asym_to_q4_128_kernel(const uint32_t* __restrict__ packed,
                                                                        const float* __restrict__ scales,
                                                                        const float* __restrict__ biases,
                                                                        uint8_t* __restrict__ blocks,
                                                                        size_t groups) {
    const size_t t = static_cast<size_t>(blockIdx.x) * kRepackThreads + threadIdx.x;
    const size_t grp = t / 16;
    const int j = static_cast<int>(t % 16);
    if (grp >= groups) return;
    const uint32_t q = packed[grp * 16 + j];
    const double sc = floor_scale(scales[grp]);
    const float zero32 = static_cast<float>(-static_cast<double>(biases[grp]) / sc);
    const float sc32 = static_cast<float>(sc);
    float v[8];
#pragma unroll
    for (int i = 0; i < 8; ++i) {
        const float d = static_cast<float>((q >> (4 * i)) & 0xFu) - zero32;
        v[i] = d * sc32;
    }
    q4_128_store(v, blocks + grp * 66, j);
}

// Q4_128 blocks -> preq2-g128: the symmetric block (scale s, levels q with
// w = (q - 8) * s) is the asymmetric group (scale s, zero 8), so meta is
// fp16 s | fp16 8.0 and the 64 nibble bytes move into the row's band slot.
// One thread per (band, group); blocks are 2-byte aligned (66-byte stride).
typedef uint32_t u32x4_a2 __attribute__((ext_vector_type(4), aligned(2)));

__global__ __launch_bounds__(kRepackThreads) void q4_128_to_preq2_kernel(const uint8_t* __restrict__ blocks,
                                                                         uint32_t* __restrict__ meta,
                                                                         uint4* __restrict__ quant, int rows, int G,
                                                                         size_t units) {
    constexpr uint32_t kZero8 = 0x4800u;  // fp16 8.0
    const size_t u = static_cast<size_t>(blockIdx.x) * kRepackThreads + threadIdx.x;
    if (u >= units) return;
    const size_t band = u / G;
    const int g = static_cast<int>(u - band * G);
#pragma unroll
    for (int r4 = 0; r4 < 4; ++r4) {
        const size_t row = band * 4 + r4;
        const bool live = row < static_cast<size_t>(rows);
        uint4 v[4];
        if (live) {
            const uint8_t* blk = blocks + (row * G + g) * 66;
            meta[row * G + g] = static_cast<uint32_t>(*reinterpret_cast<const uint16_t*>(blk)) | (kZero8 << 16);
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const u32x4_a2 w = *reinterpret_cast<const u32x4_a2*>(blk + 2 + 16 * i);
                v[i] = make_uint4(w.x, w.y, w.z, w.w);
            }
        } else {
#pragma unroll
            for (int i = 0; i < 4; ++i) v[i] = make_uint4(0u, 0u, 0u, 0u);
        }
#pragma unroll
        for (int i = 0; i < 4; ++i) quant[(u * 4 + r4) * 4 + i] = v[i];
    }
}

unsigned blocks_for(size_t threads) { return static_cast<unsigned>((threads + kRepackThreads - 1) / kRepackThreads); }

bool aligned(const void* p, size_t a) { return reinterpret_cast<uintptr_t>(p) % a == 0; }

asdsl_status check_shape(const char* fn, int rows, int cols, int gs) {
    if (rows <= 0 || cols <= 0 || cols % gs != 0) {
        set_error("%s: rows must be positive and cols a positive multiple of %d (got %d x %d)", fn, gs, rows, cols);
        return ASDSL_ERR_INVALID_ARGUMENT;
    }
    return ASDSL_OK;
}

}  // namespace
}  // namespace asdsl

using namespace asdsl;

extern "C" asdsl_status asdsl_repack_preq_to_preq2(const uint8_t* preq, uint8_t* meta, uint8_t* quant, int rows,
                                                   int cols, int group_size, asdsl_stream_t stream) {
    ASDSL_CHECK_ARG(preq && meta && quant, "repack_preq_to_preq2: null pointer");
    ASDSL_CHECK_ARG(group_size == 32, "repack_preq_to_preq2: preq2 repack requires group_size=32");
    const asdsl_status cs = check_shape("repack_preq_to_preq2", rows, cols, 32);
    if (cs != ASDSL_OK) return cs;
    ASDSL_CHECK_ARG(aligned(preq, 4) && aligned(meta, 4) && aligned(quant, 16),
                    "repack_preq_to_preq2: preq and meta must be 4-byte and quant 16-byte aligned");
    const int G = cols / 32;
    const size_t units = static_cast<size_t>((rows + 3) / 4) * G;
    return launch("preq_to_preq2_kernel", preq_to_preq2_kernel, dim3(blocks_for(units)), dim3(kRepackThreads), 0,
                  as_hip(stream), preq, reinterpret_cast<uint32_t*>(meta), reinterpret_cast<uint4*>(quant), rows, G,
                  units);
}

extern "C" asdsl_status asdsl_repack_asym_to_q4_32(const uint8_t* packed, const float* scales, const float* biases,
                                                   uint8_t* blocks, int rows, int cols, int group_size,
                                                   asdsl_stream_t stream) {
    ASDSL_CHECK_ARG(packed && scales && biases && blocks, "repack_asym_to_q4_32: null pointer");
    ASDSL_CHECK_ARG(group_size == 32, "repack_asym_to_q4_32: requires group_size=32");
    const asdsl_status cs = check_shape("repack_asym_to_q4_32", rows, cols, 32);
    if (cs != ASDSL_OK) return cs;
    ASDSL_CHECK_ARG(aligned(packed, 16) && aligned(scales, 4) && aligned(biases, 4) && aligned(blocks, 4),
                    "repack_asym_to_q4_32: packed must be 16-byte and the others 4-byte aligned");
    const size_t units = static_cast<size_t>(rows) * (cols / 32);
    return launch("asym_to_q4_32_kernel", asym_to_q4_32_kernel, dim3(blocks_for(units)), dim3(kRepackThreads), 0,
                  as_hip(stream), reinterpret_cast<const uint4*>(packed), scales, biases,
                  reinterpret_cast<uint32_t*>(blocks), units);
}

extern "C" asdsl_status asdsl_repack_asym_to_preq2(const uint8_t* packed, const float* scales, const float* biases,
                                                   uint8_t* meta, uint8_t* quant, int rows, int cols, int group_size,
                                                   asdsl_stream_t stream) {
    ASDSL_CHECK_ARG(packed && scales && biases && meta && quant, "repack_asym_to_preq2: null pointer");
    ASDSL_CHECK_ARG(group_size == 32 || group_size == 128, "repack_asym_to_preq2: group_size must be 32 or 128");
    const asdsl_status cs = check_shape("repack_asym_to_preq2", rows, cols, group_size);
    if (cs != ASDSL_OK) return cs;
    ASDSL_CHECK_ARG(aligned(packed, 16) && aligned(scales, 4) && aligned(biases, 4) && aligned(meta, 4) &&
                        aligned(quant, 16),
                    "repack_asym_to_preq2: packed and quant must be 16-byte and the others 4-byte aligned");
    const int G = cols / group_size;
    const size_t units = static_cast<size_t>((rows + 3) / 4) * G;
    const dim3 grid(blocks_for(units));
    auto* m = reinterpret_cast<uint32_t*>(meta);
    auto* q = reinterpret_cast<uint4*>(quant);
    const auto* p = reinterpret_cast<const uint4*>(packed);
    if (group_size == 32)
        return launch("asym_to_preq2_kernel", asym_to_preq2_kernel<32>, grid, dim3(kRepackThreads), 0,
                      as_hip(stream), p, scales, biases, m, q, rows, G, units);
    return launch("asym_to_preq2_kernel", asym_to_preq2_kernel<128>, grid, dim3(kRepackThreads), 0, as_hip(stream),
                  p, scales, biases, m, q, rows, G, units);
}

extern "C" asdsl_status asdsl_repack_fp32_to_q4_128(const float* weights, uint8_t* blocks, int rows, int cols,
                                                    int group_size, asdsl_stream_t stream) {
    ASDSL_CHECK_ARG(weights && blocks, "repack_fp32_to_q4_128: null pointer");
    ASDSL_CHECK_ARG(group_size == 128, "repack_fp32_to_q4_128: requires group_size=128");
    const asdsl_status cs = check_shape("repack_fp32_to_q4_128", rows, cols, 128);
    if (cs != ASDSL_OK) return cs;
    ASDSL_CHECK_ARG(aligned(weights, 16) && aligned(blocks, 2),
                    "repack_fp32_to_q4_128: weights must be 16-byte and blocks 2-byte aligned");
    const size_t groups = static_cast<size_t>(rows) * (cols / 128);
    return launch("fp32_to_q4_128_kernel", fp32_to_q4_128_kernel, dim3(blocks_for(groups * 16)),
                  dim3(kRepackThreads), 0, as_hip(stream), reinterpret_cast<const float4*>(weights), blocks, groups);
}

extern "C" asdsl_status asdsl_repack_asym_to_q4_128(const uint8_t* packed, const float* scales, const float* biases,
                                                    uint8_t* blocks, int rows, int cols, int group_size,
                                                    asdsl_stream_t stream) {
    ASDSL_CHECK_ARG(packed && scales && biases && blocks, "repack_asym_to_q4_128: null pointer");
    ASDSL_CHECK_ARG(group_size == 128, "repack_asym_to_q4_128: requires group_size=128");
    const asdsl_status cs = check_shape("repack_asym_to_q4_128", rows, cols, 128);
    if (cs != ASDSL_OK) return cs;
    ASDSL_CHECK_ARG(aligned(packed, 4) && aligned(scales, 4) && aligned(biases, 4) && aligned(blocks, 2),
                    "repack_asym_to_q4_128: packed, scales and biases must be 4-byte and blocks 2-byte aligned");
    const size_t groups = static_cast<size_t>(rows) * (cols / 128);
    return launch("asym_to_q4_128_kernel", asym_to_q4_128_kernel, dim3(blocks_for(groups * 16)),
                  dim3(kRepackThreads), 0, as_hip(stream), reinterpret_cast<const uint32_t*>(packed), scales, biases,
                  blocks, groups);
}

extern "C" asdsl_status asdsl_repack_q4_128_to_preq2(const uint8_t* blocks, uint8_t* meta, uint8_t* quant, int rows,
                                                     int cols, asdsl_stream_t stream) {
    ASDSL_CHECK_ARG(blocks && meta && quant, "repack_q4_128_to_preq2: null pointer");
    const asdsl_status cs = check_shape("repack_q4_128_to_preq2", rows, cols, 128);
    if (cs != ASDSL_OK) return cs;
    ASDSL_CHECK_ARG(aligned(blocks, 2) && aligned(meta, 4) && aligned(quant, 16),
                    "repack_q4_128_to_preq2: blocks 2-byte, meta 4-byte and quant 16-byte aligned");
    const int G = cols / 128;
    const size_t units = static_cast<size_t>((rows + 3) / 4) * G;
    return launch("q4_128_to_preq2_kernel", q4_128_to_preq2_kernel, dim3(blocks_for(units)), dim3(kRepackThreads),
                  0, as_hip(stream), blocks, reinterpret_cast<uint32_t*>(meta), reinterpret_cast<uint4*>(quant), rows,
                  G, units);
}
