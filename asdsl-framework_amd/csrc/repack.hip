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
// The preq2 producers give each lane one 16-byte piece of the output, so a
// wave's stores cover consecutive bytes and its loads read each row's
// groups as contiguous runs; the block writers (20- and 66-byte blocks, not
// a multiple of the store width) assemble a workgroup's output in LDS and
// write it out with consecutive dword stores.
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

typedef uint32_t u32x4_a4 __attribute__((ext_vector_type(4), aligned(4)));
typedef uint32_t u32x4_a2 __attribute__((ext_vector_type(4), aligned(2)));

// preq (20-byte blocks, row-major) -> preq2: one lane per 16-byte band slot
// (lane t = slot t of quant: unit t/4 = (band, group), row slot t%4), which
// also writes that row's meta word; slots of rows past `rows` are zero
// (repack_preq2.py:22-49).
__global__ __launch_bounds__(kRepackThreads) void preq_to_preq2_kernel(const uint8_t* __restrict__ preq,
                                                                       uint32_t* __restrict__ meta,
                                                                       uint4* __restrict__ quant, int rows, int G,
                                                                       size_t slots) {
    const size_t t = static_cast<size_t>(blockIdx.x) * kRepackThreads + threadIdx.x;
    if (t >= slots) return;
    const size_t u = t / 4;
    const size_t band = u / G;
    const int g = static_cast<int>(u - band * G);
    const size_t row = band * 4 + (t % 4);
    uint4 v = make_uint4(0u, 0u, 0u, 0u);
    if (row < static_cast<size_t>(rows)) {
        const uint8_t* blk = preq + (row * G + g) * 20;
        meta[row * G + g] = *reinterpret_cast<const uint32_t*>(blk);
        const u32x4_a4 w = *reinterpret_cast<const u32x4_a4*>(blk + 4);
        v = make_uint4(w.x, w.y, w.z, w.w);
    }
    quant[t] = v;
}

// asymmetric packed Q4 (gs 32) -> 20-byte preq blocks: one thread per
// (row, group) builds its block in LDS; the workgroup's 256 consecutive
// blocks then go out as consecutive dwords (repack_q4_32.py:63-102).
__global__ __launch_bounds__(kRepackThreads) void asym_to_q4_32_kernel(const uint4* __restrict__ packed,
                                                                       const float* __restrict__ scales,
                                                                       const float* __restrict__ biases,
                                                                       uint32_t* __restrict__ blocks, size_t units) {
    __shared__ uint32_t stage[kRepackThreads * 5];
    const size_t base = static_cast<size_t>(blockIdx.x) * kRepackThreads;
    const size_t u = base + threadIdx.x;
    if (u < units) {
        const uint4 q = packed[u];  // row-major packed rows of 16 bytes per group
        uint32_t* b = stage + threadIdx.x * 5;
        b[0] = meta_word(scales[u], biases[u]);
        b[1] = q.x;
        b[2] = q.y;
        b[3] = q.z;
        b[4] = q.w;
    }
    __syncthreads();
    const int nwords = static_cast<int>(min(static_cast<size_t>(kRepackThreads), units - base)) * 5;
    for (int i = static_cast<int>(threadIdx.x); i < nwords; i += kRepackThreads) blocks[base * 5 + i] = stage[i];
}

// asymmetric packed Q4 -> preq2 at group size GS (32: the composition of the
// two repackers above; 128: the same band structure with 64-byte row slots).
// One lane per 16-byte piece of quant: unit (band, group) t / (4 kVec), row
// slot (t / kVec) % 4, piece t % kVec; the piece-0 lane writes the meta word.
template <int GS>
__global__ __launch_bounds__(kRepackThreads) void asym_to_preq2_kernel(const uint4* __restrict__ packed,
                                                                       const float* __restrict__ scales,
                                                                       const float* __restrict__ biases,
                                                                       uint32_t* __restrict__ meta,
                                                                       uint4* __restrict__ quant, int rows, int G,
                                                                       size_t pieces) {
    constexpr int kVec = GS / 32;  // 16-byte pieces per row slot
    const size_t t = static_cast<size_t>(blockIdx.x) * kRepackThreads + threadIdx.x;
    if (t >= pieces) return;
    const size_t u = t / (4 * kVec);
    const int j = static_cast<int>(t % (4 * kVec));
    const size_t band = u / G;
    const int g = static_cast<int>(u - band * G);
    const size_t row = band * 4 + j / kVec;
    const int i = j % kVec;
    uint4 v = make_uint4(0u, 0u, 0u, 0u);
    if (row < static_cast<size_t>(rows)) {
        v = packed[(row * G + g) * kVec + i];
        if (i == 0) meta[row * G + g] = meta_word(scales[row * G + g], biases[row * G + g]);
    }
    quant[t] = v;
}

// Symmetric Q4_128 requantization (repack_q4_128.py:22-31), LANES lanes
// per group, 128 / LANES weights per lane: amax over the group; below 1e-12
// the block is scale 0 and nibbles 0x88; else fp16(amax / 7) (float64) and
// levels clip(rint(w * f32(7 / amax)) + 8, 0, 15) in float32.  Writes the
// 66-byte block (33 halfwords) into `blk`: lane 0 the scale, lane j nibble
// halfwords 1 + (N/4) j ...
template <int LANES>
__device__ __forceinline__ void q4_128_store(const float (&w)[128 / LANES], uint16_t* __restrict__ blk, int j) {
    constexpr int N = 128 / LANES;
    float amax = 0.0f;
#pragma unroll
    for (int i = 0; i < N; ++i) amax = fmaxf(amax, fabsf(w[i]));
#pragma unroll
    for (int o = 1; o < LANES; o <<= 1) amax = fmaxf(amax, __shfl_xor(amax, o, kWave));
    uint32_t nib[N / 8];
    uint16_t s16 = 0;
#pragma unroll
    for (int k = 0; k < N / 8; ++k) nib[k] = 0x88888888u;
    if (static_cast<double>(amax) >= 1e-12) {
        s16 = f64_to_f16(static_cast<double>(amax) / 7.0);
        const float inv = static_cast<float>(7.0 / static_cast<double>(amax));
#pragma unroll
        for (int k = 0; k < N / 8; ++k) {
            nib[k] = 0u;
#pragma unroll
            for (int i = 0; i < 8; ++i) {
                const float prod = w[8 * k + i] * inv;
                const float lv = fminf(fmaxf(rintf(prod) + 8.0f, 0.0f), 15.0f);
                nib[k] |= static_cast<uint32_t>(lv) << (4 * i);
            }
        }
    }
    if (j == 0) blk[0] = s16;
#pragma unroll
    for (int k = 0; k < N / 8; ++k) {
        blk[1 + (N / 4) * j + 2 * k] = static_cast<uint16_t>(nib[k] & 0xFFFFu);
        blk[2 + (N / 4) * j + 2 * k] = static_cast<uint16_t>(nib[k] >> 16);
    }
}

// The workgroup's NG consecutive 66-byte blocks, built in LDS, out to global
// memory: dwords when all groups are live (the span starts on a 4-byte
// boundary: NG is a multiple of 2 and blocks are 4-byte aligned), else
// halfwords.
template <int NG>
__device__ __forceinline__ void q4_128_flush(const uint16_t* __restrict__ stage, uint8_t* __restrict__ blocks,
                                             size_t g0, size_t groups) {
    __syncthreads();
    const int n = static_cast<int>(min(static_cast<size_t>(NG), groups - g0));
    if (n == NG) {
        uint32_t* dst = reinterpret_cast<uint32_t*>(blocks + g0 * 66);
        const uint32_t* src = reinterpret_cast<const uint32_t*>(stage);
        for (int i = static_cast<int>(threadIdx.x); i < NG * 66 / 4; i += kRepackThreads) dst[i] = src[i];
    } else {
        uint16_t* dst = reinterpret_cast<uint16_t*>(blocks + g0 * 66);
        for (int i = static_cast<int>(threadIdx.x); i < n * 33; i += kRepackThreads) dst[i] = stage[i];
    }
}

// fp32 weights -> Q4_128 blocks (repack_q4_128.py:72-92): 16 lanes per
// group, two float4 loads per lane (consecutive lanes, consecutive bytes).
__global__ __launch_bounds__(kRepackThreads) void fp32_to_q4_128_kernel(const float4* __restrict__ w,
                                                                        uint8_t* __restrict__ blocks, size_t groups) {
    constexpr int kLanes = 16;
    constexpr int kGroups = kRepackThreads / kLanes;
    __shared__ __align__(16) uint16_t stage[kGroups * 33];
    const size_t g0 = static_cast<size_t>(blockIdx.x) * kGroups;
    const size_t grp = g0 + threadIdx.x / kLanes;  // uniform over the lanes of a group
    const int j = static_cast<int>(threadIdx.x % kLanes);
    if (grp < groups) {
        const float4 a = w[grp * 32 + 2 * j];
        const float4 b = w[grp * 32 + 2 * j + 1];
        const float v[8] = {a.x, a.y, a.z, a.w, b.x, b.y, b.z, b.w};
        q4_128_store<kLanes>(v, stage + (threadIdx.x / kLanes) * 33, j);
    }
    q4_128_flush<kGroups>(stage, blocks, g0, groups);
}

// asymmetric packed Q4 (gs 128) -> Q4_128 blocks (repack_q4_128.py:34-69):
// the group decoded in float32 as (q - f32(zero)) * f32(max(s, 1e-8)), zero
// = -b / max(s, 1e-8) in float64, then requantized.  4 lanes per group, one
// 16-byte load of 32 nibbles each: the float64 group terms are paid once per
// 4 lanes rather than once per 16 (the kernel is bound by its ~10 VALU
// operations per weight, not by HBM).
__global__ __launch_bounds__(kRepackThreads) void asym_to_q4_128_kernel(const uint4* __restrict__ packed,
                                                                        const float* __restrict__ scales,
                                                                        const float* __restrict__ biases,
                                                                        uint8_t* __restrict__ blocks,
                                                                        size_t groups) {
    constexpr int kLanes = 4;
    constexpr int kGroups = kRepackThreads / kLanes;
    __shared__ __align__(16) uint16_t stage[kGroups * 33];
    const size_t g0 = static_cast<size_t>(blockIdx.x) * kGroups;
    const size_t grp = g0 + threadIdx.x / kLanes;
    const int j = static_cast<int>(threadIdx.x % kLanes);
    if (grp < groups) {
        const uint4 q4 = packed[grp * 4 + j];
        const uint32_t q[4] = {q4.x, q4.y, q4.z, q4.w};
        const double sc = floor_scale(scales[grp]);
        const float zero32 = static_cast<float>(-static_cast<double>(biases[grp]) / sc);
        const float sc32 = static_cast<float>(sc);
        float v[32];
#pragma unroll
        for (int i = 0; i < 32; ++i) {
            const float d = static_cast<float>((q[i / 8] >> (4 * (i % 8))) & 0xFu) - zero32;
            v[i] = d * sc32;
        }
        q4_128_store<kLanes>(v, stage + (threadIdx.x / kLanes) * 33, j);
    }
    q4_128_flush<kGroups>(stage, blocks, g0, groups);
}

// Q4_128 blocks -> preq2-g128: the symmetric block (scale s, levels q with
// w = (q - 8) * s) is the asymmetric group (scale s, zero 8), so meta is
// fp16 s | fp16 8.0 and the 64 nibble bytes move into the row's band slot.
// One thread per (band, group); blocks are 2-byte aligned (66-byte stride).
__global__ __launch_bounds__(kRepackThreads) void q4_128_to_preq2_kernel(const uint8_t* __restrict__ blocks,
                                                                         uint32_t* __restrict__ meta,
                                                                         uint4* __restrict__ quant, int rows, int G,
                                                                         size_t pieces) {
    constexpr uint32_t kZero8 = 0x4800u;  // fp16 8.0
    const size_t t = static_cast<size_t>(blockIdx.x) * kRepackThreads + threadIdx.x;
    if (t >= pieces) return;
    const size_t u = t / 16;
    const int j = static_cast<int>(t % 16);
    const size_t band = u / G;
    const int g = static_cast<int>(u - band * G);
    const size_t row = band * 4 + j / 4;
    const int i = j % 4;
    uint4 v = make_uint4(0u, 0u, 0u, 0u);
    if (row < static_cast<size_t>(rows)) {
        const uint8_t* blk = blocks + (row * G + g) * 66;
        if (i == 0) meta[row * G + g] = static_cast<uint32_t>(*reinterpret_cast<const uint16_t*>(blk)) | (kZero8 << 16);
        const u32x4_a2 w = *reinterpret_cast<const u32x4_a2*>(blk + 2 + 16 * i);
        v = make_uint4(w.x, w.y, w.z, w.w);
    }
    quant[t] = v;
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
    const size_t slots = static_cast<size_t>((rows + 3) / 4) * G * 4;
    return launch("preq_to_preq2_kernel", preq_to_preq2_kernel, dim3(blocks_for(slots)), dim3(kRepackThreads), 0,
                  as_hip(stream), preq, reinterpret_cast<uint32_t*>(meta), reinterpret_cast<uint4*>(quant), rows, G,
                  slots);
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
    const size_t pieces = static_cast<size_t>((rows + 3) / 4) * G * 4 * (group_size / 32);
    const dim3 grid(blocks_for(pieces));
    auto* m = reinterpret_cast<uint32_t*>(meta);
    auto* q = reinterpret_cast<uint4*>(quant);
    const auto* p = reinterpret_cast<const uint4*>(packed);
    if (group_size == 32)
        return launch("asym_to_preq2_kernel", asym_to_preq2_kernel<32>, grid, dim3(kRepackThreads), 0,
                      as_hip(stream), p, scales, biases, m, q, rows, G, pieces);
    return launch("asym_to_preq2_kernel", asym_to_preq2_kernel<128>, grid, dim3(kRepackThreads), 0, as_hip(stream),
                  p, scales, biases, m, q, rows, G, pieces);
}

extern "C" asdsl_status asdsl_repack_fp32_to_q4_128(const float* weights, uint8_t* blocks, int rows, int cols,
                                                    int group_size, asdsl_stream_t stream) {
    ASDSL_CHECK_ARG(weights && blocks, "repack_fp32_to_q4_128: null pointer");
    ASDSL_CHECK_ARG(group_size == 128, "repack_fp32_to_q4_128: requires group_size=128");
    const asdsl_status cs = check_shape("repack_fp32_to_q4_128", rows, cols, 128);
    if (cs != ASDSL_OK) return cs;
    ASDSL_CHECK_ARG(aligned(weights, 16) && aligned(blocks, 4),
                    "repack_fp32_to_q4_128: weights must be 16-byte and blocks 4-byte aligned");
    const size_t groups = static_cast<size_t>(rows) * (cols / 128);
    return launch("fp32_to_q4_128_kernel", fp32_to_q4_128_kernel, dim3(blocks_for(groups * 16)),  // 16 lanes a group
                  dim3(kRepackThreads), 0, as_hip(stream), reinterpret_cast<const float4*>(weights), blocks, groups);
}

extern "C" asdsl_status asdsl_repack_asym_to_q4_128(const uint8_t* packed, const float* scales, const float* biases,
                                                    uint8_t* blocks, int rows, int cols, int group_size,
                                                    asdsl_stream_t stream) {
    ASDSL_CHECK_ARG(packed && scales && biases && blocks, "repack_asym_to_q4_128: null pointer");
    ASDSL_CHECK_ARG(group_size == 128, "repack_asym_to_q4_128: requires group_size=128");
    const asdsl_status cs = check_shape("repack_asym_to_q4_128", rows, cols, 128);
    if (cs != ASDSL_OK) return cs;
    ASDSL_CHECK_ARG(aligned(packed, 4) && aligned(scales, 4) && aligned(biases, 4) && aligned(blocks, 4),
                    "repack_asym_to_q4_128: packed, scales, biases and blocks must be 4-byte aligned");
    const size_t groups = static_cast<size_t>(rows) * (cols / 128);
    ASDSL_CHECK_ARG(aligned(packed, 16), "repack_asym_to_q4_128: packed must be 16-byte aligned");
    return launch("asym_to_q4_128_kernel", asym_to_q4_128_kernel, dim3(blocks_for(groups * 4)),  // 4 lanes a group
                  dim3(kRepackThreads), 0, as_hip(stream), reinterpret_cast<const uint4*>(packed), scales, biases,
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
    const size_t pieces = static_cast<size_t>((rows + 3) / 4) * G * 16;
    return launch("q4_128_to_preq2_kernel", q4_128_to_preq2_kernel, dim3(blocks_for(pieces)), dim3(kRepackThreads),
                  0, as_hip(stream), blocks, reinterpret_cast<uint32_t*>(meta), reinterpret_cast<uint4*>(quant), rows,
                  G, pieces);
}
