// preq g32 Q4 GEMV for gfx950 (row-major 20-byte blocks).
//
// Reference: gemv_q4_32_preq_avx2 and the fused 4row/8row variants
//   (asdsl/kernels/native/gemv_q4_preq_restored.cpp:281-336,476-669),
//   block layout asdsl/quantization/repack_q4_32.py:1-7.
//
// Mapping.  A row is G consecutive 20-byte blocks.  A wave covers 64/LPR rows
// at a time with LPR lanes per row (LPR = 64, 32 or 16, the largest that
// divides G, so no lane idles); lane j of a row reads blocks j, j+LPR, ...,
// so the lanes of a row read one contiguous run of LPR*20 bytes per step.
// Each block is fetched as one dwordx4 (scale, zero, 12 nibble bytes) plus
// one dword (last 4 nibble bytes): 20-byte blocks are 4-byte aligned only.
// Row sums: butterfly over the LPR lanes.  Same per-unit math as preq2.
#include "abi_util.hpp"
#include "device_common.hpp"

namespace asdsl {

namespace {

constexpr int kThreads = 256;
constexpr int kWavesPerWg = kThreads / kWave;

typedef uint32_t u32x4_a4 __attribute__((ext_vector_type(4), aligned(4)));

template <int LPR, int UNROLL, int NCH, bool Q8>
__global__ __launch_bounds__(kThreads) void preq_gemv_kernel(const uint8_t* __restrict__ blocks,
                                                            const float* __restrict__ x,
                                                            const int8_t* __restrict__ xq8,
                                                            const float* __restrict__ xsc,
                                                            float* __restrict__ y, int M, int K) {
    extern __shared__ __align__(16) uint32_t lds[];
    constexpr int RPW = kWave / LPR;  // rows per wave step
    const int G = K >> 5;
    const XImage im = x_image(lds, K, 32);

    const int lane = static_cast<int>(threadIdx.x) & (kWave - 1);
    const int wave = static_cast<int>(threadIdx.x) >> 6;
    const int j = lane % LPR;
    const int rin = lane / LPR;
    const int ntiles = (M + RPW - 1) / RPW;

    int tile = static_cast<int>(blockIdx.x) * kWavesPerWg + wave;
    const int tile_step = static_cast<int>(gridDim.x) * kWavesPerWg;

    u32x4_a4 h[UNROLL];
    uint32_t t[UNROLL];
    // Unconditional loads at clamped, in-bounds indices; values of groups
    // >= G or rows >= M are never used.
    auto load_batch = [&](int tl, int k0) {
        const int row = min(tl * RPW + rin, M - 1);
        const uint8_t* rb = blocks + static_cast<size_t>(row) * G * 20;
#pragma unroll
        for (int u = 0; u < UNROLL; ++u) {
            const int g = min(j + (k0 + u) * LPR, G - 1);
            const uint8_t* b = rb + static_cast<size_t>(g) * 20;
            h[u] = __builtin_nontemporal_load(reinterpret_cast<const u32x4_a4*>(b));
            t[u] = __builtin_nontemporal_load(reinterpret_cast<const uint32_t*>(b + 16));
        }
    };
    ActStage<32, kThreads, NCH, Q8> act;
    act.load(x, xq8, xsc, K);  // activation loads first: they retire first
    load_batch(tile, 0);  // unconditional: indices are clamped
    act.process(K, im);
    __syncthreads();

    const int nk = (G + LPR - 1) / LPR;
    for (; tile < ntiles; tile += tile_step) {
        float acc = 0.0f;
        for (int k0 = 0; k0 < nk; k0 += UNROLL) {
            if (k0 != 0) load_batch(tile, k0);
#pragma unroll
            for (int u = 0; u < UNROLL; ++u) {
                const int g = j + (k0 + u) * LPR;
                if (g < G) {
                    const uint4 nib = make_uint4(h[u].y, h[u].z, h[u].w, t[u]);
                    const int d = unit_dot(nib, im.xq + g * 8);
                    const float s = half_bits_to_float(h[u].x);
                    const float z = half_bits_to_float(h[u].x >> 16);
                    acc = fmaf(static_cast<float>(d), s * im.scale[g], acc);
                    acc = fmaf(-(z * s), im.usum[g], acc);
                }
            }
        }
        const int next = tile + tile_step;
        if (next < ntiles) load_batch(next, 0);
        acc = group_sum<(LPR < 16 ? LPR : 16)>(acc);
        if (LPR >= 32) acc += swz_xor16(acc);
        if (LPR >= 64) acc += __shfl_xor(acc, 32, kWave);
        if (j == 0) {
            const int row = tile * RPW + rin;
            if (row < M) y[row] = acc;
        }
    }
}

template <int LPR>
asdsl_status launch_lpr(const uint8_t* blocks, const float* x, const int8_t* xq8, const float* xsc, float* y, int M,
                        int K, hipStream_t stream, int cus) {
    constexpr int RPW = kWave / LPR;
    const int ntiles = (M + RPW - 1) / RPW;
    const dim3 grid(stream_grid(ntiles, kWavesPerWg, 4, cus));
    const dim3 block(kThreads);
    const size_t lds = x_image_bytes(K, 32);
    if (xq8 != nullptr) {
        auto* k = K <= 8 * kThreads * 2   ? preq_gemv_kernel<LPR, 4, 2, true>
                  : K <= 8 * kThreads * 4 ? preq_gemv_kernel<LPR, 4, 4, true>
                                          : preq_gemv_kernel<LPR, 4, 10, true>;
        return launch("preq_gemv_kernel", k, grid, block, lds, stream, blocks, x, xq8, xsc, y, M, K);
    }
    auto* k = K <= 8 * kThreads * 2   ? preq_gemv_kernel<LPR, 4, 2, false>
              : K <= 8 * kThreads * 4 ? preq_gemv_kernel<LPR, 4, 4, false>
                                      : preq_gemv_kernel<LPR, 4, 10, false>;
    return launch("preq_gemv_kernel", k, grid, block, lds, stream, blocks, x, xq8, xsc, y, M, K);
}

asdsl_status launch_preq(const uint8_t* blocks, const float* x, const int8_t* xq8, const float* xsc, float* y,
                         int M, int K, hipStream_t stream, int cus) {
    const int G = K / 32;
    if (G % 64 == 0) return launch_lpr<64>(blocks, x, xq8, xsc, y, M, K, stream, cus);
    if (G % 32 == 0) return launch_lpr<32>(blocks, x, xq8, xsc, y, M, K, stream, cus);
    if (G % 16 == 0 || G < 32) return launch_lpr<16>(blocks, x, xq8, xsc, y, M, K, stream, cus);
    return launch_lpr<64>(blocks, x, xq8, xsc, y, M, K, stream, cus);
}

int check_preq_args(const void* blocks, const void* x, const void* y, int M, int K, int gs, const char* fn) {
    if (!blocks || !x || !y) {
        set_error("%s: null input pointer", fn);
        return 1;
    }
    if (gs != 32) {
        set_error("%s: group_size must be 32", fn);
        return 1;
    }
    if (M <= 0 || K <= 0) {
        set_error("%s: invalid dimensions", fn);
        return 1;
    }
    if (K % gs != 0) {
        set_error("%s: in_features must be divisible by group_size", fn);
        return 1;
    }
    if (K / gs > 640) {
        set_error("%s: n_groups exceeds buffer", fn);
        return 1;
    }
    return 0;
}

}  // namespace

}  // namespace asdsl

using namespace asdsl;

extern "C" asdsl_status asdsl_gemv_q4_32_preq(const uint8_t* blocks, const int8_t* x_q8, const float* x_scales,
                                              float* y, int out_features, int in_features, int group_size,
                                              asdsl_stream_t stream) {
    if (check_preq_args(blocks, x_q8, y, out_features, in_features, group_size, "gemv_q4_32_preq"))
        return ASDSL_ERR_INVALID_ARGUMENT;
    ASDSL_CHECK_ARG(x_scales != nullptr, "gemv_q4_32_preq: null input pointer");
    ASDSL_CU_COUNT(cus);
    return launch_preq(blocks, nullptr, x_q8, x_scales, y, out_features, in_features, as_hip(stream), cus);
}

extern "C" asdsl_status asdsl_gemv_q4_32_preq_fused(const uint8_t* blocks, const float* x, float* y,
                                                    int out_features, int in_features, int group_size,
                                                    asdsl_stream_t stream) {
    if (check_preq_args(blocks, x, y, out_features, in_features, group_size, "gemv_q4_32_preq_fused"))
        return ASDSL_ERR_INVALID_ARGUMENT;
    ASDSL_CU_COUNT(cus);
    return launch_preq(blocks, x, nullptr, nullptr, y, out_features, in_features, as_hip(stream), cus);
}
