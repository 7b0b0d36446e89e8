// preq2 Q4 GEMV for gfx950 (4-row band layout + sidecar fp16 scale/zero).
//
// Reference: gemv_preq2_fused_avx2 / gemv_preq2_avx2
//   (asdsl/kernels/native/gemv_preq2_avx2.cpp:196-337), layout
//   asdsl/quantization/repack_preq2.py:22-62.
//
// Mapping.  One wave owns one band (4 output rows) at a time.  The band's
// quant bytes are contiguous (K/8 units of 16 B), so lane l reads units
// l, l+64, l+128, ... : every load instruction moves 1 KiB of contiguous HBM.
// Because 64 is a multiple of 4*(GS/32), a lane always sees the same row slot
// (and, for g128, the same 32-element quarter of its group), so the 4 row sums
// fall out of a butterfly over the other lane bits.  The activation is
// quantized once per workgroup into LDS (split int8 order) together with its
// per-group scales and per-unit sums; the prologue's HBM/L2 reads are issued
// while the first band's weight loads are already in flight.
//
// Math per unit (32 elements), all in fp32 after an exact int32 dot:
//   acc += D*(s*xs) - (z*s)*(X*xs)
// which is the reference's per-group term (gemv_preq2_avx2.cpp:168-191) with
// D = sum q*xq, X = sum xq.  y is overwritten.
#include "abi_util.hpp"
#include "device_common.hpp"

namespace asdsl {

namespace {

constexpr int kThreads = 256;
constexpr int kWavesPerWg = kThreads / kWave;

// LDS image: xq (K/4 dwords) | scale (K/GS floats) | unit sums (K/32 floats)
inline size_t x_image_bytes(int K, int gs) {
    return static_cast<size_t>(K) + static_cast<size_t>(K / gs) * 4 + static_cast<size_t>(K / 32) * 4;
}

template <int GS>
__device__ __forceinline__ void stage_activation(const float* __restrict__ x, const int8_t* __restrict__ xq8,
                                                 const float* __restrict__ xsc, int K, uint32_t* s_xq,
                                                 float* s_xs, float* s_xsum) {
    const int nchunk = K >> 3;
    for (int base = 0; base < nchunk; base += kThreads) {  // uniform trip count
        const int c = base + static_cast<int>(threadIdx.x);
        const bool active = c < nchunk;
        if (xq8 != nullptr) {
            load_chunk_q8<GS>(xq8, xsc, c, active, s_xq, s_xs, s_xsum);
        } else {
            quantize_chunk_q8<GS>(x, c, active, s_xq, s_xs, s_xsum, nullptr, nullptr);
        }
    }
}

template <int GS, int UNROLL>
__global__ __launch_bounds__(kThreads) void preq2_gemv_kernel(const uint32_t* __restrict__ meta,
                                                             const uint4* __restrict__ quant,
                                                             const float* __restrict__ x,
                                                             const int8_t* __restrict__ xq8,
                                                             const float* __restrict__ xsc,
                                                             float* __restrict__ y, int M, int K) {
    extern __shared__ __align__(16) uint32_t lds[];
    constexpr int UPS = GS / 32;          // units per (row, group)
    constexpr int UPG4 = 4 * UPS;         // units per (band, group)
    const int G = K / GS;
    const int U = K >> 5;                 // units per row
    uint32_t* s_xq = lds;
    float* s_xs = reinterpret_cast<float*>(lds + (K >> 2));
    float* s_xsum = s_xs + G;

    const int lane = static_cast<int>(threadIdx.x) & (kWave - 1);
    const int wave = static_cast<int>(threadIdx.x) >> 6;
    const int nbands = (M + 3) >> 2;
    const int upb = U * 4;                // units per band
    const int part = lane % UPS;
    const int slot = (lane / UPS) & 3;

    int band = static_cast<int>(blockIdx.x) * kWavesPerWg + wave;
    const int band_step = static_cast<int>(gridDim.x) * kWavesPerWg;

    // Issue the first band's first loads before the activation prologue.
    uint4 w[UNROLL];
    uint32_t mt[UNROLL];
    auto load_batch = [&](int b, int k0) {
        const uint4* qb = quant + static_cast<size_t>(b) * upb;
        const int row = b * 4 + slot;
        const bool row_ok = row < M;
        const uint32_t* mrow = meta + static_cast<size_t>(row_ok ? row : 0) * G;
#pragma unroll
        for (int j = 0; j < UNROLL; ++j) {
            const int c = k0 + j * kWave + lane;
            if (c < upb) {
                w[j] = load_stream16(qb + c);
                mt[j] = row_ok ? mrow[c / UPG4] : 0u;
            } else {
                w[j] = make_uint4(0u, 0u, 0u, 0u);
                mt[j] = 0u;
            }
        }
    };
    if (band < nbands) load_batch(band, 0);

    stage_activation<GS>(x, xq8, xsc, K, s_xq, s_xs, s_xsum);
    __syncthreads();

    for (; band < nbands; band += band_step) {
        float acc = 0.0f;
        for (int k0 = 0; k0 < upb; k0 += kWave * UNROLL) {
            if (k0 != 0) load_batch(band, k0);
#pragma unroll
            for (int j = 0; j < UNROLL; ++j) {
                const int c = k0 + j * kWave + lane;
                if (c < upb) {
                    const int g = c / UPG4;
                    const int u = g * UPS + part;
                    const int d = unit_dot(w[j], s_xq + u * 8);
                    const float s = half_bits_to_float(mt[j]);
                    const float z = half_bits_to_float(mt[j] >> 16);
                    acc = fmaf(static_cast<float>(d), s * s_xs[g], acc);
                    acc = fmaf(-(z * s), s_xsum[u], acc);
                }
            }
        }
        // Sum the lanes that share this lane's row slot.
#pragma unroll
        for (int m = 1; m < kWave; m <<= 1) {
            if ((m & (3 * UPS)) == 0) acc += __shfl_xor(acc, m, kWave);
        }
        const int next = band + band_step;
        if (lane < UPG4 && part == 0) {
            const int row = band * 4 + slot;
            if (row < M) y[row] = acc;
        }
        if (next < nbands) load_batch(next, 0);
    }
}

// w[r*K + k] = (q - z) * s, one thread per unit.
template <int GS>
__global__ __launch_bounds__(kThreads) void preq2_dequant_kernel(const uint32_t* __restrict__ meta,
                                                                const uint4* __restrict__ quant,
                                                                float* __restrict__ out, int M, int K) {
    constexpr int UPS = GS / 32;
    const int U = K >> 5;
    const int G = K / GS;
    const long long total = static_cast<long long>(M) * U;
    for (long long t = static_cast<long long>(blockIdx.x) * kThreads + threadIdx.x; t < total;
         t += static_cast<long long>(gridDim.x) * kThreads) {
        const int r = static_cast<int>(t / U);
        const int u = static_cast<int>(t % U);
        const int g = u / UPS;
        const int part = u % UPS;
        const int band = r >> 2;
        const int slot = r & 3;
        const size_t unit = static_cast<size_t>(band) * (U * 4) + static_cast<size_t>(g) * (4 * UPS) + slot * UPS + part;
        const uint4 wq = quant[unit];
        const uint32_t m = meta[static_cast<size_t>(r) * G + g];
        const float s = half_bits_to_float(m);
        const float z = half_bits_to_float(m >> 16);
        const uint32_t wv[4] = {wq.x, wq.y, wq.z, wq.w};
        float* o = out + static_cast<size_t>(r) * K + static_cast<size_t>(u) * 32;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            float4 a, b;
            a.x = (static_cast<float>(wv[i] & 0xF) - z) * s;
            a.y = (static_cast<float>((wv[i] >> 4) & 0xF) - z) * s;
            a.z = (static_cast<float>((wv[i] >> 8) & 0xF) - z) * s;
            a.w = (static_cast<float>((wv[i] >> 12) & 0xF) - z) * s;
            b.x = (static_cast<float>((wv[i] >> 16) & 0xF) - z) * s;
            b.y = (static_cast<float>((wv[i] >> 20) & 0xF) - z) * s;
            b.z = (static_cast<float>((wv[i] >> 24) & 0xF) - z) * s;
            b.w = (static_cast<float>((wv[i] >> 28) & 0xF) - z) * s;
            reinterpret_cast<float4*>(o)[2 * i] = a;
            reinterpret_cast<float4*>(o)[2 * i + 1] = b;
        }
    }
}

// Standalone activation quantizer (natural int8 order out).
template <int GS>
__global__ __launch_bounds__(kThreads) void quantize_activation_kernel(const float* __restrict__ x,
                                                                      int8_t* __restrict__ xq,
                                                                      float* __restrict__ xs, int K) {
    // Scratch LDS image is not needed; reuse the chunk routine with
    // throw-away split/sum outputs in registers via small LDS arrays.
    __shared__ uint32_t s_split[2 * kThreads];
    __shared__ float s_scale[kThreads];
    __shared__ float s_sum[kThreads];
    const int nchunk = K >> 3;
    for (int base = static_cast<int>(blockIdx.x) * kThreads; base < nchunk; base += static_cast<int>(gridDim.x) * kThreads) {
        const int c = base + static_cast<int>(threadIdx.x);
        const bool active = c < nchunk;
        // Local image offsets: chunk index relative to `base` keeps LDS small;
        // groups never straddle `base` because kThreads*8 is a multiple of GS.
        quantize_chunk_q8<GS>(x + static_cast<size_t>(base) * 8, c - base, active, s_split, s_scale, s_sum,
                              xq + static_cast<size_t>(base) * 8, xs + base * 8 / GS);
    }
}

int check_preq2_args(const void* meta, const void* quant, const void* x, const void* y, int M, int K, int gs,
                     const char* fn) {
    if (!meta || !quant || !x || !y) {
        set_error("%s: null pointer", fn);
        return 1;
    }
    if (gs != 32 && gs != 128) {
        set_error("%s: group_size must be 32 (preq2) or 128 (preq2-g128)", fn);
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
    if (K / 32 > 640) {
        set_error("%s: n_groups exceeds buffer", fn);
        return 1;
    }
    return 0;
}

template <int GS>
asdsl_status launch_preq2(const uint8_t* meta, const uint8_t* quant, const float* x, const int8_t* xq8,
                          const float* xsc, float* y, int M, int K, hipStream_t stream, int cus) {
    const int nbands = (M + 3) / 4;
    const int grid = stream_grid(nbands, kWavesPerWg, 4, cus);
    const size_t lds = x_image_bytes(K, GS);
    const int upb = K / 8;
    if (upb <= kWave * 6) {
        preq2_gemv_kernel<GS, 6><<<grid, kThreads, lds, stream>>>(
            reinterpret_cast<const uint32_t*>(meta), reinterpret_cast<const uint4*>(quant), x, xq8, xsc, y, M, K);
    } else {
        preq2_gemv_kernel<GS, 8><<<grid, kThreads, lds, stream>>>(
            reinterpret_cast<const uint32_t*>(meta), reinterpret_cast<const uint4*>(quant), x, xq8, xsc, y, M, K);
    }
    return launch_status("preq2_gemv_kernel");
}

}  // namespace

}  // namespace asdsl

using namespace asdsl;

extern "C" asdsl_status asdsl_gemv_preq2_fused(const uint8_t* meta, const uint8_t* quant, const float* x, float* y,
                                               int out_features, int in_features, int group_size,
                                               asdsl_stream_t stream) {
    if (check_preq2_args(meta, quant, x, y, out_features, in_features, group_size, "gemv_preq2_fused"))
        return ASDSL_ERR_INVALID_ARGUMENT;
    ASDSL_CU_COUNT(cus);
    if (group_size == 32)
        return launch_preq2<32>(meta, quant, x, nullptr, nullptr, y, out_features, in_features, as_hip(stream), cus);
    return launch_preq2<128>(meta, quant, x, nullptr, nullptr, y, out_features, in_features, as_hip(stream), cus);
}

extern "C" asdsl_status asdsl_gemv_preq2(const uint8_t* meta, const uint8_t* quant, const int8_t* x_q8,
                                         const float* x_scales, float* y, int out_features, int in_features,
                                         int group_size, asdsl_stream_t stream) {
    if (check_preq2_args(meta, quant, x_q8, y, out_features, in_features, group_size, "gemv_preq2"))
        return ASDSL_ERR_INVALID_ARGUMENT;
    ASDSL_CHECK_ARG(x_scales != nullptr, "gemv_preq2: null pointer");
    ASDSL_CU_COUNT(cus);
    if (group_size == 32)
        return launch_preq2<32>(meta, quant, nullptr, x_q8, x_scales, y, out_features, in_features, as_hip(stream), cus);
    return launch_preq2<128>(meta, quant, nullptr, x_q8, x_scales, y, out_features, in_features, as_hip(stream), cus);
}

extern "C" asdsl_status asdsl_dequant_preq2(const uint8_t* meta, const uint8_t* quant, float* w, int out_features,
                                            int in_features, int group_size, asdsl_stream_t stream) {
    if (check_preq2_args(meta, quant, w, w, out_features, in_features, group_size, "dequant_preq2"))
        return ASDSL_ERR_INVALID_ARGUMENT;
    ASDSL_CU_COUNT(cus);
    const long long units = static_cast<long long>(out_features) * (in_features / 32);
    const int grid = stream_grid(units, kThreads, 16, cus);
    if (group_size == 32) {
        preq2_dequant_kernel<32><<<grid, kThreads, 0, as_hip(stream)>>>(
            reinterpret_cast<const uint32_t*>(meta), reinterpret_cast<const uint4*>(quant), w, out_features, in_features);
    } else {
        preq2_dequant_kernel<128><<<grid, kThreads, 0, as_hip(stream)>>>(
            reinterpret_cast<const uint32_t*>(meta), reinterpret_cast<const uint4*>(quant), w, out_features, in_features);
    }
    return launch_status("preq2_dequant_kernel");
}

extern "C" asdsl_status asdsl_quantize_activation(const float* x, int8_t* x_q8, float* x_scales, int in_features,
                                                  int group_size, asdsl_stream_t stream) {
    ASDSL_CHECK_ARG(x && x_q8 && x_scales, "quantize_activation: null pointer");
    ASDSL_CHECK_ARG(group_size == 32 || group_size == 64 || group_size == 128,
                    "quantize_activation: group_size must be 32, 64 or 128");
    ASDSL_CHECK_ARG(in_features > 0 && in_features % group_size == 0,
                    "quantize_activation: in_features must be a positive multiple of group_size");
    ASDSL_CU_COUNT(cus);
    const int nchunk = in_features / 8;
    const int grid = stream_grid(nchunk, kThreads, 1, cus);
    hipStream_t s = as_hip(stream);
    if (group_size == 32) quantize_activation_kernel<32><<<grid, kThreads, 0, s>>>(x, x_q8, x_scales, in_features);
    else if (group_size == 64) quantize_activation_kernel<64><<<grid, kThreads, 0, s>>>(x, x_q8, x_scales, in_features);
    else quantize_activation_kernel<128><<<grid, kThreads, 0, s>>>(x, x_q8, x_scales, in_features);
    return launch_status("quantize_activation_kernel");
}
