// preq2 Q4 GEMV for gfx950 (4-row band layout + sidecar fp16 scale/zero).
//
// Reference: gemv_preq2_fused_avx2 / gemv_preq2_avx2
//   (asdsl/kernels/native/gemv_preq2_avx2.cpp:196-337), layout
//   asdsl/quantization/repack_preq2.py:22-62.
//
// Mapping.  A band (4 output rows) is K/8 contiguous 16-byte units.  KS waves
// of a 4-wave workgroup share one band, wave ks taking the contiguous unit
// slice [ks*NU*64, (ks+1)*NU*64); lane l reads units slice+l, slice+l+64, ...
// so every load instruction moves 1 KiB of contiguous HBM and a lane issues
// all NU of its loads before using any.  64 is a multiple of 4*(GS/32), so a
// lane always sees the same row slot (and, for g128, the same 32-element
// quarter of its group); the 4 row sums fall out of a butterfly over the
// other lane bits (DPP + swizzle + one bpermute), and the KS slices are added
// in a fixed order through LDS, so results are deterministic.
//
// The activation is quantized once per workgroup into LDS (split int8 order,
// per-group scales, per-unit sums) while the first tile's weight loads are
// already in flight; the next tile's loads are issued before the current
// tile's reduction.
//
// Math per unit (32 elements), fp32 after an exact int32 dot:
//   acc += D*(s*xs) - (z*s)*(X*xs)
// the reference's per-group term (gemv_preq2_avx2.cpp:168-191) with
// D = sum q*xq, X = sum xq.  y is overwritten.
#include "abi_util.hpp"
#include "device_common.hpp"

namespace asdsl {

namespace {

constexpr int kThreads = 256;
constexpr int kWavesPerWg = kThreads / kWave;

template <int GS, int NU, int NCH, bool Q8>
__global__ __launch_bounds__(kThreads) void preq2_gemv_kernel(const uint32_t* __restrict__ meta,
                                                             const uint4* __restrict__ quant,
                                                             const float* __restrict__ x,
                                                             const int8_t* __restrict__ xq8,
                                                             const float* __restrict__ xsc,
                                                             float* __restrict__ y, int M, int K, int KS) {
    extern __shared__ __align__(16) uint32_t lds[];
    __shared__ float s_part[2][kWavesPerWg][4];
    constexpr int UPS = GS / 32;       // units per (row, group)
    constexpr int UPG4 = 4 * UPS;      // units per (band, group)
    constexpr int SB = UPS == 1 ? 0 : 2;
    const int G = K / GS;
    const XImage im = x_image(lds, K, GS);

    const int lane = static_cast<int>(threadIdx.x) & (kWave - 1);
    const int wave = static_cast<int>(threadIdx.x) >> 6;
    const int ks = wave % KS;
    const int bpt = kWavesPerWg / KS;  // bands per tile
    const int bl = wave / KS;
    const int nbands = (M + 3) >> 2;
    const int ntiles = (nbands + bpt - 1) / bpt;
    const int upb = K >> 3;            // units per band
    const int slice = (upb + KS - 1) / KS;
    const int c_begin = ks * slice;
    const int c_end = min(c_begin + slice, upb);
    const int part = lane % UPS;
    const int slot = (lane / UPS) & 3;
    const bool writer = lane < UPG4 && part == 0;

    uint4 w[NU];
    uint32_t mt[NU];
    // Loads are unconditional at clamped, in-bounds indices (so they issue
    // back to back); values past the slice or of rows >= M are never used.
    auto load_pass = [&](int band, int c0) {
        const int b = min(band, nbands - 1);
        const uint4* qb = quant + static_cast<size_t>(b) * upb;
        const int row = min(b * 4 + slot, M - 1);
        const uint32_t* mrow = meta + static_cast<size_t>(row) * G;
#pragma unroll
        for (int j = 0; j < NU; ++j) {
            const int c = min(c0 + j * kWave + lane, c_end - 1);
            w[j] = load_stream16(qb + c);
            mt[j] = mrow[c / UPG4];
        }
    };

    int tile = static_cast<int>(blockIdx.x);
    const int tile_step = static_cast<int>(gridDim.x);
    ActStage<GS, kThreads, NCH, Q8> act;
    act.load(x, xq8, xsc, K);  // activation loads first: they retire first
    load_pass(tile * bpt + bl, c_begin);  // unconditional: indices are clamped
    act.process(K, im);        // quantize while the weights are in flight
    __syncthreads();

    int parity = 0;
    for (; tile < ntiles; tile += tile_step, parity ^= 1) {  // uniform per workgroup
        const int band = tile * bpt + bl;
        float acc = 0.0f;
        for (int c0 = c_begin; c0 < c_end; c0 += NU * kWave) {
            if (c0 != c_begin) load_pass(band, c0);
#pragma unroll
            for (int j = 0; j < NU; ++j) {
                const int c = c0 + j * kWave + lane;
                if (c < c_end) {
                    const int g = c / UPG4;
                    const int u = g * UPS + part;
                    const int d = unit_dot(w[j], im.xq + u * 8);
                    const float s = half_bits_to_float(mt[j]);
                    const float z = half_bits_to_float(mt[j] >> 16);
                    acc = fmaf(static_cast<float>(d), s * im.scale[g], acc);
                    acc = fmaf(-(z * s), im.usum[u], acc);
                }
            }
        }
        const int next = tile + tile_step;
        if (next < ntiles) load_pass(next * bpt + bl, c_begin);
        acc = slot_sum<SB>(acc);
        const int row = band * 4 + slot;
        if (KS == 1) {
            if (writer && band < nbands && row < M) y[row] = acc;
        } else {
            if (writer) s_part[parity][wave][slot] = acc;
            __syncthreads();
            if (ks == 0 && writer && band < nbands && row < M) {
                float sum = s_part[parity][wave][slot];
                for (int k = 1; k < KS; ++k) sum += s_part[parity][wave + k][slot];
                y[row] = sum;
            }
        }
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

// Standalone activation quantizer (natural int8 order out); each workgroup
// quantizes a run of kThreads chunks.
template <int GS>
__global__ __launch_bounds__(kThreads) void quantize_activation_kernel(const float* __restrict__ x,
                                                                      int8_t* __restrict__ xq,
                                                                      float* __restrict__ xs, int K) {
    __shared__ __align__(16) uint32_t s_split[2 * kThreads];
    __shared__ float s_scale[kThreads];
    __shared__ float s_sum[kThreads];
    const XImage im{s_split, s_scale, s_sum};
    const int nchunk = K >> 3;
    for (int base = static_cast<int>(blockIdx.x) * kThreads; base < nchunk;
         base += static_cast<int>(gridDim.x) * kThreads) {  // uniform per workgroup
        const int c = base + static_cast<int>(threadIdx.x);
        const bool active = c < nchunk;
        float v[8];
        if (active) {
            const float4 a = reinterpret_cast<const float4*>(x)[2 * c];
            const float4 b = reinterpret_cast<const float4*>(x)[2 * c + 1];
            v[0] = a.x; v[1] = a.y; v[2] = a.z; v[3] = a.w;
            v[4] = b.x; v[5] = b.y; v[6] = b.z; v[7] = b.w;
        } else {
#pragma unroll
            for (int e = 0; e < 8; ++e) v[e] = 0.0f;
        }
        // chunk index relative to `base` keeps the LDS image small; groups
        // never straddle `base` because kThreads*8 is a multiple of GS.
        quantize_chunk<GS>(v, c - base, active, im, xq + static_cast<size_t>(base) * 8, xs + base * 8 / GS);
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

// Launch plan: the smallest K split KS in {1,2,4} that leaves each lane at
// most 4 units (loads) per band slice.  Measured on MI355X with rotated weight
// copies: K=3072 -> KS=2 (gate_up 16384x3072 8.3 us vs 8.7-9.0 us at KS=1,
// lm_head g128 52.7 us vs 54.1 us), K=8192 -> KS=4 (down 3072x8192 7.2 us vs
// 8.2 us).  Shapes with no exact split fall back to looped passes of 8 units.
struct Plan {
    int ks, nu;
};

Plan plan_preq2(int K) {
    const int upb = K / 8;
    static const int forced = env_knob("ASDSL_HIP_KSPLIT");
    Plan best{0, 0};
    for (int ks : {1, 2, 4}) {
        if (upb % (64 * ks) != 0) continue;
        if (forced > 0 && ks != forced) continue;
        const int nu = upb / (64 * ks);
        if (nu > 8) continue;
        best = Plan{ks, nu};
        if (nu <= 4) break;
    }
    if (best.ks == 0) best = Plan{1, 8};  // generic: looped passes of 8 units
    return best;
}

template <int GS, int NCH, bool Q8>
void launch_nu(Plan p, const uint8_t* meta, const uint8_t* quant, const float* x, const int8_t* xq8,
               const float* xsc, float* y, int M, int K, hipStream_t stream, int cus) {
    const int nbands = (M + 3) / 4;
    const int bpt = kWavesPerWg / p.ks;
    const int ntiles = (nbands + bpt - 1) / bpt;
    const int grid = stream_grid(ntiles, 1, 4, cus);
    const size_t lds = x_image_bytes(K, GS);
    const auto* m = reinterpret_cast<const uint32_t*>(meta);
    const auto* q = reinterpret_cast<const uint4*>(quant);
#define ASDSL_PREQ2_NU(N) \
    case N: preq2_gemv_kernel<GS, N, NCH, Q8><<<grid, kThreads, lds, stream>>>(m, q, x, xq8, xsc, y, M, K, p.ks); break;
    switch (p.nu) {
        ASDSL_PREQ2_NU(1)
        ASDSL_PREQ2_NU(2)
        ASDSL_PREQ2_NU(3)
        ASDSL_PREQ2_NU(4)
        ASDSL_PREQ2_NU(5)
        ASDSL_PREQ2_NU(6)
        ASDSL_PREQ2_NU(7)
        default: preq2_gemv_kernel<GS, 8, NCH, Q8><<<grid, kThreads, lds, stream>>>(m, q, x, xq8, xsc, y, M, K, p.ks);
    }
#undef ASDSL_PREQ2_NU
}

template <int GS>
asdsl_status launch_preq2(const uint8_t* meta, const uint8_t* quant, const float* x, const int8_t* xq8,
                          const float* xsc, float* y, int M, int K, hipStream_t stream, int cus) {
    const Plan p = plan_preq2(K);
    if (xq8 != nullptr) {
        if (K <= 8 * kThreads * 2) launch_nu<GS, 2, true>(p, meta, quant, x, xq8, xsc, y, M, K, stream, cus);
        else if (K <= 8 * kThreads * 4) launch_nu<GS, 4, true>(p, meta, quant, x, xq8, xsc, y, M, K, stream, cus);
        else launch_nu<GS, 10, true>(p, meta, quant, x, xq8, xsc, y, M, K, stream, cus);
    } else {
        if (K <= 8 * kThreads * 2) launch_nu<GS, 2, false>(p, meta, quant, x, xq8, xsc, y, M, K, stream, cus);
        else if (K <= 8 * kThreads * 4) launch_nu<GS, 4, false>(p, meta, quant, x, xq8, xsc, y, M, K, stream, cus);
        else launch_nu<GS, 10, false>(p, meta, quant, x, xq8, xsc, y, M, K, stream, cus);
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
