// Batched preq2 GEMV for speculative verification: Y[n][:] = preq2(W) x_n for
// N activation columns, each quantized to int8 independently with the A1 rule,
// so column n equals gemv_preq2_fused_avx2(x_n) of the reference
// (asdsl/kernels/native/gemv_preq2_avx2.cpp:301-319) up to fp32 summation
// order.  The reference has no batched preq2 kernel: its engine falls back to
// serial forward_token under preq2 (asdsl/kernels/native/unified_engine.cpp:1774-1789).
//
// Same band streaming as preq2_gemv_kernel (gemv_preq2.hip); each 16-byte
// weight unit is read from HBM once and dotted with all NB columns, whose int8
// images sit side by side in LDS.  Per unit and column: 8 v_dot4_i32_i8 and
// the fp32 epilogue acc_n += D*(s*xs_n) - (z*s)*(X_n*xs_n).  Column chunks of
// up to 16 (8 when K > 4096, LDS-bound) run as separate launches over the
// same weights.  Deterministic: no atomics, fixed-order K-split combine.
#include "abi_util.hpp"
#include "device_common.hpp"

namespace asdsl {
namespace {

// LDS bytes of one column's activation image, rounded up to 16 so every image
// (and its uint4-read int8 part) starts 16-byte aligned.
__host__ __device__ inline size_t batch_image_bytes(int K, int gs) { return (x_image_bytes(K, gs) + 15) & ~static_cast<size_t>(15); }

template <int GS, int NU, int WAVES, int NB>
__global__ __launch_bounds__(WAVES * kWave) void preq2_gemv_batch_kernel(const uint32_t* __restrict__ meta,
                                                                        const uint4* __restrict__ quant,
                                                                        const float* __restrict__ X,
                                                                        float* __restrict__ Y, int M, int K,
                                                                        int ncols, int lks) {
    extern __shared__ __align__(16) uint32_t lds[];
    __shared__ float s_part[2][WAVES][4][NB];
    constexpr int UPS = GS / 32;
    constexpr int UPG4 = 4 * UPS;
    constexpr int SB = UPS == 1 ? 0 : 2;
    const int G = K / GS;
    const int img_words = static_cast<int>(batch_image_bytes(K, GS) / 4);

    const int lane = static_cast<int>(threadIdx.x) & (kWave - 1);
    const int wave = static_cast<int>(threadIdx.x) >> 6;
    const int KS = 1 << lks;
    const int ks = wave & (KS - 1);
    const int bl = wave >> lks;
    const int bpt = WAVES >> lks;
    const int nbands = (M + 3) >> 2;
    const int ntiles = (nbands + bpt - 1) / bpt;
    const int upb = K >> 3;
    const int c0 = ks * (NU * kWave) + lane;  // the plan makes KS*NU*64 == K/8 exactly
    const int part = lane % UPS;
    const int slot = (lane / UPS) & 3;
    const bool writer = lane < UPG4 && part == 0;

    uint4 w[NU];
    uint32_t mt[NU];
    auto load_tile = [&](int tile) {
        const int band = min(tile * bpt + bl, nbands - 1);
        const uint4* qp = quant + static_cast<size_t>(band) * upb + c0;
        const int row = min(band * 4 + slot, M - 1);
        const uint32_t* mp = meta + static_cast<size_t>(row) * G + c0 / UPG4;
#pragma unroll
        for (int j = 0; j < NU; ++j) w[j] = load_stream16(qp + j * kWave);
#pragma unroll
        for (int j = 0; j < NU; ++j) mt[j] = mp[j * (kWave / UPG4)];
    };

    // Quantize the columns into LDS, four at a time in flight; the first
    // tile's weights are requested right after the first columns' loads.
    int tile = static_cast<int>(blockIdx.x);
    const int tile_step = static_cast<int>(gridDim.x);
    for (int n0 = 0; n0 < NB; n0 += 4) {
        ActStage<GS, WAVES * kWave, 1, false> act[4];
#pragma unroll
        for (int q = 0; q < 4; ++q)
            if (n0 + q < ncols) act[q].load(X + static_cast<size_t>(n0 + q) * K, nullptr, nullptr, K);
        if (n0 == 0) load_tile(tile);
#pragma unroll
        for (int q = 0; q < 4; ++q)
            if (n0 + q < ncols) act[q].process(K, x_image(lds + (n0 + q) * img_words, K, GS));
    }
    __syncthreads();

    int parity = 0;
    for (; tile < ntiles; tile += tile_step) {  // uniform per workgroup
        // Nibbles split once per unit (lo: even elements, hi: odd, the LDS
        // split order); then column by column, units inner, with a scheduling
        // barrier per column so the LDS reads of all columns are not hoisted
        // at once (that spilled at 16 columns).
        uint32_t lo[NU][4], hi[NU][4];
        float s_[NU], zs_[NU];
#pragma unroll
        for (int j = 0; j < NU; ++j) {
            const uint32_t wv[4] = {w[j].x, w[j].y, w[j].z, w[j].w};
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                lo[j][i] = wv[i] & 0x0F0F0F0Fu;
                hi[j][i] = (wv[i] >> 4) & 0x0F0F0F0Fu;
            }
            s_[j] = half_bits_to_float(mt[j]);
            zs_[j] = -(half_bits_to_float(mt[j] >> 16) * s_[j]);
        }
        float acc[NB];
#pragma unroll
        for (int n = 0; n < NB; ++n) {
            acc[n] = 0.0f;
            if (n < ncols) {
                const XImage im = x_image(lds + n * img_words, K, GS);
#pragma unroll
                for (int j = 0; j < NU; ++j) {
                    const int g = (c0 + j * kWave) / UPG4;
                    const int u = g * UPS + part;
                    const uint4 a = reinterpret_cast<const uint4*>(im.xq + u * 8)[0];
                    const uint4 b = reinterpret_cast<const uint4*>(im.xq + u * 8)[1];
                    int d = 0;
                    d = __builtin_amdgcn_sdot4(static_cast<int>(lo[j][0]), static_cast<int>(a.x), d, false);
                    d = __builtin_amdgcn_sdot4(static_cast<int>(hi[j][0]), static_cast<int>(a.y), d, false);
                    d = __builtin_amdgcn_sdot4(static_cast<int>(lo[j][1]), static_cast<int>(a.z), d, false);
                    d = __builtin_amdgcn_sdot4(static_cast<int>(hi[j][1]), static_cast<int>(a.w), d, false);
                    d = __builtin_amdgcn_sdot4(static_cast<int>(lo[j][2]), static_cast<int>(b.x), d, false);
                    d = __builtin_amdgcn_sdot4(static_cast<int>(hi[j][2]), static_cast<int>(b.y), d, false);
                    d = __builtin_amdgcn_sdot4(static_cast<int>(lo[j][3]), static_cast<int>(b.z), d, false);
                    d = __builtin_amdgcn_sdot4(static_cast<int>(hi[j][3]), static_cast<int>(b.w), d, false);
                    acc[n] = fmaf(static_cast<float>(d), s_[j] * im.scale[g], acc[n]);
                    acc[n] = fmaf(zs_[j], im.usum[u], acc[n]);
                }
            }
            __builtin_amdgcn_sched_barrier(0);
        }
        const int band = tile * bpt + bl;
#pragma unroll
        for (int n = 0; n < NB; ++n) acc[n] = slot_sum<SB>(acc[n]);
        if (tile + tile_step < ntiles) load_tile(tile + tile_step);
        const int row = band * 4 + slot;
        if (lks == 0) {
            if (writer && band < nbands && row < M) {
#pragma unroll
                for (int n = 0; n < NB; ++n)
                    if (n < ncols) Y[static_cast<size_t>(n) * M + row] = acc[n];
            }
        } else {
            if (writer) {
#pragma unroll
                for (int n = 0; n < NB; ++n) s_part[parity][wave][slot][n] = acc[n];
            }
            __syncthreads();
            if (ks == 0 && writer && band < nbands && row < M) {
#pragma unroll
                for (int n = 0; n < NB; ++n) {
                    if (n < ncols) {
                        float sum = s_part[parity][wave][slot][n];
                        for (int k = 1; k < KS; ++k) sum += s_part[parity][wave + k][slot][n];
                        Y[static_cast<size_t>(n) * M + row] = sum;
                    }
                }
            }
            parity ^= 1;
        }
    }
}

struct BatchPlan {
    int lks, nu, waves, grid, nb;
    bool exact;
};

// Tiling: the largest K split (KS <= 8) that divides the band exactly, i.e.
// the fewest units per lane, since every unit's nibbles stay in registers
// while all columns are dotted; then columns per launch capped so no
// instantiation spills (measured VGPRs: 8 waves, NU <= 4: 16 columns within
// 208 VGPRs; 16 waves: 128-VGPR budget, 8 columns at NU <= 4) and the column
// images stay within ~96 KB of LDS.
BatchPlan plan_batch(int M, int K, int gs, int cus) {
    const int upb = K / 8;
    const int nbands = (M + 3) / 4;
    BatchPlan p{0, 0, K > 4096 ? 16 : 8, 0, 16, false};
    auto tiles_of = [&](int l) {
        const int bpt = p.waves >> l;
        return (nbands + bpt - 1) / bpt;
    };
    int best = -1;
    for (int l = 0; l <= 3; ++l)
        if (upb % (kWave << l) == 0 && (p.waves >> l) >= 1) best = l;
    if (best < 0) {  // no exact split: the caller falls back to per-column GEMVs
        p.exact = false;
        return p;
    }
    p.lks = best;
    p.nu = upb / (kWave << p.lks);
    p.exact = p.nu <= 6;
    const int cap = cus * (32 / p.waves);
    const int tiles = tiles_of(p.lks);
    p.grid = tiles < cap ? tiles : cap;
    if (p.waves == 8) p.nb = p.nu <= 4 ? 16 : 8;
    else p.nb = p.nu <= 4 ? 8 : 4;
    const size_t img = batch_image_bytes(K, gs);
    while (p.nb > 2 && static_cast<size_t>(p.nb) * img > 96 * 1024) p.nb >>= 1;
    return p;
}

template <int GS, int WAVES, int NB>
asdsl_status launch_batch_nb(const BatchPlan& p, const uint32_t* m, const uint4* q, const float* X, float* Y, int M,
                             int K, int ncols, hipStream_t stream) {
    const size_t lds = static_cast<size_t>(NB) * batch_image_bytes(K, GS);
    const dim3 block(WAVES * kWave);
#define ASDSL_BATCH_NU(N)                                                                                  \
    case N:                                                                                                \
        return launch("preq2_gemv_batch_kernel", preq2_gemv_batch_kernel<GS, N, WAVES, NB>, dim3(p.grid),  \
                      block, lds, stream, m, q, X, Y, M, K, ncols, p.lks);
    switch (p.nu) {
        ASDSL_BATCH_NU(1)
        ASDSL_BATCH_NU(2)
        ASDSL_BATCH_NU(3)
        ASDSL_BATCH_NU(4)
        ASDSL_BATCH_NU(5)
        default: ASDSL_BATCH_NU(6)
    }
#undef ASDSL_BATCH_NU
}

template <int GS, int WAVES>
asdsl_status launch_batch_waves(const BatchPlan& p, const uint32_t* m, const uint4* q, const float* X, float* Y,
                                int M, int K, int ncols, hipStream_t stream) {
    if (ncols <= 2) return launch_batch_nb<GS, WAVES, 2>(p, m, q, X, Y, M, K, ncols, stream);
    if (ncols <= 4) return launch_batch_nb<GS, WAVES, 4>(p, m, q, X, Y, M, K, ncols, stream);
    if (ncols <= 8) return launch_batch_nb<GS, WAVES, 8>(p, m, q, X, Y, M, K, ncols, stream);
    return launch_batch_nb<GS, WAVES, 16>(p, m, q, X, Y, M, K, ncols, stream);
}

}  // namespace
}  // namespace asdsl

using namespace asdsl;

extern "C" asdsl_status asdsl_gemv_preq2_fused(const uint8_t* meta, const uint8_t* quant, const float* x, float* y,
                                               int out_features, int in_features, int group_size,
                                               asdsl_stream_t stream);

extern "C" asdsl_status asdsl_gemv_preq2_fused_batch(const uint8_t* meta, const uint8_t* quant, const float* X,
                                                     float* Y, int out_features, int in_features, int group_size,
                                                     int n_cols, asdsl_stream_t stream) {
    ASDSL_CHECK_ARG(meta && quant && X && Y, "gemv_preq2_fused_batch: null pointer");
    ASDSL_CHECK_ARG(group_size == 32 || group_size == 128,
                    "gemv_preq2_fused_batch: group_size must be 32 (preq2) or 128 (preq2-g128)");
    ASDSL_CHECK_ARG(out_features > 0 && in_features > 0, "gemv_preq2_fused_batch: invalid dimensions");
    ASDSL_CHECK_ARG(in_features % group_size == 0,
                    "gemv_preq2_fused_batch: in_features must be divisible by group_size");
    ASDSL_CHECK_ARG(in_features / 32 <= 640, "gemv_preq2_fused_batch: n_groups exceeds buffer");
    ASDSL_CHECK_ARG(n_cols >= 1 && n_cols <= 64, "gemv_preq2_fused_batch: n_cols must be in [1, 64]");
    ASDSL_CHECK_ARG(reinterpret_cast<uintptr_t>(X) % 16 == 0, "gemv_preq2_fused_batch: X must be 16-byte aligned");
    ASDSL_CU_COUNT(cus);
    hipStream_t s = as_hip(stream);
    const BatchPlan p = plan_batch(out_features, in_features, group_size, cus);
    const int M = out_features, K = in_features;
    // one column, or shapes outside the batched kernel's tiling: per-column GEMVs
    if (n_cols == 1 || !p.exact || K > 8192) {
        for (int n = 0; n < n_cols; ++n) {
            const asdsl_status st = asdsl_gemv_preq2_fused(meta, quant, X + static_cast<size_t>(n) * K,
                                                           Y + static_cast<size_t>(n) * M, M, K, group_size, stream);
            if (st != ASDSL_OK) return st;
        }
        return ASDSL_OK;
    }
    const auto* m = reinterpret_cast<const uint32_t*>(meta);
    const auto* q = reinterpret_cast<const uint4*>(quant);
    for (int n0 = 0; n0 < n_cols; n0 += p.nb) {
        const int nc = n_cols - n0 < p.nb ? n_cols - n0 : p.nb;
        const float* Xc = X + static_cast<size_t>(n0) * K;
        float* Yc = Y + static_cast<size_t>(n0) * M;
        asdsl_status st;
        if (group_size == 32) {
            st = p.waves == 8 ? launch_batch_waves<32, 8>(p, m, q, Xc, Yc, M, K, nc, s)
                              : launch_batch_waves<32, 16>(p, m, q, Xc, Yc, M, K, nc, s);
        } else {
            st = p.waves == 8 ? launch_batch_waves<128, 8>(p, m, q, Xc, Yc, M, K, nc, s)
                              : launch_batch_waves<128, 16>(p, m, q, Xc, Yc, M, K, nc, s);
        }
        if (st != ASDSL_OK) return st;
    }
    return ASDSL_OK;
}
