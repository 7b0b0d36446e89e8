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
#include <cstdlib>
#include <type_traits>

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
                                                                        const float* __restrict__ inv,
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
    // 8-element chunks per thread: K <= 4096 at 8 waves, <= 8192 at 16, and
    // 12 waves (K <= 8192) need two
    constexpr int NCHB = WAVES == 12 ? 2 : 1;
    for (int n0 = 0; n0 < NB; n0 += 4) {
        ActStage<GS, WAVES * kWave, NCHB, false> act[4];
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
        if (inv) {  // the norm-fed single-column GEMV's 1/rms, before the K-split sum
#pragma unroll
            for (int n = 0; n < NB; ++n)
                if (n < ncols) acc[n] *= inv[n];
        }
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

// ---------------------------------------------------------------- MFMA path
// The batch is a sum over groups of int8 matrix products, GS/32
// v_mfma_i32_16x16x32_i8 per (group, 16-row tile) for 16 columns at once,
// accumulated in one exact int32 tile (the 32-element K slices of a 128-group
// chain through the MFMA's accumulator), then one fp32 epilogue per group:
//   D[n][r] = sum_{k in g} xq[n][k] * q[r][k]      (exact int32)
//   Y[n][r] += D*(s_r*xs_n) - (z_r*s_r)*(X_n*xs_n)  (the reference's per-group
//                                                     term, X_n = sum_g xq[n])
// The MFMA's A operand is the activations (its rows = columns n), B the
// weights (its columns = rows r), so lane l ends with rows r0 + l%16 and
// columns 4*(l/16) + v, v = 0..3: one row's (s, z) per lane per group.  Any
// permutation of k inside a group applied to both operands leaves D alone,
// so the weight operand is the nibble split (lo: even elements, hi: odd) and
// the activation operand the split order (even elements, odd elements).
//
// Pass 1 quantizes the 16 columns once (A1 rule per GS-group; zero columns
// past ncols) into a slice-major image in a device buffer:
//   img[t][n][4] uint2 : split-order int8 of column n in 32-element slice t, per chunk
//   fac[g][n]    float2: (xs, X*xs), X = sum of group g's int8
// Pass 2: workgroup = W waves over all groups of a 16-row tile (wave w:
// groups [w*GPW, (w+1)*GPW), their activation operands held in registers);
// the W partial tiles are added in LDS in fixed order.  Quantizing inside
// pass 2 instead was measured slower: every workgroup re-reads all of X.
constexpr int kMfmaCols = 16;

static_assert(kMfmaCols == kImageCols, "one image layout");

template <int GS>
__global__ __launch_bounds__(256) void batch_quantize_kernel(const float* __restrict__ X, uint2* __restrict__ img,
                                                             float2* __restrict__ fac, int K, int ncols) {
    const int n = static_cast<int>(blockIdx.y);
    const int c = static_cast<int>(blockIdx.x) * 256 + static_cast<int>(threadIdx.x);
    const int nchunk = K >> 3;  // a multiple of 4: lanes past the end form whole groups
    const int cc = min(c, nchunk - 1);
    float v[8];
    if (n < ncols) {
        const float4* xp = reinterpret_cast<const float4*>(X + static_cast<size_t>(n) * K) + 2 * cc;
        const float4 a = xp[0], b = xp[1];
        v[0] = a.x; v[1] = a.y; v[2] = a.z; v[3] = a.w;
        v[4] = b.x; v[5] = b.y; v[6] = b.z; v[7] = b.w;
    } else {
#pragma unroll
        for (int i = 0; i < 8; ++i) v[i] = 0.0f;
    }
    image_store8<GS>(v, c, n, c < nchunk, img, fac);
}

typedef int v4i32 __attribute__((ext_vector_type(4)));

// LDS bytes of one band's GPW groups (GS/2 bytes each: 4 rows x GS/32
// 16-byte slices) in a wave's staging area, padded by 64 B so that the four
// bands of a tile fall on different LDS banks.
__host__ __device__ constexpr int mfma_band_bytes(int gs, int gpw) { return gpw * (gs * 2) + 64; }
// Per wave: the weight staging area (4 bands of one tile) and the wave's
// (xs, X*xs) pairs (GPW groups x 16 columns x 8 B); per workgroup: two
// buffers of the fixed-order K-slice sum.
__host__ __device__ constexpr int mfma_wave_bytes(int gs, int gpw) { return 4 * mfma_band_bytes(gs, gpw) + gpw * 128; }
__host__ __device__ constexpr size_t mfma_lds_bytes(int gs, int gpw, int waves) {
    return static_cast<size_t>(waves) * mfma_wave_bytes(gs, gpw) + 2 * static_cast<size_t>(waves) * 4 * kWave * 4;
}

// Workgroups loop over 16-row tiles (tile = blockIdx.x, += gridDim.x).  With
// PF each wave requests the next tile's weights and (s, z) pairs before it
// computes the current one, so HBM streams while the fp32 epilogue runs;
// without PF (one tile per workgroup) the second register set is not needed.
template <int GS, int GPW, int W, bool PF>
__global__ __launch_bounds__(W * kWave) void preq2_batch_mfma_kernel(const uint32_t* __restrict__ meta,
                                                                    const uint8_t* __restrict__ quant,
                                                                    const uint2* __restrict__ img,
                                                                    const float2* __restrict__ fac,
                                                                    float* __restrict__ Y, int M, int K, int ncols) {
    constexpr int UPS = GS / 32;                    // 32-element slices per group
    constexpr int kBand = mfma_band_bytes(GS, GPW);
    constexpr int kGroupBytes = GS * 2;             // one group of a band: 4 rows x UPS slices x 16 B
    constexpr int kUnits = GPW * 4 * UPS;           // 16-byte units per band
    constexpr int kLoads = (4 * kUnits) / kWave;    // dwordx4 loads per lane per tile
    static_assert((4 * kUnits) % kWave == 0, "a tile's four bands are whole wave loads");
    extern __shared__ __align__(16) uint32_t lds_words[];
    uint8_t* lds = reinterpret_cast<uint8_t*>(lds_words);
    const int lane = static_cast<int>(threadIdx.x) & (kWave - 1);
    const int wave = static_cast<int>(threadIdx.x) >> 6;
    const int r16 = lane & 15;
    const int q = lane >> 4;
    const int G = K / GS;  // == W * GPW (the plan guarantees it)
    const int g0 = wave * GPW;
    const int ntiles = (M + 15) >> 4;
    const int nbands = (M + 3) >> 2;
    uint8_t* stage = lds + static_cast<size_t>(wave) * mfma_wave_bytes(GS, GPW);
    uint8_t* wfac = stage + 4 * kBand;
    float* red = reinterpret_cast<float*>(lds + static_cast<size_t>(W) * mfma_wave_bytes(GS, GPW));  // [2][W][4][kWave]

    // Weights: a tile's four bands x GPW groups are contiguous runs of
    // GPW*GS*2 bytes in HBM (within a group, 16-byte unit r*UPS + t holds
    // slice t of the band's row r), read with whole 16-byte lanes.
    auto load_tile = [&](uint4 (&wv)[kLoads], uint32_t (&mt)[GPW], int tile) {
#pragma unroll
        for (int i = 0; i < kLoads; ++i) {
            const int e = i * kWave + lane;
            const int band = min(tile * 4 + e / kUnits, nbands - 1);  // past M: the last band, never stored
            wv[i] = load_stream16(
                reinterpret_cast<const uint4*>(quant + (static_cast<size_t>(band) * G + g0) * kGroupBytes) +
                e % kUnits);
        }
        const int row = min(tile * 16 + r16, M - 1);
        const uint32_t* mrow = meta + static_cast<size_t>(row) * G + g0;
        if constexpr (GPW % 4 == 0) {
            const uint4* mp = reinterpret_cast<const uint4*>(mrow);
#pragma unroll
            for (int j4 = 0; j4 < GPW / 4; ++j4) {
                const uint4 m4 = mp[j4];
                mt[4 * j4 + 0] = m4.x;
                mt[4 * j4 + 1] = m4.y;
                mt[4 * j4 + 2] = m4.z;
                mt[4 * j4 + 3] = m4.w;
            }
        } else {
#pragma unroll
            for (int j = 0; j < GPW; ++j) mt[j] = mrow[j];
        }
    };

    int tile = static_cast<int>(blockIdx.x);
    const int step = static_cast<int>(gridDim.x);
    // two register sets, used alternately, so that the prefetch is never
    // copied (a copy would wait for the prefetch to land)
    uint4 w0[kLoads], w1[PF ? kLoads : 1];
    uint32_t m0[GPW], m1[PF ? GPW : 1];

    // activation operands (column r16, chunk q of each slice of the wave's
    // groups) and the wave's (xs, X*xs) pairs (GPW*128 contiguous bytes, to LDS)
    long a[GPW][UPS];
#pragma unroll
    for (int j = 0; j < GPW; ++j)
#pragma unroll
        for (int t = 0; t < UPS; ++t) {
            const uint2 v = img[(static_cast<size_t>((g0 + j) * UPS + t) * kMfmaCols + r16) * 4 + q];
            a[j][t] = static_cast<long>(static_cast<uint64_t>(v.x) | (static_cast<uint64_t>(v.y) << 32));
        }
    constexpr int kFacLoads = (GPW * 8 + kWave - 1) / kWave;
    uint4 fv[kFacLoads];
    const uint4* fsrc = reinterpret_cast<const uint4*>(fac + static_cast<size_t>(g0) * kMfmaCols);
#pragma unroll
    for (int i = 0; i < kFacLoads; ++i) fv[i] = fsrc[min(i * kWave + lane, GPW * 8 - 1)];
    load_tile(w0, m0, tile);  // the grid never exceeds the tile count
#pragma unroll
    for (int i = 0; i < kFacLoads; ++i)
        if (i * kWave + lane < GPW * 8) reinterpret_cast<uint4*>(wfac)[i * kWave + lane] = fv[i];

    const v4i32 zero = {0, 0, 0, 0};
    const int rd = (r16 >> 2) * kBand + (r16 & 3) * (UPS * 16) + q * 4;  // row r16, chunk q of slice 0
    auto run_tile = [&](auto prefetch, uint4 (&wc)[kLoads], uint32_t (&mc)[GPW], auto& wn, auto& mn, int parity) {
        // stage this tile's weights (the wave reads back only what it wrote;
        // LDS operations of a wave complete in order), then request the next
        // tile's before computing
#pragma unroll
        for (int i = 0; i < kLoads; ++i) {
            const int e = i * kWave + lane;
            *reinterpret_cast<uint4*>(stage + (e / kUnits) * kBand + (e % kUnits) * 16) = wc[i];
        }
        // (s, z) decoded before the prefetch is issued (uses after it would
        // wait for it as well)
        float sf[GPW], zsf[GPW];
#pragma unroll
        for (int j = 0; j < GPW; ++j) {
            sf[j] = half_bits_to_float(mc[j]);
            zsf[j] = -(half_bits_to_float(mc[j] >> 16) * sf[j]);
        }
        __builtin_amdgcn_sched_barrier(0);
        // (a workgroup's last tile requests nothing: a wave ends only once its
        // loads have landed)
        if constexpr (decltype(prefetch)::value) load_tile(wn, mn, tile + step);
        __builtin_amdgcn_sched_barrier(0);

        float acc[4] = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
        for (int j = 0; j < GPW; ++j) {
            const float4 f0 = reinterpret_cast<const float4*>(wfac + j * 128 + q * 32)[0];
            const float4 f1 = reinterpret_cast<const float4*>(wfac + j * 128 + q * 32)[1];
            const float xs[4] = {f0.x, f0.z, f1.x, f1.z};
            const float xx[4] = {f0.y, f0.w, f1.y, f1.w};
            v4i32 d = zero;
#pragma unroll
            for (int t = 0; t < UPS; ++t) {
                const uint32_t w = *reinterpret_cast<const uint32_t*>(stage + rd + j * kGroupBytes + t * 16);
                const uint64_t b = static_cast<uint64_t>(w & 0x0F0F0F0Fu) |
                                   (static_cast<uint64_t>((w >> 4) & 0x0F0F0F0Fu) << 32);
                d = __builtin_amdgcn_mfma_i32_16x16x32_i8(a[j][t], static_cast<long>(b), d, 0, 0, 0);
            }
#pragma unroll
            for (int v = 0; v < 4; ++v) {
                acc[v] = fmaf(static_cast<float>(d[v]), sf[j] * xs[v], acc[v]);
                acc[v] = fmaf(zsf[j], xx[v], acc[v]);
            }
        }

        // add the W K-slices in fixed order; the two buffers alternate, so
        // one barrier per tile suffices
        float* rb = red + parity * (W * 4 * kWave);
#pragma unroll
        for (int v = 0; v < 4; ++v) rb[(wave * 4 + v) * kWave + lane] = acc[v];
        __syncthreads();
        for (int e = static_cast<int>(threadIdx.x); e < 4 * kWave; e += W * kWave) {
            float sum = rb[e];
#pragma unroll
            for (int k = 1; k < W; ++k) sum += rb[k * 4 * kWave + e];
            const int v = e / kWave;
            const int l = e & (kWave - 1);
            const int n = 4 * (l >> 4) + v;
            const int row = tile * 16 + (l & 15);
            if (n < ncols && row < M) Y[static_cast<size_t>(n) * M + row] = sum;
        }
    };
    const std::true_type pf_on;
    const std::false_type pf_off;
    if constexpr (PF) {
        // every path has a fixed number of requests in flight at each wait (a
        // conditional request would make every wait drain all of them)
        while (true) {  // uniform per workgroup
            if (tile + step >= ntiles) {
                run_tile(pf_off, w0, m0, w0, m0, 0);
                break;
            }
            run_tile(pf_on, w0, m0, w1, m1, 0);
            tile += step;
            if (tile + step >= ntiles) {
                run_tile(pf_off, w1, m1, w1, m1, 1);
                break;
            }
            run_tile(pf_on, w1, m1, w0, m0, 1);
            tile += step;
        }
    } else {
        int parity = 0;
        while (true) {  // uniform per workgroup
            run_tile(pf_off, w0, m0, w0, m0, parity);
            tile += step;
            if (tile >= ntiles) break;
            load_tile(w0, m0, tile);
            parity ^= 1;
        }
    }
}

struct MfmaPlan {
    int waves = 0, gpw = 0, grid = 0;
    bool ok = false, prefetch = false;
};

// Waves x groups-per-wave cover the K/GS groups exactly; the grid holds
// ASDSL_HIP_BATCH_WG_PER_CU workgroups per compute unit (default 1), capped
// at the tile count.
MfmaPlan plan_mfma(int M, int K, int gs, int cus) {
    MfmaPlan p;
    if (K % 128 != 0) return p;
    const int G = K / gs;
    static const int pairs32[][2] = {{8, 12}, {16, 16}, {8, 16}, {16, 12}, {8, 8}, {16, 8}, {8, 20}, {4, 16}, {4, 8}};
    static const int pairs128[][2] = {{8, 3}, {16, 4}, {8, 4}, {8, 5}, {4, 4}};
    auto pick = [&](const auto& pairs) {
        for (const auto& wg : pairs)
            if (wg[0] * wg[1] == G) return std::pair<int, int>(wg[0], wg[1]);
        return std::pair<int, int>(0, 0);
    };
    const auto wg = gs == 32 ? pick(pairs32) : pick(pairs128);
    p.waves = wg.first;
    p.gpw = wg.second;
    if (p.waves == 0) return p;
    static const int knob = env_knob("ASDSL_HIP_BATCH_WG_PER_CU");
    const int per_cu = knob > 0 ? knob : 1;
    const int tiles = (M + 15) / 16;
    p.grid = tiles < per_cu * cus ? tiles : per_cu * cus;
    p.prefetch = tiles > p.grid;
    p.ok = true;
    return p;
}

template <int GS, int GPW, int W>
asdsl_status launch_mfma_shape(const MfmaPlan& p, const uint32_t* m, const uint8_t* q, const uint2* img,
                               const float2* fac, float* Y, int M, int K, int ncols, hipStream_t s) {
    if constexpr (W < 16) {  // 16 waves: 128 registers, no room for the second register set
        if (p.prefetch)
            return launch("preq2_batch_mfma_kernel", preq2_batch_mfma_kernel<GS, GPW, W, true>, dim3(p.grid),
                          dim3(W * kWave), mfma_lds_bytes(GS, GPW, W), s, m, q, img, fac, Y, M, K, ncols);
    }
    return launch("preq2_batch_mfma_kernel", preq2_batch_mfma_kernel<GS, GPW, W, false>, dim3(p.grid),
                  dim3(W * kWave), mfma_lds_bytes(GS, GPW, W), s, m, q, img, fac, Y, M, K, ncols);
}

asdsl_status launch_mfma(const MfmaPlan& p, int gs, const uint32_t* m, const uint8_t* q, const uint2* img,
                         const float2* fac, float* Y, int M, int K, int ncols, hipStream_t s) {
#define ASDSL_MFMA_CASE(GS_, W_, GPW_)          \
    if (gs == GS_ && p.waves == W_ && p.gpw == GPW_) \
        return launch_mfma_shape<GS_, GPW_, W_>(p, m, q, img, fac, Y, M, K, ncols, s);
    ASDSL_MFMA_CASE(32, 8, 12)
    ASDSL_MFMA_CASE(32, 16, 16)
    ASDSL_MFMA_CASE(32, 8, 16)
    ASDSL_MFMA_CASE(32, 16, 12)
    ASDSL_MFMA_CASE(32, 8, 8)
    ASDSL_MFMA_CASE(32, 16, 8)
    ASDSL_MFMA_CASE(32, 8, 20)
    ASDSL_MFMA_CASE(32, 4, 16)
    ASDSL_MFMA_CASE(32, 4, 8)
    ASDSL_MFMA_CASE(128, 8, 3)
    ASDSL_MFMA_CASE(128, 16, 4)
    ASDSL_MFMA_CASE(128, 8, 4)
    ASDSL_MFMA_CASE(128, 8, 5)
    ASDSL_MFMA_CASE(128, 4, 4)
#undef ASDSL_MFMA_CASE
    set_error("gemv_preq2_fused_batch: no MFMA tiling for this shape");
    return ASDSL_ERR_UNSUPPORTED;
}

struct BatchPlan {
    int lks, nu, waves, grid, nb;
    bool exact;
    int cus;
};

// Tiling: the largest K split (KS <= 8) that divides the band exactly, i.e.
// the fewest units per lane, since every unit's nibbles stay in registers
// while all columns are dotted; then columns per launch capped so no
// instantiation spills and enough waves stay resident (16 waves: 128-VGPR
// budget, 8 columns at NU <= 4; 8 waves, NU = 3: 16 columns take 208 VGPRs,
// two waves per SIMD, 8 columns 128, four -- measured at 16 columns, gate_up
// 16384x3072 g128 36.6 us in two launches of 8 vs 41.4 in one of 16,
// lm_head 200064x3072 239 vs 383 us) and the column images stay within
// ~96 KB of LDS.
BatchPlan plan_batch(int M, int K, int gs, int cus) {
    const int upb = K / 8;
    const int nbands = (M + 3) / 4;
    BatchPlan p{0, 0, K > 4096 ? 16 : 8, 0, 16, false, cus};
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
    p.grid = tiles_of(p.lks);  // capped at the resident workgroups at launch
    if (p.waves == 8) p.nb = p.nu <= 2 ? 16 : 8;
    else p.nb = p.nu <= 4 ? 8 : 4;
    const size_t img = batch_image_bytes(K, gs);
    while (p.nb > 2 && static_cast<size_t>(p.nb) * img > 96 * 1024) p.nb >>= 1;
    static const int nb_knob = env_knob("ASDSL_HIP_BATCH_MAX_COLS");  // tuning: a lower cap
    while (nb_knob > 0 && p.nb > 2 && p.nb > nb_knob) p.nb >>= 1;
    return p;
}

// One workgroup per tile up to the workgroups that fit on the chip at once
// (VGPRs and LDS decide); past that each workgroup loops over tiles, so
// its column staging is paid once for several tiles.
template <typename Kern>
int resident_grid(Kern kern, const BatchPlan& p, int threads, size_t lds) {
    int per_cu = 0;
    if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, kern, threads, lds) != hipSuccess || per_cu < 1)
        per_cu = 1;
    static const int knob = env_knob("ASDSL_HIP_BATCH_WG_PER_CU");
    if (knob > 0 && knob < per_cu) per_cu = knob;
    const long long cap = static_cast<long long>(p.cus) * per_cu;
    return p.grid < cap ? p.grid : static_cast<int>(cap);
}

template <int GS, int WAVES, int NB>
asdsl_status launch_batch_nb(const BatchPlan& p, const uint32_t* m, const uint4* q, const float* X, const float* inv,
                             float* Y, int M, int K, int ncols, hipStream_t stream) {
    const size_t lds = static_cast<size_t>(NB) * batch_image_bytes(K, GS);
    const dim3 block(WAVES * kWave);
#define ASDSL_BATCH_NU(N)                                                                                        \
    case N: {                                                                                                    \
        auto* kern = preq2_gemv_batch_kernel<GS, N, WAVES, NB>;                                                 \
        return launch("preq2_gemv_batch_kernel", kern, dim3(resident_grid(kern, p, WAVES * kWave, lds)), block, \
                      lds, stream, m, q, X, inv, Y, M, K, ncols, p.lks);                                        \
    }
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
                                int M, int K, int ncols, hipStream_t stream, const float* inv = nullptr) {
    if (ncols <= 2) return launch_batch_nb<GS, WAVES, 2>(p, m, q, X, inv, Y, M, K, ncols, stream);
    if (ncols <= 4) return launch_batch_nb<GS, WAVES, 4>(p, m, q, X, inv, Y, M, K, ncols, stream);
    if (ncols <= 8) return launch_batch_nb<GS, WAVES, 8>(p, m, q, X, inv, Y, M, K, ncols, stream);
    return launch_batch_nb<GS, WAVES, 16>(p, m, q, X, inv, Y, M, K, ncols, stream);
}

// plan_batch's column count and grid on the single-column GEMV's launch
// shape (preq2_plan_shape): K split, units per lane and waves (8, 12 or 16).
// columns from which the batched GEMV takes the MFMA form (dot4 below)
constexpr int kBatchMfmaMinN = 5;

// ------------------------------------------------------- exact MFMA form
// Copies n <= PER * THREADS 16-byte units from global memory to LDS, thread
// tid taking units tid, tid + THREADS, ...  All of a thread's loads are
// requested before its first LDS write, so the copy costs one memory round
// trip; a strided copy loop waits for each load before requesting the next.
// Indexes past n are clamped to unit n - 1 (a repeated load and an identical
// write), which keeps the copy free of branches and of a loop, whose back
// edge would make the compiler wait for every earlier load at its head.
template <int THREADS, int PER>
__device__ __forceinline__ void copy_to_lds(uint4* __restrict__ dst, const uint4* __restrict__ src, int n, int tid) {
    uint4 v[PER];
#pragma unroll
    for (int i = 0; i < PER; ++i) v[i] = src[min(i * THREADS + tid, n - 1)];
#pragma unroll
    for (int i = 0; i < PER; ++i) dst[min(i * THREADS + tid, n - 1)] = v[i];
}

// The batched GEMV with the single-column GEMV's fp32 order (plan_preq2's
// shape: K split KS = 1 << lks, NU units per lane), on an activation image
// that carries the per-slice sums (image_store8 with `us`).  In the
// single-column kernel the lane at virtual position v of a band's wave ks
// accumulates, unit by unit in unit order, acc = fma(d, s*xs, acc);
// acc = fma(-(z*s), xu, acc), where d is the exact int32 dot of the unit's 32
// nibbles with 32 int8 activations; slot_sum then reduces the 16 lanes of a
// row in a fixed tree and the KS partial rows are added in ks order.  Here
// the int32 dots come from v_mfma_i32_16x16x32_i8 (16 rows x 16 columns per
// 32-element slice, exact in any order) and the float steps are repeated in
// the same order:
//   GS 32:  the 16 accumulators of a row are the quads qd = g mod 16 (lane
//           bits 2-5; in-row position qd & 3, DPP row qd >> 2).  Wave w of
//           a K-range takes qd in [4w, 4w + 4): in every block of 16 groups
//           its 4 consecutive groups, in block order.
//   GS 128: the accumulators are (g mod 4, slice t) (lane bits 4-5 and 0-1).
//           Wave w takes the groups with g mod 4 = w, in group order, all
//           four slices of each.
// The tree: each wave folds its four accumulators as slot_sum's in-row steps
// do (GS 32: row_ror 4 then row_ror 8, so position 0 ends with (x0 + x3) +
// (x2 + x1); GS 128: quad xor 1 then xor 2, (x0 + x1) + (x2 + x3)); the four
// waves' values then pair as xor 16 and xor 32 do, (R0 + R1) + (R2 + R3); the
// K-ranges add in order.  Workgroup = 4 * KS waves (wave 4 * ks + w) over
// 16-row tiles (tile = blockIdx.x, += gridDim.x): the waves' activation
// operands stay in registers and the columns' scales in LDS for every tile.
// A tile step: 4 bands x 256 contiguous bytes, one 16-byte unit per lane,
// staged in the wave's LDS area (bands 16 bytes apart against bank
// conflicts), from which lane (r16, q) reads dword q of its row's unit for
// each of the step's four MFMAs.  With PF each wave requests the next tile's
// weights and (s, z) pairs before it computes the current one (two register
// sets, used alternately).
template <int GS, int NU, int KS, bool PF>
__global__ __launch_bounds__(4 * KS * kWave) void preq2_batch_exact_mfma_kernel(
    const uint32_t* __restrict__ meta, const uint8_t* __restrict__ quant, const uint2* __restrict__ img,
    const float2* __restrict__ fac, const float* __restrict__ us, float* __restrict__ Y, int M, int K, int ncols) {
#pragma clang fp contract(off)
    constexpr int UPS = GS / 32;
    constexpr int kGroupBytes = GS * 2;            // a band's group: 4 rows x UPS 16-byte slices
    constexpr int kStepGroups = GS == 32 ? 4 : 1;  // groups of one wave step
    constexpr int kRangeGroups = GS == 32 ? 16 * NU : 4 * NU;
    extern __shared__ __align__(16) uint32_t lds_words[];
    const int G = K / GS;
    float2* sfac = reinterpret_cast<float2*>(lds_words);                                  // [G][16]
    float* sus = reinterpret_cast<float*>(sfac + static_cast<size_t>(G) * kMfmaCols);    // [K/32][16] (GS 128)
    float* red = sus + (GS == 128 ? static_cast<size_t>(K / 32) * kMfmaCols : 0);        // [2][KS][4][4][kWave]
    uint8_t* stage_all = reinterpret_cast<uint8_t*>(red + 2 * static_cast<size_t>(KS) * 16 * kWave);

    const int tid = static_cast<int>(threadIdx.x);
    const int lane = tid & (kWave - 1);
    const int wave = tid >> 6;
    const int ks = wave >> 2;
    const int w = wave & 3;
    const int r16 = lane & 15;
    const int q = lane >> 4;
    const int ntiles = (M + 15) >> 4;
    const int nbands = (M + 3) >> 2;

    auto first_group = [&](int st) {
        return GS == 32 ? ks * kRangeGroups + 16 * st + 4 * w : ks * kRangeGroups + 4 * st + w;
    };
    // a tile's weights (lane e: unit e % 16 of band e / 16's 256-byte run)
    // and (s, z) pairs for this wave's NU steps.  Rows past M read the last
    // row and are never stored.
    auto load_tile = [&](uint4 (&wq)[NU], uint32_t (&mt)[NU][kStepGroups], int tile) {
        const int lband = min(tile * 4 + (lane >> 4), nbands - 1);
        const int row = min(tile * 16 + r16, M - 1);
#pragma unroll
        for (int st = 0; st < NU; ++st)
            wq[st] = load_stream16(
                reinterpret_cast<const uint4*>(quant + (static_cast<size_t>(lband) * G + first_group(st)) * kGroupBytes) +
                (lane & 15));
#pragma unroll
        for (int st = 0; st < NU; ++st) {
            const uint32_t* mp = meta + static_cast<size_t>(row) * G + first_group(st);
            if constexpr (kStepGroups == 4) {
                const uint4 m4 = *reinterpret_cast<const uint4*>(mp);  // 4 consecutive groups: 16-byte aligned
                mt[st][0] = m4.x;
                mt[st][1 % kStepGroups] = m4.y;
                mt[st][2 % kStepGroups] = m4.z;
                mt[st][3 % kStepGroups] = m4.w;
            } else {
                mt[st][0] = mp[0];
            }
        }
    };

    // the wave's activation operands (column r16, chunk q of each slice) and,
    // in LDS, the columns' (xs, X*xs) and slice sums for every group
    long av[NU][4];
#pragma unroll
    for (int st = 0; st < NU; ++st)
#pragma unroll
        for (int k = 0; k < 4; ++k) {
            // MFMA k of the step: GS 32 group g0 + k; GS 128 slice k of group g0
            const int slice = GS == 32 ? first_group(st) + k : first_group(st) * UPS + k;
            const uint2 v = img[(static_cast<size_t>(slice) * kMfmaCols + r16) * 4 + q];
            av[st][k] = static_cast<long>(static_cast<uint64_t>(v.x) | (static_cast<uint64_t>(v.y) << 32));
        }
    int tile = static_cast<int>(blockIdx.x);
    const int step = static_cast<int>(gridDim.x);
    uint4 wq0[NU], wq1[PF ? NU : 1];
    constexpr int kBandStride = 256 + 16;
    constexpr int kStepBytes = 4 * kBandStride;
    uint8_t* stage = stage_all + static_cast<size_t>(wave) * NU * kStepBytes;
    uint32_t mt0[NU][kStepGroups], mt1[PF ? NU : 1][kStepGroups];
    // the scale tables first, all of a thread's loads in flight together:
    // the LDS writes then wait for these alone, not for the weights
    // (K <= 8192: at most 8192 / GS * 8 pair units and 1024 sum units)
    constexpr int kThreads = 4 * KS * kWave;
    copy_to_lds<kThreads, (8192 / GS * 8 + kThreads - 1) / kThreads>(
        reinterpret_cast<uint4*>(sfac), reinterpret_cast<const uint4*>(fac), G * kMfmaCols / 2, tid);
    if constexpr (GS == 128)
        copy_to_lds<kThreads, (1024 + kThreads - 1) / kThreads>(
            reinterpret_cast<uint4*>(sus), reinterpret_cast<const uint4*>(us), (K / 32) * kMfmaCols / 4, tid);
    load_tile(wq0, mt0, tile);  // the grid never exceeds the tile count
    __syncthreads();

    const v4i32 zero = {0, 0, 0, 0};
    auto run_tile = [&](auto prefetch, uint4 (&wq)[NU], uint32_t (&mt)[NU][kStepGroups], auto& wn, auto& mn,
                        int parity) {
        // stage this tile's weights (the wave reads back only what it wrote;
        // a wave's LDS operations complete in order)
#pragma unroll
        for (int st = 0; st < NU; ++st)
            *reinterpret_cast<uint4*>(stage + st * kStepBytes + (lane >> 4) * kBandStride + (lane & 15) * 16) = wq[st];
        float sf[NU][kStepGroups], zs[NU][kStepGroups];
#pragma unroll
        for (int st = 0; st < NU; ++st)
#pragma unroll
            for (int k = 0; k < kStepGroups; ++k) {
                sf[st][k] = half_bits_to_float(mt[st][k]);
                zs[st][k] = -(half_bits_to_float(mt[st][k] >> 16) * sf[st][k]);
            }
        __builtin_amdgcn_sched_barrier(0);
        if constexpr (decltype(prefetch)::value) load_tile(wn, mn, tile + step);
        __builtin_amdgcn_sched_barrier(0);
        float acc[4][4];  // [column 4q + v][accumulator j of this wave]
#pragma unroll
        for (int v = 0; v < 4; ++v)
#pragma unroll
            for (int j = 0; j < 4; ++j) acc[v][j] = 0.0f;
#pragma unroll
        for (int st = 0; st < NU; ++st) {
#pragma unroll
            for (int k = 0; k < 4; ++k) {
                // the 16-byte unit of MFMA k in a band's run: GS 32, group
                // k's row r16 & 3 (unit 4k + r); GS 128, slice k of row r
                // (unit 4r + k); its dword q holds elements 8q..8q+7 (low
                // nibble even), split as the activation operand is
                const int unit = GS == 32 ? 4 * k + (r16 & 3) : 4 * (r16 & 3) + k;
                const uint32_t wsel = *reinterpret_cast<const uint32_t*>(
                    stage + st * kStepBytes + (r16 >> 2) * kBandStride + unit * 16 + q * 4);
                const uint64_t b = static_cast<uint64_t>(wsel & 0x0F0F0F0Fu) |
                                   (static_cast<uint64_t>((wsel >> 4) & 0x0F0F0F0Fu) << 32);
                const v4i32 d = __builtin_amdgcn_mfma_i32_16x16x32_i8(av[st][k], static_cast<long>(b), zero, 0, 0, 0);
                const int g = GS == 32 ? first_group(st) + k : first_group(st);
                const int mk = GS == 32 ? k : 0;
                const float4 f0 = reinterpret_cast<const float4*>(sfac + static_cast<size_t>(g) * kMfmaCols + 4 * q)[0];
                const float4 f1 = reinterpret_cast<const float4*>(sfac + static_cast<size_t>(g) * kMfmaCols + 4 * q)[1];
                const float xs[4] = {f0.x, f0.z, f1.x, f1.z};
                float xu[4] = {f0.y, f0.w, f1.y, f1.w};
                if constexpr (GS == 128) {
                    const float4 u = reinterpret_cast<const float4*>(
                        sus + static_cast<size_t>(g * UPS + k) * kMfmaCols + 4 * q)[0];
                    xu[0] = u.x; xu[1] = u.y; xu[2] = u.z; xu[3] = u.w;
                }
                // accumulator: GS 32 in-row position g mod 4 = k; GS 128 slice k
#pragma unroll
                for (int v = 0; v < 4; ++v) {
                    acc[v][k] = fmaf(static_cast<float>(d[v]), sf[st][mk] * xs[v], acc[v][k]);
                    acc[v][k] = fmaf(zs[st][mk], xu[v], acc[v][k]);
                }
            }
        }
        // the wave's in-row fold, then the four waves and the K-ranges in LDS
        // (two buffers by tile parity: one barrier per tile suffices)
        float* rb = red + static_cast<size_t>(parity) * KS * 16 * kWave;
#pragma unroll
        for (int v = 0; v < 4; ++v) {
            const float r = GS == 32 ? (acc[v][0] + acc[v][3]) + (acc[v][2] + acc[v][1])
                                     : (acc[v][0] + acc[v][1]) + (acc[v][2] + acc[v][3]);
            rb[((ks * 4 + w) * 4 + v) * kWave + lane] = r;
        }
        __syncthreads();
        if (wave < 4) {  // wave w stores column 4q + w
            const int v = w;
            float sum = 0.0f;
#pragma unroll
            for (int k2 = 0; k2 < KS; ++k2) {
                const float* rr = rb + static_cast<size_t>(k2) * 16 * kWave;
                const float p = (rr[(0 * 4 + v) * kWave + lane] + rr[(1 * 4 + v) * kWave + lane]) +
                                (rr[(2 * 4 + v) * kWave + lane] + rr[(3 * 4 + v) * kWave + lane]);
                sum = k2 == 0 ? p : sum + p;
            }
            const int n = 4 * q + v;
            const int orow = tile * 16 + r16;
            if (n < ncols && orow < M) Y[static_cast<size_t>(n) * M + orow] = sum;
        }
    };
    const std::true_type pf_on;
    const std::false_type pf_off;
    if constexpr (PF) {
        while (true) {  // uniform per workgroup
            if (tile + step >= ntiles) {
                run_tile(pf_off, wq0, mt0, wq0, mt0, 0);
                break;
            }
            run_tile(pf_on, wq0, mt0, wq1, mt1, 0);
            tile += step;
            if (tile + step >= ntiles) {
                run_tile(pf_off, wq1, mt1, wq1, mt1, 1);
                break;
            }
            run_tile(pf_on, wq1, mt1, wq0, mt0, 1);
            tile += step;
        }
    } else {
        int parity = 0;
        while (true) {  // uniform per workgroup
            run_tile(pf_off, wq0, mt0, wq0, mt0, parity);
            tile += step;
            if (tile >= ntiles) break;
            load_tile(wq0, mt0, tile);
            parity ^= 1;
        }
    }
}

// The exact MFMA form for at most 8 columns, two 16-row tiles per step.
// With 8 columns half of each MFMA's 16 columns is padding, and the fp32
// steps run over all 64 lanes anyway.  Here the activation operands carry
// columns 0..7 twice (operand rows c and c + 8), one MFMA runs per tile of
// the pair, and lanes q < 2 take tile A's dots (columns 4q + v) while lanes
// q >= 2 take tile B's (columns 4(q - 2) + v): one pass of fp32 steps
// serves both tiles.  Every (row, column) accumulator still sees the
// single-column GEMV's steps in its order, so the results are those of the
// one-tile kernel bit for bit.  Tile pair p is tiles 2p and 2p + 1 (rows
// past M read the last row and are never stored); workgroups loop over pairs.
template <int GS, int NU, int KS>
__global__ __launch_bounds__(4 * KS * kWave) void preq2_batch_exact_mfma_pair_kernel(
    const uint32_t* __restrict__ meta, const uint8_t* __restrict__ quant, const uint2* __restrict__ img,
    const float2* __restrict__ fac, const float* __restrict__ us, float* __restrict__ Y, int M, int K, int ncols) {
#pragma clang fp contract(off)
    constexpr int UPS = GS / 32;
    constexpr int kGroupBytes = GS * 2;
    constexpr int kStepGroups = GS == 32 ? 4 : 1;
    constexpr int kRangeGroups = GS == 32 ? 16 * NU : 4 * NU;
    extern __shared__ __align__(16) uint32_t lds_words[];
    const int G = K / GS;
    float2* sfac = reinterpret_cast<float2*>(lds_words);                                  // [G][16]
    float* sus = reinterpret_cast<float*>(sfac + static_cast<size_t>(G) * kMfmaCols);    // [K/32][16] (GS 128)
    float* red = sus + (GS == 128 ? static_cast<size_t>(K / 32) * kMfmaCols : 0);        // [2][KS][4][4][kWave]
    uint8_t* stage_all = reinterpret_cast<uint8_t*>(red + 2 * static_cast<size_t>(KS) * 16 * kWave);

    const int tid = static_cast<int>(threadIdx.x);
    const int lane = tid & (kWave - 1);
    const int wave = tid >> 6;
    const int ks = wave >> 2;
    const int w = wave & 3;
    const int r16 = lane & 15;
    const int q = lane >> 4;
    const bool upper = q >= 2;  // this lane takes tile B of the pair
    const int qc = q & 1;       // its columns: 4 qc .. 4 qc + 3
    const int ntiles = (M + 15) >> 4;
    const int npairs = (ntiles + 1) >> 1;
    const int nbands = (M + 3) >> 2;

    auto first_group = [&](int st) {
        return GS == 32 ? ks * kRangeGroups + 16 * st + 4 * w : ks * kRangeGroups + 4 * st + w;
    };
    // a tile's weights, staged by the whole wave
    auto load_weights = [&](uint4 (&wq)[NU], int tile) {
        const int lband = min(tile * 4 + (lane >> 4), nbands - 1);
#pragma unroll
        for (int st = 0; st < NU; ++st)
            wq[st] = load_stream16(
                reinterpret_cast<const uint4*>(quant + (static_cast<size_t>(lband) * G + first_group(st)) * kGroupBytes) +
                (lane & 15));
    };
    // the (s, z) pairs of row r16 of this lane's own tile of the pair
    auto load_meta = [&](uint32_t (&mt)[NU][kStepGroups], int tile) {
        const int row = min(tile * 16 + r16, M - 1);
#pragma unroll
        for (int st = 0; st < NU; ++st) {
            const uint32_t* mp = meta + static_cast<size_t>(row) * G + first_group(st);
            if constexpr (kStepGroups == 4) {
                const uint4 m4 = *reinterpret_cast<const uint4*>(mp);
                mt[st][0] = m4.x;
                mt[st][1 % kStepGroups] = m4.y;
                mt[st][2 % kStepGroups] = m4.z;
                mt[st][3 % kStepGroups] = m4.w;
            } else {
                mt[st][0] = mp[0];
            }
        }
    };

    // activation operands: operand row r16 holds column r16 & 7
    long av[NU][4];
#pragma unroll
    for (int st = 0; st < NU; ++st)
#pragma unroll
        for (int k = 0; k < 4; ++k) {
            const int slice = GS == 32 ? first_group(st) + k : first_group(st) * UPS + k;
            const uint2 v = img[(static_cast<size_t>(slice) * kMfmaCols + (r16 & 7)) * 4 + q];
            av[st][k] = static_cast<long>(static_cast<uint64_t>(v.x) | (static_cast<uint64_t>(v.y) << 32));
        }
    int pair = static_cast<int>(blockIdx.x);
    const int step = static_cast<int>(gridDim.x);
    uint4 wa[NU], wb[NU];
    uint32_t mt[NU][kStepGroups];
    constexpr int kBandStride = 256 + 16;
    constexpr int kStepBytes = 4 * kBandStride;
    uint8_t* stage_a = stage_all + static_cast<size_t>(wave) * 2 * NU * kStepBytes;
    uint8_t* stage_b = stage_a + NU * kStepBytes;
    constexpr int kThreads = 4 * KS * kWave;
    copy_to_lds<kThreads, (8192 / GS * 8 + kThreads - 1) / kThreads>(
        reinterpret_cast<uint4*>(sfac), reinterpret_cast<const uint4*>(fac), G * kMfmaCols / 2, tid);
    if constexpr (GS == 128)
        copy_to_lds<kThreads, (1024 + kThreads - 1) / kThreads>(
            reinterpret_cast<uint4*>(sus), reinterpret_cast<const uint4*>(us), (K / 32) * kMfmaCols / 4, tid);
    load_weights(wa, 2 * pair);  // the grid never exceeds the pair count
    load_weights(wb, 2 * pair + 1);
    load_meta(mt, 2 * pair + (upper ? 1 : 0));
    __syncthreads();

    const v4i32 zero = {0, 0, 0, 0};
    int parity = 0;
    while (true) {  // uniform per workgroup
#pragma unroll
        for (int st = 0; st < NU; ++st) {
            const int off = st * kStepBytes + (lane >> 4) * kBandStride + (lane & 15) * 16;
            *reinterpret_cast<uint4*>(stage_a + off) = wa[st];
            *reinterpret_cast<uint4*>(stage_b + off) = wb[st];
        }
        float sf[NU][kStepGroups], zs[NU][kStepGroups];
#pragma unroll
        for (int st = 0; st < NU; ++st)
#pragma unroll
            for (int k = 0; k < kStepGroups; ++k) {
                sf[st][k] = half_bits_to_float(mt[st][k]);
                zs[st][k] = -(half_bits_to_float(mt[st][k] >> 16) * sf[st][k]);
            }
        float acc[4][4];  // [column 4 qc + v][accumulator j of this wave]
#pragma unroll
        for (int v = 0; v < 4; ++v)
#pragma unroll
            for (int j = 0; j < 4; ++j) acc[v][j] = 0.0f;
#pragma unroll
        for (int st = 0; st < NU; ++st) {
#pragma unroll
            for (int k = 0; k < 4; ++k) {
                const int unit = GS == 32 ? 4 * k + (r16 & 3) : 4 * (r16 & 3) + k;
                const int rd = st * kStepBytes + (r16 >> 2) * kBandStride + unit * 16 + q * 4;
                const uint32_t wsa = *reinterpret_cast<const uint32_t*>(stage_a + rd);
                const uint32_t wsb = *reinterpret_cast<const uint32_t*>(stage_b + rd);
                const uint64_t ba = static_cast<uint64_t>(wsa & 0x0F0F0F0Fu) |
                                    (static_cast<uint64_t>((wsa >> 4) & 0x0F0F0F0Fu) << 32);
                const uint64_t bb = static_cast<uint64_t>(wsb & 0x0F0F0F0Fu) |
                                    (static_cast<uint64_t>((wsb >> 4) & 0x0F0F0F0Fu) << 32);
                const v4i32 da = __builtin_amdgcn_mfma_i32_16x16x32_i8(av[st][k], static_cast<long>(ba), zero, 0, 0, 0);
                const v4i32 db = __builtin_amdgcn_mfma_i32_16x16x32_i8(av[st][k], static_cast<long>(bb), zero, 0, 0, 0);
                const int g = GS == 32 ? first_group(st) + k : first_group(st);
                const int mk = GS == 32 ? k : 0;
                const float4 f0 = reinterpret_cast<const float4*>(sfac + static_cast<size_t>(g) * kMfmaCols + 4 * qc)[0];
                const float4 f1 = reinterpret_cast<const float4*>(sfac + static_cast<size_t>(g) * kMfmaCols + 4 * qc)[1];
                const float xs[4] = {f0.x, f0.z, f1.x, f1.z};
                float xu[4] = {f0.y, f0.w, f1.y, f1.w};
                if constexpr (GS == 128) {
                    const float4 u = reinterpret_cast<const float4*>(
                        sus + static_cast<size_t>(g * UPS + k) * kMfmaCols + 4 * qc)[0];
                    xu[0] = u.x; xu[1] = u.y; xu[2] = u.z; xu[3] = u.w;
                }
#pragma unroll
                for (int v = 0; v < 4; ++v) {
                    const int d = upper ? db[v] : da[v];
                    acc[v][k] = fmaf(static_cast<float>(d), sf[st][mk] * xs[v], acc[v][k]);
                    acc[v][k] = fmaf(zs[st][mk], xu[v], acc[v][k]);
                }
            }
        }
        const int tile = 2 * pair + (upper ? 1 : 0);
        pair += step;
        const bool more = pair < npairs;  // uniform
        float* rb = red + static_cast<size_t>(parity) * KS * 16 * kWave;
#pragma unroll
        for (int v = 0; v < 4; ++v) {
            const float r = GS == 32 ? (acc[v][0] + acc[v][3]) + (acc[v][2] + acc[v][1])
                                     : (acc[v][0] + acc[v][1]) + (acc[v][2] + acc[v][3]);
            rb[((ks * 4 + w) * 4 + v) * kWave + lane] = r;
        }
        __syncthreads();
        if (wave < 4) {  // wave w stores column 4 qc + w of its lane's tile
            const int v = w;
            float sum = 0.0f;
#pragma unroll
            for (int k2 = 0; k2 < KS; ++k2) {
                const float* rr = rb + static_cast<size_t>(k2) * 16 * kWave;
                const float p = (rr[(0 * 4 + v) * kWave + lane] + rr[(1 * 4 + v) * kWave + lane]) +
                                (rr[(2 * 4 + v) * kWave + lane] + rr[(3 * 4 + v) * kWave + lane]);
                sum = k2 == 0 ? p : sum + p;
            }
            const int n = 4 * qc + v;
            const int orow = tile * 16 + r16;
            if (n < ncols && orow < M) Y[static_cast<size_t>(n) * M + orow] = sum;
        }
        if (!more) break;
        load_weights(wa, 2 * pair);
        load_weights(wb, 2 * pair + 1);
        load_meta(mt, 2 * pair + (upper ? 1 : 0));
        parity ^= 1;
    }
}

size_t exact_mfma_lds_bytes(int K, int gs, int ks, int nu, bool pair = false) {
    return static_cast<size_t>(K / gs) * kMfmaCols * sizeof(float2) +
           (gs == 128 ? static_cast<size_t>(K / 32) * kMfmaCols * sizeof(float) : 0) +
           2 * static_cast<size_t>(ks) * 4 * 4 * kWave * sizeof(float) +
           static_cast<size_t>(4 * ks) * nu * 4 * (256 + 16) * (pair ? 2 : 1);  // per wave: nu steps of 4 padded bands (per tile)
}

BatchPlan plan_batch_single(int M, int K, int gs, int cus) {
    BatchPlan p{0, 0, 8, 0, 16, false, cus};
    preq2_plan_shape(M, K, cus, &p.lks, &p.nu, &p.waves, &p.exact);
    // The single-column plan's 16-wave workgroups for K <= 4096 (one tile
    // per compute unit) keep its K split and units per lane, so 8 waves give
    // the same per-column bits here; the batched kernel stages every column
    // per workgroup and measured slower at 16 (4-token verify pass at ctx
    // 1024: 2334 against 1917 us).
    if (p.waves == 16 && K <= 4096) p.waves = 8;
    if (!p.exact || K > 8192) {
        p.exact = false;
        return p;
    }
    const int bpt = p.waves >> p.lks;
    p.grid = ((M + 3) / 4 + bpt - 1) / bpt;
    if (p.waves == 8) p.nb = p.nu <= 2 ? 16 : 8;
    else p.nb = p.nu <= 4 ? 8 : 4;
    const size_t img = batch_image_bytes(K, gs);
    while (p.nb > 2 && static_cast<size_t>(p.nb) * img > 96 * 1024) p.nb >>= 1;
    return p;
}

}  // namespace
}  // namespace asdsl

using namespace asdsl;

extern "C" asdsl_status asdsl_gemv_preq2_fused(const uint8_t* meta, const uint8_t* quant, const float* x, float* y,
                                               int out_features, int in_features, int group_size,
                                               asdsl_stream_t stream);

// allow_mfma = false keeps every column on the dot4 kernels, whose
// per-column arithmetic follows the single-column GEMV; the multi-token
// decode pass uses that form (see preq2_fused_batch in abi_util.hpp).
asdsl_status asdsl::preq2_fused_batch(const uint8_t* meta, const uint8_t* quant, const float* X, float* Y,
                                      int out_features, int in_features, int group_size, int n_cols,
                                      asdsl_stream_t stream, bool allow_mfma, void* work, size_t work_bytes) {
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
    const auto* m = reinterpret_cast<const uint32_t*>(meta);
    // At least ASDSL_HIP_BATCH_MFMA_MIN_N columns: 16 columns per pass.
    // Default where the MFMA path was measured to overtake the dot4 kernel
    // (graph-replayed over rotated weights, pre-pass included): N >= 5
    // (gate_up 16384x3072 g32: N = 4 12.6 vs 11.6 us, N = 5 12.2 vs 13.8;
    // down 3072x8192: N = 4 10.6 vs 10.3, N = 5 10.6 vs 12.6).
    static const int mfma_knob = env_knob("ASDSL_HIP_BATCH_MFMA_MIN_N");
    const int mfma_min = mfma_knob > 0 ? mfma_knob : kBatchMfmaMinN;
    const MfmaPlan mp = plan_mfma(M, K, group_size, cus);
    if (allow_mfma && n_cols >= mfma_min && mp.ok && reinterpret_cast<uintptr_t>(meta) % 16 == 0 &&
        reinterpret_cast<uintptr_t>(quant) % 4 == 0) {
        const size_t img_bytes = static_cast<size_t>(K / 32) * kMfmaCols * 32;
        void* ws = nullptr;
        const asdsl_status st0 = work_buffer(
            s, work, work_bytes, img_bytes + static_cast<size_t>(K / group_size) * kMfmaCols * sizeof(float2), &ws,
            "gemv_preq2_fused_batch");
        if (st0 != ASDSL_OK) return st0;
        auto* img = static_cast<uint2*>(ws);
        auto* fac = reinterpret_cast<float2*>(static_cast<uint8_t*>(ws) + img_bytes);
        for (int n0 = 0; n0 < n_cols; n0 += kMfmaCols) {
            const int nc = n_cols - n0 < kMfmaCols ? n_cols - n0 : kMfmaCols;
            const dim3 qgrid((K / 8 + 255) / 256, kMfmaCols);
            asdsl_status st = group_size == 32
                                  ? launch("batch_quantize_kernel", batch_quantize_kernel<32>, qgrid, dim3(256), 0, s,
                                           X + static_cast<size_t>(n0) * K, img, fac, K, nc)
                                  : launch("batch_quantize_kernel", batch_quantize_kernel<128>, qgrid, dim3(256), 0, s,
                                           X + static_cast<size_t>(n0) * K, img, fac, K, nc);
            if (st != ASDSL_OK) return st;
            st = launch_mfma(mp, group_size, m, quant, img, fac, Y + static_cast<size_t>(n0) * M, M, K, nc, s);
            if (st != ASDSL_OK) return st;
        }
        return ASDSL_OK;
    }
    // one column, or shapes outside the batched kernel's tiling: per-column GEMVs
    if (n_cols == 1 || !p.exact || K > 8192) {
        for (int n = 0; n < n_cols; ++n) {
            const asdsl_status st = asdsl_gemv_preq2_fused(meta, quant, X + static_cast<size_t>(n) * K,
                                                           Y + static_cast<size_t>(n) * M, M, K, group_size, stream);
            if (st != ASDSL_OK) return st;
        }
        return ASDSL_OK;
    }
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

asdsl_status asdsl::preq2_batch_exact(const uint8_t* meta, const uint8_t* quant, const float* X, const float* inv,
                                      float* Y, int out_features, int in_features, int group_size, int n_cols,
                                      asdsl_stream_t stream) {
    ASDSL_CHECK_ARG(meta && quant && X && Y, "gemv_preq2_batch_exact: null pointer");
    ASDSL_CHECK_ARG(group_size == 32 || group_size == 128, "gemv_preq2_batch_exact: group_size must be 32 or 128");
    ASDSL_CHECK_ARG(out_features > 0 && in_features > 0 && in_features % group_size == 0 && in_features / 32 <= 640,
                    "gemv_preq2_batch_exact: invalid dimensions");
    ASDSL_CHECK_ARG(n_cols >= 1 && n_cols <= 64, "gemv_preq2_batch_exact: n_cols must be in [1, 64]");
    ASDSL_CHECK_ARG(reinterpret_cast<uintptr_t>(X) % 16 == 0, "gemv_preq2_batch_exact: X must be 16-byte aligned");
    ASDSL_CU_COUNT(cus);
    const int M = out_features, K = in_features;
    const BatchPlan p = plan_batch_single(M, K, group_size, cus);
    if (!p.exact) {
        set_error("gemv_preq2_batch_exact: the single-column launch shape of %dx%d leaves masked units", M, K);
        return ASDSL_ERR_UNSUPPORTED;
    }
    const auto* m = reinterpret_cast<const uint32_t*>(meta);
    const auto* q = reinterpret_cast<const uint4*>(quant);
    hipStream_t s = as_hip(stream);
    for (int n0 = 0; n0 < n_cols; n0 += p.nb) {
        const int nc = n_cols - n0 < p.nb ? n_cols - n0 : p.nb;
        const float* Xc = X + static_cast<size_t>(n0) * K;
        float* Yc = Y + static_cast<size_t>(n0) * M;
        const float* ic = inv ? inv + n0 : nullptr;
        asdsl_status st;
        if (group_size == 32) {
            st = p.waves == 8    ? launch_batch_waves<32, 8>(p, m, q, Xc, Yc, M, K, nc, s, ic)
                 : p.waves == 12 ? launch_batch_waves<32, 12>(p, m, q, Xc, Yc, M, K, nc, s, ic)
                                 : launch_batch_waves<32, 16>(p, m, q, Xc, Yc, M, K, nc, s, ic);
        } else {
            st = p.waves == 8    ? launch_batch_waves<128, 8>(p, m, q, Xc, Yc, M, K, nc, s, ic)
                 : p.waves == 12 ? launch_batch_waves<128, 12>(p, m, q, Xc, Yc, M, K, nc, s, ic)
                                 : launch_batch_waves<128, 16>(p, m, q, Xc, Yc, M, K, nc, s, ic);
        }
        if (st != ASDSL_OK) return st;
    }
    return ASDSL_OK;
}

namespace asdsl {
namespace {

template <int GS, int NU, int KS>
asdsl_status launch_exact_mfma_ks(bool pf, dim3 grid, size_t lds, hipStream_t s, const uint32_t* m, const uint8_t* q,
                                  const uint2* img, const float2* fac, const float* us, float* Y, int M, int K,
                                  int ncols) {
    // K split 4 (16 waves, 128 registers): no room for the second register
    // set; the caller gives such launches one workgroup per tile
    if constexpr (KS < 4) {
        if (pf)
            return launch("preq2_batch_exact_mfma_kernel", preq2_batch_exact_mfma_kernel<GS, NU, KS, true>, grid,
                          dim3(4 * KS * kWave), lds, s, m, q, img, fac, us, Y, M, K, ncols);
    }
    return launch("preq2_batch_exact_mfma_kernel", preq2_batch_exact_mfma_kernel<GS, NU, KS, false>, grid,
                  dim3(4 * KS * kWave), lds, s, m, q, img, fac, us, Y, M, K, ncols);
}

template <int GS, int NU>
asdsl_status launch_exact_mfma_nu(int ks, bool pf, dim3 grid, size_t lds, hipStream_t s, const uint32_t* m,
                                  const uint8_t* q, const uint2* img, const float2* fac, const float* us, float* Y,
                                  int M, int K, int ncols) {
    switch (ks) {
        case 1: return launch_exact_mfma_ks<GS, NU, 1>(pf, grid, lds, s, m, q, img, fac, us, Y, M, K, ncols);
        case 2: return launch_exact_mfma_ks<GS, NU, 2>(pf, grid, lds, s, m, q, img, fac, us, Y, M, K, ncols);
        default:
            // K split 4 with K <= 8192 leaves at most 4 units per lane
            if constexpr (NU <= 4)
                return launch_exact_mfma_ks<GS, NU, 4>(pf, grid, lds, s, m, q, img, fac, us, Y, M, K, ncols);
            set_error("gemv_preq2_batch_exact_mfma: no kernel for K split 4 with %d units per lane", NU);
            return ASDSL_ERR_UNSUPPORTED;
    }
}

template <int GS, int NU>
asdsl_status launch_exact_mfma_pair(int ks, dim3 grid, size_t lds, hipStream_t s, const uint32_t* m,
                                   const uint8_t* q, const uint2* img, const float2* fac, const float* us, float* Y,
                                   int M, int K, int ncols) {
    if (ks == 1)
        return launch("preq2_batch_exact_mfma_pair_kernel", preq2_batch_exact_mfma_pair_kernel<GS, NU, 1>, grid,
                      dim3(4 * kWave), lds, s, m, q, img, fac, us, Y, M, K, ncols);
    return launch("preq2_batch_exact_mfma_pair_kernel", preq2_batch_exact_mfma_pair_kernel<GS, NU, 2>, grid,
                  dim3(8 * kWave), lds, s, m, q, img, fac, us, Y, M, K, ncols);
}

template <int GS>
asdsl_status launch_exact_mfma_pairs(int nu, int ks, dim3 grid, size_t lds, hipStream_t s, const uint32_t* m,
                                     const uint8_t* q, const uint2* img, const float2* fac, const float* us,
                                     float* Y, int M, int K, int ncols) {
    switch (nu) {
        case 1: return launch_exact_mfma_pair<GS, 1>(ks, grid, lds, s, m, q, img, fac, us, Y, M, K, ncols);
        case 2: return launch_exact_mfma_pair<GS, 2>(ks, grid, lds, s, m, q, img, fac, us, Y, M, K, ncols);
        case 3: return launch_exact_mfma_pair<GS, 3>(ks, grid, lds, s, m, q, img, fac, us, Y, M, K, ncols);
        case 4: return launch_exact_mfma_pair<GS, 4>(ks, grid, lds, s, m, q, img, fac, us, Y, M, K, ncols);
        case 5: return launch_exact_mfma_pair<GS, 5>(ks, grid, lds, s, m, q, img, fac, us, Y, M, K, ncols);
        default: return launch_exact_mfma_pair<GS, 6>(ks, grid, lds, s, m, q, img, fac, us, Y, M, K, ncols);
    }
}

template <int GS>
asdsl_status launch_exact_mfma(int nu, int ks, bool pf, dim3 grid, size_t lds, hipStream_t s, const uint32_t* m,
                               const uint8_t* q, const uint2* img, const float2* fac, const float* us, float* Y, int M,
                               int K, int ncols) {
    switch (nu) {
        case 1: return launch_exact_mfma_nu<GS, 1>(ks, pf, grid, lds, s, m, q, img, fac, us, Y, M, K, ncols);
        case 2: return launch_exact_mfma_nu<GS, 2>(ks, pf, grid, lds, s, m, q, img, fac, us, Y, M, K, ncols);
        case 3: return launch_exact_mfma_nu<GS, 3>(ks, pf, grid, lds, s, m, q, img, fac, us, Y, M, K, ncols);
        case 4: return launch_exact_mfma_nu<GS, 4>(ks, pf, grid, lds, s, m, q, img, fac, us, Y, M, K, ncols);
        case 5: return launch_exact_mfma_nu<GS, 5>(ks, pf, grid, lds, s, m, q, img, fac, us, Y, M, K, ncols);
        default: return launch_exact_mfma_nu<GS, 6>(ks, pf, grid, lds, s, m, q, img, fac, us, Y, M, K, ncols);
    }
}

}  // namespace
}  // namespace asdsl

bool asdsl::preq2_batch_exact_mfma_applies(int out_features, int in_features, int group_size, int n_cols) {
    if ((group_size != 32 && group_size != 128) || out_features <= 0 || in_features <= 0 ||
        in_features % group_size != 0 || in_features > 8192 || n_cols < 1 || n_cols > kMfmaCols)
        return false;
    const int cus = cu_count_current();
    if (cus < 0) return false;
    int lks = 0, nu = 0, waves = 0;
    bool exact = false;
    preq2_plan_shape(out_features, in_features, cus, &lks, &nu, &waves, &exact);
    return exact && lks <= 2 && nu >= 1 && nu <= (lks == 2 ? 4 : 6);
}

asdsl_status asdsl::preq2_batch_exact_mfma_image(const uint8_t* meta, const uint8_t* quant, const void* image,
                                                 float* Y, int out_features, int in_features, int group_size,
                                                 int n_cols, asdsl_stream_t stream) {
    ASDSL_CHECK_ARG(meta && quant && image && Y, "gemv_preq2_batch_exact_mfma: null pointer");
    ASDSL_CHECK_ARG(preq2_batch_exact_mfma_applies(out_features, in_features, group_size, n_cols),
                    "gemv_preq2_batch_exact_mfma: the form does not apply to this call");
    ASDSL_CHECK_ARG(reinterpret_cast<uintptr_t>(image) % 16 == 0 && reinterpret_cast<uintptr_t>(quant) % 4 == 0,
                    "gemv_preq2_batch_exact_mfma: image must be 16-byte and quant 4-byte aligned");
    ASDSL_CU_COUNT(cus);
    const int M = out_features, K = in_features;
    int lks = 0, nu = 0, waves = 0;
    bool exact = false;
    preq2_plan_shape(M, K, cus, &lks, &nu, &waves, &exact);
    const int ks = 1 << lks;
    const auto* base = static_cast<const uint8_t*>(image);
    const auto* img = reinterpret_cast<const uint2*>(base);
    const auto* fac = reinterpret_cast<const float2*>(base + image_fac_offset(K));
    const auto* us = reinterpret_cast<const float*>(base + image_us_offset(K));
    // workgroups per compute unit (ASDSL_HIP_EXACT_WG_PER_CU, default 2),
    // capped at the tile count; more tiles than workgroups: prefetch
    static const int knob = env_knob("ASDSL_HIP_EXACT_WG_PER_CU");
    const int per_cu = knob > 0 ? knob : 2;
    const int tiles = (M + 15) / 16;
    const auto* base_m = reinterpret_cast<const uint32_t*>(meta);
    // up to 8 columns: two tiles per step (ASDSL_HIP_EXACT_PAIR=0, read per
    // call, turns it off).  Not at K split 4, whose 16 waves have no room for
    // the second tile's registers, nor with fewer pairs than half the compute
    // units (o_proj 3072x3072, 96 pairs: 6.7 against 5.7 us at 8 columns;
    // qkv 5120x3072, 160 pairs: 8.0 against 9.0; gate_up 10.8 against 12.4;
    // lm_head 72.6 against 84.3)
    const char* pair_env = std::getenv("ASDSL_HIP_EXACT_PAIR");
    const int pairs = (tiles + 1) / 2;
    if (n_cols <= 8 && ks < 4 && 2 * pairs >= cus && !(pair_env && pair_env[0] == '0')) {
        const dim3 pgrid(pairs < per_cu * cus ? pairs : per_cu * cus);
        const size_t plds = exact_mfma_lds_bytes(K, group_size, ks, nu, true);
        hipStream_t ps = as_hip(stream);
        return group_size == 32
                   ? launch_exact_mfma_pairs<32>(nu, ks, pgrid, plds, ps, base_m, quant, img, fac, us, Y, M, K, n_cols)
                   : launch_exact_mfma_pairs<128>(nu, ks, pgrid, plds, ps, base_m, quant, img, fac, us, Y, M, K,
                                                  n_cols);
    }
    const int gridn = ks == 4 || tiles < per_cu * cus ? tiles : per_cu * cus;
    const bool pf = tiles > gridn;
    const dim3 grid(gridn);
    const size_t lds = exact_mfma_lds_bytes(K, group_size, ks, nu);
    const auto* m = reinterpret_cast<const uint32_t*>(meta);
    hipStream_t s = as_hip(stream);
    return group_size == 32 ? launch_exact_mfma<32>(nu, ks, pf, grid, lds, s, m, quant, img, fac, us, Y, M, K, n_cols)
                            : launch_exact_mfma<128>(nu, ks, pf, grid, lds, s, m, quant, img, fac, us, Y, M, K, n_cols);
}

extern "C" asdsl_status asdsl_gemv_preq2_fused_batch(const uint8_t* meta, const uint8_t* quant, const float* X,
                                                     float* Y, int out_features, int in_features, int group_size,
                                                     int n_cols, asdsl_stream_t stream) {
    return preq2_fused_batch(meta, quant, X, Y, out_features, in_features, group_size, n_cols, stream, true);
}

// The MFMA form's column image: per 32-group 16 columns x 32 int8 operands
// and a (scale, scaled sum) pair.
bool asdsl::preq2_batch_image_applies(const uint8_t* meta, const uint8_t* quant, int out_features, int in_features,
                                      int group_size, int n_cols, bool allow_mfma) {
    if (!allow_mfma || !meta || !quant || (group_size != 32 && group_size != 128) || out_features <= 0 ||
        in_features <= 0 || in_features % group_size != 0 || in_features / 32 > 640 || n_cols < 1 ||
        n_cols > kMfmaCols)
        return false;
    const int cus = cu_count_current();
    if (cus < 0) return false;
    // The image comes from the kernel before (no quantize pre-pass), so the
    // MFMA form pays from fewer columns than in the standalone batched GEMV:
    // 4, or 3 once K >= 4096 (the verify pass's own-order form measured 1713
    // against 1973 us per 4-token pass with the dot4 kernel instead).
    static const int mfma_knob = env_knob("ASDSL_HIP_BATCH_MFMA_MIN_N");
    const int mfma_min = mfma_knob > 0 ? mfma_knob : (in_features >= 4096 ? 3 : 4);
    return n_cols >= mfma_min && plan_mfma(out_features, in_features, group_size, cus).ok &&
           reinterpret_cast<uintptr_t>(meta) % 16 == 0 && reinterpret_cast<uintptr_t>(quant) % 4 == 0;
}

asdsl_status asdsl::preq2_batch_mfma_image(const uint8_t* meta, const uint8_t* quant, const void* image, float* Y,
                                           int out_features, int in_features, int group_size, int n_cols,
                                           asdsl_stream_t stream) {
    ASDSL_CHECK_ARG(image && Y, "gemv_preq2_batch_image: null pointer");
    ASDSL_CHECK_ARG(preq2_batch_image_applies(meta, quant, out_features, in_features, group_size, n_cols, true),
                    "gemv_preq2_batch_image: the MFMA form does not apply to this call");
    ASDSL_CU_COUNT(cus);
    const int M = out_features, K = in_features;
    const MfmaPlan mp = plan_mfma(M, K, group_size, cus);
    const size_t img_bytes = static_cast<size_t>(K / 32) * kMfmaCols * 32;
    const auto* img = static_cast<const uint2*>(image);
    const auto* fac = reinterpret_cast<const float2*>(static_cast<const uint8_t*>(image) + img_bytes);
    return launch_mfma(mp, group_size, reinterpret_cast<const uint32_t*>(meta), quant, img, fac, Y, M, K, n_cols,
                       as_hip(stream));
}

extern "C" size_t asdsl_gemv_preq2_fused_batch_work_bytes(int in_features) {
    if (in_features <= 0 || in_features % 32 != 0) return 0;
    return image_bytes(in_features);  // int8 image, group (scale, sum) pairs, slice sums
}

extern "C" asdsl_status asdsl_gemv_preq2_fused_batch_ws(const uint8_t* meta, const uint8_t* quant, const float* X,
                                                        float* Y, int out_features, int in_features, int group_size,
                                                        int n_cols, void* work, size_t work_bytes,
                                                        asdsl_stream_t stream) {
    ASDSL_CHECK_ARG(work != nullptr, "gemv_preq2_fused_batch_ws: null work buffer");
    ASDSL_CHECK_ARG(work_bytes >= asdsl_gemv_preq2_fused_batch_work_bytes(in_features),
                    "gemv_preq2_fused_batch_ws: work buffer of %zu bytes, "
                    "asdsl_gemv_preq2_fused_batch_work_bytes gives %zu", work_bytes,
                    asdsl_gemv_preq2_fused_batch_work_bytes(in_features));
    return preq2_fused_batch(meta, quant, X, Y, out_features, in_features, group_size, n_cols, stream, true, work,
                             work_bytes);
}
