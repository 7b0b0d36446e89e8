// Row-major block-quantized Q4 GEMV for gfx950, shared by four layouts:
//
//   preq    20-byte block per (row, 32-group): fp16 s | fp16 z | 16 B nibbles
//           (asdsl/quantization/repack_q4_32.py:1-7); activation groups of 32.
//   Q4_128  66-byte block per (row, 128-group): fp16 s | 64 B nibbles, zero 8
//           (asdsl/quantization/repack_q4_128.py:1-6); activation groups of 128.
//   packed  K/2 nibble bytes per row, fp32 scale per (row, group) in a side
//           array, zero 8 (gemv_q4_q8_avx2, asdsl/kernels/native/gemv_q4_avx2.cpp:131-253);
//           activation groups of group_size (32, 64 or 128).
//   Q4_K    144-byte superblock per (row, 256): fp16 d | fp16 dmin | 12 B of
//           6-bit scales (0-7) and mins (8-15), LSB-first | 8 x 16 B nibbles
//           (gemv_q4km_q8_avx2, gemv_q4_avx2.cpp:110-120,283-420); activation
//           groups of 32 under the round-half-away rule.
//
// In all, a row is a sequence of 16-byte "units" (32 nibbles = 32 consecutive
// K elements), unit t covering K elements [32t, 32t+32): preq and packed have
// one unit per block, Q4_128 four, Q4_K eight.  Lane j of the LPR lanes serving a row owns units
// j, j+LPR, ..., j+(NU-1)*LPR, so the lanes of a row read LPR consecutive units
// (LPR*20 contiguous bytes for preq, 4-block runs with 2-byte header gaps for
// Q4_128) and a lane's K positions are the same for every row: its activation
// units are read from LDS into registers once per workgroup.  A 66-byte block
// is 2-byte aligned only; gfx950 global loads are unaligned-capable, so a unit
// is one dwordx4 either way.
//
// Math per unit, fp32 after an exact int32 dot (D = sum q*xq, X = sum xq):
//   acc += D*(s*xs) - (z*s)*(X*xs)
// with z the block's zero-point (preq) or 8 (Q4_128, packed): the reference's
// per-group terms (gemv_q4_preq_restored.cpp:318-336; gemv_q4_128.cpp:174-217;
// gemv_q4_avx2.cpp:225-248) split per 32-element unit; for Q4_K
//   acc += (d*sc*D - dmin*m*X) * xs          (gemv_q4_avx2.cpp:316)
// y is overwritten.
//
// Launch: workgroups of WAVES waves, each wave serving 64/LPR rows at a time;
// LPR in {16, 32, 64} is the smallest with NU <= 6 units per lane, doubled
// while fewer than CUs/2 workgroups would run.  Rows of more than 6*64 units
// (K > 12288) are walked in passes of 4 units per lane.
#pragma once

#include <type_traits>

#include "abi_util.hpp"
#include "device_common.hpp"

namespace asdsl {

enum class RowLayout { kPreq, kQ4_128, kPacked, kQ4K, kQ4S256 };

// kBlockBytes: bytes per block; kUnitsPerBlock: 16-byte units per block;
// kDataOffset: offset of the first unit in a block.
template <RowLayout L>
struct RowFmt;

template <>
struct RowFmt<RowLayout::kPreq> {
    static constexpr int kBlockBytes = 20, kUnitsPerBlock = 1, kDataOffset = 4;
};

template <>
struct RowFmt<RowLayout::kQ4_128> {
    static constexpr int kBlockBytes = 66, kUnitsPerBlock = 4, kDataOffset = 2;
};

template <>
struct RowFmt<RowLayout::kPacked> {
    static constexpr int kBlockBytes = 16, kUnitsPerBlock = 1, kDataOffset = 0;
};

template <>
struct RowFmt<RowLayout::kQ4K> {
    static constexpr int kBlockBytes = 144, kUnitsPerBlock = 8, kDataOffset = 16;
};

// Q4_S256: 8 fp16 sub-scales (one per 32 weights) then 128 nibble bytes,
// symmetric about 8 (gemv_q4_s256.cpp:3-8).
template <>
struct RowFmt<RowLayout::kQ4S256> {
    static constexpr int kBlockBytes = 144, kUnitsPerBlock = 8, kDataOffset = 16;
};

// Blocks whose 16-byte header serves all 8 units.
template <RowLayout L>
constexpr bool kWideHeader = L == RowLayout::kQ4K || L == RowLayout::kQ4S256;

// 6-bit field idx of the Q4_K scale bitstream held in 3 dwords (12 bytes,
// LSB-first), as get_6bit_packed reads it (gemv_q4_avx2.cpp:110-120).
__device__ __forceinline__ uint32_t q4k_field(uint32_t b0, uint32_t b1, uint32_t b2, int idx) {
    const uint64_t lo = static_cast<uint64_t>(b0) | (static_cast<uint64_t>(b1) << 32);
    const int bit = idx * 6;
    if (bit + 6 <= 64) return static_cast<uint32_t>(lo >> bit) & 0x3Fu;
    if (bit >= 64) return (b2 >> (bit - 64)) & 0x3Fu;
    return static_cast<uint32_t>((lo >> bit) | (static_cast<uint64_t>(b2) << (64 - bit))) & 0x3Fu;
}

typedef uint32_t u32x4_a2 __attribute__((ext_vector_type(4), aligned(2)));

// side: per-(row, group) fp32 scales for kPacked, unused otherwise.
template <RowLayout L, int GSX, int NU, int WAVES, int NCH, bool Q8, bool EXACT, bool MULTI>
__global__ __launch_bounds__(WAVES * kWave) void rowblk_gemv_kernel(const uint8_t* __restrict__ blocks,
                                                                   const float* __restrict__ side,
                                                                   const float* __restrict__ x,
                                                                   const int8_t* __restrict__ xq8,
                                                                   const float* __restrict__ xsc,
                                                                   float* __restrict__ y, int M, int K,
                                                                   int llpr) {
    using F = RowFmt<L>;
    using Hd = typename std::conditional<kWideHeader<L>, uint4, uint32_t>::type;
    constexpr int UPG = GSX / 32;  // units per activation group
    constexpr QRule kRule = L == RowLayout::kQ4K ? QRule::kRoundAway : QRule::kRne;
    extern __shared__ __align__(16) uint32_t lds[];
    const XImage im = x_image(lds, K, GSX);

    const int lane = static_cast<int>(threadIdx.x) & (kWave - 1);
    const int wave = static_cast<int>(threadIdx.x) >> 6;
    const int lpr = 1 << llpr;
    const int j = lane & (lpr - 1);
    const int rin = lane >> llpr;
    const int rpw = kWave >> llpr;         // rows per wave pass
    const int rpt = rpw * WAVES;           // rows per tile
    const int U = K >> 5;                  // units per row
    const int G = K / GSX;                 // activation (and kPacked scale) groups per row
    const size_t row_bytes = static_cast<size_t>(U / F::kUnitsPerBlock) * F::kBlockBytes;
    const int ntiles = (M + rpt - 1) / rpt;
    // MULTI: rows longer than NU*LPR units are walked in passes, with the
    // activation read from LDS per unit; otherwise one pass, activation in
    // registers.
    const int per_pass = NU << llpr;
    const int npass = MULTI ? (U + per_pass - 1) / per_pass : 1;

    int tu[NU];
    bool valid[NU];
    auto set_units = [&](int pass) {
#pragma unroll
        for (int i = 0; i < NU; ++i) {
            const int t = pass * per_pass + j + i * lpr;
            valid[i] = EXACT || t < U;
            tu[i] = EXACT ? t : min(t, U - 1);
        }
    };
    set_units(0);

    uint4 w[NU];
    Hd hd[NU];
    // STAGE (blocks whose header serves several units: Q4_128, Q4_K; one
    // pass): a wave's rpw rows are one contiguous byte range, requested with
    // aligned 16-byte loads into registers, written to the wave's LDS area at
    // the start of the tile and read back per unit (Q4_128's units are 2-byte
    // aligned, which gfx950 LDS serves) and per header.  Measured: Q4_128
    // lm_head 80.3 -> 61.7 us, Q4_K gate_up 10.4 -> 10.2 us; for preq (one
    // unit per block) it was slower (gate_up 8.1 -> 10.0 us), so preq keeps
    // per-unit loads.
    constexpr bool STAGE = (L == RowLayout::kQ4_128 || kWideHeader<L>) && !MULTI;
    constexpr int kStageLoads = STAGE ? (NU * kWave * F::kBlockBytes / F::kUnitsPerBlock + 32 + 16 * kWave - 1) /
                                            (16 * kWave) : 1;
    uint4 cw[kStageLoads];
    const size_t stage_bytes = static_cast<size_t>(rpw) * row_bytes;  // one tile's rows of this wave
    const size_t total_bytes = static_cast<size_t>(M) * row_bytes;
    uint8_t* wstage = reinterpret_cast<uint8_t*>(lds) + ((x_image_bytes(K, GSX) + 15) & ~static_cast<size_t>(15)) +
                      static_cast<size_t>(wave) * ((stage_bytes + 47) & ~static_cast<size_t>(15));
    size_t st_a0 = 0, st_lead = 0;  // aligned start of the staged range, and the range's offset in it
    int st_count = 0;                // 16-byte chunks of the staged range
    auto load_stage = [&](int tile) {
        const int r0 = min(tile * rpt + wave * rpw, M - 1);
        const size_t a = static_cast<size_t>(r0) * row_bytes;
        const size_t end = min(a + stage_bytes, total_bytes);  // rows past M: not loaded, never stored
        st_a0 = a & ~static_cast<size_t>(15);
        st_lead = a - st_a0;
        st_count = static_cast<int>((end - st_a0 + 15) / 16);
#pragma unroll
        for (int k = 0; k < kStageLoads; ++k) {
            const int c = min(k * kWave + lane, st_count - 1);
            // the last chunk may run past the buffer's end: it is read ending there
            const size_t at = min(st_a0 + static_cast<size_t>(c) * 16, total_bytes - 16);
            const u32x4_a2 v = __builtin_nontemporal_load(reinterpret_cast<const u32x4_a2*>(blocks + at));
            cw[k] = make_uint4(v.x, v.y, v.z, v.w);
        }
    };
    auto unstage = [&]() {
#pragma unroll
        for (int k = 0; k < kStageLoads; ++k) {
            const int c = k * kWave + lane;
            if (c < st_count) {
                const size_t at = min(st_a0 + static_cast<size_t>(c) * 16, total_bytes - 16);
                *reinterpret_cast<u32x4_a2*>(wstage + (at - st_a0)) = u32x4_a2{cw[k].x, cw[k].y, cw[k].z, cw[k].w};
            }
        }
        const uint8_t* rb = wstage + st_lead + static_cast<size_t>(rin) * row_bytes;
#pragma unroll
        for (int i = 0; i < NU; ++i) {
            const int t = tu[i];
            const uint8_t* bp = rb + static_cast<size_t>(t / F::kUnitsPerBlock) * F::kBlockBytes;
            const u32x4_a2 v = *reinterpret_cast<const u32x4_a2*>(bp + F::kDataOffset + 16 * (t % F::kUnitsPerBlock));
            w[i] = make_uint4(v.x, v.y, v.z, v.w);
            if constexpr (L == RowLayout::kPreq) hd[i] = *reinterpret_cast<const uint32_t*>(bp);
            else if constexpr (L == RowLayout::kQ4_128) hd[i] = *reinterpret_cast<const uint16_t*>(bp);
            else if constexpr (kWideHeader<L>) hd[i] = *reinterpret_cast<const uint4*>(bp);
        }
    };
    // Unconditional loads at clamped, in-bounds rows; rows >= M are never stored.
    auto load_units = [&](int tile) {
        if constexpr (STAGE) {
            load_stage(tile);
            return;
        }
        const int row = min(tile * rpt + wave * rpw + rin, M - 1);
        const uint8_t* rb = blocks + static_cast<size_t>(row) * row_bytes;
#pragma unroll
        for (int i = 0; i < NU; ++i) {
            const int t = tu[i];
            const uint8_t* bp = rb + static_cast<size_t>(t / F::kUnitsPerBlock) * F::kBlockBytes;
            const u32x4_a2 v = __builtin_nontemporal_load(
                reinterpret_cast<const u32x4_a2*>(bp + F::kDataOffset + 16 * (t % F::kUnitsPerBlock)));
            w[i] = make_uint4(v.x, v.y, v.z, v.w);
        }
#pragma unroll
        for (int i = 0; i < NU; ++i) {
            const int t = tu[i];
            const uint8_t* bp = rb + static_cast<size_t>(t / F::kUnitsPerBlock) * F::kBlockBytes;
            if constexpr (L == RowLayout::kPreq) hd[i] = *reinterpret_cast<const uint32_t*>(bp);
            else if constexpr (L == RowLayout::kQ4_128) hd[i] = *reinterpret_cast<const uint16_t*>(bp);
            else if constexpr (L == RowLayout::kPacked)
                hd[i] = __float_as_uint(side[static_cast<size_t>(row) * G + t / UPG]);
            else hd[i] = *reinterpret_cast<const uint4*>(bp);
        }
    };

    int tile = static_cast<int>(blockIdx.x);
    const int tile_step = static_cast<int>(gridDim.x);
    ActStage<GSX, WAVES * kWave, NCH, Q8, kRule> act;
    act.load(x, xq8, xsc, K);  // activation loads first: they retire first
    load_units(tile);          // grid <= ntiles, so this tile exists
    act.process(K, im);
    __syncthreads();

    auto read_x = [&](int t, uint32_t (&dst)[8], float& sc, float& us) {
        const uint4 a = reinterpret_cast<const uint4*>(im.xq + t * 8)[0];
        const uint4 b = reinterpret_cast<const uint4*>(im.xq + t * 8)[1];
        dst[0] = a.x; dst[1] = a.y; dst[2] = a.z; dst[3] = a.w;
        dst[4] = b.x; dst[5] = b.y; dst[6] = b.z; dst[7] = b.w;
        sc = im.scale[t / UPG];
        us = im.usum[t];
    };
    uint32_t xr[MULTI ? 1 : NU][8];
    float xs[MULTI ? 1 : NU], xu[MULTI ? 1 : NU];
    if (!MULTI) {
#pragma unroll
        for (int i = 0; i < NU; ++i) read_x(tu[i], xr[MULTI ? 0 : i], xs[MULTI ? 0 : i], xu[MULTI ? 0 : i]);
    }
    auto dots = [&](float acc) {
        if constexpr (STAGE) unstage();
#pragma unroll
        for (int i = 0; i < NU; ++i) {
            if (valid[i]) {
                uint32_t xt[8];
                float sc, us;
                if (MULTI) read_x(tu[i], xt, sc, us);
                const int ii = MULTI ? 0 : i;
                const uint32_t(&xv)[8] = MULTI ? xt : xr[ii];
                const float xsv = MULTI ? sc : xs[ii];
                const int d = unit_dot(w[i], xv);
                if constexpr (L == RowLayout::kQ4S256) {
                    const uint4 h = hd[i];
                    const int sb = tu[i] % 8;
                    const uint32_t pair = sb < 2 ? h.x : (sb < 4 ? h.y : (sb < 6 ? h.z : h.w));
                    const float s = half_bits_to_float(pair >> (16 * (sb & 1)));
                    acc = fmaf(static_cast<float>(d), s * xsv, acc);
                    acc = fmaf(-(8.0f * s), MULTI ? us : xu[ii], acc);
                } else if constexpr (L == RowLayout::kQ4K) {
                    const uint4 h = hd[i];
                    const int sb = tu[i] % 8;
                    const float sub_scale = half_bits_to_float(h.x) * static_cast<float>(q4k_field(h.y, h.z, h.w, sb));
                    const float sub_min = half_bits_to_float(h.x >> 16) * static_cast<float>(q4k_field(h.y, h.z, h.w, sb + 8));
                    int xsum = 0;
#pragma unroll
                    for (int k = 0; k < 8; ++k) xsum = __builtin_amdgcn_sdot4(static_cast<int>(xv[k]), 0x01010101, xsum, false);
                    acc = fmaf(sub_scale * static_cast<float>(d) - sub_min * static_cast<float>(xsum), xsv, acc);
                } else {
                    const float s = L == RowLayout::kPacked ? __uint_as_float(hd[i]) : half_bits_to_float(hd[i]);
                    const float z = L == RowLayout::kPreq ? half_bits_to_float(hd[i] >> 16) : 8.0f;
                    acc = fmaf(static_cast<float>(d), s * xsv, acc);
                    acc = fmaf(-(z * s), MULTI ? us : xu[ii], acc);
                }
            }
        }
        return acc;
    };

    for (; tile < ntiles; tile += tile_step) {  // uniform per workgroup
        float acc = dots(0.0f);
        for (int pass = 1; pass < npass; ++pass) {  // MULTI only
            set_units(pass);
            load_units(tile);
            acc = dots(acc);
        }
        acc = group_sum<16>(acc);
        if (lpr >= 32) acc += swz_xor16(acc);
        if (lpr >= 64) acc += __shfl_xor(acc, 32, kWave);
        const int row = tile * rpt + wave * rpw + rin;
        if (tile + tile_step < ntiles) {
            if (MULTI) set_units(0);
            load_units(tile + tile_step);
        }
        if (j == 0 && row < M) y[row] = acc;
    }
}

struct RowPlan {
    int llpr, nu, waves, grid;
    bool exact, multi;
};

inline RowPlan plan_rowblk(int M, int K, int cus) {
    const int U = K / 32;
    RowPlan p{4, 0, K > 4096 ? 16 : 8, 0, false, false};
    auto nu_of = [&](int llpr) { return (U + (1 << llpr) - 1) >> llpr; };
    auto tiles_of = [&](int llpr) {
        const int rpt = (kWave >> llpr) * p.waves;
        return (M + rpt - 1) / rpt;
    };
    while (p.llpr < 6 && nu_of(p.llpr) > 6) ++p.llpr;
    while (p.llpr < 6 && tiles_of(p.llpr) < cus / 2 && U % (1 << (p.llpr + 1)) == 0) ++p.llpr;
    p.nu = nu_of(p.llpr);
    if (p.nu > 6) {  // rows longer than 6*64 units: passes of 4 units per lane
        p.multi = true;
        p.nu = 4;
    }
    p.exact = !p.multi && (p.nu << p.llpr) == U;
    const int cap = cus * (32 / p.waves);  // at most 32 waves per compute unit
    const int tiles = tiles_of(p.llpr);
    p.grid = tiles < cap ? tiles : cap;
    return p;
}

template <RowLayout L, int GSX, int WAVES, int NCH, bool Q8, bool EXACT, bool MULTI>
asdsl_status launch_rowblk_exact(const RowPlan& p, const uint8_t* blocks, const float* side, const float* x,
                                 const int8_t* xq8, const float* xsc, float* y, int M, int K, hipStream_t stream) {
    using F = RowFmt<L>;
    constexpr bool STAGE = (L == RowLayout::kQ4_128 || kWideHeader<L>) && !MULTI;
    const size_t row_bytes = static_cast<size_t>(K / 32 / F::kUnitsPerBlock) * F::kBlockBytes;
    const size_t stage = STAGE ? WAVES * (((static_cast<size_t>(kWave >> p.llpr) * row_bytes) + 47) & ~static_cast<size_t>(15))
                               : 0;
    const size_t lds = ((x_image_bytes(K, GSX) + 15) & ~static_cast<size_t>(15)) + stage;
    const dim3 block(WAVES * kWave);
#define ASDSL_ROWBLK_NU(N)                                                                                  \
    case N:                                                                                                 \
        return launch("rowblk_gemv_kernel", rowblk_gemv_kernel<L, GSX, N, WAVES, NCH, Q8, EXACT, MULTI>,    \
                      dim3(p.grid), block, lds, stream, blocks, side, x, xq8, xsc, y, M, K, p.llpr);
    switch (p.nu) {
        ASDSL_ROWBLK_NU(1)
        ASDSL_ROWBLK_NU(2)
        ASDSL_ROWBLK_NU(3)
        ASDSL_ROWBLK_NU(4)
        ASDSL_ROWBLK_NU(5)
        default: ASDSL_ROWBLK_NU(6)
    }
#undef ASDSL_ROWBLK_NU
}

template <RowLayout L, int GSX, int WAVES, int NCH, bool Q8>
asdsl_status launch_rowblk_waves(const RowPlan& p, const uint8_t* blocks, const float* side, const float* x,
                                 const int8_t* xq8, const float* xsc, float* y, int M, int K, hipStream_t stream) {
    if (p.multi)
        return launch_rowblk_exact<L, GSX, WAVES, NCH, Q8, false, true>(p, blocks, side, x, xq8, xsc, y, M, K, stream);
    if (p.exact)
        return launch_rowblk_exact<L, GSX, WAVES, NCH, Q8, true, false>(p, blocks, side, x, xq8, xsc, y, M, K, stream);
    return launch_rowblk_exact<L, GSX, WAVES, NCH, Q8, false, false>(p, blocks, side, x, xq8, xsc, y, M, K, stream);
}

// x (fp32, quantized inside) or xq8/xsc (pre-quantized, when Q8) — one of them.
template <RowLayout L, int GSX, bool Q8>
asdsl_status launch_rowblk(const uint8_t* blocks, const float* side, const float* x, const int8_t* xq8,
                           const float* xsc, float* y, int M, int K, hipStream_t stream, int cus) {
    const RowPlan p = plan_rowblk(M, K, cus);
    if (p.waves == 8) return launch_rowblk_waves<L, GSX, 8, 1, Q8>(p, blocks, side, x, xq8, xsc, y, M, K, stream);
    if (K <= 8192) return launch_rowblk_waves<L, GSX, 16, 1, Q8>(p, blocks, side, x, xq8, xsc, y, M, K, stream);
    if (K <= 16384) return launch_rowblk_waves<L, GSX, 16, 2, Q8>(p, blocks, side, x, xq8, xsc, y, M, K, stream);
    return launch_rowblk_waves<L, GSX, 16, 3, Q8>(p, blocks, side, x, xq8, xsc, y, M, K, stream);
}

}  // namespace asdsl
