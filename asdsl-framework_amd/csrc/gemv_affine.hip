// fp32-affine quantized GEMVs for gfx950: y = sum_g s_g * (sum_k q_k x_k) + b_g * (sum_k x_k)
//
// One kernel serves the reference's fp32 GEMVs over row-major weights with fp32
// per-group scale (and bias), the activation NOT quantized:
//   gemv_q4_packed      4-bit, 2 nibbles per byte, low nibble = even column
//                       (asdsl/kernels/native/gemv_q4_avx2.cpp:665-749)
//   gemv_q4_unpacked    one byte per value, value used as is (755-806)
//   gemv_q4_avx2_gs64   4-bit, scales only, group 64 (gemv_q4_kernel.cpp:96-122)
//   fused_dequant_gemv / gemv_q8_unpacked
//                       one byte per value (asdsl/kernels/native/gemv_q8_avx2.cpp:67-144)
//   gemv_sparse_unpacked / gemv_sparse_with_indices
//                       one byte per value, only active columns count
//                       (asdsl/kernels/native/gemv_sparse_avx2.cpp:66-139)
//
// The sparse forms are the dense form on a masked activation: x~_k = c_k x_k
// with c_k the number of times column k is active (0 or 1 for a bitmask), so
// inactive columns drop out of both sums.  A 32-column unit whose mask word is
// zero skips its weight loads (row-major weights save bytes only for such
// whole-unit runs of inactive columns).
//
// Mapping: a unit = 32 consecutive columns of one row (16 bytes packed, 32
// bytes unpacked).  LPR lanes serve a row, lane j taking units j, j+LPR, ...
// in passes of NU.  The activation sits in LDS as fp32 (masked), one unit per
// 36-float slot (the 4-float pad rotates consecutive units onto different LDS
// banks: lanes of a row read consecutive units in the same instruction), with
// the sum of each unit's 32 values after the slots; per unit a lane adds
//   s_g * dot_unit + b_g * sum_unit
// (the reference's per-group terms split per unit).  Requires group_size % 32
// == 0; other multiples of 8 take affine_gemv_generic (one wave per row).
#include <algorithm>
#include <type_traits>

#include "abi_util.hpp"
#include "device_common.hpp"

namespace asdsl {
namespace {

constexpr int kThreads = 256;
constexpr int kXStride = 36;  // floats per unit slot in LDS (32 values + pad)

// LDS: x~ (K/32 slots of kXStride floats) then per-unit sums (K/32 floats).
template <int WAVES, bool MASKED>
__device__ __forceinline__ void stage_x(const float* __restrict__ x, const uint32_t* __restrict__ mask,
                                        float* __restrict__ xs, float* __restrict__ usum, int K) {
    // one float4 per thread and pass; 8 consecutive threads = one unit
    const int n4 = K >> 2;
    for (int base = 0; base < n4; base += WAVES * kWave) {  // uniform
        const int c = base + static_cast<int>(threadIdx.x);
        const bool active = c < n4;
        float4 v = active ? reinterpret_cast<const float4*>(x)[c] : make_float4(0.f, 0.f, 0.f, 0.f);
        if (MASKED && active) {
            const uint32_t m = mask[c >> 3] >> ((c & 7) * 4);
            v.x = (m & 1u) ? v.x : 0.0f;
            v.y = (m & 2u) ? v.y : 0.0f;
            v.z = (m & 4u) ? v.z : 0.0f;
            v.w = (m & 8u) ? v.w : 0.0f;
        }
        const float s = group_sum<8>((v.x + v.y) + (v.z + v.w));
        if (active) {
            reinterpret_cast<float4*>(xs)[(c >> 3) * (kXStride / 4) + (c & 7)] = v;
            if ((c & 7) == 0) usum[c >> 3] = s;
        }
    }
}

template <int BITS>
__device__ __forceinline__ float unit_dot_f32(const uint4 (&w)[BITS / 4], const float* __restrict__ xu) {
    float d = 0.0f;
    const float4* x4 = reinterpret_cast<const float4*>(xu);
    if (BITS == 4) {
        const uint32_t wv[4] = {w[0].x, w[0].y, w[0].z, w[0].w};
#pragma unroll
        for (int i = 0; i < 4; ++i) {  // dword i = columns 8i..8i+7
            const uint32_t lo = wv[i] & 0x0F0F0F0Fu;
            const uint32_t hi = (wv[i] >> 4) & 0x0F0F0F0Fu;
            const float4 a = x4[2 * i];
            const float4 b = x4[2 * i + 1];
            d = fmaf(static_cast<float>(lo & 0xFFu), a.x, d);
            d = fmaf(static_cast<float>(hi & 0xFFu), a.y, d);
            d = fmaf(static_cast<float>((lo >> 8) & 0xFFu), a.z, d);
            d = fmaf(static_cast<float>((hi >> 8) & 0xFFu), a.w, d);
            d = fmaf(static_cast<float>((lo >> 16) & 0xFFu), b.x, d);
            d = fmaf(static_cast<float>((hi >> 16) & 0xFFu), b.y, d);
            d = fmaf(static_cast<float>(lo >> 24), b.z, d);
            d = fmaf(static_cast<float>(hi >> 24), b.w, d);
        }
    } else {
        const uint32_t wv[8] = {w[0].x, w[0].y, w[0].z, w[0].w, w[1].x, w[1].y, w[1].z, w[1].w};
#pragma unroll
        for (int i = 0; i < 8; ++i) {  // dword i = columns 4i..4i+3
            const float4 a = x4[i];
            d = fmaf(static_cast<float>(wv[i] & 0xFFu), a.x, d);
            d = fmaf(static_cast<float>((wv[i] >> 8) & 0xFFu), a.y, d);
            d = fmaf(static_cast<float>((wv[i] >> 16) & 0xFFu), a.z, d);
            d = fmaf(static_cast<float>(wv[i] >> 24), a.w, d);
        }
    }
    return d;
}

typedef uint32_t u32x4_a2 __attribute__((ext_vector_type(4), aligned(2)));

// Q128: weights are Q4_128 66-byte blocks (fp16 scale | 64 B nibbles, zero 8)
// instead of packed nibbles with side scale/bias arrays: per unit
// acc += ws * (dot - 8 * sum_x) (gemm_q4_128_q8_avx2's w = (q - 8) * ws).
template <int BITS, bool BIAS, bool MASKED, int NU, int WAVES, bool Q128 = false>
__global__ __launch_bounds__(WAVES * kWave) void affine_gemv_kernel(const uint8_t* __restrict__ w,
                                                                   const float* __restrict__ x,
                                                                   const float* __restrict__ scales,
                                                                   const float* __restrict__ biases,
                                                                   const uint32_t* __restrict__ mask,
                                                                   float* __restrict__ y, int M, int K, int gs,
                                                                   int llpr) {
    constexpr int UB = BITS * 4;  // bytes per unit: 16 packed, 32 unpacked
    extern __shared__ __align__(16) float lds_f[];
    float* xs = lds_f;
    float* usum = lds_f + (K >> 5) * kXStride;

    const int lane = static_cast<int>(threadIdx.x) & (kWave - 1);
    const int wave = static_cast<int>(threadIdx.x) >> 6;
    const int lpr = 1 << llpr;
    const int j = lane & (lpr - 1);
    const int rin = lane >> llpr;
    const int rpw = kWave >> llpr;
    const int rpt = rpw * WAVES;
    const int U = K >> 5;
    const int G = K / gs;
    const int upg = gs >> 5;  // units per group
    const size_t row_bytes = Q128 ? static_cast<size_t>(U / 4) * 66 : static_cast<size_t>(U) * UB;
    const int ntiles = (M + rpt - 1) / rpt;
    const int per_pass = NU << llpr;
    const int npass = (U + per_pass - 1) / per_pass;
    const int bx = static_cast<int>(blockIdx.x);
    const int gx = static_cast<int>(gridDim.x);
    const int iters = ((ntiles - 1 - bx) / gx + 1) * npass;  // (tile, pass) steps; the grid never exceeds ntiles

    // One step's weights, scales (Q128: the block scale) and biases, requested
    // one step ahead.  Units past U are loaded clamped and not used; the
    // masked form skips the loads of units whose mask word is zero.
    auto load_step = [&](int it, uint4 (&wu)[NU][BITS / 4], float (&sc)[NU], float (&bi)[NU], uint32_t& live) {
        const int tile = bx + (it / npass) * gx;
        const int pass = it % npass;
        const int row = min(tile * rpt + wave * rpw + rin, M - 1);
        const uint8_t* rb = w + static_cast<size_t>(row) * row_bytes;
        live = 0;
#pragma unroll
        for (int i = 0; i < NU; ++i) {
            const int t = pass * per_pass + j + i * lpr;
            const bool on = t < U && (!MASKED || mask[t] != 0u);
            live |= static_cast<uint32_t>(on) << i;
            if (MASKED && !on) continue;
            const int tc = min(t, U - 1);
            if constexpr (Q128) {
                const uint8_t* bp = rb + static_cast<size_t>(tc / 4) * 66;
                const u32x4_a2 v = __builtin_nontemporal_load(reinterpret_cast<const u32x4_a2*>(bp + 2 + 16 * (tc % 4)));
                wu[i][0] = make_uint4(v.x, v.y, v.z, v.w);
                sc[i] = half_bits_to_float(*reinterpret_cast<const uint16_t*>(bp));
            } else {
#pragma unroll
                for (int h = 0; h < BITS / 4; ++h)
                    wu[i][h] = load_stream16(reinterpret_cast<const uint4*>(rb + static_cast<size_t>(tc) * UB) + h);
                const size_t gi = static_cast<size_t>(row) * G + tc / upg;
                sc[i] = scales[gi];
                if constexpr (BIAS) bi[i] = biases[gi];
            }
        }
    };

    float acc = 0.0f;
    auto compute_step = [&](int it, const uint4 (&wu)[NU][BITS / 4], const float (&sc)[NU], const float (&bi)[NU],
                            uint32_t live) {
        const int tile = bx + (it / npass) * gx;
        const int pass = it % npass;
#pragma unroll
        for (int i = 0; i < NU; ++i) {
            const int t = pass * per_pass + j + i * lpr;
            if ((live >> i) & 1u) {
                const float d = unit_dot_f32<BITS>(wu[i], xs + t * kXStride);
                acc = fmaf(sc[i], d, acc);
                if constexpr (Q128) acc = fmaf(-8.0f * sc[i], usum[t], acc);
                if constexpr (BIAS) acc = fmaf(bi[i], usum[t], acc);
            }
        }
        if (pass == npass - 1) {  // uniform
            float r = group_sum<16>(acc);
            if (lpr >= 32) r += swz_xor16(r);
            if (lpr >= 64) r += __shfl_xor(r, 32, kWave);
            const int row = tile * rpt + wave * rpw + rin;
            if (j == 0 && row < M) y[row] = r;
            acc = 0.0f;
        }
    };

    // two register sets used alternately (a copy of a prefetch would wait for
    // it); the first step's loads are in flight while x is staged.  The last
    // step requests nothing (a wave ends only once its loads have landed).
    uint4 wa[NU][BITS / 4], wb[NU][BITS / 4];
    float sa[NU], sb[NU], ba[NU], bb[NU];
    uint32_t la, lb;
    load_step(0, wa, sa, ba, la);
    stage_x<WAVES, MASKED>(x, mask, xs, usum, K);
    __syncthreads();
    for (int it = 0;; it += 2) {  // uniform per workgroup
        if (it + 1 >= iters) {
            compute_step(it, wa, sa, ba, la);
            break;
        }
        load_step(it + 1, wb, sb, bb, lb);
        __builtin_amdgcn_sched_barrier(0);
        compute_step(it, wa, sa, ba, la);
        if (it + 2 >= iters) {
            compute_step(it + 1, wb, sb, bb, lb);
            break;
        }
        load_step(it + 2, wa, sa, ba, la);
        __builtin_amdgcn_sched_barrier(0);
        compute_step(it + 1, wb, sb, bb, lb);
    }
}

// Any group size that is a multiple of 8: one wave per row, lanes over
// 8-column chunks, per-group sums combined through LDS-free shuffles by
// accumulating s_g*dot + b_g*sum per chunk.
template <int BITS, bool BIAS, bool MASKED>
__global__ __launch_bounds__(kThreads) void affine_gemv_generic(const uint8_t* __restrict__ w,
                                                               const float* __restrict__ x,
                                                               const float* __restrict__ scales,
                                                               const float* __restrict__ biases,
                                                               const uint32_t* __restrict__ mask,
                                                               float* __restrict__ y, int M, int K, int gs) {
    const int lane = static_cast<int>(threadIdx.x) & (kWave - 1);
    const int G = K / gs;
    const int nch = K >> 3;
    for (int row = static_cast<int>(blockIdx.x) * (kThreads / kWave) + (static_cast<int>(threadIdx.x) >> 6);
         row < M; row += static_cast<int>(gridDim.x) * (kThreads / kWave)) {
        float acc = 0.0f;
        for (int c = lane; c < nch; c += kWave) {
            const int k0 = c * 8;
            float d = 0.0f, sx = 0.0f;
            uint32_t bits = 0xFFu;
            if (MASKED) bits = (mask[k0 >> 5] >> (k0 & 31)) & 0xFFu;
            for (int e = 0; e < 8; ++e) {
                const int k = k0 + e;
                const float xv = ((bits >> e) & 1u) ? x[k] : 0.0f;
                uint32_t q;
                if (BITS == 4) {
                    const uint8_t byte = w[static_cast<size_t>(row) * (K / 2) + (k >> 1)];
                    q = (k & 1) ? (byte >> 4) : (byte & 0x0F);
                } else {
                    q = w[static_cast<size_t>(row) * K + k];
                }
                d = fmaf(static_cast<float>(q), xv, d);
                sx += xv;
            }
            const int g = k0 / gs;  // 8 | gs: a chunk lies in one group
            acc = fmaf(scales[static_cast<size_t>(row) * G + g], d, acc);
            if (BIAS) acc = fmaf(biases[static_cast<size_t>(row) * G + g], sx, acc);
        }
        acc = group_sum<16>(acc);
        acc += swz_xor16(acc);
        acc += __shfl_xor(acc, 32, kWave);
        if (lane == 0) y[row] = acc;
    }
}

// Builds the masked activation's bitmask from an index list: mask bit k set for
// k listed at least once; counts[k] = times listed (duplicates count again).
__global__ __launch_bounds__(kThreads) void scatter_indices_kernel(const int32_t* __restrict__ idx, int n,
                                                                  uint32_t* __restrict__ mask,
                                                                  float* __restrict__ xs_out,
                                                                  const float* __restrict__ x, int K) {
    for (int i = static_cast<int>(blockIdx.x) * kThreads + static_cast<int>(threadIdx.x); i < n;
         i += static_cast<int>(gridDim.x) * kThreads) {
        const int k = idx[i];
        if (k < 0 || k >= K) continue;  // ignored (the reference would read out of bounds)
        atomicOr(mask + (k >> 5), 1u << (k & 31));
        atomicAdd(xs_out + k, x[k]);  // equal addends: any order gives c*x exactly as summed
    }
}

__global__ __launch_bounds__(kThreads) void fill_zero_kernel(uint32_t* __restrict__ p, int n) {
    for (int i = static_cast<int>(blockIdx.x) * kThreads + static_cast<int>(threadIdx.x); i < n;
         i += static_cast<int>(gridDim.x) * kThreads)
        p[i] = 0u;
}

__global__ __launch_bounds__(kThreads) void compute_bitmask_kernel(const float* __restrict__ x,
                                                                  uint32_t* __restrict__ mask, int K,
                                                                  float thr) {
    // one 32-bit word per 32 lanes: ballot of |x| >= thr (ordered: NaN inactive)
    const int nw = (K + 31) >> 5;
    for (int base = static_cast<int>(blockIdx.x) * kThreads; base < nw * 32;
         base += static_cast<int>(gridDim.x) * kThreads) {  // uniform
        const int k = base + static_cast<int>(threadIdx.x);
        const bool on = k < K && (x[k] >= thr || x[k] <= -thr);
        const unsigned long long b = __ballot(on);
        const int lane = static_cast<int>(threadIdx.x) & (kWave - 1);
        if ((lane & 31) == 0 && k < nw * 32)
            mask[k >> 5] = static_cast<uint32_t>(lane == 0 ? (b & 0xFFFFFFFFull) : (b >> 32));
    }
}

struct AffinePlan {
    int llpr, nu, grid;
};

AffinePlan plan_affine(int M, int K, int cus) {
    const int U = K / 32;
    AffinePlan p{4, 0, 0};
    constexpr int kWaves = 8;
    auto nu_of = [&](int l) { return (U + (1 << l) - 1) >> l; };
    auto tiles_of = [&](int l) {
        const int rpt = (kWave >> l) * kWaves;
        return (M + rpt - 1) / rpt;
    };
    while (p.llpr < 6 && nu_of(p.llpr) > 4) ++p.llpr;
    while (p.llpr < 6 && tiles_of(p.llpr) < cus / 2 && U % (1 << (p.llpr + 1)) == 0) ++p.llpr;
    p.nu = nu_of(p.llpr) > 4 ? 4 : nu_of(p.llpr);  // longer rows: passes of 4 units
    static const int knob = env_knob("ASDSL_HIP_AFFINE_WG_PER_CU");
    const int cap = cus * (knob > 0 ? knob : 2);
    const int tiles = tiles_of(p.llpr);
    p.grid = tiles < cap ? tiles : cap;
    return p;
}

template <int BITS, bool BIAS, bool MASKED, bool Q128 = false>
asdsl_status launch_affine(const uint8_t* w, const float* x, const float* s, const float* b, const uint32_t* mask,
                           float* y, int M, int K, int gs, hipStream_t stream, int cus) {
    if (!Q128 && (gs % 32 != 0 || K % 32 != 0)) {
        const int grid = stream_grid(M, kThreads / kWave, 8, cus);
        return launch("affine_gemv_generic", affine_gemv_generic<BITS, BIAS, MASKED>, dim3(grid), dim3(kThreads), 0,
                      stream, w, x, s, b, mask, y, M, K, gs);
    }
    const AffinePlan p = plan_affine(M, K, cus);
    const size_t lds = static_cast<size_t>(K / 32) * (kXStride + 1) * 4;
    constexpr int W = 8;
    switch (p.nu) {
#define ASDSL_AFFINE_NU(N)                                                                                    \
    case N:                                                                                                   \
        return launch("affine_gemv_kernel", affine_gemv_kernel<BITS, BIAS, MASKED, N, W, Q128>, dim3(p.grid), \
                      dim3(W * kWave), lds, stream, w, x, s, b, mask, y, M, K, gs, p.llpr);
        ASDSL_AFFINE_NU(1)
        ASDSL_AFFINE_NU(2)
        ASDSL_AFFINE_NU(3)
        default: ASDSL_AFFINE_NU(4)
#undef ASDSL_AFFINE_NU
    }
}

// ---------------------------------------------------------- batched (MFMA) path
// Up to 16 activation columns per weight pass, v_mfma_f32_16x16x32_f16 per
// (unit, 16-row tile).  The pre-pass scales each column by 2^e (its amax to
// [2^14, 2^15)) and splits x' = 2^e x into two fp16 digits, hi = fp16(x') and
// lo = fp16(x' - hi), together x' to ~2^-22 relative (elements below fp16's
// normal range keep an absolute error under 2^-25, i.e. 2^-39 of the column's
// amax); a 4-bit weight is exact in fp16 and each product q*digit exact in
// fp32, so per group g (UPG units of 32 columns)
//   C[n][r]   = sum_{k in g} q[r][k] * (hi + lo)[n][k]          (fp32 MFMA)
//   acc[n][r] += s[r][g] * C + b[r][g] * sum_{k in g} x'[n][k]
//   Y[n][r]   = 2^-e[n] * acc
// (the reference's w = fma(q, s, b) summed against fp32 x, per group).
// A = digits (its rows = columns n), B = weights (its columns = rows r), so
// lane l ends with row r0 + l%16 and columns 4*(l/16) + v, v = 0..3.
//
// Operand order inside a unit's dword d (8 nibbles, nibble i = column 8d+i):
// the weight operand takes the four halfword pairs
//   (w & 0x000F000F), (w & 0x00F000F0), (w>>8 & 0x000F000F), (w>>8 & 0x00F000F0)
// each OR 0x6400 per half (fp16 1024 + v) minus 1024, i.e. slots 2p, 2p+1 hold
// columns p and p+4 (p = 0..3), the odd pairs 16x the nibble; the digit
// operand holds the same columns in the same slots, the odd pairs' x' / 16.
//
// Pre-pass image (device work buffer):
//   img[t][digit][lane]  uint4: unit t's digits for lane l = 16*d + n
//   xsum[g][n]           float: sum of x' over group g
//   down[n]              float: 2^-e of column n
//
// Measured alternatives (gate_up 16384x3072, B = 4): the digit operands in
// LDS with independent waves streaming their K share (no per-tile barrier)
// ran 19.2 us against this kernel's 16.4; 32-row tiles and a second tile of
// prefetch both spill registers and ran 20-22 us.
constexpr int kBatchCols = 16;
constexpr int kSplitThreads = 1024;

typedef _Float16 v8h __attribute__((ext_vector_type(8)));
typedef _Float16 h2v __attribute__((ext_vector_type(2)));
typedef float v4f __attribute__((ext_vector_type(4)));

__device__ __forceinline__ uint32_t pack_h2(float a, float b) {
    const h2v h = {static_cast<_Float16>(a), static_cast<_Float16>(b)};
    return __builtin_bit_cast(uint32_t, h);
}

// (a & m) | o in one instruction: the mask from an SGPR, o from a VGPR (one
// constant-bus operand on gfx9)
__device__ __forceinline__ uint32_t and_or(uint32_t a, uint32_t m, uint32_t o) {
    uint32_t r;
    asm("v_and_or_b32 %0, %1, %2, %3" : "=v"(r) : "v"(a), "s"(m), "v"(o));
    return r;
}

// One workgroup per column n < ncols: its amax, then its digits and group sums.
template <int UPG>
__global__ __launch_bounds__(kSplitThreads) void affine_split_kernel(const float* __restrict__ X,
                                                                     uint4* __restrict__ img,
                                                                     float* __restrict__ xsum,
                                                                     float* __restrict__ down_out, int K) {
    constexpr int kGroupLanes = 4 * UPG;  // 8-element chunks (threads) per group
    __shared__ float red[kSplitThreads / kWave];
    const int n = static_cast<int>(blockIdx.x);
    const int tid = static_cast<int>(threadIdx.x);
    const float* x = X + static_cast<size_t>(n) * K;
    float am = 0.0f;
    for (int c = tid; c < K / 4; c += kSplitThreads) {
        const float4 v = reinterpret_cast<const float4*>(x)[c];
        am = fmaxf(am, fmaxf(fmaxf(fabsf(v.x), fabsf(v.y)), fmaxf(fabsf(v.z), fabsf(v.w))));
    }
    for (int o = 32; o >= 1; o >>= 1) am = fmaxf(am, __shfl_xor(am, o, kWave));
    if ((tid & (kWave - 1)) == 0) red[tid >> 6] = am;
    __syncthreads();
    am = red[0];
#pragma unroll
    for (int i = 1; i < kSplitThreads / kWave; ++i) am = fmaxf(am, red[i]);
    // 2^se brings amax to [2^14, 2^15); both 2^se and 2^-se stay normal
    const int E = static_cast<int>((__float_as_uint(am) >> 23) & 0xFFu);
    const int se = min(max(141 - E, -126), 126);
    const float up = __uint_as_float(static_cast<uint32_t>(se + 127) << 23);
    if (tid == 0) down_out[n] = __uint_as_float(static_cast<uint32_t>(127 - se) << 23);

    // chunks of 8: groups are whole runs of kGroupLanes threads (K/8 is a
    // multiple of kGroupLanes), so a partly active pass has whole groups
    for (int c = tid; c < K / 8; c += kSplitThreads) {
        const float4 a = reinterpret_cast<const float4*>(x)[2 * c];
        const float4 b = reinterpret_cast<const float4*>(x)[2 * c + 1];
        const float v[8] = {a.x * up, a.y * up, a.z * up, a.w * up, b.x * up, b.y * up, b.z * up, b.w * up};
        float sm = 0.0f;
#pragma unroll
        for (int i = 0; i < 8; ++i) sm += v[i];
        sm = group_sum<kGroupLanes>(sm);
        uint32_t hi[4], lo[4];
#pragma unroll
        for (int p = 0; p < 4; ++p) {
            float yh[2], yl[2];
#pragma unroll
            for (int h = 0; h < 2; ++h) {
                const float y = v[p + 4 * h] * ((p & 1) ? 0.0625f : 1.0f);
                const float t = static_cast<float>(static_cast<_Float16>(y));
                yh[h] = t;
                yl[h] = y - t;  // exact
            }
            hi[p] = pack_h2(yh[0], yh[1]);
            lo[p] = pack_h2(yl[0], yl[1]);
        }
        const int t = c >> 2;
        const int lane = 16 * (c & 3) + n;
        img[(static_cast<size_t>(t) * 2 + 0) * kWave + lane] = make_uint4(hi[0], hi[1], hi[2], hi[3]);
        img[(static_cast<size_t>(t) * 2 + 1) * kWave + lane] = make_uint4(lo[0], lo[1], lo[2], lo[3]);
        if (c % kGroupLanes == 0) xsum[static_cast<size_t>(c / kGroupLanes) * kBatchCols + n] = sm;
    }
}

// LDS per wave: the staged weights of one 16-row tile (pitch GPW*16 + 16
// bytes, so that the 16 rows start on different banks), its scales and
// biases ([16][GPW/UPG] floats each) and the wave's group sums ([GPW/UPG][16]
// floats); per workgroup two buffers of the fixed-order K-slice sum.
__host__ __device__ constexpr int ab_pitch(int gpw) { return gpw * 16 + 16; }
__host__ __device__ constexpr int ab_wave_bytes(int gpw, int upg) {
    return 16 * ab_pitch(gpw) + 2 * 16 * (gpw / upg) * 4 + (gpw / upg) * 64;
}
__host__ __device__ constexpr size_t ab_lds_bytes(int gpw, int upg, int waves) {
    return static_cast<size_t>(waves) * ab_wave_bytes(gpw, upg) + 2 * static_cast<size_t>(waves) * 4 * kWave * 4;
}

// Workgroup = W waves over one K-slab of W*GPW units (slab = blockIdx.y),
// looping over 16-row tiles; the W partial tiles are added in LDS in fixed
// order and written to out + slab * slab_stride (Y itself for one slab).
// Each wave requests the next tile's weights, scales and biases before it
// computes the current one (two register sets in turn).  Q128: the weights
// are Q4_128 66-byte blocks (fp16 scale, 64 B nibbles; UPG = 4), s = the
// block scale and b = -8 s (gemm_q4_128_q8_avx2's w = (q - 8) * ws).
template <int UPG, int GPW, int W, bool BIAS, bool Q128 = false>
__global__ __launch_bounds__(W * kWave) void affine_batch_mfma_kernel(
    const uint8_t* __restrict__ w, const float* __restrict__ scales, const float* __restrict__ biases,
    const uint4* __restrict__ img, const float* __restrict__ xsum, const float* __restrict__ down,
    float* __restrict__ out, int M, int K, int ncols, size_t slab_stride) {
    static_assert(GPW % 4 == 0 && GPW % UPG == 0, "whole loads and whole groups per wave");
    constexpr int NG = GPW / UPG;
    constexpr int kPitch = ab_pitch(GPW);
    constexpr int kLoads = GPW / 4;  // 16 rows x GPW units x 16 B = GPW/4 uint4 per lane
    constexpr int kSB = 16 * NG;     // a tile's scales (and biases), read row-contiguous
    constexpr int kSBLoads = (kSB + kWave - 1) / kWave;
    extern __shared__ __align__(16) uint32_t ab_lds[];
    uint8_t* lds = reinterpret_cast<uint8_t*>(ab_lds);
    const int lane = static_cast<int>(threadIdx.x) & (kWave - 1);
    const int wave = static_cast<int>(threadIdx.x) >> 6;
    const int r16 = lane & 15;
    const int q = lane >> 4;
    const int G = (K >> 5) / UPG;
    const int slab = static_cast<int>(blockIdx.y);
    const int u0 = (slab * W + wave) * GPW;
    const int g0 = u0 / UPG;
    static_assert(!Q128 || (UPG == 4 && BIAS), "Q4_128 blocks: group 128, bias -8 * scale");
    const size_t rowb = Q128 ? static_cast<size_t>(K / 128) * 66 : static_cast<size_t>(K) >> 1;
    const int ntiles = (M + 15) >> 4;
    uint8_t* stage = lds + static_cast<size_t>(wave) * ab_wave_bytes(GPW, UPG);
    float* sst = reinterpret_cast<float*>(stage + 16 * kPitch);  // [16][NG] scales
    float* bst = sst + kSB;                                        // [16][NG] biases
    float* wsum = bst + kSB;                                       // [NG][16] group sums
    float* red = reinterpret_cast<float*>(lds + static_cast<size_t>(W) * ab_wave_bytes(GPW, UPG));
    out += static_cast<size_t>(slab) * slab_stride;

    auto load_tile = [&](uint4 (&wv)[kLoads], float (&sv)[kSBLoads], float (&bv)[BIAS ? kSBLoads : 1], int tile) {
#pragma unroll
        for (int i = 0; i < kLoads; ++i) {
            const int e = i * kWave + lane;
            const int row = min(tile * 16 + e / GPW, M - 1);  // past M: the last row, never stored
            const int u = u0 + e % GPW;
            if constexpr (Q128) {
                const u32x4_a2 v = __builtin_nontemporal_load(reinterpret_cast<const u32x4_a2*>(
                    w + static_cast<size_t>(row) * rowb + static_cast<size_t>(u / 4) * 66 + 2 + 16 * (u % 4)));
                wv[i] = make_uint4(v.x, v.y, v.z, v.w);
            } else {
                wv[i] = load_stream16(reinterpret_cast<const uint4*>(w + static_cast<size_t>(row) * rowb +
                                                                     static_cast<size_t>(u) * 16));
            }
        }
#pragma unroll
        for (int i = 0; i < kSBLoads; ++i) {
            const int e = min(i * kWave + lane, kSB - 1);
            const int row = min(tile * 16 + e / NG, M - 1);
            if constexpr (Q128) {
                sv[i] = half_bits_to_float(*reinterpret_cast<const uint16_t*>(
                    w + static_cast<size_t>(row) * rowb + static_cast<size_t>(g0 + e % NG) * 66));
            } else {
                const size_t so = static_cast<size_t>(row) * G + g0 + e % NG;
                sv[i] = scales[so];
                if constexpr (BIAS) bv[i] = biases[so];
            }
        }
    };

    const int bx = static_cast<int>(blockIdx.x);
    const int step = static_cast<int>(gridDim.x);
    const int nt = (ntiles - 1 - bx) / step + 1;  // this workgroup's tiles bx + i*step; the grid never exceeds ntiles
    uint4 w0[kLoads], w1[kLoads];
    float s0[kSBLoads], s1[kSBLoads], b0[BIAS ? kSBLoads : 1], b1[BIAS ? kSBLoads : 1];

    // the first tile's weights go out first; then the digit operands (column
    // r16, dword q of each of the wave's units: lanes of columns past ncols
    // hold zeros and load nothing) and the wave's group sums (to LDS)
    load_tile(w0, s0, b0, bx);
    v8h ahi[GPW], alo[GPW];
    const bool col_live = r16 < ncols;
#pragma unroll
    for (int j = 0; j < GPW; ++j) {
        uint4 h = make_uint4(0u, 0u, 0u, 0u), l = h;
        if (col_live) {
            h = img[(static_cast<size_t>(u0 + j) * 2 + 0) * kWave + lane];
            l = img[(static_cast<size_t>(u0 + j) * 2 + 1) * kWave + lane];
        }
        ahi[j] = __builtin_bit_cast(v8h, h);
        alo[j] = __builtin_bit_cast(v8h, l);
    }
    if constexpr (BIAS) {
        constexpr int kSumLoads = (NG * 16 + kWave - 1) / kWave;
        float sv[kSumLoads];
#pragma unroll
        for (int i = 0; i < kSumLoads; ++i)
            sv[i] = xsum[static_cast<size_t>(g0) * kBatchCols + min(i * kWave + lane, NG * 16 - 1)];
#pragma unroll
        for (int i = 0; i < kSumLoads; ++i)
            if (i * kWave + lane < NG * 16) wsum[i * kWave + lane] = sv[i];
    }

    const v4f zero = {0.0f, 0.0f, 0.0f, 0.0f};
    const h2v k1024 = {static_cast<_Float16>(1024.0f), static_cast<_Float16>(1024.0f)};
    uint32_t magic;  // fp16 1024 in both halves, held in a VGPR for v_and_or_b32
    asm volatile("v_mov_b32 %0, 0x64006400" : "=v"(magic));
    // tile i of this workgroup from register set (wc, sc, bc); with prefetch,
    // tile i + 1 is requested into (wn, sn, bn)
    auto run_tile = [&](auto prefetch, int i, uint4 (&wc)[kLoads], float (&sc)[kSBLoads],
                        float (&bc)[BIAS ? kSBLoads : 1], auto& wn, auto& sn, auto& bn) {
        const int tile = bx + i * step;
        // stage this tile's weights, scales and biases (the wave reads back
        // only what it wrote; LDS operations of a wave complete in order),
        // then request the next tile's before computing
#pragma unroll
        for (int k = 0; k < kLoads; ++k) {
            const int e = k * kWave + lane;
            *reinterpret_cast<uint4*>(stage + (e / GPW) * kPitch + (e % GPW) * 16) = wc[k];
        }
#pragma unroll
        for (int k = 0; k < kSBLoads; ++k) {
            const int e = k * kWave + lane;
            if (e < kSB) {
                sst[e] = sc[k];
                if constexpr (Q128)
                    bst[e] = -8.0f * sc[k];
                else if constexpr (BIAS)
                    bst[e] = bc[k];
            }
        }
        __builtin_amdgcn_sched_barrier(0);
        // (a workgroup's last tile requests nothing: a wave ends only once its
        // loads have landed)
        if constexpr (decltype(prefetch)::value) load_tile(wn, sn, bn, tile + step);
        __builtin_amdgcn_sched_barrier(0);

        float acc[4] = {0.0f, 0.0f, 0.0f, 0.0f};
        v4f c = zero;
#pragma unroll
        for (int j = 0; j < GPW; ++j) {
            const uint32_t wd = *reinterpret_cast<const uint32_t*>(stage + r16 * kPitch + j * 16 + q * 4);
            const uint32_t w8 = wd >> 8;
            const uint32_t pr[4] = {and_or(wd, 0x000F000Fu, magic), and_or(wd, 0x00F000F0u, magic),
                                    and_or(w8, 0x000F000Fu, magic), and_or(w8, 0x00F000F0u, magic)};
            uint32_t bw[4];
#pragma unroll
            for (int p = 0; p < 4; ++p) bw[p] = __builtin_bit_cast(uint32_t, __builtin_bit_cast(h2v, pr[p]) - k1024);
            const v8h bop = __builtin_bit_cast(v8h, make_uint4(bw[0], bw[1], bw[2], bw[3]));
            c = __builtin_amdgcn_mfma_f32_16x16x32_f16(ahi[j], bop, (j % UPG == 0) ? zero : c, 0, 0, 0);
            c = __builtin_amdgcn_mfma_f32_16x16x32_f16(alo[j], bop, c, 0, 0, 0);
            if (j % UPG == UPG - 1) {
                const int jg = j / UPG;
                const float sr = sst[r16 * NG + jg];
#pragma unroll
                for (int v = 0; v < 4; ++v) acc[v] = fmaf(c[v], sr, acc[v]);
                if constexpr (BIAS) {
                    const float br = bst[r16 * NG + jg];
                    const float4 xs = *reinterpret_cast<const float4*>(wsum + jg * 16 + q * 4);
                    acc[0] = fmaf(br, xs.x, acc[0]);
                    acc[1] = fmaf(br, xs.y, acc[1]);
                    acc[2] = fmaf(br, xs.z, acc[2]);
                    acc[3] = fmaf(br, xs.w, acc[3]);
                }
            }
        }

        // add the W K-slices in fixed order; the two buffers alternate, so
        // one barrier per tile suffices
        float* rb = red + (i & 1) * (W * 4 * kWave);
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
            if (n < ncols && row < M) out[static_cast<size_t>(n) * M + row] = sum * down[n];
        }
    };
    const std::true_type pf_on;
    const std::false_type pf_off;
    // Every path has a fixed number of requests in flight at each wait (a
    // conditional request would make every wait drain all of them): at the
    // loop head tile i is in set 0.
    for (int i = 0;; i += 2) {  // uniform per workgroup
        if (i + 1 >= nt) {
            run_tile(pf_off, i, w0, s0, b0, w0, s0, b0);
            break;
        }
        run_tile(pf_on, i, w0, s0, b0, w1, s1, b1);
        if (i + 2 >= nt) {
            run_tile(pf_off, i + 1, w1, s1, b1, w1, s1, b1);
            break;
        }
        run_tile(pf_on, i + 1, w1, s1, b1, w0, s0, b0);
    }
}

// Y[n][m] = sum over slabs of part[slab][n][m], slabs in order.
__global__ __launch_bounds__(256) void affine_batch_sum_kernel(const float* __restrict__ part, float* __restrict__ Y,
                                                               int M, int ncols, int slabs) {
    const size_t total = static_cast<size_t>(ncols) * M;
    const size_t stride = static_cast<size_t>(kBatchCols) * M;
    for (size_t i = static_cast<size_t>(blockIdx.x) * 256 + threadIdx.x; i < total;
         i += static_cast<size_t>(gridDim.x) * 256) {
        float s = part[i];
        for (int p = 1; p < slabs; ++p) s += part[static_cast<size_t>(p) * stride + i];
        Y[i] = s;
    }
}

struct BatchPlan {
    int waves = 0, gpw = 0, slabs = 0, grid = 0;
    bool ok = false;
};

// (waves, units per wave) covering K/32 units in the fewest K-slabs
// (ASDSL_HIP_AFFINE_BATCH_SHAPE = 1..6 forces one); the grid holds
// ASDSL_HIP_AFFINE_BATCH_WG_PER_CU slab-workgroups per compute unit (default
// 1), capped at the tile count.
BatchPlan plan_affine_batch(int M, int K, int upg, int cus) {
    BatchPlan p;
    if (K % 128 != 0) return p;
    const int U = K / 32;
    static const int shapes[][2] = {{8, 12}, {8, 8}, {4, 12}, {8, 4}, {4, 8}, {4, 4}};
    static const int force = env_knob("ASDSL_HIP_AFFINE_BATCH_SHAPE");
    for (int si = 0; si < 6; ++si) {
        const auto& s = shapes[si];
        const int per = s[0] * s[1];
        if (U % per != 0 || s[1] % upg != 0 || (force > 0 && force != si + 1)) continue;
        if (p.slabs == 0 || U / per < p.slabs) {
            p.waves = s[0];
            p.gpw = s[1];
            p.slabs = U / per;
        }
    }
    if (p.slabs == 0) return p;
    static const int knob = env_knob("ASDSL_HIP_AFFINE_BATCH_WG_PER_CU");
    const int per_cu = knob > 0 ? knob : 1;
    const int tiles = (M + 15) / 16;
    const int want = std::max(1, per_cu * cus / p.slabs);
    p.grid = tiles < want ? tiles : want;
    p.ok = true;
    return p;
}

template <int UPG, int GPW, int W, bool BIAS, bool Q128>
asdsl_status launch_batch_shape(const BatchPlan& p, const uint8_t* w, const float* s, const float* b,
                                const uint4* img, const float* xsum, const float* down, float* out, int M, int K,
                                int ncols, size_t slab_stride, hipStream_t st) {
    return launch("affine_batch_mfma_kernel", affine_batch_mfma_kernel<UPG, GPW, W, BIAS, Q128>, dim3(p.grid, p.slabs),
                  dim3(W * kWave), ab_lds_bytes(GPW, UPG, W), st, w, s, b, img, xsum, down, out, M, K, ncols,
                  slab_stride);
}

template <int UPG, bool BIAS, bool Q128>
asdsl_status launch_batch_upg(const BatchPlan& p, const uint8_t* w, const float* s, const float* b,
                              const uint4* img, const float* xsum, const float* down, float* out, int M, int K,
                              int ncols, size_t slab_stride, hipStream_t st) {
#define ASDSL_AB_CASE(W_, GPW_)                                                                               \
    if constexpr (GPW_ % UPG == 0)                                                                            \
        if (p.waves == W_ && p.gpw == GPW_)                                                                   \
            return launch_batch_shape<UPG, GPW_, W_, BIAS, Q128>(p, w, s, b, img, xsum, down, out, M, K, ncols, \
                                                                 slab_stride, st);
    ASDSL_AB_CASE(8, 12)
    ASDSL_AB_CASE(8, 8)
    ASDSL_AB_CASE(4, 12)
    ASDSL_AB_CASE(8, 4)
    ASDSL_AB_CASE(4, 8)
    ASDSL_AB_CASE(4, 4)
#undef ASDSL_AB_CASE
    set_error("affine batch: no MFMA tiling for this shape");
    return ASDSL_ERR_UNSUPPORTED;
}

// The batched fp32-activation GEMV over packed 4-bit weights with scales (and
// biases), or over Q4_128 blocks (Q128, gs = 128): Y[n] = W x[n] for n < B,
// B columns of X, 16 per weight pass.  Returns ASDSL_ERR_UNSUPPORTED (nothing
// launched) when the shape has no MFMA tiling; the caller then runs one GEMV
// per column.
// Work bytes of affine_batch: the column image (K/32 units x 2 digits x 64 x 16
// bytes), per-group sums and scale exponents, and the K-slab partial rows.
size_t affine_batch_work_bytes(int M, int K, int upg, int slabs) {
    const int U = K / 32;
    const size_t img_bytes = static_cast<size_t>(U) * 2 * kWave * 16;
    const size_t sum_bytes = static_cast<size_t>(U / upg) * kBatchCols * 4 + kBatchCols * 4;
    const size_t part_floats = slabs > 1 ? static_cast<size_t>(slabs) * kBatchCols * M : 0;
    return img_bytes + sum_bytes + part_floats * 4;
}

template <bool BIAS, bool Q128 = false>
asdsl_status affine_batch(const uint8_t* w, const float* s, const float* b, const float* X, float* Y, int M, int K,
                          int B, int gs, hipStream_t st, int cus, const char* what, void* work = nullptr,
                          size_t work_bytes = 0) {
    const int upg = gs / 32;
    if (gs % 32 != 0 || (upg != 1 && upg != 2 && upg != 4) || reinterpret_cast<uintptr_t>(X) % 16 != 0)
        return ASDSL_ERR_UNSUPPORTED;
    const BatchPlan p = plan_affine_batch(M, K, upg, cus);
    if (!p.ok) return ASDSL_ERR_UNSUPPORTED;
    const int U = K / 32;
    const size_t img_bytes = static_cast<size_t>(U) * 2 * kWave * 16;
    const size_t sum_bytes = static_cast<size_t>(U / upg) * kBatchCols * 4 + kBatchCols * 4;
    void* ws = nullptr;
    asdsl_status r = work_buffer(st, work, work_bytes, affine_batch_work_bytes(M, K, upg, p.slabs), &ws, what);
    if (r != ASDSL_OK) return r;
    uint4* img = static_cast<uint4*>(ws);
    float* xsum = reinterpret_cast<float*>(static_cast<uint8_t*>(ws) + img_bytes);
    float* down = xsum + static_cast<size_t>(U / upg) * kBatchCols;
    float* part = reinterpret_cast<float*>(static_cast<uint8_t*>(ws) + img_bytes + sum_bytes);
    for (int n0 = 0; n0 < B; n0 += kBatchCols) {
        const int nc = std::min(kBatchCols, B - n0);
        const float* Xc = X + static_cast<size_t>(n0) * K;
        float* Yc = Y + static_cast<size_t>(n0) * M;
        if (upg == 1)
            r = launch("affine_split_kernel", affine_split_kernel<1>, dim3(nc), dim3(kSplitThreads), 0, st, Xc, img,
                       xsum, down, K);
        else if (upg == 2)
            r = launch("affine_split_kernel", affine_split_kernel<2>, dim3(nc), dim3(kSplitThreads), 0, st, Xc, img,
                       xsum, down, K);
        else
            r = launch("affine_split_kernel", affine_split_kernel<4>, dim3(nc), dim3(kSplitThreads), 0, st, Xc, img,
                       xsum, down, K);
        if (r != ASDSL_OK) return r;
        float* out = p.slabs > 1 ? part : Yc;
        const size_t stride = p.slabs > 1 ? static_cast<size_t>(kBatchCols) * M : 0;
        if constexpr (Q128)
            r = launch_batch_upg<4, true, true>(p, w, s, b, img, xsum, down, out, M, K, nc, stride, st);
        else if (upg == 1)
            r = launch_batch_upg<1, BIAS, false>(p, w, s, b, img, xsum, down, out, M, K, nc, stride, st);
        else if (upg == 2)
            r = launch_batch_upg<2, BIAS, false>(p, w, s, b, img, xsum, down, out, M, K, nc, stride, st);
        else
            r = launch_batch_upg<4, BIAS, false>(p, w, s, b, img, xsum, down, out, M, K, nc, stride, st);
        if (r != ASDSL_OK) return r;
        if (p.slabs > 1) {
            const int g = stream_grid(static_cast<long long>(nc) * M, 256, 4, cus);
            r = launch("affine_batch_sum_kernel", affine_batch_sum_kernel, dim3(g), dim3(256), 0, st, part, Yc, M, nc,
                       p.slabs);
            if (r != ASDSL_OK) return r;
        }
    }
    return ASDSL_OK;
}

// LDS budget of the fast path: K/32 * 148 bytes (151552 at the maximum K).
constexpr int kMaxAffineK = 32768;

int check_affine(const void* w, const void* x, const void* s, const void* y, int M, int K, int gs, int batch,
                 const char* fn) {
    if (!w || !x || !s || !y) {
        set_error("%s: null pointer", fn);
        return 1;
    }
    if (M <= 0 || K <= 0 || gs <= 0) {
        set_error("%s: M, K, group_size must be positive", fn);
        return 1;
    }
    if (batch < 1) {
        set_error("%s: batch must be >= 1", fn);
        return 1;
    }
    if (K % 2 != 0) {
        set_error("%s: K must be even for 4-bit packing", fn);
        return 1;
    }
    if (K % gs != 0) {
        set_error("%s: K must be divisible by group_size", fn);
        return 1;
    }
    if (gs % 8 != 0) {
        set_error("%s: group_size must be a multiple of 8", fn);
        return 1;
    }
    if (K > kMaxAffineK) {
        set_error("%s: K must be <= %d", fn, kMaxAffineK);
        return 1;
    }
    if (reinterpret_cast<uintptr_t>(x) % 16 != 0 || reinterpret_cast<uintptr_t>(w) % 16 != 0) {
        set_error("%s: weights and x must be 16-byte aligned", fn);
        return 1;
    }
    return 0;
}

}  // namespace
}  // namespace asdsl

using namespace asdsl;

extern "C" size_t asdsl_affine_batch_work_bytes(int M, int K, int group_size) {
    if (M <= 0 || K <= 0 || group_size <= 0 || group_size % 32 != 0) return 0;
    const int upg = group_size / 32;
    if (upg != 1 && upg != 2 && upg != 4) return 0;
    const BatchPlan p = plan_affine_batch(M, K, upg, 256);  // the slab count does not depend on the CU count
    return p.ok ? affine_batch_work_bytes(M, K, upg, p.slabs) : 0;
}

extern "C" asdsl_status asdsl_gemv_q4_packed_ws(const uint8_t* w_packed, const float* x, const float* scales,
                                                const float* biases, float* y, int M, int K, int group_size,
                                                int batch, void* work, size_t work_bytes, asdsl_stream_t stream) {
    if (check_affine(w_packed, x, scales, y, M, K, group_size, batch, "gemv_q4_packed"))
        return ASDSL_ERR_INVALID_ARGUMENT;
    ASDSL_CHECK_ARG(biases != nullptr, "gemv_q4_packed: null pointer");
    ASDSL_CHECK_ARG(group_size % 16 == 0, "gemv_q4_packed: group_size must be a multiple of 16");
    ASDSL_CU_COUNT(cus);
    if (batch > 1) {
        const asdsl_status st = affine_batch<true>(w_packed, scales, biases, x, y, M, K, batch, group_size,
                                                   as_hip(stream), cus, "gemv_q4_packed", work, work_bytes);
        if (st != ASDSL_ERR_UNSUPPORTED) return st;
    }
    for (int bi = 0; bi < batch; ++bi) {
        const asdsl_status st = launch_affine<4, true, false>(w_packed, x + static_cast<size_t>(bi) * K, scales, biases,
                                                              nullptr, y + static_cast<size_t>(bi) * M, M, K,
                                                              group_size, as_hip(stream), cus);
        if (st != ASDSL_OK) return st;
    }
    return ASDSL_OK;
}

extern "C" asdsl_status asdsl_gemv_q4_packed(const uint8_t* w_packed, const float* x, const float* scales,
                                             const float* biases, float* y, int M, int K, int group_size,
                                             int batch, asdsl_stream_t stream) {
    return asdsl_gemv_q4_packed_ws(w_packed, x, scales, biases, y, M, K, group_size, batch, nullptr, 0, stream);
}

extern "C" asdsl_status asdsl_gemv_q4_unpacked(const uint8_t* w, const float* x, const float* scales,
                                               const float* biases, float* y, int M, int K, int group_size,
                                               asdsl_stream_t stream) {
    if (check_affine(w, x, scales, y, M, K, group_size, 1, "gemv_q4_unpacked")) return ASDSL_ERR_INVALID_ARGUMENT;
    ASDSL_CHECK_ARG(biases != nullptr, "gemv_q4_unpacked: null pointer");
    ASDSL_CU_COUNT(cus);
    return launch_affine<8, true, false>(w, x, scales, biases, nullptr, y, M, K, group_size, as_hip(stream), cus);
}

extern "C" asdsl_status asdsl_gemv_q4_gs64_ws(const uint8_t* w_packed, const float* x, const float* scales, float* y,
                                              int rows, int cols, int batch, void* work, size_t work_bytes,
                                              asdsl_stream_t stream) {
    if (check_affine(w_packed, x, scales, y, rows, cols, 64, batch, "gemv_q4_avx2_gs64"))
        return ASDSL_ERR_INVALID_ARGUMENT;
    ASDSL_CU_COUNT(cus);
    if (batch > 1) {
        const asdsl_status st = affine_batch<false>(w_packed, scales, nullptr, x, y, rows, cols, batch, 64,
                                                    as_hip(stream), cus, "gemv_q4_avx2_gs64", work, work_bytes);
        if (st != ASDSL_ERR_UNSUPPORTED) return st;
    }
    for (int bi = 0; bi < batch; ++bi) {
        const asdsl_status st = launch_affine<4, false, false>(w_packed, x + static_cast<size_t>(bi) * cols, scales,
                                                               nullptr, nullptr, y + static_cast<size_t>(bi) * rows,
                                                               rows, cols, 64, as_hip(stream), cus);
        if (st != ASDSL_OK) return st;
    }
    return ASDSL_OK;
}

extern "C" asdsl_status asdsl_gemv_q4_gs64(const uint8_t* w_packed, const float* x, const float* scales, float* y,
                                           int rows, int cols, int batch, asdsl_stream_t stream) {
    return asdsl_gemv_q4_gs64_ws(w_packed, x, scales, y, rows, cols, batch, nullptr, 0, stream);
}

extern "C" asdsl_status asdsl_gemv_q8_unpacked(const uint8_t* w, const float* x, const float* scales,
                                               const float* biases, float* y, int M, int K, int group_size,
                                               asdsl_stream_t stream) {
    if (check_affine(w, x, scales, y, M, K, group_size, 1, "gemv_q8_unpacked")) return ASDSL_ERR_INVALID_ARGUMENT;
    ASDSL_CHECK_ARG(biases != nullptr, "gemv_q8_unpacked: null pointer");
    ASDSL_CU_COUNT(cus);
    return launch_affine<8, true, false>(w, x, scales, biases, nullptr, y, M, K, group_size, as_hip(stream), cus);
}

extern "C" asdsl_status asdsl_compute_bitmask(const float* x, uint32_t* bitmask, int K, float threshold,
                                              asdsl_stream_t stream) {
    ASDSL_CHECK_ARG(x && bitmask, "compute_bitmask: null pointer");
    ASDSL_CHECK_ARG(K > 0, "compute_bitmask: K must be positive");
    ASDSL_CU_COUNT(cus);
    const int grid = stream_grid(static_cast<long long>((K + 31) / 32) * 32, kThreads, 4, cus);
    return launch("compute_bitmask_kernel", compute_bitmask_kernel, dim3(grid), dim3(kThreads), 0, as_hip(stream), x,
                  bitmask, K, threshold);
}

extern "C" asdsl_status asdsl_gemv_sparse_unpacked(const uint8_t* w, const float* x, const float* scales,
                                                   const float* biases, const uint32_t* bitmask, float* y, int M,
                                                   int K, int group_size, asdsl_stream_t stream) {
    if (check_affine(w, x, scales, y, M, K, group_size, 1, "gemv_sparse_unpacked")) return ASDSL_ERR_INVALID_ARGUMENT;
    ASDSL_CHECK_ARG(biases && bitmask, "gemv_sparse_unpacked: null pointer");
    ASDSL_CU_COUNT(cus);
    return launch_affine<8, true, true>(w, x, scales, biases, bitmask, y, M, K, group_size, as_hip(stream), cus);
}

extern "C" asdsl_status asdsl_gemv_sparse_with_indices(const uint8_t* w, const float* x, const float* scales,
                                                       const float* biases, const int32_t* active_indices,
                                                       int n_active, float* y, int M, int K, int group_size,
                                                       uint32_t* work_mask, float* work_x, asdsl_stream_t stream) {
    if (check_affine(w, x, scales, y, M, K, group_size, 1, "gemv_sparse_with_indices"))
        return ASDSL_ERR_INVALID_ARGUMENT;
    ASDSL_CHECK_ARG(biases && work_mask && work_x, "gemv_sparse_with_indices: null pointer");
    ASDSL_CHECK_ARG(n_active >= 0 && (n_active == 0 || active_indices != nullptr),
                    "gemv_sparse_with_indices: invalid active index list");
    ASDSL_CHECK_ARG(reinterpret_cast<uintptr_t>(work_x) % 16 == 0, "gemv_sparse_with_indices: work_x must be 16-byte aligned");
    ASDSL_CU_COUNT(cus);
    hipStream_t s = as_hip(stream);
    const int nw = (K + 31) / 32;
    asdsl_status st = launch("fill_zero_kernel", fill_zero_kernel, dim3(stream_grid(nw, kThreads, 1, cus)),
                             dim3(kThreads), 0, s, work_mask, nw);
    if (st != ASDSL_OK) return st;
    st = launch("fill_zero_kernel", fill_zero_kernel, dim3(stream_grid(K, kThreads, 1, cus)), dim3(kThreads), 0, s,
                reinterpret_cast<uint32_t*>(work_x), K);
    if (st != ASDSL_OK) return st;
    if (n_active > 0) {
        st = launch("scatter_indices_kernel", scatter_indices_kernel, dim3(stream_grid(n_active, kThreads, 1, cus)),
                    dim3(kThreads), 0, s, active_indices, n_active, work_mask, work_x, x, K);
        if (st != ASDSL_OK) return st;
    }
    // work_x holds c_k*x_k on listed columns and 0 elsewhere; work_mask marks them
    return launch_affine<8, true, true>(w, work_x, scales, biases, work_mask, y, M, K, group_size, s, cus);
}

extern "C" asdsl_status asdsl_matmul_batch_q4_ws(const uint8_t* w_packed, const float* scales, const float* biases,
                                                 const float* X, float* Y, int M, int K, int B, int group_size,
                                                 void* work, size_t work_bytes, asdsl_stream_t stream) {
    if (check_affine(w_packed, X, scales, Y, M, K, group_size, B, "matmul_batch_q4")) return ASDSL_ERR_INVALID_ARGUMENT;
    ASDSL_CHECK_ARG(biases != nullptr, "matmul_batch_q4: null pointer");
    ASDSL_CHECK_ARG(B <= 64, "matmul_batch_q4: B must be <= 64 (the reference's accumulator limit)");
    ASDSL_CHECK_ARG(group_size % 16 == 0, "matmul_batch_q4: group_size must be a multiple of 16");
    ASDSL_CU_COUNT(cus);
    if (B > 1) {
        const asdsl_status st = affine_batch<true>(w_packed, scales, biases, X, Y, M, K, B, group_size,
                                                   as_hip(stream), cus, "matmul_batch_q4", work, work_bytes);
        if (st != ASDSL_ERR_UNSUPPORTED) return st;
    }
    for (int bi = 0; bi < B; ++bi) {
        const asdsl_status st = launch_affine<4, true, false>(w_packed, X + static_cast<size_t>(bi) * K, scales, biases,
                                                              nullptr, Y + static_cast<size_t>(bi) * M, M, K,
                                                              group_size, as_hip(stream), cus);
        if (st != ASDSL_OK) return st;
    }
    return ASDSL_OK;
}

extern "C" asdsl_status asdsl_matmul_batch_q4(const uint8_t* w_packed, const float* scales, const float* biases,
                                              const float* X, float* Y, int M, int K, int B, int group_size,
                                              asdsl_stream_t stream) {
    return asdsl_matmul_batch_q4_ws(w_packed, scales, biases, X, Y, M, K, B, group_size, nullptr, 0, stream);
}

extern "C" asdsl_status asdsl_gemm_q4_128_ws(const uint8_t* blocks, const float* X, float* Y, int out_features,
                                             int in_features, int group_size, int batch_size, void* work,
                                             size_t work_bytes, asdsl_stream_t stream) {
    ASDSL_CHECK_ARG(blocks && X && Y, "gemm_q4_128_q8_avx2: null pointer");
    ASDSL_CHECK_ARG(group_size == 128, "gemm_q4_128_q8_avx2: group_size must be 128");
    ASDSL_CHECK_ARG(out_features > 0 && in_features > 0 && in_features % 128 == 0,
                    "gemm_q4_128_q8_avx2: in_features must be a positive multiple of 128");
    ASDSL_CHECK_ARG(in_features <= kMaxAffineK, "gemm_q4_128_q8_avx2: in_features too large");
    ASDSL_CHECK_ARG(batch_size >= 1 && batch_size <= 64, "gemm_q4_128_q8_avx2: batch_size must be in [1, 64]");
    ASDSL_CHECK_ARG(reinterpret_cast<uintptr_t>(blocks) % 2 == 0 && reinterpret_cast<uintptr_t>(X) % 16 == 0,
                    "gemm_q4_128_q8_avx2: blocks must be 2-byte and X 16-byte aligned");
    ASDSL_CU_COUNT(cus);
    if (batch_size > 1) {
        const asdsl_status st = affine_batch<true, true>(blocks, nullptr, nullptr, X, Y, out_features, in_features,
                                                         batch_size, 128, as_hip(stream), cus, "gemm_q4_128_q8_avx2",
                                                         work, work_bytes);
        if (st != ASDSL_ERR_UNSUPPORTED) return st;
    }
    for (int bi = 0; bi < batch_size; ++bi) {
        const asdsl_status st = launch_affine<4, false, false, true>(
            blocks, X + static_cast<size_t>(bi) * in_features, nullptr, nullptr, nullptr,
            Y + static_cast<size_t>(bi) * out_features, out_features, in_features, 128, as_hip(stream), cus);
        if (st != ASDSL_OK) return st;
    }
    return ASDSL_OK;
}

extern "C" asdsl_status asdsl_gemm_q4_128(const uint8_t* blocks, const float* X, float* Y, int out_features,
                                          int in_features, int group_size, int batch_size, asdsl_stream_t stream) {
    return asdsl_gemm_q4_128_ws(blocks, X, Y, out_features, in_features, group_size, batch_size, nullptr, 0, stream);
}
