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
// in passes of NU.  The activation sits in LDS as fp32 (masked), with the sum
// of each unit's 32 values next to it; per unit a lane adds
//   s_g * dot_unit + b_g * sum_unit
// (the reference's per-group terms split per unit).  Requires group_size % 32
// == 0; other multiples of 8 take affine_gemv_generic (one wave per row).
#include "abi_util.hpp"
#include "device_common.hpp"

namespace asdsl {
namespace {

constexpr int kThreads = 256;

// LDS: x~ (K floats) then per-unit sums (K/32 floats).
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
            reinterpret_cast<float4*>(xs)[c] = v;
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
    float* usum = lds_f + K;

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

    stage_x<WAVES, MASKED>(x, mask, xs, usum, K);
    __syncthreads();

    for (int tile = static_cast<int>(blockIdx.x); tile < ntiles; tile += static_cast<int>(gridDim.x)) {
        const int row = min(tile * rpt + wave * rpw + rin, M - 1);
        const uint8_t* rb = w + static_cast<size_t>(row) * row_bytes;
        const float* srow = Q128 ? nullptr : scales + static_cast<size_t>(row) * G;
        const float* brow = BIAS ? biases + static_cast<size_t>(row) * G : nullptr;
        float acc = 0.0f;
        for (int pass = 0; pass < npass; ++pass) {
            uint4 wu[NU][BITS / 4];
            bool live[NU];
#pragma unroll
            for (int i = 0; i < NU; ++i) {
                const int t = pass * per_pass + j + i * lpr;
                live[i] = t < U && (!MASKED || mask[t] != 0u);
                if (live[i]) {
                    if (Q128) {
                        const u32x4_a2 v = __builtin_nontemporal_load(
                            reinterpret_cast<const u32x4_a2*>(rb + static_cast<size_t>(t / 4) * 66 + 2 + 16 * (t % 4)));
                        wu[i][0] = make_uint4(v.x, v.y, v.z, v.w);
                    } else {
#pragma unroll
                        for (int h = 0; h < BITS / 4; ++h)
                            wu[i][h] = load_stream16(reinterpret_cast<const uint4*>(rb + static_cast<size_t>(t) * UB) + h);
                    }
                }
            }
#pragma unroll
            for (int i = 0; i < NU; ++i) {
                const int t = pass * per_pass + j + i * lpr;
                if (live[i]) {
                    const float d = unit_dot_f32<BITS>(wu[i], xs + t * 32);
                    if (Q128) {
                        const float ws = half_bits_to_float(*reinterpret_cast<const uint16_t*>(rb + static_cast<size_t>(t / 4) * 66));
                        acc = fmaf(ws, d, acc);
                        acc = fmaf(-8.0f * ws, usum[t], acc);
                    } else {
                        const int g = t / upg;
                        acc = fmaf(srow[g], d, acc);
                        if (BIAS) acc = fmaf(brow[g], usum[t], acc);
                    }
                }
            }
        }
        acc = group_sum<16>(acc);
        if (lpr >= 32) acc += swz_xor16(acc);
        if (lpr >= 64) acc += __shfl_xor(acc, 32, kWave);
        const int r = tile * rpt + wave * rpw + rin;
        if (j == 0 && r < M) y[r] = acc;
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
    const int cap = cus * 4;
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
    const size_t lds = static_cast<size_t>(K) * 4 + static_cast<size_t>(K / 32) * 4;
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

// LDS budget of the fast path: K*4 + K/8 bytes.
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

extern "C" asdsl_status asdsl_gemv_q4_packed(const uint8_t* w_packed, const float* x, const float* scales,
                                             const float* biases, float* y, int M, int K, int group_size,
                                             int batch, asdsl_stream_t stream) {
    if (check_affine(w_packed, x, scales, y, M, K, group_size, batch, "gemv_q4_packed"))
        return ASDSL_ERR_INVALID_ARGUMENT;
    ASDSL_CHECK_ARG(biases != nullptr, "gemv_q4_packed: null pointer");
    ASDSL_CHECK_ARG(group_size % 16 == 0, "gemv_q4_packed: group_size must be a multiple of 16");
    ASDSL_CU_COUNT(cus);
    for (int bi = 0; bi < batch; ++bi) {
        const asdsl_status st = launch_affine<4, true, false>(w_packed, x + static_cast<size_t>(bi) * K, scales, biases,
                                                              nullptr, y + static_cast<size_t>(bi) * M, M, K,
                                                              group_size, as_hip(stream), cus);
        if (st != ASDSL_OK) return st;
    }
    return ASDSL_OK;
}

extern "C" asdsl_status asdsl_gemv_q4_unpacked(const uint8_t* w, const float* x, const float* scales,
                                               const float* biases, float* y, int M, int K, int group_size,
                                               asdsl_stream_t stream) {
    if (check_affine(w, x, scales, y, M, K, group_size, 1, "gemv_q4_unpacked")) return ASDSL_ERR_INVALID_ARGUMENT;
    ASDSL_CHECK_ARG(biases != nullptr, "gemv_q4_unpacked: null pointer");
    ASDSL_CU_COUNT(cus);
    return launch_affine<8, true, false>(w, x, scales, biases, nullptr, y, M, K, group_size, as_hip(stream), cus);
}

extern "C" asdsl_status asdsl_gemv_q4_gs64(const uint8_t* w_packed, const float* x, const float* scales, float* y,
                                           int rows, int cols, int batch, asdsl_stream_t stream) {
    if (check_affine(w_packed, x, scales, y, rows, cols, 64, batch, "gemv_q4_avx2_gs64"))
        return ASDSL_ERR_INVALID_ARGUMENT;
    ASDSL_CU_COUNT(cus);
    for (int bi = 0; bi < batch; ++bi) {
        const asdsl_status st = launch_affine<4, false, false>(w_packed, x + static_cast<size_t>(bi) * cols, scales,
                                                               nullptr, nullptr, y + static_cast<size_t>(bi) * rows,
                                                               rows, cols, 64, as_hip(stream), cus);
        if (st != ASDSL_OK) return st;
    }
    return ASDSL_OK;
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

extern "C" asdsl_status asdsl_matmul_batch_q4(const uint8_t* w_packed, const float* scales, const float* biases,
                                              const float* X, float* Y, int M, int K, int B, int group_size,
                                              asdsl_stream_t stream) {
    if (check_affine(w_packed, X, scales, Y, M, K, group_size, B, "matmul_batch_q4")) return ASDSL_ERR_INVALID_ARGUMENT;
    ASDSL_CHECK_ARG(biases != nullptr, "matmul_batch_q4: null pointer");
    ASDSL_CHECK_ARG(B <= 64, "matmul_batch_q4: B must be <= 64 (the reference's accumulator limit)");
    ASDSL_CHECK_ARG(group_size % 16 == 0, "matmul_batch_q4: group_size must be a multiple of 16");
    ASDSL_CU_COUNT(cus);
    for (int bi = 0; bi < B; ++bi) {
        const asdsl_status st = launch_affine<4, true, false>(w_packed, X + static_cast<size_t>(bi) * K, scales, biases,
                                                              nullptr, Y + static_cast<size_t>(bi) * M, M, K,
                                                              group_size, as_hip(stream), cus);
        if (st != ASDSL_OK) return st;
    }
    return ASDSL_OK;
}

extern "C" asdsl_status asdsl_gemm_q4_128(const uint8_t* blocks, const float* X, float* Y, int out_features,
                                          int in_features, int group_size, int batch_size, asdsl_stream_t stream) {
    ASDSL_CHECK_ARG(blocks && X && Y, "gemm_q4_128_q8_avx2: null pointer");
    ASDSL_CHECK_ARG(group_size == 128, "gemm_q4_128_q8_avx2: group_size must be 128");
    ASDSL_CHECK_ARG(out_features > 0 && in_features > 0 && in_features % 128 == 0,
                    "gemm_q4_128_q8_avx2: in_features must be a positive multiple of 128");
    ASDSL_CHECK_ARG(in_features <= kMaxAffineK, "gemm_q4_128_q8_avx2: in_features too large");
    ASDSL_CHECK_ARG(batch_size >= 1 && batch_size <= 64, "gemm_q4_128_q8_avx2: batch_size must be in [1, 64]");
    ASDSL_CHECK_ARG(reinterpret_cast<uintptr_t>(blocks) % 2 == 0 && reinterpret_cast<uintptr_t>(X) % 16 == 0,
                    "gemm_q4_128_q8_avx2: blocks must be 2-byte and X 16-byte aligned");
    ASDSL_CU_COUNT(cus);
    for (int bi = 0; bi < batch_size; ++bi) {
        const asdsl_status st = launch_affine<4, false, false, true>(
            blocks, X + static_cast<size_t>(bi) * in_features, nullptr, nullptr, nullptr,
            Y + static_cast<size_t>(bi) * out_features, out_features, in_features, 128, as_hip(stream), cus);
        if (st != ASDSL_OK) return st;
    }
    return ASDSL_OK;
}
