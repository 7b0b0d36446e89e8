// FATReLU-sparse down-projection over K-major (transposed) packed Q4 weights.
//
// Reference: sparse_down_proj_T (asdsl/kernels/native/gemv_sparse_avx2.cpp:273-418),
//   weights built by load_transposed_down_proj (experiments/phi4_cpu_run.py:2074-2185):
//   w_T[in_dim][out_dim/2] packed nibbles (low = even output), fp32 scale and
//   bias per (input row, out group).  For each listed row r with x[r] != 0
//   (and 0 <= r < in_dim):
//       y[o] += fma(q[r][o], s[r][o/gs] * x[r], b[r][o/gs] * x[r])
//   A row listed twice adds twice.  Only listed rows are read: at 80 % zeros
//   the kernel streams a fifth of the matrix.
//
// Pass 1: P workgroups each take a contiguous chunk of the active list; a
//   wave walks rows of the chunk (two rows' loads in flight), its lanes owning
//   fixed 32-output units (lane l: units l, l+64, ...), so the per-lane
//   accumulators stay in registers.  Waves add their partial y in LDS in a
//   fixed order and the workgroup writes work[p][:].
// Pass 2: y[o] = sum_p work[p][o] in order p = 0..P-1.
// No atomics: results are reproducible run to run (the reference's own
// per-thread buffers race across pool chunks, gemv_sparse_avx2.cpp:297-300).
#include "abi_util.hpp"
#include "device_common.hpp"

namespace asdsl {
namespace {

constexpr int kWaves = 8;
constexpr int kMaxSlice = 4096;   // outputs per launch: 64 lanes x 2 units x 32
constexpr int kUnitsPerLane = kMaxSlice / (32 * kWave);

__global__ __launch_bounds__(kWaves * kWave) void sparse_down_pass1(
    const uint8_t* __restrict__ wT, const float* __restrict__ sT, const float* __restrict__ bT,
    const float* __restrict__ x, const int32_t* __restrict__ rows, int n, float* __restrict__ work,
    int in_dim, int out_dim, int gs, int o_off, int o_len, int per_wg) {
    extern __shared__ __align__(16) float part[];  // [kWaves][o_len]
    const int lane = static_cast<int>(threadIdx.x) & (kWave - 1);
    const int wave = static_cast<int>(threadIdx.x) >> 6;
    const int G = out_dim / gs;
    const int units = o_len >> 5;
    const int a0 = static_cast<int>(blockIdx.x) * per_wg;
    const int a1 = min(a0 + per_wg, n);

    float acc[kUnitsPerLane][32];
#pragma unroll
    for (int i = 0; i < kUnitsPerLane; ++i)
#pragma unroll
        for (int e = 0; e < 32; ++e) acc[i][e] = 0.0f;

    for (int a = a0 + wave; a < a1; a += kWaves) {
        const int r = rows[a];
        if (r < 0 || r >= in_dim) continue;  // skipped, as the reference does
        const float xv = x[r];
        if (xv == 0.0f) continue;
        const uint8_t* rp = wT + static_cast<size_t>(r) * (out_dim / 2) + o_off / 2;
        const float* sp = sT + static_cast<size_t>(r) * G;
        const float* bp = bT + static_cast<size_t>(r) * G;
#pragma unroll
        for (int i = 0; i < kUnitsPerLane; ++i) {
            const int u = lane + i * kWave;
            if (u < units) {
                const uint4 w = load_stream16(reinterpret_cast<const uint4*>(rp) + u);
                const uint32_t wv[4] = {w.x, w.y, w.z, w.w};
#pragma unroll
                for (int dw = 0; dw < 4; ++dw) {  // 8 outputs per dword, one group (8 | gs)
                    const int g = (o_off + u * 32 + dw * 8) / gs;
                    const float s = sp[g] * xv;
                    const float b = bp[g] * xv;
#pragma unroll
                    for (int e = 0; e < 8; ++e) {
                        const float q = static_cast<float>((wv[dw] >> (4 * e)) & 0xFu);
                        acc[i][dw * 8 + e] += fmaf(q, s, b);
                    }
                }
            }
        }
    }
    // fixed-order combine of the waves' partials
#pragma unroll
    for (int i = 0; i < kUnitsPerLane; ++i) {
        const int u = lane + i * kWave;
        if (u < units) {
            float* dst = part + wave * o_len + u * 32;
#pragma unroll
            for (int e = 0; e < 32; e += 4)
                *reinterpret_cast<float4*>(dst + e) = make_float4(acc[i][e], acc[i][e + 1], acc[i][e + 2], acc[i][e + 3]);
        }
    }
    __syncthreads();
    float* out = work + static_cast<size_t>(blockIdx.x) * o_len;
    for (int o = static_cast<int>(threadIdx.x); o < o_len; o += kWaves * kWave) {
        float sum = part[o];
        for (int v = 1; v < kWaves; ++v) sum += part[v * o_len + o];
        out[o] = sum;
    }
}

__global__ __launch_bounds__(256) void sparse_down_pass2(const float* __restrict__ work, int P, float* __restrict__ y,
                                                        int o_off, int o_len) {
    const int o = static_cast<int>(blockIdx.x) * 256 + static_cast<int>(threadIdx.x);
    if (o >= o_len) return;
    float sum = 0.0f;
    for (int p = 0; p < P; ++p) sum += work[static_cast<size_t>(p) * o_len + o];
    y[o_off + o] = sum;
}

// Workgroups for n listed rows: enough to keep ~8 rows per wave in flight
// territory without multiplying the partial traffic (P * o_len * 4 bytes).
int sparse_down_wgs(int n, int cus) {
    int p = (n + kWaves * 4 - 1) / (kWaves * 4);  // ~4 rows per wave
    const int cap = cus / 2 > 0 ? cus / 2 : 1;
    if (p > cap) p = cap;
    return p < 1 ? 1 : p;
}

}  // namespace
}  // namespace asdsl

using namespace asdsl;

extern "C" size_t asdsl_sparse_down_proj_T_workspace_bytes(int n_active, int out_dim) {
    const int cus = cu_count_current();
    const int P = sparse_down_wgs(n_active > 0 ? n_active : 1, cus > 0 ? cus : 256);
    const int slice = out_dim < kMaxSlice ? out_dim : kMaxSlice;
    return static_cast<size_t>(P) * static_cast<size_t>(slice > 0 ? slice : 1) * sizeof(float);
}

extern "C" asdsl_status asdsl_sparse_down_proj_T(const uint8_t* w_T_packed, const float* scales_T,
                                                 const float* biases_T, const float* sparse_x,
                                                 const int32_t* active_rows, int n_active, float* y, int in_dim,
                                                 int out_dim, int group_size, float* work, size_t work_bytes,
                                                 asdsl_stream_t stream) {
    ASDSL_CHECK_ARG(in_dim > 0 && out_dim > 0 && group_size > 0, "in_dim, out_dim, group_size must be positive");
    ASDSL_CHECK_ARG(out_dim % group_size == 0, "out_dim must be divisible by group_size");
    ASDSL_CHECK_ARG(w_T_packed && scales_T && biases_T && sparse_x && y, "sparse_down_proj_T: null pointer");
    ASDSL_CHECK_ARG(n_active >= 0 && (n_active == 0 || active_rows != nullptr),
                    "sparse_down_proj_T: invalid active row list");
    ASDSL_CHECK_ARG(out_dim % 32 == 0 && group_size % 8 == 0,
                    "sparse_down_proj_T: out_dim must be a multiple of 32 and group_size of 8");
    ASDSL_CHECK_ARG(reinterpret_cast<uintptr_t>(w_T_packed) % 16 == 0 && (out_dim / 2) % 16 == 0,
                    "sparse_down_proj_T: weight rows must be 16-byte aligned");
    ASDSL_CU_COUNT(cus);
    hipStream_t s = as_hip(stream);
    const int P = sparse_down_wgs(n_active > 0 ? n_active : 1, cus);
    const int per_wg = (n_active + P - 1) / P > 0 ? (n_active + P - 1) / P : 1;
    for (int o_off = 0; o_off < out_dim; o_off += kMaxSlice) {
        const int o_len = out_dim - o_off < kMaxSlice ? out_dim - o_off : kMaxSlice;
        ASDSL_CHECK_ARG(work != nullptr && work_bytes >= static_cast<size_t>(P) * o_len * sizeof(float),
                        "sparse_down_proj_T: workspace too small (asdsl_sparse_down_proj_T_workspace_bytes)");
        const size_t lds = static_cast<size_t>(kWaves) * o_len * sizeof(float);
        asdsl_status st = launch("sparse_down_pass1", sparse_down_pass1, dim3(P), dim3(kWaves * kWave), lds, s,
                                 w_T_packed, scales_T, biases_T, sparse_x, active_rows, n_active, work, in_dim,
                                 out_dim, group_size, o_off, o_len, per_wg);
        if (st != ASDSL_OK) return st;
        st = launch("sparse_down_pass2", sparse_down_pass2, dim3((o_len + 255) / 256), dim3(256), 0, s,
                    static_cast<const float*>(work), P, y, o_off, o_len);
        if (st != ASDSL_OK) return st;
    }
    return ASDSL_OK;
}
