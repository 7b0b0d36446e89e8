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
// The active list is cut into P contiguous parts and the outputs into slices
// of 256; workgroup (slice, part) walks its part's rows for its slice.  Per
// listed row a workgroup touches one 128-byte nibble line and one scale and
// one bias segment, so the cost is set by rows per workgroup (scattered line
// lookups in the compute unit's cache), and splitting the list is what spreads
// it over the chip.  Eight lanes serve a row (16 bytes = 32 outputs each), a
// wave load covers 8 rows and every lane requests its 4 rows before using any.
// Each lane keeps its 32 sums in registers; the 8 rows of a wave fold with DPP
// and lane swizzles, the 4 waves through LDS in fixed order.
//   P == 1: the workgroup writes y.
//   P > 1:  it writes part[p][slice], and a second launch adds the P parts of
//           each output in order p = 0..P-1.
// A last-arriving-workgroup reduction in one launch was measured 2-5x slower:
// its device-scope fences cost more than the second launch.  No atomics, so
// results are reproducible run to run on a device (P follows n and the CU
// count).  The reference's own per-thread buffers race across pool chunks
// (gemv_sparse_avx2.cpp:297-300).
#include <mutex>

#include "abi_util.hpp"
#include "device_common.hpp"

namespace asdsl {

ASDSL_TIMELINE_BUFFER

namespace {

constexpr int kWaves = 4;
constexpr int kLanesPerRow = 8;                    // 8 x 16 bytes = 256 outputs
constexpr int kSliceOut = kLanesPerRow * 32;
constexpr int kRowsPerWave = kWave / kLanesPerRow;
constexpr int kDepth = 4;                          // rows per lane in flight
constexpr int kXcds = 8;                           // MI355X: workgroup i runs on XCD i % 8
constexpr int kMaxParts = 32;
constexpr int kMinRowsPerPart = 32;

// WIDE: group_size % 32 == 0, so a lane's 32 outputs share one (scale, bias)
// and a row costs the lane one load of each; otherwise one per 8 outputs.
template <bool WIDE>
__global__ __launch_bounds__(kWaves * kWave) void sparse_down_kernel(
    const uint8_t* __restrict__ wT, const float* __restrict__ sT, const float* __restrict__ bT,
    const float* __restrict__ x, const int32_t* __restrict__ rows, int n, float* __restrict__ out, int in_dim,
    int out_dim, int gs, int nslices, int nparts, int per_part) {
    __shared__ __align__(16) float red[kWaves][kSliceOut];
    // Consecutive tiles t run on one XCD, so neighbouring slices (which share
    // scale lines) of one part meet in one L2.  The grid is a multiple of 8.
    const int bid = static_cast<int>(blockIdx.x);
    const int per_xcd = static_cast<int>(gridDim.x) / kXcds;
    const int t = (bid % kXcds) * per_xcd + bid / kXcds;
    if (t >= nslices * nparts) return;  // padding workgroup: the whole workgroup leaves
    ASDSL_TIMELINE_STAMP(5, t, 0);
    const int slice = t % nslices;
    const int p = t / nslices;

    const int lane = static_cast<int>(threadIdx.x) & (kWave - 1);
    const int wave = static_cast<int>(threadIdx.x) >> 6;
    const int sub = lane / kLanesPerRow;  // row within the wave load
    const int j = lane % kLanesPerRow;
    const int o0 = slice * kSliceOut + j * 32;  // this lane's first output
    const bool live_out = o0 < out_dim;
    const int G = out_dim / gs;
    const size_t row_bytes = static_cast<size_t>(out_dim / 2);
    const int a_begin = p * per_part;
    const int a_end = min(a_begin + per_part, n);

    float acc[32];
#pragma unroll
    for (int e = 0; e < 32; ++e) acc[e] = 0.0f;

    constexpr int stride = kWaves * kRowsPerWave;
    for (int a0 = a_begin + wave * kRowsPerWave + sub; a0 < a_end; a0 += kDepth * stride) {
        int r[kDepth];
        float xv[kDepth];
        uint4 w[kDepth];
        float s[kDepth][4], b[kDepth][4];
        bool ok[kDepth];
#pragma unroll
        for (int d = 0; d < kDepth; ++d) {
            const int a = a0 + d * stride;
            r[d] = a < a_end ? rows[a] : -1;
        }
#pragma unroll
        for (int d = 0; d < kDepth; ++d) {
            ok[d] = live_out && r[d] >= 0 && r[d] < in_dim;
            const int rr = ok[d] ? r[d] : 0;  // in-bounds row for the loads below
            const int oo = live_out ? o0 : 0;
            xv[d] = x[rr];
            w[d] = load_stream16(reinterpret_cast<const uint4*>(wT + static_cast<size_t>(rr) * row_bytes + oo / 2));
            if (WIDE) {
                const size_t at = static_cast<size_t>(rr) * G + oo / gs;
                s[d][0] = sT[at];
                b[d][0] = bT[at];
#pragma unroll
                for (int dw = 1; dw < 4; ++dw) {
                    s[d][dw] = s[d][0];
                    b[d][dw] = b[d][0];
                }
            } else {
#pragma unroll
                for (int dw = 0; dw < 4; ++dw) {  // 8 outputs per dword lie in one group (8 | gs)
                    const size_t at = static_cast<size_t>(rr) * G + (oo + dw * 8) / gs;
                    s[d][dw] = sT[at];
                    b[d][dw] = bT[at];
                }
            }
        }
        ASDSL_TIMELINE_STAMP(5, t, 1);  // the row indices arrived, the rows requested
#pragma unroll
        for (int d = 0; d < kDepth; ++d) {
            if (ok[d] && xv[d] != 0.0f) {
                const uint32_t wv[4] = {w[d].x, w[d].y, w[d].z, w[d].w};
#pragma unroll
                for (int dw = 0; dw < 4; ++dw) {
                    const float sx = s[d][dw] * xv[d];
                    const float bx = b[d][dw] * xv[d];
#pragma unroll
                    for (int e = 0; e < 8; ++e)
                        acc[dw * 8 + e] += fmaf(static_cast<float>((wv[dw] >> (4 * e)) & 0xFu), sx, bx);
                }
            }
        }
    }

    ASDSL_TIMELINE_STAMP(5, t, 2);  // the rows arrived and were accumulated
    // fold the 8 rows of a wave load: lanes that agree in bits 0-2 (the unit j)
#pragma unroll
    for (int e = 0; e < 32; ++e) {
        float v = acc[e];
        v += dpp<kDppRowRor8>(v);       // lane bit 3
        v += swz_xor16(v);              // bit 4
        v += __shfl_xor(v, 32, kWave);  // bit 5
        acc[e] = v;
    }
    ASDSL_TIMELINE_STAMP(5, t, 3);
    if (sub == 0) {
        float* dst = &red[wave][j * 32];
#pragma unroll
        for (int e = 0; e < 32; e += 4)
            *reinterpret_cast<float4*>(dst + e) = make_float4(acc[e], acc[e + 1], acc[e + 2], acc[e + 3]);
    }
    __syncthreads();
    for (int o = static_cast<int>(threadIdx.x); o < kSliceOut; o += kWaves * kWave) {
        const int og = slice * kSliceOut + o;
        if (og < out_dim) {
            float sum = red[0][o];
#pragma unroll
            for (int v = 1; v < kWaves; ++v) sum += red[v][o];
            out[static_cast<size_t>(p) * out_dim + og] = sum;
        }
    }
    ASDSL_TIMELINE_STAMP(5, t, 4);
}

// y[o] = part[0][o] + part[1][o] + ... + part[P-1][o], in that order.  All P
// loads are issued before the first add, so the kernel waits on memory once.
__global__ __launch_bounds__(64) void sparse_down_sum_parts(const float* __restrict__ part, float* __restrict__ y,
                                                            int out_dim, int nparts) {
    const int o = static_cast<int>(blockIdx.x) * 64 + static_cast<int>(threadIdx.x);
    if (o >= out_dim) return;
    float v[kMaxParts];
#pragma unroll
    for (int p = 0; p < kMaxParts; ++p) v[p] = p < nparts ? part[static_cast<size_t>(p) * out_dim + o] : 0.0f;
    float sum = v[0];
#pragma unroll
    for (int p = 1; p < kMaxParts; ++p)
        if (p < nparts) sum += v[p];
    y[o] = sum;
}

}  // namespace

#ifdef ASDSL_WG_TIMELINE
asdsl_status timeline_set_sparse(void* buf) {
    const hipError_t e = hipMemcpyToSymbol(HIP_SYMBOL(g_timeline), &buf, sizeof(buf));
    if (e != hipSuccess) {
        set_error("timeline: %s", hipGetErrorString(e));
        return ASDSL_ERR_HIP;
    }
    return ASDSL_OK;
}
#endif
}  // namespace asdsl

using namespace asdsl;

namespace {

// Partial rows of the no-allocation entry point: at most kMaxParts rows of
// kNoAllocMaxOut outputs (2 MiB), one array per device for the life of the
// process.  In host code `g_sparse_scratch` names a host-side stand-in, not
// device memory: kernels get the per-device address that
// hipGetSymbolAddress returns (sparse_scratch_ptr).
constexpr int kNoAllocMaxOut = 16384;
static __device__ __align__(256) float g_sparse_scratch[kMaxParts * kNoAllocMaxOut];

struct ScratchSlot {
    std::once_flag once;
    void* ptr = nullptr;
    hipError_t err = hipSuccess;
};
ScratchSlot g_scratch_slots[64];

// Device address of this device's g_sparse_scratch, looked up once per device
// (with that device current) on its first use.
asdsl_status sparse_scratch_ptr(float** out) {
    int dev = -1;
    const hipError_t e = hipGetDevice(&dev);
    if (e != hipSuccess || dev < 0 || dev >= 64) {
        set_error("sparse_down_proj_T_noalloc: no usable HIP device: %s", hipGetErrorString(e));
        return ASDSL_ERR_HIP;
    }
    ScratchSlot& slot = g_scratch_slots[dev];
    std::call_once(slot.once, [&] {
        void* p = nullptr;
        slot.err = hipGetSymbolAddress(&p, HIP_SYMBOL(g_sparse_scratch));
        slot.ptr = slot.err == hipSuccess ? p : nullptr;
    });
    if (slot.err != hipSuccess || slot.ptr == nullptr) {
        set_error("sparse_down_proj_T_noalloc: hipGetSymbolAddress failed: %s", hipGetErrorString(slot.err));
        return ASDSL_ERR_HIP;
    }
    *out = static_cast<float*>(slot.ptr);
    return ASDSL_OK;
}

struct SparsePlan {
    int nslices, nparts, per_part, grid;
};

SparsePlan plan_sparse_down(int n_active, int out_dim, int cus) {
    SparsePlan p{};
    p.nslices = (out_dim + kSliceOut - 1) / kSliceOut;
    // about 3 workgroups per 4 compute units, at least 32 rows per part
    int nparts = (3 * cus / 4) / p.nslices;
    nparts = min(nparts, (n_active + kMinRowsPerPart - 1) / kMinRowsPerPart);
    p.nparts = max(1, min(nparts, kMaxParts));
    p.per_part = max(1, (n_active + p.nparts - 1) / p.nparts);
    const int tiles = p.nslices * p.nparts;
    p.grid = (tiles + kXcds - 1) / kXcds * kXcds;
    return p;
}

asdsl_status check_sparse_down(const uint8_t* w_T_packed, const float* scales_T, const float* biases_T,
                               const float* sparse_x, const int32_t* active_rows, int n_active, const float* y,
                               int in_dim, int out_dim, int group_size) {
    ASDSL_CHECK_ARG(in_dim > 0 && out_dim > 0 && group_size > 0, "in_dim, out_dim, group_size must be positive");
    ASDSL_CHECK_ARG(out_dim % group_size == 0, "out_dim must be divisible by group_size");
    ASDSL_CHECK_ARG(w_T_packed && scales_T && biases_T && sparse_x && y, "sparse_down_proj_T: null pointer");
    ASDSL_CHECK_ARG(n_active >= 0 && (n_active == 0 || active_rows != nullptr),
                    "sparse_down_proj_T: invalid active row list");
    ASDSL_CHECK_ARG(out_dim % 32 == 0 && group_size % 8 == 0,
                    "sparse_down_proj_T: out_dim must be a multiple of 32 and group_size of 8");
    ASDSL_CHECK_ARG(reinterpret_cast<uintptr_t>(w_T_packed) % 16 == 0,
                    "sparse_down_proj_T: w_T_packed must be 16-byte aligned");
    return ASDSL_OK;
}

// The two launches; `part` (nparts x out_dim floats) is only touched when
// the plan has more than one part.
asdsl_status run_sparse_down(const SparsePlan& p, const uint8_t* w_T_packed, const float* scales_T,
                             const float* biases_T, const float* sparse_x, const int32_t* active_rows, int n_active,
                             float* y, float* part, int in_dim, int out_dim, int group_size, hipStream_t s) {
    auto kernel = group_size % 32 == 0 ? sparse_down_kernel<true> : sparse_down_kernel<false>;
    if (p.nparts == 1)
        return launch("sparse_down_kernel", kernel, dim3(p.grid), dim3(kWaves * kWave), 0, s, w_T_packed, scales_T,
                      biases_T, sparse_x, active_rows, n_active, y, in_dim, out_dim, group_size, p.nslices, p.nparts,
                      p.per_part);
    const asdsl_status st1 = launch("sparse_down_kernel", kernel, dim3(p.grid), dim3(kWaves * kWave), 0, s,
                                    w_T_packed, scales_T, biases_T, sparse_x, active_rows, n_active, part, in_dim,
                                    out_dim, group_size, p.nslices, p.nparts, p.per_part);
    if (st1 != ASDSL_OK) return st1;
    return launch("sparse_down_sum_parts", sparse_down_sum_parts, dim3((out_dim + 63) / 64), dim3(64), 0, s,
                  static_cast<const float*>(part), y, out_dim, p.nparts);
}

}  // namespace

extern "C" size_t asdsl_sparse_down_work_bytes(int out_dim) {
    return out_dim > 0 ? static_cast<size_t>(kMaxParts) * out_dim * sizeof(float) : 0;
}

extern "C" asdsl_status asdsl_sparse_down_proj_T_ws(const uint8_t* w_T_packed, const float* scales_T,
                                                    const float* biases_T, const float* sparse_x,
                                                    const int32_t* active_rows, int n_active, float* y, int in_dim,
                                                    int out_dim, int group_size, void* work, size_t work_bytes,
                                                    asdsl_stream_t stream) {
    const asdsl_status cs = check_sparse_down(w_T_packed, scales_T, biases_T, sparse_x, active_rows, n_active, y,
                                              in_dim, out_dim, group_size);
    if (cs != ASDSL_OK) return cs;
    ASDSL_CHECK_ARG(work == nullptr || work_bytes >= asdsl_sparse_down_work_bytes(out_dim),
                    "sparse_down_proj_T: work buffer of %zu bytes, asdsl_sparse_down_work_bytes gives %zu", work_bytes,
                    asdsl_sparse_down_work_bytes(out_dim));
    ASDSL_CU_COUNT(cus);
    const SparsePlan p = plan_sparse_down(n_active, out_dim, cus);
    hipStream_t s = as_hip(stream);
    void* part = nullptr;
    if (p.nparts > 1) {
        const asdsl_status st = work_buffer(s, work, work_bytes, static_cast<size_t>(p.nparts) * out_dim * sizeof(float),
                                            &part, "sparse_down_proj_T");
        if (st != ASDSL_OK) return st;
    }
    return run_sparse_down(p, w_T_packed, scales_T, biases_T, sparse_x, active_rows, n_active, y,
                           static_cast<float*>(part), in_dim, out_dim, group_size, s);
}

extern "C" asdsl_status asdsl_sparse_down_proj_T(const uint8_t* w_T_packed, const float* scales_T,
                                                 const float* biases_T, const float* sparse_x,
                                                 const int32_t* active_rows, int n_active, float* y, int in_dim,
                                                 int out_dim, int group_size, asdsl_stream_t stream) {
    return asdsl_sparse_down_proj_T_ws(w_T_packed, scales_T, biases_T, sparse_x, active_rows, n_active, y, in_dim,
                                       out_dim, group_size, nullptr, 0, stream);
}

extern "C" asdsl_status asdsl_sparse_down_proj_T_noalloc(const uint8_t* w_T_packed, const float* scales_T,
                                                         const float* biases_T, const float* sparse_x,
                                                         const int32_t* active_rows, int n_active, float* y,
                                                         int in_dim, int out_dim, int group_size,
                                                         asdsl_stream_t stream) {
    const asdsl_status cs = check_sparse_down(w_T_packed, scales_T, biases_T, sparse_x, active_rows, n_active, y,
                                              in_dim, out_dim, group_size);
    if (cs != ASDSL_OK) return cs;
    ASDSL_CHECK_ARG(out_dim <= kNoAllocMaxOut, "sparse_down_proj_T_noalloc: out_dim %d exceeds the %d outputs of its "
                    "device scratch array", out_dim, kNoAllocMaxOut);
    ASDSL_CU_COUNT(cus);
    const SparsePlan p = plan_sparse_down(n_active, out_dim, cus);
    float* part = nullptr;
    if (p.nparts > 1) {
        const asdsl_status st = sparse_scratch_ptr(&part);
        if (st != ASDSL_OK) return st;
    }
    return run_sparse_down(p, w_T_packed, scales_T, biases_T, sparse_x, active_rows, n_active, y, part, in_dim,
                           out_dim, group_size, as_hip(stream));
}
