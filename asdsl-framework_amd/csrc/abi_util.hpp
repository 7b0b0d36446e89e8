// Host-side helpers for the C ABI: per-thread error text, argument checks,
// launch checks and the cached device shape used to size grids.
#pragma once

#include <hip/hip_ext.h>
#include <hip/hip_runtime.h>

#include <tuple>
#include <utility>

#include "asdsl_hip.h"

namespace asdsl {

void set_error(const char* fmt, ...) __attribute__((format(printf, 1, 2)));
void clear_error();

// Compute units of the current device; -1 (error text set) when no device.
int cu_count_current();

// Checks hipGetLastError() after a launch; maps a failure to ASDSL_ERR_HIP.
asdsl_status launch_status(const char* what);

inline hipStream_t as_hip(asdsl_stream_t s) { return reinterpret_cast<hipStream_t>(s); }

// Timing events of one launch.
struct LaunchEvents {
    hipEvent_t start = nullptr;
    hipEvent_t stop = nullptr;
};

// Stage label of the calling thread's launches (a string literal), kept by the
// stage recorder (asdsl_profile_stages_begin/_end) beside each launch's
// events; a launch outside any StageScope is recorded under its kernel name.
extern thread_local const char* g_stage;
struct StageScope {
    const char* prev;
    explicit StageScope(const char* label) : prev(g_stage) { g_stage = label; }
    ~StageScope() { g_stage = prev; }
    StageScope(const StageScope&) = delete;
    StageScope& operator=(const StageScope&) = delete;
};

// Events for the calling thread's next launch: the pair armed by
// asdsl_profile_next_launch (returned and cleared), else, while the stage
// recorder is armed, a pair of its own recorded under the current stage label
// (ASDSL_ERR_UNSUPPORTED on a stream under graph capture, ASDSL_ERR_INVALID_ARGUMENT
// past its launch limit), else none.
asdsl_status take_launch_events(const char* what, hipStream_t stream, LaunchEvents* ev);

// Launches `kernel` on `stream`.  With events the launch goes through
// hipExtLaunchKernel, which records them as part of the kernel's own dispatch
// (start and end of its execution, no extra packets on the stream).
// Returns ASDSL_OK or ASDSL_ERR_HIP with the error text set.
template <typename... P, typename... A>
asdsl_status launch(const char* what, void (*kernel)(P...), dim3 grid, dim3 block, size_t lds, hipStream_t stream,
                    A... args) {
    static_assert(sizeof...(P) == sizeof...(A), "kernel argument count");
    LaunchEvents ev;
    const asdsl_status es = take_launch_events(what, stream, &ev);
    if (es != ASDSL_OK) return es;
    if (ev.start == nullptr && ev.stop == nullptr) {
        kernel<<<grid, block, lds, stream>>>(args...);
        return launch_status(what);
    }
    std::tuple<P...> held{static_cast<P>(args)...};
    void* ptrs[sizeof...(P)];
    std::apply([&](auto&... v) {
        size_t i = 0;
        ((ptrs[i++] = static_cast<void*>(&v)), ...);
    }, held);
    const hipError_t e = hipExtLaunchKernel(reinterpret_cast<const void*>(kernel), grid, block, ptrs, lds, stream,
                                            ev.start, ev.stop, 0);
    if (e != hipSuccess) {
        set_error("%s: kernel launch failed: %s", what, hipGetErrorString(e));
        return ASDSL_ERR_HIP;
    }
    return launch_status(what);
}

// Device buffer private to the library, one per device, grown on demand;
// every buffer it hands out stays allocated until the process ends.  Calls
// that use it and overlap on one device (different streams, no ordering
// between them) race on it; calls ordered by a stream or by events do not.
// Growing calls hipMalloc, which a stream under graph capture does not allow:
// an earlier call of at least the same size sizes it first
// (ASDSL_ERR_UNSUPPORTED otherwise).  After reserve_workspace(n > 0) on the
// device it is never grown: a request beyond it is ASDSL_ERR_INVALID_ARGUMENT.
asdsl_status device_workspace(hipStream_t stream, size_t bytes, void** out, const char* what);

// asdsl_reserve_workspace: allocate the current device's library buffer to
// at least `bytes` now and fix it (no later call allocates); 0 returns to
// growth on demand.
asdsl_status reserve_workspace(size_t bytes);

// The work buffer of one call: the caller's (`work`, `work_bytes`; at least
// `need` bytes, 256-byte aligned, else ASDSL_ERR_INVALID_ARGUMENT) when
// `work` is not null, the library-held one (device_workspace) otherwise.
asdsl_status work_buffer(hipStream_t stream, void* work, size_t work_bytes, size_t need, void** out,
                         const char* what);

// Integer tuning knob from the environment, read once (0 = unset).  Knobs
// only change launch shapes (and with them the fp32 summation order), never
// the formula: ASDSL_HIP_WG_PER_CU caps workgroups per compute unit,
// ASDSL_HIP_KSPLIT forces the K split of the preq2 kernels.
int env_knob(const char* name);

// The batched preq2 GEMV behind asdsl_gemv_preq2_fused_batch.  allow_mfma =
// false keeps every column on the dot4 kernels.  The MFMA form sums each
// column's groups in another fp32 order (~1e-7 apart); a consumer that
// quantizes the result to int8 again (the next layer's GEMV) can see such a
// difference move one element across a rounding boundary, about 5e-4 of that
// GEMV's output per flipped level.  A pass that must track the single-token
// step's arithmetic therefore uses the dot4 form.
asdsl_status preq2_fused_batch(const uint8_t* meta, const uint8_t* quant, const float* X, float* Y,
                               int out_features, int in_features, int group_size, int n_cols, asdsl_stream_t stream,
                               bool allow_mfma, void* work = nullptr, size_t work_bytes = 0);

// Whether the norm-fed preq2 GEMVs take the factored form (quantize h * nw,
// scale the reduced outputs by 1/rms) instead of the reference's order
// (quantize (h * inv_rms) * nw): ASDSL_HIP_NORM_FACTORED=1, read per call.
bool preq2_norm_factored();

// The launch shape of the single-column preq2 GEMV for M x K (K split
// 1 << lks, nu units per lane, waves per workgroup, exact = the split covers
// a band with no masked unit): the per-row fp32 order of its result.
void preq2_plan_shape(int M, int K, int cus, int* lks, int* nu, int* waves, bool* exact);

// The batched dot4 GEMV in the single-column GEMV's launch shape, so column
// n of Y is bit for bit what that GEMV gives on column n of X (same units
// per lane, same row reduction, same K-split sum); inv (per column, may be
// null) scales each partial row after its reduction and before the K-split
// sum, as the norm-fed single-column GEMVs apply 1/rms.  Returns
// ASDSL_ERR_UNSUPPORTED (nothing launched) where that shape leaves masked
// units or K > 8192.  1 <= n_cols <= 64.
asdsl_status preq2_batch_exact(const uint8_t* meta, const uint8_t* quant, const float* X, const float* inv, float* Y,
                               int out_features, int in_features, int group_size, int n_cols, asdsl_stream_t stream);

// The MFMA form of preq2_fused_batch (up to 16 columns) on an activation
// image another kernel already wrote at `image` (image_store8 layout: img,
// then fac at image + in_features * 16 bytes; columns past n_cols zero).
// preq2_batch_image_applies says whether preq2_fused_batch would take the
// MFMA form for this call (allow_mfma included); only then is
// preq2_batch_mfma_image valid (ASDSL_ERR_INVALID_ARGUMENT otherwise).
bool preq2_batch_image_applies(const uint8_t* meta, const uint8_t* quant, int out_features, int in_features,
                               int group_size, int n_cols, bool allow_mfma);
asdsl_status preq2_batch_mfma_image(const uint8_t* meta, const uint8_t* quant, const void* image, float* Y,
                                    int out_features, int in_features, int group_size, int n_cols,
                                    asdsl_stream_t stream);

// The MFMA batched GEMV in the single-column GEMV's fp32 order (up to 16
// columns): column n of Y is bit for bit what that GEMV gives on column n
// (same per-lane unit order, row reduction tree and K-split sum), the int32
// dots from MFMA.  Reads an image with its per-slice sums (image_store8 with
// `us`; image_fac_offset / image_us_offset).  preq2_batch_exact_mfma_applies
// says whether the single-column shape of M x K allows it (exact split, K
// split <= 4, K <= 8192, 1..16 columns).
bool preq2_batch_exact_mfma_applies(int out_features, int in_features, int group_size, int n_cols);
asdsl_status preq2_batch_exact_mfma_image(const uint8_t* meta, const uint8_t* quant, const void* image, float* Y,
                                          int out_features, int in_features, int group_size, int n_cols,
                                          asdsl_stream_t stream);

// The decode step's o_proj: gemv_preq2_fused of the attention output, which
// the GEMV's prologue merges itself from the split partials (part: per head
// nsplit rows of part_stride floats, m, l, acc[head_dim]) of a position
// *pos in [0, min(max_seq, pos_limit)): nt = pos / tile + 1 tiles in splits
// of ceil(nt / max_splits) tiles (max_splits <= 8).  A position outside that
// range reads `att` (the attention kernel zeroed it).
asdsl_status preq2_fused_combine(const uint8_t* meta, const uint8_t* quant, const float* att, float* y,
                                 int out_features, int in_features, int group_size, const float* part, const int* pos,
                                 int nsplit, int tile, int max_splits, int part_stride, int head_dim, int max_seq,
                                 int pos_limit, asdsl_stream_t stream);

// The decode step's first qkv GEMV: the RMSNorm prologue reads h as the fp16
// embedding row of *token (row 0 for a token outside [0, vocab)), workgroup 0
// stores h to h_out (fp32) and clears *clear_key (may be null).
asdsl_status preq2_embed_rmsnorm(const uint8_t* meta, const uint8_t* quant, const uint16_t* embed, const int* token,
                                 int vocab, const float* norm_w, float* h_out, float* y, int out_features,
                                 int in_features, int group_size, float eps, unsigned long long* clear_key,
                                 asdsl_stream_t stream);

#ifdef ASDSL_WG_TIMELINE
// Timing build: the preq2 GEMVs' and the sparse down-projection's timeline
// buffers (see device_common.hpp).
asdsl_status timeline_set_preq2(void* buf);
asdsl_status timeline_set_sparse(void* buf);
#endif

// Workgroups for a streaming kernel: enough tiles for every wave, capped at
// `per_cu` workgroups per compute unit (waves then loop over tiles).
inline int stream_grid(long long tiles, int waves_per_wg, int per_cu, int cus) {
    long long wgs = (tiles + waves_per_wg - 1) / waves_per_wg;
    static const int knob = env_knob("ASDSL_HIP_WG_PER_CU");
    if (knob > 0) per_cu = knob;
    const long long cap = static_cast<long long>(per_cu) * (cus > 0 ? cus : 256);
    if (wgs > cap) wgs = cap;
    if (wgs < 1) wgs = 1;
    return static_cast<int>(wgs);
}

}  // namespace asdsl

#define ASDSL_CHECK_ARG(cond, ...)                 \
    do {                                           \
        if (!(cond)) {                             \
            ::asdsl::set_error(__VA_ARGS__);       \
            return ASDSL_ERR_INVALID_ARGUMENT;     \
        }                                          \
    } while (0)

#define ASDSL_CU_COUNT(var)                        \
    const int var = ::asdsl::cu_count_current();   \
    if (var < 0) return ASDSL_ERR_HIP
