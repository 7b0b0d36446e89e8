/*
 * asdsl_hip.h — C ABI of the MI355X (gfx950) Q4 GEMV family.
 *
 * Every entry point is stream-ordered and asynchronous: pointers are DEVICE
 * pointers and the call returns as soon as its kernels are queued on
 * `stream` (0 = the null stream).  Nothing is allocated, with one exception:
 * the calls that need a work buffer (asdsl_sparse_down_proj_T, and the
 * batched GEMVs: asdsl_gemv_preq2_fused_batch with n_cols >= 4 (>= 3 when
 * in_features >= 4096), asdsl_matmul_batch_q4, asdsl_gemm_q4_128 and
 * asdsl_gemv_q4_packed / asdsl_gemv_q4_gs64 with batch > 1 and
 * K % 128 == 0) each have a *_ws form that takes a caller-owned work buffer
 * (size from the matching *_work_bytes query) and allocates nothing; the
 * plain forms use one buffer per device that the library grows on first use
 * and keeps (calls that overlap on one device on unordered streams race on
 * it; growing is refused under graph capture).  A caller that must not see
 * hipMalloc on the call path reserves that buffer once at load,
 * asdsl_reserve_workspace(bytes): the plain forms then never allocate, and
 * one that needs more than was reserved returns ASDSL_ERR_INVALID_ARGUMENT.
 * Buffers are owned by the
 * caller, exactly as in the reference kernels, which take caller-owned
 * host buffers (asdsl/kernels/native/gemv_q4_kernel.h:25-121).
 *
 * Byte layouts are the reference's, unchanged:
 *   preq    20-byte block per (row, 32-group): fp16 scale | fp16 zero | 16 B nibbles
 *           (asdsl/quantization/repack_q4_32.py:1-7)
 *   preq2   meta[M][G][4] (fp16 scale, fp16 zero) + quant[ceil(M/4)][G][64]
 *           4-row bands, slot r%4 at byte 16*(r%4) (asdsl/quantization/repack_preq2.py:1-9)
 *   Q4_128  66-byte block per (row, 128-group): fp16 scale=amax/7 | 64 B nibbles,
 *           implicit zero 8 (asdsl/quantization/repack_q4_128.py:1-6)
 *   nibbles low nibble = even element (asdsl/quantization/core.py:556-563)
 *
 * Return value: ASDSL_OK, or an error code; asdsl_last_error() then holds a
 * message for the calling thread.  Argument errors are detected before any
 * HIP call, so they are reported even on a machine without a GPU.
 */
#ifndef ASDSL_HIP_H
#define ASDSL_HIP_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* Same type as hipStream_t (hip/hip_runtime_api.h), so a hipStream_t, or
 * torch.cuda.current_stream().cuda_stream, is passed unchanged. */
struct ihipStream_t;
typedef struct ihipStream_t* asdsl_stream_t;

typedef enum asdsl_status {
    ASDSL_OK = 0,
    ASDSL_ERR_INVALID_ARGUMENT = 1, /* reference: std::invalid_argument -> ValueError */
    ASDSL_ERR_HIP = 2,              /* a HIP runtime call or kernel launch failed */
    ASDSL_ERR_UNSUPPORTED = 3       /* valid request outside what the kernels handle */
} asdsl_status;

#define ASDSL_ABI_VERSION 3

/* Library identity and error text. No reference counterpart (pybind11 raises). */
int asdsl_abi_version(void);
const char* asdsl_last_error(void);

/* Number of compute units of the current device, or -1 (and an error) when
 * no HIP device is usable.  Replaces the reference's thread-count probes
 * get_num_threads/has_openmp (asdsl/kernels/native/gemv_q4_avx2.cpp:1490-1505). */
int asdsl_device_cu_count(void);

/* Allocates the current device's library work buffer (the one the plain
 * forms of the work-buffer calls use) to at least `bytes` now and fixes it:
 * from then on no call on this device allocates, and a plain-form call that
 * needs more than `bytes` returns ASDSL_ERR_INVALID_ARGUMENT (the matching
 * *_work_bytes query gives each call's need).  bytes = 0 returns to growth on
 * demand.  Call it once per device at load, outside graph capture.  No
 * reference counterpart: the reference kernels allocate only thread-local
 * host scratch (gemv_q4_preq_restored.cpp:483-484, gemv_preq2_avx2.cpp:315-316). */
asdsl_status asdsl_reserve_workspace(size_t bytes);

/* Instrumentation, no reference counterpart: arms two HIP events (hipEvent_t,
 * created by the caller; either may be NULL) for the calling thread's next
 * kernel launch by this library.  The launch records them as part of the
 * kernel's own dispatch (hipExtLaunchKernel), at the start and end of its
 * execution, so hipEventElapsedTime(start, stop) is that kernel's duration
 * alone, with no extra commands on the stream. */
asdsl_status asdsl_profile_next_launch(void* start_event, void* stop_event);

/* Per-stage timing of a decode step, replacing the reference's
 * ASDSL_ENGINE_PROFILE breakdown (asdsl/kernels/native/unified_engine.cpp:58-95,
 * 1668-1687, which times each stage of UnifiedEngine::forward_token with a
 * host clock).  Between begin and end, every kernel this library launches from
 * the calling thread (at most max_launches, 1..65536) records two HIP events
 * through its own dispatch, as asdsl_profile_next_launch does, under a stage
 * label: the decode step's launches are labelled "embed", "qkv", "attention",
 * "attention_combine", "o_proj", "gate_up", "down", "lm_head" and "finalize";
 * any other launch carries its kernel's name.  begin creates the events it
 * needs (kept for later sessions of the thread) and fails on a thread already
 * armed; a launch while armed on a stream under graph capture fails with
 * ASDSL_ERR_UNSUPPORTED.  end disarms, waits for the last recorded launch and
 * writes launch i's label (a static string) and duration in ms to labels[i]
 * and ms[i] in launch order, their number to *count (capacity at least that),
 * and the time from the first launch's start to the last one's end to
 * *span_ms; it fails when more launches than max_launches were made, or when
 * one used events armed by asdsl_profile_next_launch instead. */
asdsl_status asdsl_profile_stages_begin(int max_launches);
asdsl_status asdsl_profile_stages_end(int capacity, const char** labels, float* ms, int* count, float* span_ms);

/* Calibration, no reference counterpart: reads `bytes` (a multiple of 16)
 * from the 16-byte-aligned device buffer `data` with 16-byte non-temporal
 * loads over `grid` workgroups of 512 threads (<= 0: one per compute unit)
 * and writes nothing in practice (`sink`, one device word, is written only
 * if the loaded words fold to a fixed sentinel).  Timed like a GEMV it gives
 * the practical ceiling for streaming that many bytes in one launch. */
asdsl_status asdsl_stream_read(const void* data, size_t bytes, uint32_t* sink, int grid, asdsl_stream_t stream);

/* The same read in the launch shapes a sweep of the single-launch ceiling
 * covers: `threads` (256, 512 or 1024) per workgroup, `inflight` (4, 8 or
 * 16) 16-byte loads in flight per lane, grid-stride units (slab = 0) or one
 * contiguous slab of bytes/grid per workgroup (slab = 1, a GEMV
 * workgroup's access).  slab = 2 is the one-shot read a GEMV tile makes:
 * workgroup w reads slabs of threads * inflight consecutive 16-byte units
 * (threads 256 or 512, inflight 2, 3, 4, 6, 8 or 12 loads per lane, all
 * requested before any is used), slabs w, w + grid, ...  No reference
 * counterpart (calibration). */
asdsl_status asdsl_stream_read_ex(const void* data, size_t bytes, uint32_t* sink, int grid, int threads,
                                  int inflight, int slab, asdsl_stream_t stream);

/* Calibration, no reference counterpart: the cost of a grid-wide handoff
 * inside one kernel.  One cooperative launch of `grid` workgroups (256
 * threads each; all must fit on the device at once, else
 * ASDSL_ERR_UNSUPPORTED) runs `rounds` waits for every workgroup.  mode 0:
 * each workgroup stores its own flag word, one wave polls all of them;
 * mode 1: the same with a 4096-float vector written in slices before the
 * flags and read whole after (plus a second wait before it is rewritten);
 * mode 2: one atomic add per workgroup on a shared counter, polled.  Flags
 * and data use agent-scope atomic loads and stores, no cache flushes.
 * work: asdsl_grid_sync_probe_work_bytes(grid) bytes, zeroed by the caller
 * before every call.  Every wait gives up after spin_limit polls: the run
 * then stops early with word 0 of work set to 1 (0 after a complete run). */
size_t asdsl_grid_sync_probe_work_bytes(int grid);
asdsl_status asdsl_grid_sync_probe(int mode, int rounds, int grid, void* work, size_t work_bytes, int spin_limit,
                                   asdsl_stream_t stream);

/* ------------------------------------------------------------------ A1 ---
 * Per-group int8 activation quantizer.
 * Replaces quantize_activation_avx2
 *   (asdsl/kernels/native/gemv_q4_preq_restored.cpp:505-549;
 *    pybind asdsl/kernels/native/gemv_q4_avx2.cpp:1352-1365).
 * amax=max|x|; amax<1e-9 -> q=0, scale=1; else scale=amax*(1/127),
 * q=sat8(rne(x*(127/amax))).  x[in_features] -> x_q8[in_features],
 * x_scales[in_features/group_size].  group_size in {32, 64, 128}. */
asdsl_status asdsl_quantize_activation(const float* x, int8_t* x_q8, float* x_scales,
                                       int in_features, int group_size,
                                       asdsl_stream_t stream);

/* ------------------------------------------------------------------ A3 ---
 * preq g32 GEMV on 20-byte blocks, activation already quantized.
 * Replaces gemv_q4_32_preq_avx2 (asdsl/kernels/native/gemv_q4_preq_restored.cpp:551-573).
 * y[r] = sum_g s*xs*D_g - z*s*xs*X_g (D_g = sum q*xq, X_g = sum xq).  y overwritten. */
asdsl_status asdsl_gemv_q4_32_preq(const uint8_t* blocks, const int8_t* x_q8,
                                   const float* x_scales, float* y,
                                   int out_features, int in_features, int group_size,
                                   asdsl_stream_t stream);

/* Same, quantizing the fp32 activation inside the call.
 * Replaces gemv_q4_32_preq_fused_avx2 / _4row_avx2 / _8row_avx2
 *   (asdsl/kernels/native/gemv_q4_preq_restored.cpp:575-669); the 4/8-row
 *   unroll of the reference is a CPU scheduling choice with identical math. */
asdsl_status asdsl_gemv_q4_32_preq_fused(const uint8_t* blocks, const float* x, float* y,
                                         int out_features, int in_features, int group_size,
                                         asdsl_stream_t stream);

/* ------------------------------------------------------------------ A5 ---
 * preq2 GEMV (4-row band quant + sidecar meta), fp32 activation quantized inside.
 * Replaces gemv_preq2_fused_avx2 (asdsl/kernels/native/gemv_preq2_avx2.cpp:301-319).
 * group_size 32 is the reference layout.  group_size 128 selects the
 * asymmetric preq2-g128 layout, which the reference does not have:
 * meta[M][K/128][4] + quant[ceil(M/4)][K/128][256] (4 rows x 64 B per band),
 * activation quantized per 128. */
asdsl_status asdsl_gemv_preq2_fused(const uint8_t* meta, const uint8_t* quant,
                                    const float* x, float* y,
                                    int out_features, int in_features, int group_size,
                                    asdsl_stream_t stream);

/* Batched preq2 GEMV for speculative verification: X[n_cols][in_features]
 * (16-byte aligned) -> Y[n_cols][out_features]; every column quantized
 * independently, so Y[n] equals asdsl_gemv_preq2_fused on X[n] up to fp32
 * summation order.  Each weight byte is read once per launch: group size 32
 * with n_cols >= 4 (>= 3 when in_features >= 4096) runs the MFMA form, 16
 * columns per launch; otherwise the dot4 form takes 16 columns per launch
 * when each lane holds at most 2 weight units of a band (8-wave workgroups,
 * in_features <= 4096), else 8 (16-wave workgroups at most 4 units per lane)
 * or 4, and fewer when the columns' int8 images would pass 96 KB of LDS
 * (at in_features 3072: 8 columns; at 8192: 8).  n_cols in [1, 64].
 * No reference counterpart: the reference engine verifies preq2 drafts with
 * serial forward_token calls (asdsl/kernels/native/unified_engine.cpp:1768-1789);
 * this is the batched kernel its forward_verify_batch would call. */
asdsl_status asdsl_gemv_preq2_fused_batch(const uint8_t* meta, const uint8_t* quant, const float* X, float* Y,
                                          int out_features, int in_features, int group_size, int n_cols,
                                          asdsl_stream_t stream);

/* Bytes of work buffer asdsl_gemv_preq2_fused_batch_ws needs for this
 * in_features (any out_features and n_cols); 0 for an invalid size. */
size_t asdsl_gemv_preq2_fused_batch_work_bytes(int in_features);

/* asdsl_gemv_preq2_fused_batch with a caller-owned work buffer (256-byte
 * aligned, at least asdsl_gemv_preq2_fused_batch_work_bytes bytes; contents
 * after the call unspecified): allocates nothing.  Calls that share a work
 * buffer must be ordered (one stream, or events). */
asdsl_status asdsl_gemv_preq2_fused_batch_ws(const uint8_t* meta, const uint8_t* quant, const float* X, float* Y,
                                             int out_features, int in_features, int group_size, int n_cols,
                                             void* work, size_t work_bytes, asdsl_stream_t stream);

/* preq2 GEMV on a pre-quantized activation.
 * Replaces gemv_preq2_avx2 (asdsl/kernels/native/gemv_preq2_avx2.cpp:321-337).
 * group_size as for asdsl_gemv_preq2_fused; x_scales has in_features/group_size entries. */
asdsl_status asdsl_gemv_preq2(const uint8_t* meta, const uint8_t* quant,
                              const int8_t* x_q8, const float* x_scales, float* y,
                              int out_features, int in_features, int group_size,
                              asdsl_stream_t stream);

/* ------------------------------------------------------------------ A6 ---
 * Q4_128 symmetric GEMV: 66-byte blocks per (row, 128-group), fp16 scale,
 * implicit zero 8; activation pre-quantized per 128 (x_scales has
 * in_features/128 entries).  blocks must be 2-byte aligned.
 * Replaces gemv_q4_128_preq_avx2 (asdsl/kernels/native/gemv_q4_128.cpp:94-257;
 *   pybind asdsl/kernels/native/gemv_q4_avx2.cpp:1461-1477).
 * y[r] = sum_g D_g*(ws*xs) - 8*X_g*xs*ws.  group_size must be 128, y overwritten. */
asdsl_status asdsl_gemv_q4_128_preq(const uint8_t* blocks, const int8_t* x_q8, const float* x_scales, float* y,
                                    int out_features, int in_features, int group_size,
                                    asdsl_stream_t stream);

/* Same, quantizing the fp32 activation per 128 inside the call (the A1 rule).
 * Replaces the engine's quantize-then-GEMV pair for the g128 lm_head
 * (asdsl/kernels/native/unified_engine.cpp:1646-1653). */
asdsl_status asdsl_gemv_q4_128_fused(const uint8_t* blocks, const float* x, float* y,
                                     int out_features, int in_features, int group_size,
                                     asdsl_stream_t stream);

/* ---------------------------------------------------------------- A9(ii) ---
 * Symmetric packed Q4 (nibbles row-major, K/2 bytes per row, low = even
 * column, zero 8) with fp32 scales[M][K/group_size]; x quantized per
 * group_size inside the call (the A1 rule).  y[r] = sum_g D'(q-8, xq)*ws*xs.
 * group_size in {32, 64, 128}; weights 16-byte aligned.
 * Replaces gemv_q4_q8_avx2 (asdsl/kernels/native/gemv_q4_avx2.cpp:131-253;
 * pybind 1301-1316; reached from gemv_q4_packed(use_q8=True), asdsl/kernels/gemv_q4.py:269-273). */
asdsl_status asdsl_gemv_q4_q8(const uint8_t* weights_packed, const float* scales, const float* x, float* y,
                              int out_features, int in_features, int group_size, asdsl_stream_t stream);

/* ------------------------------------------------------------------- A8 ---
 * Q4_K (ASDSL variant) GEMV: 144-byte superblock per (row, 256): fp16 d |
 * fp16 dmin | 12 bytes of 6-bit fields (0-7 scales, 8-15 mins; LSB-first
 * bitstream) | 8 x 16 bytes of nibbles.  x quantized per 32 inside the call
 * with round-half-away, clamp +-127, amax < 1e-12 -> scale 0.
 * y[r] = sum_sb (d*sc*D - dmin*m*X) * xs.  in_features % 256 == 0.
 * Replaces gemv_q4km_q8_avx2 (asdsl/kernels/native/gemv_q4_avx2.cpp:283-420;
 * pybind 1318-1348). */
asdsl_status asdsl_gemv_q4km_q8(const uint8_t* weights_q4km, const float* x, float* y, int out_features,
                                int in_features, asdsl_stream_t stream);

/* ------------------------------------------------------------- A10 / A9(i) ---
 * fp32-affine GEMVs, activation not quantized:
 *   y[r] = sum_g scales[r,g] * (sum_{k in g} q[r,k] * x[k]) + biases[r,g] * (sum_{k in g} x[k])
 * Weights row-major; x and weights 16-byte aligned; K <= 32768.
 * Argument rules and messages follow validate_gemv_args
 *   (asdsl/kernels/native/gemv_q4_avx2.cpp:901-929). */

/* 4-bit, 2 nibbles per byte (low = even column); x is [batch][K], y [batch][M].
 * Replaces gemv_q4_packed (gemv_q4_avx2.cpp:665-749, pybind 1084-1126).
 * group_size must be a multiple of 16. */
asdsl_status asdsl_gemv_q4_packed(const uint8_t* w_packed, const float* x, const float* scales,
                                  const float* biases, float* y, int M, int K, int group_size, int batch,
                                  asdsl_stream_t stream);

/* Bytes of work buffer the batched fp32-affine GEMMs need at this shape:
 * asdsl_gemv_q4_packed_ws, asdsl_gemv_q4_gs64_ws (group_size 64),
 * asdsl_matmul_batch_q4_ws and asdsl_gemm_q4_128_ws (group_size 128); any
 * batch.  0 when the shape has no batched form (those calls then run one
 * GEMV per column and need no buffer) or the arguments are invalid. */
size_t asdsl_affine_batch_work_bytes(int M, int K, int group_size);

/* The same as asdsl_gemv_q4_packed with a caller-owned work buffer
 * (256-byte aligned, asdsl_affine_batch_work_bytes(M, K, group_size) bytes;
 * may be NULL when batch == 1): allocates nothing. */
asdsl_status asdsl_gemv_q4_packed_ws(const uint8_t* w_packed, const float* x, const float* scales,
                                     const float* biases, float* y, int M, int K, int group_size, int batch,
                                     void* work, size_t work_bytes, asdsl_stream_t stream);

/* One byte per value, used as is.  Replaces gemv_q4_unpacked
 * (gemv_q4_avx2.cpp:755-806, pybind 1128-1160). */
asdsl_status asdsl_gemv_q4_unpacked(const uint8_t* w, const float* x, const float* scales,
                                    const float* biases, float* y, int M, int K, int group_size,
                                    asdsl_stream_t stream);

/* 4-bit packed, scales only, group 64; x [batch][cols], y [batch][rows].
 * Replaces gemv_q4_avx2 / gemv_q4_avx2_gs64 (asdsl/kernels/native/gemv_q4_kernel.cpp:96-122;
 * pybind gemv_q4_avx2.cpp:1211-1268). */
asdsl_status asdsl_gemv_q4_gs64(const uint8_t* w_packed, const float* x, const float* scales, float* y,
                                int rows, int cols, int batch, asdsl_stream_t stream);

/* The same with a caller-owned work buffer (asdsl_affine_batch_work_bytes(rows,
 * cols, 64) bytes, 256-byte aligned; may be NULL when batch == 1). */
asdsl_status asdsl_gemv_q4_gs64_ws(const uint8_t* w_packed, const float* x, const float* scales, float* y,
                                   int rows, int cols, int batch, void* work, size_t work_bytes,
                                   asdsl_stream_t stream);

/* ------------------------------------------------------------------ A11 ---
 * Batched fp32 Q4 GEMM over packed weights: Y[b][r] = sum_k dequant(W[r,k]) X[b][k]
 * with dequant = q*s + b per group; X [B][K], Y [B][M] overwritten, B <= 64.
 * For B >= 2, group_size 32/64/128 and K % 128 == 0 one weight pass serves 16
 * columns (MFMA on fp16 hi/lo digits of each column, within 1e-5 of fp32);
 * other shapes run one GEMV per column.
 * Replaces matmul_batch_q4 (asdsl/kernels/native/gemv_q4_avx2.cpp:950-1059). */
asdsl_status asdsl_matmul_batch_q4(const uint8_t* w_packed, const float* scales, const float* biases,
                                   const float* X, float* Y, int M, int K, int B, int group_size,
                                   asdsl_stream_t stream);

/* The same with a caller-owned work buffer (asdsl_affine_batch_work_bytes(M, K,
 * group_size) bytes, 256-byte aligned; may be NULL when B == 1). */
asdsl_status asdsl_matmul_batch_q4_ws(const uint8_t* w_packed, const float* scales, const float* biases,
                                      const float* X, float* Y, int M, int K, int B, int group_size, void* work,
                                      size_t work_bytes, asdsl_stream_t stream);

/* Batched Q4_128 GEMM with an fp32 activation, not quantized:
 * Y[b][r] = sum_g ws * sum_k (q-8) X[b][k]; X [B][K], Y [B][M], B <= 64.
 * Replaces gemm_q4_128_q8_avx2 (asdsl/kernels/native/gemv_q4_128.cpp:262-306),
 * the engine's forward_batch GEMM under g128 (unified_engine.cpp:1153-1158). */
asdsl_status asdsl_gemm_q4_128(const uint8_t* blocks, const float* X, float* Y, int out_features,
                               int in_features, int group_size, int batch_size, asdsl_stream_t stream);

/* The same with a caller-owned work buffer (asdsl_affine_batch_work_bytes(
 * out_features, in_features, 128) bytes, 256-byte aligned; may be NULL when
 * batch_size == 1). */
asdsl_status asdsl_gemm_q4_128_ws(const uint8_t* blocks, const float* X, float* Y, int out_features,
                                  int in_features, int group_size, int batch_size, void* work, size_t work_bytes,
                                  asdsl_stream_t stream);

/* uint8 weights (one per byte), fp32 scale and bias per group.
 * Replaces fused_dequant_gemv / gemv_q8_unpacked
 * (asdsl/kernels/native/gemv_q8_avx2.cpp:67-144, pybind 159-215); the
 * reference's cache_tiling flag changes loop blocking only and has no
 * counterpart here. */
asdsl_status asdsl_gemv_q8_unpacked(const uint8_t* w, const float* x, const float* scales,
                                    const float* biases, float* y, int M, int K, int group_size,
                                    asdsl_stream_t stream);

/* --------------------------------------------------------------- A12(ii) ---
 * Bit k of bitmask[(K+31)/32] set iff |x[k]| >= threshold (NaN: clear).
 * Replaces compute_bitmask (asdsl/kernels/native/gemv_sparse_avx2.cpp:144-179). */
asdsl_status asdsl_compute_bitmask(const float* x, uint32_t* bitmask, int K, float threshold,
                                   asdsl_stream_t stream);

/* Activation-sparse GEMV over uint8 weights: only columns whose bit is set
 * count (in both sums).  32-column runs with a zero mask word skip their
 * weight loads.  Replaces gemv_sparse_unpacked
 * (asdsl/kernels/native/gemv_sparse_avx2.cpp:66-139, bitmask path). */
asdsl_status asdsl_gemv_sparse_unpacked(const uint8_t* w, const float* x, const float* scales,
                                        const float* biases, const uint32_t* bitmask, float* y, int M, int K,
                                        int group_size, asdsl_stream_t stream);

/* Same over an explicit list of active columns (a column listed c times counts
 * c times; indices outside [0, K) are ignored).  work_mask[(K+31)/32] and
 * work_x[K] (16-byte aligned) are caller-provided device scratch, overwritten.
 * Replaces gemv_sparse_with_indices (gemv_sparse_avx2.cpp:66-110, index path). */
asdsl_status asdsl_gemv_sparse_with_indices(const uint8_t* w, const float* x, const float* scales,
                                            const float* biases, const int32_t* active_indices, int n_active,
                                            float* y, int M, int K, int group_size, uint32_t* work_mask,
                                            float* work_x, asdsl_stream_t stream);

/* ---------------------------------------------------------------- A12(i) ---
 * FATReLU-sparse down-projection over K-major packed Q4:
 * w_T[in_dim][out_dim/2] (low nibble = even output), scales_T/biases_T
 * [in_dim][out_dim/group_size] fp32.  For every listed row r with
 * 0 <= r < in_dim and sparse_x[r] != 0:
 *     y[o] += fma(q[r][o], scales_T[r][o/gs]*x[r], biases_T[r][o/gs]*x[r])
 * y[out_dim] is overwritten (starts from zero).  A row listed twice adds twice.
 * out_dim % 32 == 0, group_size % 8 == 0, w_T 16-byte aligned.
 * Long lists are summed in parts through a device buffer the library keeps
 * per device: calls that overlap on one device (unordered streams) race on
 * it.  Sizing it allocates, so under graph capture a call with at least the
 * same n_active and out_dim must have run on the device before (else
 * ASDSL_ERR_UNSUPPORTED); asdsl_sparse_down_proj_T_ws takes the buffer from
 * the caller instead.  Repeat calls are bitwise equal.
 * Replaces sparse_down_proj_T (asdsl/kernels/native/gemv_sparse_avx2.cpp:273-418),
 * called from experiments/phi4_cpu_run.py:3949-3967. */
asdsl_status asdsl_sparse_down_proj_T(const uint8_t* w_T_packed, const float* scales_T, const float* biases_T,
                                      const float* sparse_x, const int32_t* active_rows, int n_active, float* y,
                                      int in_dim, int out_dim, int group_size, asdsl_stream_t stream);

/* Bytes of work buffer asdsl_sparse_down_proj_T_ws needs for out_dim outputs
 * (any list length); 0 for out_dim <= 0. */
size_t asdsl_sparse_down_work_bytes(int out_dim);

/* asdsl_sparse_down_proj_T with a caller-owned work buffer (256-byte aligned,
 * asdsl_sparse_down_work_bytes(out_dim) bytes; contents after the call
 * unspecified): allocates nothing.  Calls that share a work buffer must be
 * ordered (one stream, or events). */
asdsl_status asdsl_sparse_down_proj_T_ws(const uint8_t* w_T_packed, const float* scales_T, const float* biases_T,
                                         const float* sparse_x, const int32_t* active_rows, int n_active, float* y,
                                         int in_dim, int out_dim, int group_size, void* work, size_t work_bytes,
                                         asdsl_stream_t stream);

/* asdsl_sparse_down_proj_T for callers that cannot allocate at all (code
 * under HIP graph capture, tight serving loops, harnesses that forbid
 * hipMalloc); no counterpart in the reference.  The partial rows live in a
 * static device array of this library: 32 rows of at most 16384 outputs
 * (2 MiB per device, held until the process ends), so out_dim > 16384 is
 * refused (ASDSL_ERR_INVALID_ARGUMENT).  The array's device address is
 * looked up once per device on the first call there.  Every call on a
 * device shares that device's array: calls that overlap on one device
 * (unordered streams) race on it; calls ordered by one stream or by events
 * do not.  Same bits as asdsl_sparse_down_proj_T. */
asdsl_status asdsl_sparse_down_proj_T_noalloc(const uint8_t* w_T_packed, const float* scales_T,
                                              const float* biases_T, const float* sparse_x,
                                              const int32_t* active_rows, int n_active, float* y, int in_dim,
                                              int out_dim, int group_size, asdsl_stream_t stream);

/* Debug dequantization of a preq2 matrix to fp32 W[M][K]: w = (q - z) * s,
 * bit-exact with the reference's dequant (experiments/phi4_cpu_run.py:3450-3467). */
asdsl_status asdsl_dequant_preq2(const uint8_t* meta, const uint8_t* quant, float* w,
                                 int out_features, int in_features, int group_size,
                                 asdsl_stream_t stream);

/* ------------------------------------------------------------------ A13 ---
 * Batch-1 decode step (the glue around the GEMVs).
 *
 * preq2 GEMV whose fp32 input is rmsnorm(h) with h = h_in + delta (delta may
 * be NULL): inv_rms = 1/sqrt(sum(h^2)/K + eps), x = (h*inv_rms)*norm_w, then
 * quantized inside as asdsl_gemv_preq2_fused.  The positive factor inv_rms
 * leaves the int8 codes unchanged and scales every group scale, so it is
 * applied to the outputs instead: y = inv_rms * GEMV(h*norm_w), equal to the
 * normed form up to fp32 rounding (a value within rounding of a code
 * boundary may take the neighbouring code).  If h_out is not NULL, h is
 * stored there (the new residual stream; must not alias h_in or delta).  If
 * argmax_key is not NULL (zeroed before the call), the largest y and its row
 * (first on ties) are folded into it: key = order-preserving float bits << 32
 * | (0xFFFFFFFF - row).  in_features <= 8192.
 * Replaces residual_add_rmsnorm_f32 / rmsnorm_f32 + the fused preq GEMV and
 * argmax_f32_avx2 (asdsl/kernels/native/unified_engine.cpp:499-524,651-688,207-233,
 * call sites 1377-1421,1521-1528,1634-1648). */
asdsl_status asdsl_gemv_preq2_rmsnorm(const uint8_t* meta, const uint8_t* quant, const float* h_in,
                                      const float* delta, const float* norm_w, float* h_out, float* y,
                                      int out_features, int in_features, int group_size, float eps,
                                      unsigned long long* argmax_key, asdsl_stream_t stream);

/* preq2 GEMV whose fp32 input is swiglu(gate_up[0:K], gate_up[K:2K]):
 * v = (g * 1/(1 + exp(-g))) * u with the reference's polynomial exp, zeroed
 * where |v| < threshold if threshold > 0 (FATReLU).  in_features <= 8192.
 * Replaces swiglu_inplace + the down GEMV (unified_engine.cpp:781-857, call
 * sites 1581-1628). */
asdsl_status asdsl_gemv_preq2_swiglu(const uint8_t* meta, const uint8_t* quant, const float* gate_up,
                                     float* y, int out_features, int in_features, int group_size,
                                     float threshold, asdsl_stream_t stream);

/* gate_up GEMV with the residual add + RMSNorm prologue of
 * asdsl_gemv_preq2_rmsnorm and SwiGLU in its epilogue: the weight rows are
 * [gate ffn | up ffn] x in_features (preq2), and s_out[ffn] =
 * swiglu(gate, up) with the reference's polynomial exp and the FATReLU
 * threshold, bit for bit what asdsl_gemv_preq2_rmsnorm followed by the
 * SwiGLU prologue of asdsl_gemv_preq2_swiglu computes.  A workgroup takes
 * gate and up rows together, so the 2*ffn outputs never reach memory.
 * ffn % 16 == 0, in_features <= 8192; ASDSL_ERR_UNSUPPORTED when the shape
 * has no paired tiling (nothing is launched then).
 * Replaces residual_add_rmsnorm_f32 + the gate_up GEMV + swiglu_inplace
 * (unified_engine.cpp:651-688,1524-1575). */
asdsl_status asdsl_gemv_preq2_rmsnorm_swiglu(const uint8_t* meta, const uint8_t* quant, const float* h_in,
                                             const float* delta, const float* norm_w, float* h_out, float* s_out,
                                             int ffn, int in_features, int group_size, float eps, float threshold,
                                             asdsl_stream_t stream);

/* Floats of device work buffer asdsl_attention_f16kv / _q8kv need. */
size_t asdsl_attention_work_floats(int n_heads, int max_seq);

/* RoPE + KV write + attention for one token at position *pos (device int):
 * qkv = [q n_heads*128 | k n_kv_heads*128 | v n_kv_heads*128] fp32.  RoPE
 * rotates the first rotary_dim dims of every q and k head, half split
 * (x[i], x[i+rotary_dim/2]) with rope_cos/rope_sin[pos][rotary_dim/2].  The new
 * k, v are rounded to fp16 and stored at [kv_head][pos] of the caches
 * (fp16 [n_kv_heads][max_seq][128]); att_out[h] = softmax(q_h.K/sqrt(128)) V
 * over positions 0..pos of kv head h / (n_heads/n_kv_heads).  head_dim = 128,
 * work: asdsl_attention_work_floats floats of scratch.
 * Replaces rope_apply_inplace + set_kv_cache + compute_attention_flash_q8
 * (unified_engine.cpp:768-801,859-1027), with an fp16 instead of int8 cache. */
asdsl_status asdsl_attention_f16kv(const float* qkv, uint16_t* k_cache, uint16_t* v_cache,
                                   const float* rope_cos, const float* rope_sin, const int* pos,
                                   float* att_out, float* work, int n_heads, int n_kv_heads,
                                   int head_dim, int rotary_dim, int max_seq, asdsl_stream_t stream);

/* The same with the reference's cache form: int8 codes [n_kv_heads][max_seq][128]
 * and one fp32 scale per 64 dims, k_scale/v_scale [n_kv_heads][max_seq][2].
 * The new k and v are quantized per 64-dim block as set_kv_cache does
 * (scale = amax * (1/127), or 1e-12 when amax <= 1e-12; code =
 * round-half-even(x / scale) clamped to [-127, 127]) and every K/V element
 * of the attention, the new row's included, is float(code) * scale.
 * Replaces rope_apply_inplace + set_kv_cache + compute_attention_flash_q8
 * (unified_engine.cpp:768-801,859-1027). */
asdsl_status asdsl_attention_q8kv(const float* qkv, int8_t* k_cache, int8_t* v_cache, float* k_scale,
                                  float* v_scale, const float* rope_cos, const float* rope_sin, const int* pos,
                                  float* att_out, float* work, int n_heads, int n_kv_heads, int head_dim,
                                  int rotary_dim, int max_seq, asdsl_stream_t stream);

/* KV cache forms of asdsl_decode_model.kv_format. */
#define ASDSL_KV_FP16 0 /* fp16 rows */
#define ASDSL_KV_INT8 1 /* int8 rows + fp32 scale per 64 dims (the reference's form) */

/* Weights of one decoder layer (device pointers). */
typedef struct asdsl_decode_layer {
    const uint8_t* qkv_meta;  const uint8_t* qkv_quant;   /* preq2, [(h + 2 kv) * 128] x hidden, gs_attn */
    const uint8_t* o_meta;    const uint8_t* o_quant;     /* preq2, hidden x hidden, gs_attn */
    const uint8_t* gu_meta;   const uint8_t* gu_quant;    /* preq2, [gate ffn | up ffn] x hidden, gs_ffn */
    const uint8_t* down_meta; const uint8_t* down_quant;  /* preq2, hidden x ffn, gs_ffn */
    const float* rms_att;     const float* rms_ffn;       /* [hidden] */
    void* k_cache;            void* v_cache;              /* [n_kv_heads][max_seq][128], fp16 or int8
                                                             (kv_format), 16-byte aligned */
    float fatrelu_threshold;                              /* 0: plain SwiGLU */
    float* k_scale;           float* v_scale;             /* int8 cache: fp32 [n_kv_heads][max_seq][2];
                                                             unused (may be null) for fp16 */
} asdsl_decode_layer;

/* A Phi-4-shaped decoder (layers is a HOST array of n_layers entries). */
typedef struct asdsl_decode_model {
    int hidden, ffn, vocab, n_layers, n_heads, n_kv_heads, head_dim, rotary_dim, max_seq;
    int gs_attn, gs_ffn, gs_lm;                           /* preq2 group sizes: 32 or 128 */
    float rms_eps;
    const asdsl_decode_layer* layers;
    const uint16_t* embed;                                /* fp16 [vocab][hidden] */
    const float* rms_out;                                 /* [hidden] */
    const uint8_t* lm_meta;   const uint8_t* lm_quant;    /* preq2, vocab x hidden, gs_lm */
    const float* rope_cos;    const float* rope_sin;      /* fp32 [max_seq][rotary_dim/2] */
    int kv_format;                                        /* ASDSL_KV_FP16 or ASDSL_KV_INT8 */
} asdsl_decode_model;

/* Bytes of device work buffer asdsl_decode_token needs (0 for an invalid model). */
size_t asdsl_decode_work_bytes(const asdsl_decode_model* model);

/* Bits of the decode step's flags word (a uint32 in the work buffer at
 * asdsl_decode_flags_offset(model) bytes).  The step only sets them; the
 * caller zeroes the word before the first step (with the whole buffer) and
 * after reading a raised bit.  A step that raises one computed its attention
 * as zero and wrote no K/V row, so its logits are not the model's. */
#define ASDSL_DECODE_FLAG_POS_LIMIT 1u /* *pos was at or past asdsl_decode_token_upto's pos_limit */
#define ASDSL_DECODE_FLAG_POS_RANGE 2u /* *pos was outside [0, max_seq) */

/* Byte offset of the flags word in the decode work buffer (0 for an invalid
 * model; a valid model's word is never at offset 0).  No reference
 * counterpart (the reference throws std::out_of_range on the host,
 * unified_engine.cpp:1352-1354). */
size_t asdsl_decode_flags_offset(const asdsl_decode_model* model);

/* Queues one greedy decode step on `stream`: embeds *token (device int),
 * runs every layer at position *pos (device int), writes logits[vocab], then
 * sets *token to the argmax and increments *pos.  Nothing else changes on
 * the host side between steps, so a HIP graph of one call replays step after
 * step.  work: asdsl_decode_work_bytes() bytes, 256-byte aligned, zeroed
 * before the first step; apart from the flags word its contents after a call
 * are unspecified.  A position outside [0, max_seq) raises
 * ASDSL_DECODE_FLAG_POS_RANGE.
 * Replaces UnifiedEngine::forward_token + greedy argmax
 * (asdsl/kernels/native/unified_engine.cpp:1339-1688,207-233). */
asdsl_status asdsl_decode_token(const asdsl_decode_model* model, int* token, int* pos, float* logits,
                                void* work, asdsl_stream_t stream);

/* The same step for a position *pos < pos_limit (asdsl_decode_token is
 * pos_limit = max_seq).  The launch is shaped for that range: the attention
 * grid covers only the splits such positions use (one per 64 positions, at
 * most 32), and below 512 the o_proj GEMV merges them in its prologue, with
 * no combine launch (same bits as the combine kernel).  A HIP graph of one
 * call then replays for every position below pos_limit.  A replay at a
 * position at or past pos_limit is detected on the device: its attention is
 * zero, no K/V row is written, ASDSL_DECODE_FLAG_POS_LIMIT is raised, and
 * *token and *pos still advance.  No reference counterpart (the reference
 * passes the position by value, unified_engine.cpp:1339). */
asdsl_status asdsl_decode_token_upto(const asdsl_decode_model* model, int* token, int* pos, int pos_limit,
                                     float* logits, void* work, asdsl_stream_t stream);

/* Bytes of device work buffer asdsl_decode_verify needs for up to max_tokens
 * tokens (1..16); 0 for an invalid model or count. */
size_t asdsl_decode_verify_work_bytes(const asdsl_decode_model* model, int max_tokens);

/* Queues one multi-token pass (speculative verify): tokens[0..n) (device) at
 * positions *pos .. *pos + n - 1 (device int, not advanced) run through every
 * layer with the projections as batched GEMVs over the n columns; each
 * column's K/V are written to the caches at its position and its attention
 * covers positions <= its own; logits[n][vocab] (16-byte aligned) and
 * next_tokens[n] = the greedy argmax of each column (first on ties).  Columns
 * at or past max_seq produce zero attention and write no K/V.  1 <= n <= 16;
 * work: asdsl_decode_verify_work_bytes(model, >= n) bytes, 256-byte aligned.
 * Replaces UnifiedEngine::forward_verify_batch
 * (asdsl/kernels/native/unified_engine.cpp:1774-1789), whose preq2 path falls
 * back to serial forward_token calls. */
asdsl_status asdsl_decode_verify(const asdsl_decode_model* model, const int* tokens, int n_tokens, const int* pos,
                                 float* logits, int* next_tokens, void* work, asdsl_stream_t stream);

/* The int8 cache's form of asdsl_kv_zero_from: codes 0 and scales 1.0 in rows
 * [from_pos, max_seq), as zero_kv_from leaves them
 * (asdsl/kernels/native/unified_engine.cpp:1263-1283). */
asdsl_status asdsl_kv_zero_from_q8(int8_t* k_cache, int8_t* v_cache, float* k_scale, float* v_scale,
                                   int n_kv_heads, int head_dim, int max_seq, int from_pos, asdsl_stream_t stream);

/* Zeroes rows [from_pos, max_seq) of every head of one layer's fp16 K and V
 * caches ([n_kv_heads][max_seq][head_dim], 16-byte aligned); from_pos < 0
 * counts as 0, from_pos >= max_seq does nothing.
 * Replaces UnifiedEngine::zero_kv_from (asdsl/kernels/native/unified_engine.cpp:1263-1283),
 * used by truncate_kv / restore_kv (1285-1307). */
asdsl_status asdsl_kv_zero_from(uint16_t* k_cache, uint16_t* v_cache, int n_kv_heads, int head_dim, int max_seq,
                                int from_pos, asdsl_stream_t stream);

/* Q4_S256 superblock GEMV: blocks[out][in/256][144] = 8 fp16 sub-scales
 * (one per 32 weights) then 128 nibble bytes (low nibble = even weight),
 * weights (q - 8) * s; x_q8/x_scales pre-quantized per 32 (group_size must
 * be 32; x_q8 16-byte aligned); in_features % 256 == 0, <= 20480; blocks
 * 16-byte aligned.
 * Replaces gemv_q4_s256_preq_avx2 (asdsl/kernels/native/gemv_q4_s256.cpp:79-209). */
asdsl_status asdsl_gemv_q4_s256(const uint8_t* blocks, const int8_t* x_q8, const float* x_scales, float* y,
                                int out_features, int in_features, int group_size, asdsl_stream_t stream);

/* The same with the fp32 activation quantized inside (A1 rule, groups of 32),
 * as the reference's engine does before calling it (unified_engine.cpp:1414-1416). */
asdsl_status asdsl_gemv_q4_s256_fused(const uint8_t* blocks, const float* x, float* y, int out_features,
                                      int in_features, asdsl_stream_t stream);

/* ------------------------------------------------------------- repackers
 * Load-time conversions of the quantized store's weights into the layouts
 * above, on the GPU; every output byte equals the reference's.  Inputs are
 * the asymmetric packed Q4 of the store (row-major, two nibbles per byte,
 * low nibble = even column) with fp32 scale and bias per (row, group), or
 * preq blocks.  All pointers are device memory; rows >= 1, cols a multiple
 * of the group size. */

/* preq (20-byte blocks) -> preq2 meta[rows][cols/32][4] +
 * quant[ceil(rows/4)][cols/32][64]; group_size must be 32.  preq and meta
 * 4-byte, quant 16-byte aligned.
 * Replaces repack_preq_blocks_to_preq2 (asdsl/quantization/repack_preq2.py:22-49). */
asdsl_status asdsl_repack_preq_to_preq2(const uint8_t* preq, uint8_t* meta, uint8_t* quant, int rows, int cols,
                                        int group_size, asdsl_stream_t stream);

/* packed + scales + biases (gs 32) -> 20-byte preq blocks[rows][cols/32]:
 * fp16(max(s, 1e-8)), fp16(-b / max(s, 1e-8)) (float64 division), the 16
 * packed bytes.  packed 16-byte, the rest 4-byte aligned.
 * Replaces repack_asymmetric_to_q4_32_blocks (asdsl/quantization/repack_q4_32.py:63-102). */
asdsl_status asdsl_repack_asym_to_q4_32(const uint8_t* packed, const float* scales, const float* biases,
                                        uint8_t* blocks, int rows, int cols, int group_size,
                                        asdsl_stream_t stream);

/* packed + scales + biases -> preq2 (meta, quant) at group_size 32 (the
 * composition repack_q4_32 -> repack_preq2, byte for byte) or 128 (the same
 * fp16 pair per group; 4-row bands of 64-byte row slots per group).  packed
 * and quant 16-byte, the rest 4-byte aligned.
 * Replaces repack_asymmetric_to_q4_32_blocks + repack_preq_blocks_to_preq2
 * (asdsl/quantization/repack_q4_32.py:63-102; repack_preq2.py:22-49) in the
 * preq cache build (experiments/phi4_cpu_run.py:627-787). */
asdsl_status asdsl_repack_asym_to_preq2(const uint8_t* packed, const float* scales, const float* biases,
                                        uint8_t* meta, uint8_t* quant, int rows, int cols, int group_size,
                                        asdsl_stream_t stream);

/* fp32 weights[rows][cols] -> 66-byte Q4_128 blocks: fp16(amax/7), levels
 * clip(round_half_even(w * f32(7/amax)) + 8, 0, 15); amax < 1e-12: scale 0,
 * nibbles 0x88.  group_size must be 128; weights 16-byte, blocks 4-byte aligned.
 * Replaces repack_fp32_to_q4_128_blocks (asdsl/quantization/repack_q4_128.py:72-92). */
asdsl_status asdsl_repack_fp32_to_q4_128(const float* weights, uint8_t* blocks, int rows, int cols, int group_size,
                                         asdsl_stream_t stream);

/* packed + scales + biases (gs 128) -> Q4_128 blocks: each group decoded in
 * float32 as (q - f32(zero)) * f32(max(s, 1e-8)), then requantized as above.
 * packed 16-byte, scales, biases and blocks 4-byte aligned.
 * Replaces repack_asymmetric_to_q4_128_blocks (asdsl/quantization/repack_q4_128.py:34-69). */
asdsl_status asdsl_repack_asym_to_q4_128(const uint8_t* packed, const float* scales, const float* biases,
                                         uint8_t* blocks, int rows, int cols, int group_size,
                                         asdsl_stream_t stream);

/* Q4_128 blocks[rows][cols/128][66] -> preq2-g128 (meta, quant): meta =
 * fp16 block scale | fp16 8.0 (the symmetric group as scale s, zero 8, so
 * every weight decodes to the same (q - 8) * s); the 64 nibble bytes move
 * into 4-row bands of 64-byte slots.  blocks 2-byte, meta 4-byte, quant
 * 16-byte aligned.  No counterpart in the reference (its g128 tensors stay
 * Q4_128 blocks, experiments/phi4_cpu_run.py:637-646); it lets the preq
 * cache at group size 128 feed the preq2-g128 GEMVs and decode step. */
asdsl_status asdsl_repack_q4_128_to_preq2(const uint8_t* blocks, uint8_t* meta, uint8_t* quant, int rows, int cols,
                                          asdsl_stream_t stream);

/* ------------------------------------------------------------- GGUF weights
 * K-quant tensors of a GGUF file, in the file's row-major block order (rows =
 * out_features, cols = in_features, a multiple of 256), on the device. */

/* ggml Q4_K blocks[rows][cols/256][144] -> fp32 weights[rows][cols]:
 * w = (d * sc) * q - (dmin * m) per 32-weight sub-block.  blocks and
 * weights 16-byte aligned.  Replaces dequant_tensor for Q4_K
 * (asdsl/io/gguf_loader.py:150-181, which calls gguf.quants.dequantize). */
asdsl_status asdsl_dequant_gguf_q4k(const uint8_t* blocks, float* weights, int rows, int cols,
                                   asdsl_stream_t stream);

/* ggml Q6_K blocks[rows][cols/256][210] -> fp32 weights[rows][cols]:
 * w = (d * scale) * (code - 32) per 16-weight group.  weights 16-byte
 * aligned.  Replaces dequant_tensor for Q6_K (asdsl/io/gguf_loader.py:150-181). */
asdsl_status asdsl_dequant_gguf_q6k(const uint8_t* blocks, float* weights, int rows, int cols,
                                   asdsl_stream_t stream);

/* ggml Q5_K blocks[rows][cols/256][176] -> fp32 weights[rows][cols]:
 * w = (d * sc) * q - (dmin * m) per 32-weight sub-block, q = the 4-bit code
 * with its fifth bit from the 32 high-bit bytes.  blocks and weights 16-byte
 * aligned.  Replaces dequant_tensor for Q5_K (asdsl/io/gguf_loader.py:150-181). */
asdsl_status asdsl_dequant_gguf_q5k(const uint8_t* blocks, float* weights, int rows, int cols,
                                   asdsl_stream_t stream);

/* ggml Q8_0 blocks[rows][cols/32][34] -> fp32 weights[rows][cols] (cols a
 * multiple of 32): w = code * d, one fp16 d per 32 int8 codes.  blocks 2-byte
 * and weights 16-byte aligned.  Replaces dequant_tensor for Q8_0
 * (asdsl/io/gguf_loader.py:150-181). */
asdsl_status asdsl_dequant_gguf_q8_0(const uint8_t* blocks, float* weights, int rows, int cols,
                                    asdsl_stream_t stream);

/* ggml's legacy 32-weight blocks[rows][cols/32] -> fp32 weights[rows][cols]
 * (cols a multiple of 32; blocks 2-byte and weights 16-byte aligned).  Nibble
 * byte j holds weight j (low) and j + 16 (high); Q5 blocks add a 32-bit word
 * of fifth bits (bit i: weight i).
 *   Q4_0 (18 B): fp16 d | nibbles;                 w = (q - 8) * d
 *   Q4_1 (20 B): fp16 d | fp16 m | nibbles;        w = d * q + m
 *   Q5_0 (22 B): fp16 d | high bits | nibbles;     w = (q - 16) * d
 *   Q5_1 (24 B): fp16 d | fp16 m | high bits | nibbles; w = d * q + m
 * Replace dequant_tensor for these types (asdsl/io/gguf_loader.py:150-181). */
asdsl_status asdsl_dequant_gguf_q4_0(const uint8_t* blocks, float* weights, int rows, int cols,
                                    asdsl_stream_t stream);
asdsl_status asdsl_dequant_gguf_q4_1(const uint8_t* blocks, float* weights, int rows, int cols,
                                    asdsl_stream_t stream);
asdsl_status asdsl_dequant_gguf_q5_0(const uint8_t* blocks, float* weights, int rows, int cols,
                                    asdsl_stream_t stream);
asdsl_status asdsl_dequant_gguf_q5_1(const uint8_t* blocks, float* weights, int rows, int cols,
                                    asdsl_stream_t stream);

/* ggml Q2_K blocks[rows][cols/256][84] and Q3_K blocks[rows][cols/256][110]
 * -> fp32 weights[rows][cols] (blocks 2-byte, weights 16-byte aligned).
 * Weight 128n + 32j + 16h + i sits in bits 2j..2j+1 of code byte
 * 32n + 16h + i under scale 8n + 2j + h.  Q2_K (16 scale bytes | codes |
 * fp16 d | fp16 dmin): w = (d * (s & 15)) * q - dmin * (s >> 4).  Q3_K
 * (32 high-mask bytes | codes | 12 bytes of 6-bit scales | fp16 d): q -= 4
 * unless mask bit 4n + j of byte 16h + i is set, w = (d * (scale - 32)) * q.
 * Replace dequant_tensor for Q2_K and Q3_K (asdsl/io/gguf_loader.py:150-181). */
asdsl_status asdsl_dequant_gguf_q2k(const uint8_t* blocks, float* weights, int rows, int cols,
                                   asdsl_stream_t stream);
asdsl_status asdsl_dequant_gguf_q3k(const uint8_t* blocks, float* weights, int rows, int cols,
                                   asdsl_stream_t stream);

/* ggml Q4_K blocks -> the ASDSL Q4_K variant blocks that asdsl_gemv_q4km_q8
 * reads (6-bit scales and mins as one linear bitstream, each sub-block's
 * codes in its own 16 bytes), losslessly, so that the GEMV computes ggml's
 * weights.  Both 16-byte aligned.  The reference hands the GGUF bytes to its
 * Q4_K GEMV unchanged (asdsl/io/gguf_loader.py:184-205 q4k_blocks_rowmajor,
 * experiments/phi4_cpu_run.py:1480-1521), which reads ggml's fields in the
 * variant's places; this entry point has no counterpart there. */
asdsl_status asdsl_repack_gguf_q4k_to_q4km(const uint8_t* gguf_blocks, uint8_t* q4km_blocks, int rows, int cols,
                                          asdsl_stream_t stream);

/* fp32 weights[rows][cols] -> symmetric group-wise Q4: packed[rows*cols/2]
 * (low nibble = even element), scales[groups] = f32(f16(max(amax, 1e-5) /
 * 7.5)), biases[groups] = -7.5 * scale; q = clip(rne(w / max(scale, 1e-4) +
 * 7.5), 0, 15).  group_size 32, 64 or 128 dividing cols; weights 16-byte,
 * packed 2-byte, scales and biases 4-byte aligned.  Replaces
 * quantize_weights(bits=4, symmetric=True) (asdsl/quantization/core.py:358-420)
 * with the scale/bias form of load_from_gguf (experiments/phi4_cpu_run.py:1444-1459);
 * asdsl_repack_asym_to_preq2 then builds the preq2 operands. */
asdsl_status asdsl_quantize_q4_symmetric(const float* weights, uint8_t* packed, float* scales, float* biases,
                                        int rows, int cols, int group_size, asdsl_stream_t stream);

#ifdef __cplusplus
}
#endif

#endif /* ASDSL_HIP_H */
