// Symmetric packed Q4 x Q8 GEMV and the Q4_K (ASDSL variant) superblock GEMV.
//
// Reference: gemv_q4_q8_avx2 (asdsl/kernels/native/gemv_q4_avx2.cpp:131-253) and
//   gemv_q4km_q8_avx2 (gemv_q4_avx2.cpp:283-420).  Both quantize the fp32
//   activation inside the call (per group_size with the A1 rule, resp. per 32
//   with the Q4_K rule).  Kernel: the shared row-major block GEMV of
//   rowblk_gemv.hpp.
#include "rowblk_gemv.hpp"

using namespace asdsl;

extern "C" asdsl_status asdsl_gemv_q4_q8(const uint8_t* weights_packed, const float* scales, const float* x, float* y,
                                         int out_features, int in_features, int group_size, asdsl_stream_t stream) {
    ASDSL_CHECK_ARG(weights_packed && scales && x && y, "gemv_q4_q8_avx2: null pointer");
    ASDSL_CHECK_ARG(out_features > 0 && in_features > 0, "gemv_q4_q8_avx2: invalid dimensions");
    ASDSL_CHECK_ARG(group_size == 32 || group_size == 64 || group_size == 128,
                    "gemv_q4_q8_avx2: group_size must be 32, 64 or 128");
    ASDSL_CHECK_ARG(in_features % group_size == 0, "gemv_q4_q8_avx2: in_features must be divisible by group_size");
    ASDSL_CHECK_ARG(in_features <= 20480, "gemv_q4_q8_avx2: in_features must be <= 20480");
    ASDSL_CHECK_ARG(reinterpret_cast<uintptr_t>(weights_packed) % 16 == 0,
                    "gemv_q4_q8_avx2: weights must be 16-byte aligned");
    ASDSL_CU_COUNT(cus);
    hipStream_t s = as_hip(stream);
    if (group_size == 32)
        return launch_rowblk<RowLayout::kPacked, 32, false>(weights_packed, scales, x, nullptr, nullptr, y,
                                                             out_features, in_features, s, cus);
    if (group_size == 64)
        return launch_rowblk<RowLayout::kPacked, 64, false>(weights_packed, scales, x, nullptr, nullptr, y,
                                                             out_features, in_features, s, cus);
    return launch_rowblk<RowLayout::kPacked, 128, false>(weights_packed, scales, x, nullptr, nullptr, y, out_features,
                                                          in_features, s, cus);
}

extern "C" asdsl_status asdsl_gemv_q4km_q8(const uint8_t* weights_q4km, const float* x, float* y, int out_features,
                                           int in_features, asdsl_stream_t stream) {
    ASDSL_CHECK_ARG(weights_q4km && x && y, "gemv_q4km_q8_avx2: null pointer");
    ASDSL_CHECK_ARG(out_features > 0 && in_features > 0, "gemv_q4km_q8_avx2: invalid dimensions");
    ASDSL_CHECK_ARG(in_features % 256 == 0, "in_features must be divisible by 256 for Q4_K_M");
    ASDSL_CHECK_ARG(in_features <= 20480, "gemv_q4km_q8_avx2: in_features must be <= 20480");
    ASDSL_CHECK_ARG(reinterpret_cast<uintptr_t>(weights_q4km) % 16 == 0,
                    "gemv_q4km_q8_avx2: weights must be 16-byte aligned");
    ASDSL_CU_COUNT(cus);
    return launch_rowblk<RowLayout::kQ4K, 32, false>(weights_q4km, nullptr, x, nullptr, nullptr, y, out_features,
                                                      in_features, as_hip(stream), cus);
}

// Q4_S256 superblock GEMV (asdsl/kernels/native/gemv_q4_s256.cpp:79-209):
// y[r] = sum_sub s_sub * xs_sub * (sum q*x8 - 8 * sum x8) over 32-weight
// sub-blocks, with the activation quantized per 32 (A1 rule) -- given as
// x_q8/x_scales (the reference's interface) or quantized inside (_fused).
static asdsl_status check_s256(const uint8_t* blocks, float* y, int out_features, int in_features, const char* fn) {
    ASDSL_CHECK_ARG(blocks && y, "%s: null pointer", fn);
    ASDSL_CHECK_ARG(out_features > 0 && in_features > 0, "%s: invalid dimensions", fn);
    ASDSL_CHECK_ARG(in_features % 256 == 0, "gemv_q4_s256: in_features must be divisible by 256");
    ASDSL_CHECK_ARG(in_features <= 20480, "%s: in_features must be <= 20480", fn);
    ASDSL_CHECK_ARG(reinterpret_cast<uintptr_t>(blocks) % 16 == 0, "%s: blocks must be 16-byte aligned", fn);
    return ASDSL_OK;
}

extern "C" asdsl_status asdsl_gemv_q4_s256(const uint8_t* blocks, const int8_t* x_q8, const float* x_scales, float* y,
                                           int out_features, int in_features, int group_size, asdsl_stream_t stream) {
    const asdsl_status cs = check_s256(blocks, y, out_features, in_features, "gemv_q4_s256_preq_avx2");
    if (cs != ASDSL_OK) return cs;
    ASDSL_CHECK_ARG(x_q8 && x_scales, "gemv_q4_s256_preq_avx2: null pointer");
    ASDSL_CHECK_ARG(group_size == 32, "gemv_q4_s256_preq_avx2: group_size (activation groups) must be 32");
    ASDSL_CHECK_ARG(reinterpret_cast<uintptr_t>(x_q8) % 16 == 0, "gemv_q4_s256_preq_avx2: x_q8 must be 16-byte aligned");
    ASDSL_CU_COUNT(cus);
    return launch_rowblk<RowLayout::kQ4S256, 32, true>(blocks, nullptr, nullptr, x_q8, x_scales, y, out_features,
                                                        in_features, as_hip(stream), cus);
}

extern "C" asdsl_status asdsl_gemv_q4_s256_fused(const uint8_t* blocks, const float* x, float* y, int out_features,
                                                 int in_features, asdsl_stream_t stream) {
    const asdsl_status cs = check_s256(blocks, y, out_features, in_features, "gemv_q4_s256_fused");
    if (cs != ASDSL_OK) return cs;
    ASDSL_CHECK_ARG(x != nullptr, "gemv_q4_s256_fused: null pointer");
    ASDSL_CU_COUNT(cus);
    return launch_rowblk<RowLayout::kQ4S256, 32, false>(blocks, nullptr, x, nullptr, nullptr, y, out_features,
                                                         in_features, as_hip(stream), cus);
}
