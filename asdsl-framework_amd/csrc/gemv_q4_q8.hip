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
