// preq g32 Q4 GEMV entry points (row-major 20-byte blocks).
//
// Reference: gemv_q4_32_preq_avx2 and the fused 4row/8row variants
//   (asdsl/kernels/native/gemv_q4_preq_restored.cpp:281-336,476-669),
//   block layout asdsl/quantization/repack_q4_32.py:1-7.  The kernel is the
//   shared row-major block GEMV of rowblk_gemv.hpp.
#include "rowblk_gemv.hpp"

namespace asdsl {
namespace {

int check_preq_args(const void* blocks, const void* x, const void* y, int M, int K, int gs, const char* fn) {
    if (!blocks || !x || !y) {
        set_error("%s: null input pointer", fn);
        return 1;
    }
    if (reinterpret_cast<uintptr_t>(blocks) % 4 != 0) {
        set_error("%s: blocks must be 4-byte aligned", fn);
        return 1;
    }
    if (gs != 32) {
        set_error("%s: group_size must be 32", fn);
        return 1;
    }
    if (M <= 0 || K <= 0) {
        set_error("%s: invalid dimensions", fn);
        return 1;
    }
    if (K % gs != 0) {
        set_error("%s: in_features must be divisible by group_size", fn);
        return 1;
    }
    if (K / gs > 640) {
        set_error("%s: n_groups exceeds buffer", fn);
        return 1;
    }
    return 0;
}

}  // namespace
}  // namespace asdsl

using namespace asdsl;

extern "C" asdsl_status asdsl_gemv_q4_32_preq(const uint8_t* blocks, const int8_t* x_q8, const float* x_scales,
                                              float* y, int out_features, int in_features, int group_size,
                                              asdsl_stream_t stream) {
    if (check_preq_args(blocks, x_q8, y, out_features, in_features, group_size, "gemv_q4_32_preq"))
        return ASDSL_ERR_INVALID_ARGUMENT;
    ASDSL_CHECK_ARG(x_scales != nullptr, "gemv_q4_32_preq: null input pointer");
    ASDSL_CU_COUNT(cus);
    return launch_rowblk<RowLayout::kPreq, 32, true>(blocks, nullptr, nullptr, x_q8, x_scales, y, out_features, in_features,
                                           as_hip(stream), cus);
}

extern "C" asdsl_status asdsl_gemv_q4_32_preq_fused(const uint8_t* blocks, const float* x, float* y,
                                                    int out_features, int in_features, int group_size,
                                                    asdsl_stream_t stream) {
    if (check_preq_args(blocks, x, y, out_features, in_features, group_size, "gemv_q4_32_preq_fused"))
        return ASDSL_ERR_INVALID_ARGUMENT;
    ASDSL_CU_COUNT(cus);
    return launch_rowblk<RowLayout::kPreq, 32, false>(blocks, nullptr, x, nullptr, nullptr, y, out_features, in_features,
                                           as_hip(stream), cus);
}
