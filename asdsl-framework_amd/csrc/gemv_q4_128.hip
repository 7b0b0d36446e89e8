// Q4_128 (symmetric g128, 66-byte blocks) GEMV entry points.
//
// Reference: gemv_q4_128_preq_avx2 (asdsl/kernels/native/gemv_q4_128.cpp:94-257),
//   block layout asdsl/quantization/repack_q4_128.py:1-6 and 192-262.  The
//   kernel is the shared row-major block GEMV of rowblk_gemv.hpp with the
//   implicit zero-point 8.
#include "rowblk_gemv.hpp"

namespace asdsl {
namespace {

int check_q4_128_args(const void* blocks, const void* x, const void* y, int M, int K, int gs, const char* fn) {
    if (!blocks || !x || !y) {
        set_error("%s: null pointer", fn);
        return 1;
    }
    if (reinterpret_cast<uintptr_t>(blocks) % 2 != 0) {
        set_error("%s: blocks must be 2-byte aligned", fn);
        return 1;
    }
    if (gs != 128) {
        set_error("%s: group_size must be 128", fn);
        return 1;
    }
    if (M <= 0 || K <= 0) {
        set_error("%s: invalid dimensions", fn);
        return 1;
    }
    if (K % 128 != 0) {
        set_error("%s: in_features must be divisible by 128", fn);
        return 1;
    }
    if (K / 128 > 140) {  // the reference keeps per-group sums in x_sums[140]
        set_error("%s: n_groups exceeds buffer", fn);
        return 1;
    }
    return 0;
}

}  // namespace
}  // namespace asdsl

using namespace asdsl;

extern "C" asdsl_status asdsl_gemv_q4_128_preq(const uint8_t* blocks, const int8_t* x_q8, const float* x_scales,
                                               float* y, int out_features, int in_features, int group_size,
                                               asdsl_stream_t stream) {
    if (check_q4_128_args(blocks, x_q8, y, out_features, in_features, group_size, "gemv_q4_128_preq_avx2"))
        return ASDSL_ERR_INVALID_ARGUMENT;
    ASDSL_CHECK_ARG(x_scales != nullptr, "gemv_q4_128_preq_avx2: null pointer");
    ASDSL_CU_COUNT(cus);
    return launch_rowblk<RowLayout::kQ4_128, 128, true>(blocks, nullptr, nullptr, x_q8, x_scales, y, out_features, in_features,
                                             as_hip(stream), cus);
}

extern "C" asdsl_status asdsl_gemv_q4_128_fused(const uint8_t* blocks, const float* x, float* y, int out_features,
                                                int in_features, int group_size, asdsl_stream_t stream) {
    if (check_q4_128_args(blocks, x, y, out_features, in_features, group_size, "gemv_q4_128_fused"))
        return ASDSL_ERR_INVALID_ARGUMENT;
    ASDSL_CU_COUNT(cus);
    return launch_rowblk<RowLayout::kQ4_128, 128, false>(blocks, nullptr, x, nullptr, nullptr, y, out_features, in_features,
                                             as_hip(stream), cus);
}
