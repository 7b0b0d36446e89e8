// Build wrapper for the reference's asdsl/kernels/native/gemv_q4_s256.cpp
// (test infrastructure, oracle/_ref only).  That kernel has no Python
// binding in the reference (UnifiedEngine calls it for weight_format 1), so
// the source is compiled unchanged and given one C entry point for ctypes.
#include "gemv_q4_s256.cpp"

extern "C" void ref_gemv_q4_s256(const uint8_t* blocks, const int8_t* x_q8, const float* x_scales, float* y,
                                 int out_features, int in_features) {
    gemv_q4_s256_preq_avx2(blocks, x_q8, x_scales, y, out_features, in_features, 32);
}
