// Build wrapper for the reference's asdsl/kernels/native/gemv_q4_avx2.cpp
// (test infrastructure, oracle/_ref only).  That file defines its own
// _cvtsh_ss helper (gemv_q4_avx2.cpp:1510), which collides with the one in
// GCC's <f16cintrin.h>.  Including the intrinsics first and renaming the
// file's helper with a macro compiles the reference source unchanged.
#include <immintrin.h>
#define _cvtsh_ss asdsl_ref_local_cvtsh_ss
#include "gemv_q4_avx2.cpp"
