// Streaming-read calibration kernel (no counterpart in the reference).
//
// Reads `bytes` bytes with 16-byte non-temporal loads, four in flight per
// lane, and folds them into a value that is stored only if it equals a fixed
// sentinel (so the loads cannot be dropped and nothing is written in
// practice).  Timed the same way as a GEMV (back-to-back launches in a HIP
// graph over rotated buffers), it gives the practical ceiling for streaming
// that many bytes in one launch, which the GEMV roofline figures are read
// against: at 31.5 MB a launch cannot reach 8 TB/s because of its dispatch
// and ramp time.
#include "abi_util.hpp"

namespace asdsl {
namespace {

typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
constexpr int kReadThreads = 512;

__global__ __launch_bounds__(kReadThreads) void stream_read_kernel(const u32x4* __restrict__ p, size_t n16,
                                                                    uint32_t* __restrict__ sink) {
    uint32_t acc = 0;
    const size_t stride = static_cast<size_t>(gridDim.x) * kReadThreads;
    size_t i = static_cast<size_t>(blockIdx.x) * kReadThreads + threadIdx.x;
    for (; i + 3 * stride < n16; i += 4 * stride) {
        const u32x4 a = __builtin_nontemporal_load(p + i);
        const u32x4 b = __builtin_nontemporal_load(p + i + stride);
        const u32x4 c = __builtin_nontemporal_load(p + i + 2 * stride);
        const u32x4 d = __builtin_nontemporal_load(p + i + 3 * stride);
        acc ^= (a.x ^ a.y ^ a.z ^ a.w) ^ (b.x ^ b.y ^ b.z ^ b.w) ^ (c.x ^ c.y ^ c.z ^ c.w) ^ (d.x ^ d.y ^ d.z ^ d.w);
    }
    for (; i < n16; i += stride) {
        const u32x4 a = __builtin_nontemporal_load(p + i);
        acc ^= a.x ^ a.y ^ a.z ^ a.w;
    }
    if (acc == 0x9E3779B9u) sink[0] = acc;
}

}  // namespace
}  // namespace asdsl

using namespace asdsl;

extern "C" asdsl_status asdsl_stream_read(const void* data, size_t bytes, uint32_t* sink, int grid,
                                          asdsl_stream_t stream) {
    ASDSL_CHECK_ARG(data && sink, "stream_read: null pointer");
    ASDSL_CHECK_ARG(bytes >= 16 && bytes % 16 == 0, "stream_read: bytes must be a positive multiple of 16");
    ASDSL_CHECK_ARG(reinterpret_cast<uintptr_t>(data) % 16 == 0, "stream_read: data must be 16-byte aligned");
    ASDSL_CU_COUNT(cus);
    const int g = grid > 0 ? grid : cus;
    return launch("stream_read_kernel", stream_read_kernel, dim3(g), dim3(kReadThreads), 0, as_hip(stream),
                  static_cast<const u32x4*>(data), bytes / 16, sink);
}
