// Calibration of cross-workgroup synchronisation (no counterpart in the
// reference): the cost of one grid-wide handoff between phases of a kernel
// whose workgroups all run at once, which decides whether a decode step can
// live in one persistent kernel instead of six launches per layer.
//
// One cooperative launch of `grid` workgroups runs `rounds` rounds; a round
// is one wait for every workgroup.  Modes:
//   0  flag barrier: each workgroup stores its own flag word (agent scope),
//      one wave polls all flags (agent-scope loads);
//   1  flag barrier with a data handoff: before its flag each workgroup
//      stores its 16-float slice of a 4096-float vector, and after the wait
//      every workgroup reads the whole vector back (agent-scope loads) and
//      folds it into the next round's values; a second wait (its own flag
//      array) keeps the next round from overwriting a vector still read;
//   2  counter barrier: one agent-scope atomic add per workgroup on a shared
//      counter, one wave polls the counter.
// Every wait is bounded (grid_sync.hpp); a timed-out run raises word 0 of
// the work buffer and every workgroup exits.
#include "abi_util.hpp"
#include "grid_sync.hpp"

namespace asdsl {
namespace {

constexpr int kProbeThreads = 256;
constexpr int kVec = 4096;
constexpr int kFlagsAt = 64;  // words: abort, counter, then flags from here

__global__ __launch_bounds__(kProbeThreads) void grid_sync_probe_kernel(uint32_t* __restrict__ work, int mode,
                                                                         int rounds, int spin_limit) {
    uint32_t* abort = work;
    uint32_t* counter = work + 1;
    const int fstride = static_cast<int>((gridDim.x + 63) / 64) * 64;
    uint32_t* flags = work + kFlagsAt;
    uint32_t* flags2 = flags + fstride;  // mode 1: "the vector has been read" flags
    float* vec = reinterpret_cast<float*>(flags2 + fstride);
    __shared__ int s_ok;
    __shared__ float s_red[kProbeThreads / 64];
    const int tid = static_cast<int>(threadIdx.x);
    const int nwg = static_cast<int>(gridDim.x);
    float carry = static_cast<float>(blockIdx.x);
    for (int r = 1; r <= rounds; ++r) {
        const uint32_t epoch = static_cast<uint32_t>(r);
        if (mode == 1 && tid < 16 && static_cast<int>(blockIdx.x) * 16 < kVec)
            agent_store_f(vec + blockIdx.x * 16 + tid, carry + static_cast<float>(tid));
        wait_vm_stores();
        __syncthreads();
        if (tid < 64) {
            bool ok;
            if (mode == 2) {
                if (tid == 0) __hip_atomic_fetch_add(counter, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                const uint32_t target = static_cast<uint32_t>(nwg) * epoch;
                ok = true;
                for (int spins = 0;; ++spins) {
                    if (agent_load(counter) >= target) break;
                    if (agent_load(abort) != 0u) { ok = false; break; }
                    if (spins >= spin_limit) {
                        if (tid == 0) agent_store(abort, 1u);
                        ok = false;
                        break;
                    }
                    __builtin_amdgcn_s_sleep(1);
                }
            } else {
                if (tid == 0) agent_store(flags + blockIdx.x, epoch);
                ok = wave_wait_flags(flags, nwg, epoch, abort, spin_limit);
            }
            if (tid == 0) s_ok = ok ? 1 : 0;
        }
        __syncthreads();
        if (!s_ok) return;  // uniform per workgroup
        if (mode == 1) {
            float sum = 0.0f;
            for (int i = tid; i < kVec && i < nwg * 16; i += kProbeThreads) sum += agent_load_f(vec + i);
            for (int o = 32; o >= 1; o >>= 1) sum += __shfl_xor(sum, o, 64);
            if ((tid & 63) == 0) s_red[tid >> 6] = sum;
            __syncthreads();
            carry = s_red[0] + s_red[1] + s_red[2] + s_red[3];
            // the next round's stores overwrite the vector: everyone must
            // have read it first (a second wait, on the second flag array)
            __syncthreads();
            if (tid < 64) {
                if (tid == 0) agent_store(flags2 + blockIdx.x, epoch);
                const bool ok = wave_wait_flags(flags2, nwg, epoch, abort, spin_limit);
                if (tid == 0) s_ok = ok ? 1 : 0;
            }
            __syncthreads();
            if (!s_ok) return;
        }
    }
    if (blockIdx.x == 0 && tid == 0) agent_store_f(reinterpret_cast<float*>(work + 2), carry);
}

}  // namespace
}  // namespace asdsl

using namespace asdsl;

extern "C" size_t asdsl_grid_sync_probe_work_bytes(int grid) {
    if (grid <= 0) return 0;
    return (static_cast<size_t>(kFlagsAt) + 2 * static_cast<size_t>((grid + 63) / 64) * 64 + kVec) *
           sizeof(uint32_t);
}

extern "C" asdsl_status asdsl_grid_sync_probe(int mode, int rounds, int grid, void* work, size_t work_bytes,
                                              int spin_limit, asdsl_stream_t stream) {
    ASDSL_CHECK_ARG(mode >= 0 && mode <= 2, "grid_sync_probe: mode must be 0, 1 or 2");
    ASDSL_CHECK_ARG(rounds > 0 && rounds < (1 << 30), "grid_sync_probe: rounds must be positive");
    ASDSL_CHECK_ARG(grid > 0 && grid <= 4096, "grid_sync_probe: grid must be in [1, 4096]");
    ASDSL_CHECK_ARG(work && work_bytes >= asdsl_grid_sync_probe_work_bytes(grid),
                    "grid_sync_probe: work must hold asdsl_grid_sync_probe_work_bytes(grid) bytes");
    ASDSL_CHECK_ARG(spin_limit > 0, "grid_sync_probe: spin_limit must be positive");
    ASDSL_CU_COUNT(cus);
    int per_cu = 0;
    if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, grid_sync_probe_kernel, kProbeThreads, 0) !=
            hipSuccess ||
        static_cast<long long>(per_cu) * cus < grid) {
        set_error("grid_sync_probe: %d workgroups do not fit on the device at once", grid);
        return ASDSL_ERR_UNSUPPORTED;
    }
    uint32_t* w = static_cast<uint32_t*>(work);
    void* args[] = {&w, &mode, &rounds, &spin_limit};
    const hipError_t e = hipLaunchCooperativeKernel(reinterpret_cast<const void*>(grid_sync_probe_kernel), dim3(grid),
                                                    dim3(kProbeThreads), args, 0, as_hip(stream));
    if (e != hipSuccess) {
        set_error("grid_sync_probe: cooperative launch failed: %s", hipGetErrorString(e));
        return ASDSL_ERR_HIP;
    }
    return ASDSL_OK;
}
