// Cross-workgroup signalling for kernels whose workgroups all run at once
// (grid <= co-resident capacity; launched cooperatively or sized from the
// occupancy query).
//
// MI355X has one L2 per XCD and the L2s are not coherent with each other,
// so a value one workgroup stores is not seen by a workgroup on another XCD
// through ordinary loads.  Signals and the small vectors passed between
// phases therefore use agent-scope atomic loads and stores (relaxed), which
// the compiler emits with the device-scope cache bits: they are performed at
// the device's coherence point instead of in a private L2.  No read-modify-
// write atomics and no whole-cache write-back or invalidate are needed:
//   producer: agent-scope stores of its data, wait for them to complete
//             (s_waitcnt vmcnt(0)), then an agent-scope store of its flag;
//   consumer: polls the flags with agent-scope loads, then reads the data
//             with agent-scope loads.
// Every wait is bounded: after `spin_limit` polls the waiter raises the
// shared abort word and gives up, and every other waiter sees the abort word
// on its next poll and gives up too, so the grid always drains.  Epochs are
// compared modulo 2^32.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace asdsl {

__device__ __forceinline__ void agent_store(uint32_t* p, uint32_t v) {
    __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

__device__ __forceinline__ uint32_t agent_load(const uint32_t* p) {
    return __hip_atomic_load(const_cast<uint32_t*>(p), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

__device__ __forceinline__ void agent_store_f(float* p, float v) {
    __hip_atomic_store(reinterpret_cast<uint32_t*>(p), __float_as_uint(v), __ATOMIC_RELAXED,
                       __HIP_MEMORY_SCOPE_AGENT);
}

__device__ __forceinline__ float agent_load_f(const float* p) {
    return __uint_as_float(__hip_atomic_load(reinterpret_cast<uint32_t*>(const_cast<float*>(p)), __ATOMIC_RELAXED,
                                             __HIP_MEMORY_SCOPE_AGENT));
}

// Waits until this wave's earlier vector-memory operations (the agent-scope
// stores above all) have completed; also a compiler barrier.
__device__ __forceinline__ void wait_vm_stores() { asm volatile("s_waitcnt vmcnt(0)" ::: "memory"); }

__device__ __forceinline__ bool epoch_reached(uint32_t flag, uint32_t epoch) {
    return static_cast<int32_t>(flag - epoch) >= 0;
}

// Called by one whole wave: polls flags[0..n) until every one has reached
// `epoch`.  Returns false (and raises *abort) after spin_limit polls, or
// false at once when another waiter raised *abort.
__device__ __forceinline__ bool wave_wait_flags(const uint32_t* flags, int n, uint32_t epoch, uint32_t* abort,
                                                int spin_limit) {
    const int lane = static_cast<int>(threadIdx.x) & 63;
    for (int spins = 0;; ++spins) {
        bool ok = true;
        for (int i = lane; i < n; i += 64) ok = ok && epoch_reached(agent_load(flags + i), epoch);
        if (__all(ok)) return true;
        if (agent_load(abort) != 0u) return false;
        if (spins >= spin_limit) {
            if (lane == 0) agent_store(abort, 1u);
            return false;
        }
        __builtin_amdgcn_s_sleep(1);
    }
}

}  // namespace asdsl
