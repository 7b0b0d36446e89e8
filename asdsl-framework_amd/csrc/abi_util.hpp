// Host-side helpers for the C ABI: per-thread error text, argument checks,
// launch checks and the cached device shape used to size grids.
#pragma once

#include <hip/hip_runtime.h>

#include "asdsl_hip.h"

namespace asdsl {

void set_error(const char* fmt, ...) __attribute__((format(printf, 1, 2)));
void clear_error();

// Compute units of the current device; -1 (error text set) when no device.
int cu_count_current();

// Checks hipGetLastError() after a launch; maps a failure to ASDSL_ERR_HIP.
asdsl_status launch_status(const char* what);

inline hipStream_t as_hip(asdsl_stream_t s) { return reinterpret_cast<hipStream_t>(s); }

// Integer tuning knob from the environment, read once (0 = unset).  Knobs
// only change launch shapes (and with them the fp32 summation order), never
// the formula: ASDSL_HIP_WG_PER_CU caps workgroups per compute unit,
// ASDSL_HIP_KSPLIT forces the K split of the preq2 kernels.
int env_knob(const char* name);

// Workgroups for a streaming kernel: enough tiles for every wave, capped at
// `per_cu` workgroups per compute unit (waves then loop over tiles).
inline int stream_grid(long long tiles, int waves_per_wg, int per_cu, int cus) {
    long long wgs = (tiles + waves_per_wg - 1) / waves_per_wg;
    static const int knob = env_knob("ASDSL_HIP_WG_PER_CU");
    if (knob > 0) per_cu = knob;
    const long long cap = static_cast<long long>(per_cu) * (cus > 0 ? cus : 256);
    if (wgs > cap) wgs = cap;
    if (wgs < 1) wgs = 1;
    return static_cast<int>(wgs);
}

}  // namespace asdsl

#define ASDSL_CHECK_ARG(cond, ...)                 \
    do {                                           \
        if (!(cond)) {                             \
            ::asdsl::set_error(__VA_ARGS__);       \
            return ASDSL_ERR_INVALID_ARGUMENT;     \
        }                                          \
    } while (0)

#define ASDSL_CU_COUNT(var)                        \
    const int var = ::asdsl::cu_count_current();   \
    if (var < 0) return ASDSL_ERR_HIP
