// Error text, device queries and the library identity entry points.
#include <stdarg.h>
#include <stdio.h>
#include <stdlib.h>

#include <mutex>

#include "abi_util.hpp"

namespace asdsl {

namespace {
thread_local char g_error[512] = "";
thread_local LaunchEvents g_events;

struct DeviceShape {
    int cus = -1;
};
std::mutex g_shape_mu;
DeviceShape g_shape[64];

struct Workspace {
    void* ptr = nullptr;
    size_t bytes = 0;
};
std::mutex g_ws_mu;
Workspace g_ws[64];
}  // namespace

void set_error(const char* fmt, ...) {
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(g_error, sizeof(g_error), fmt, ap);
    va_end(ap);
}

void clear_error() { g_error[0] = '\0'; }

LaunchEvents take_launch_events() {
    const LaunchEvents ev = g_events;
    g_events = LaunchEvents{};
    return ev;
}

int cu_count_current() {
    int dev = -1;
    hipError_t e = hipGetDevice(&dev);
    if (e != hipSuccess || dev < 0 || dev >= 64) {
        set_error("no usable HIP device: %s", hipGetErrorString(e));
        return -1;
    }
    std::lock_guard<std::mutex> lock(g_shape_mu);
    if (g_shape[dev].cus < 0) {
        int cus = 0;
        e = hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev);
        if (e != hipSuccess || cus <= 0) {
            set_error("hipDeviceGetAttribute(MultiprocessorCount) failed: %s", hipGetErrorString(e));
            return -1;
        }
        g_shape[dev].cus = cus;
    }
    return g_shape[dev].cus;
}

asdsl_status device_workspace(hipStream_t stream, size_t bytes, void** out, const char* what) {
    int dev = -1;
    hipError_t e = hipGetDevice(&dev);
    if (e != hipSuccess || dev < 0 || dev >= 64) {
        set_error("%s: no usable HIP device: %s", what, hipGetErrorString(e));
        return ASDSL_ERR_HIP;
    }
    std::lock_guard<std::mutex> lock(g_ws_mu);
    Workspace& ws = g_ws[dev];
    if (ws.bytes < bytes) {
        hipStreamCaptureStatus cap = hipStreamCaptureStatusNone;
        e = hipStreamIsCapturing(stream, &cap);
        if (e != hipSuccess) {
            set_error("%s: hipStreamIsCapturing failed: %s", what, hipGetErrorString(e));
            return ASDSL_ERR_HIP;
        }
        if (cap != hipStreamCaptureStatusNone) {
            set_error("%s: needs a %zu-byte work buffer, which cannot be allocated under graph capture; "
                      "make one call of this size before capturing", what, bytes);
            return ASDSL_ERR_UNSUPPORTED;
        }
        // A smaller buffer is kept, not freed: queued work or a graph captured
        // earlier may still use it.
        const size_t grown = (bytes + (1u << 20) - 1) & ~static_cast<size_t>((1u << 20) - 1);
        void* fresh = nullptr;
        e = hipMalloc(&fresh, grown);
        if (e != hipSuccess) {
            set_error("%s: hipMalloc(%zu) for the work buffer failed: %s", what, grown, hipGetErrorString(e));
            return ASDSL_ERR_HIP;
        }
        ws.ptr = fresh;
        ws.bytes = grown;
    }
    *out = ws.ptr;
    return ASDSL_OK;
}

asdsl_status work_buffer(hipStream_t stream, void* work, size_t work_bytes, size_t need, void** out,
                         const char* what) {
    if (work == nullptr) return device_workspace(stream, need, out, what);
    if (work_bytes < need) {
        set_error("%s: work buffer of %zu bytes, %zu needed", what, work_bytes, need);
        return ASDSL_ERR_INVALID_ARGUMENT;
    }
    if (reinterpret_cast<uintptr_t>(work) % 256 != 0) {
        set_error("%s: work buffer must be 256-byte aligned", what);
        return ASDSL_ERR_INVALID_ARGUMENT;
    }
    *out = work;
    return ASDSL_OK;
}

int env_knob(const char* name) {
    const char* v = getenv(name);
    if (!v || !*v) return 0;
    const int n = atoi(v);
    return n > 0 ? n : 0;
}

asdsl_status launch_status(const char* what) {
    const hipError_t e = hipGetLastError();
    if (e != hipSuccess) {
        set_error("%s: kernel launch failed: %s", what, hipGetErrorString(e));
        return ASDSL_ERR_HIP;
    }
    return ASDSL_OK;
}

}  // namespace asdsl

extern "C" int asdsl_abi_version(void) { return ASDSL_ABI_VERSION; }

extern "C" const char* asdsl_last_error(void) { return asdsl::g_error; }

extern "C" int asdsl_device_cu_count(void) { return asdsl::cu_count_current(); }

extern "C" asdsl_status asdsl_profile_next_launch(void* start_event, void* stop_event) {
    asdsl::g_events.start = static_cast<hipEvent_t>(start_event);
    asdsl::g_events.stop = static_cast<hipEvent_t>(stop_event);
    return ASDSL_OK;
}
