// Error text, device queries and the library identity entry points.
#include <stdarg.h>
#include <stdio.h>
#include <stdlib.h>

#include <mutex>
#include <vector>

#include "abi_util.hpp"

namespace asdsl {

thread_local const char* g_stage = nullptr;

namespace {
thread_local char g_error[512] = "";
thread_local LaunchEvents g_events;

// The stage recorder of asdsl_profile_stages_begin/_end: one event pair per
// launch from a pool that is created at begin and kept for later sessions.
constexpr int kMaxStageLaunches = 65536;
struct StageRecord {
    const char* label;
    LaunchEvents ev;
};
struct StageRecorder {
    bool armed = false;
    int max = 0;
    int launches = 0;  // launches while armed, recorded or not
    std::vector<StageRecord> recs;
    std::vector<hipEvent_t> pool;
};
thread_local StageRecorder g_rec;

struct DeviceShape {
    int cus = -1;
};
std::mutex g_shape_mu;
DeviceShape g_shape[64];

struct Workspace {
    void* ptr = nullptr;
    size_t bytes = 0;
    bool fixed = false;  // asdsl_reserve_workspace: never grown again
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

asdsl_status take_launch_events(const char* what, hipStream_t stream, LaunchEvents* ev) {
    *ev = g_events;
    g_events = LaunchEvents{};
    if (!g_rec.armed) return ASDSL_OK;
    ++g_rec.launches;
    if (ev->start != nullptr || ev->stop != nullptr) return ASDSL_OK;  // explicit pair wins (end reports it)
    hipStreamCaptureStatus cs = hipStreamCaptureStatusNone;
    if (hipStreamIsCapturing(stream, &cs) == hipSuccess && cs != hipStreamCaptureStatusNone) {
        set_error("%s: stage recording is armed on a stream under graph capture", what);
        return ASDSL_ERR_UNSUPPORTED;
    }
    const size_t i = g_rec.recs.size();
    if (static_cast<int>(i) >= g_rec.max) return ASDSL_OK;  // past the limit: end reports it
    ev->start = g_rec.pool[2 * i];
    ev->stop = g_rec.pool[2 * i + 1];
    g_rec.recs.push_back(StageRecord{g_stage != nullptr ? g_stage : what, *ev});
    return ASDSL_OK;
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
    if (ws.bytes < bytes && ws.fixed) {
        set_error("%s: needs a %zu-byte work buffer; %zu bytes were reserved by asdsl_reserve_workspace "
                  "(reserve more, or pass a work buffer)", what, bytes, ws.bytes);
        return ASDSL_ERR_INVALID_ARGUMENT;
    }
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

asdsl_status reserve_workspace(size_t bytes) {
    int dev = -1;
    hipError_t e = hipGetDevice(&dev);
    if (e != hipSuccess || dev < 0 || dev >= 64) {
        set_error("reserve_workspace: no usable HIP device: %s", hipGetErrorString(e));
        return ASDSL_ERR_HIP;
    }
    std::lock_guard<std::mutex> lock(g_ws_mu);
    Workspace& ws = g_ws[dev];
    if (bytes == 0) {
        ws.fixed = false;
        return ASDSL_OK;
    }
    if (ws.bytes < bytes) {
        const size_t grown = (bytes + 255) & ~static_cast<size_t>(255);  // what was asked, not the growth step
        void* fresh = nullptr;
        e = hipMalloc(&fresh, grown);
        if (e != hipSuccess) {
            set_error("reserve_workspace: hipMalloc(%zu) failed: %s", grown, hipGetErrorString(e));
            return ASDSL_ERR_HIP;
        }
        ws.ptr = fresh;  // a smaller earlier buffer is kept (queued work or a graph may use it)
        ws.bytes = grown;
    }
    ws.fixed = true;
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

extern "C" asdsl_status asdsl_profile_stages_begin(int max_launches) {
    using asdsl::g_rec;
    ASDSL_CHECK_ARG(!g_rec.armed, "profile_stages_begin: already armed on this thread");
    ASDSL_CHECK_ARG(max_launches >= 1 && max_launches <= asdsl::kMaxStageLaunches,
                    "profile_stages_begin: max_launches must be in [1, 65536]");
    while (g_rec.pool.size() < 2 * static_cast<size_t>(max_launches)) {
        hipEvent_t e = nullptr;
        const hipError_t err = hipEventCreate(&e);
        if (err != hipSuccess) {
            asdsl::set_error("profile_stages_begin: hipEventCreate failed: %s", hipGetErrorString(err));
            return ASDSL_ERR_HIP;
        }
        g_rec.pool.push_back(e);
    }
    g_rec.recs.clear();
    g_rec.recs.reserve(max_launches);
    g_rec.max = max_launches;
    g_rec.launches = 0;
    g_rec.armed = true;
    return ASDSL_OK;
}

extern "C" asdsl_status asdsl_profile_stages_end(int capacity, const char** labels, float* ms, int* count,
                                                 float* span_ms) {
    using asdsl::g_rec;
    ASDSL_CHECK_ARG(g_rec.armed, "profile_stages_end: not armed on this thread");
    g_rec.armed = false;
    ASDSL_CHECK_ARG(labels && ms && count && span_ms, "profile_stages_end: null pointer");
    const int n = static_cast<int>(g_rec.recs.size());
    if (g_rec.launches != n) {
        asdsl::set_error("profile_stages_end: %d launches, %d recorded (limit %d, or a launch armed by "
                         "asdsl_profile_next_launch)", g_rec.launches, n, g_rec.max);
        return ASDSL_ERR_INVALID_ARGUMENT;
    }
    ASDSL_CHECK_ARG(capacity >= n, "profile_stages_end: capacity below the launch count");
    *count = n;
    *span_ms = 0.0f;
    if (n == 0) return ASDSL_OK;
    hipError_t err = hipEventSynchronize(g_rec.recs.back().ev.stop);
    for (int i = 0; i < n && err == hipSuccess; ++i) {
        labels[i] = g_rec.recs[i].label;
        err = hipEventElapsedTime(&ms[i], g_rec.recs[i].ev.start, g_rec.recs[i].ev.stop);
    }
    if (err == hipSuccess) err = hipEventElapsedTime(span_ms, g_rec.recs.front().ev.start, g_rec.recs.back().ev.stop);
    if (err != hipSuccess) {
        asdsl::set_error("profile_stages_end: %s", hipGetErrorString(err));
        return ASDSL_ERR_HIP;
    }
    return ASDSL_OK;
}

extern "C" asdsl_status asdsl_reserve_workspace(size_t bytes) { return asdsl::reserve_workspace(bytes); }
