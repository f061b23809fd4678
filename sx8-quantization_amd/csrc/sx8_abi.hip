// sx8_abi.hip -- library-wide C-ABI plumbing: version, last-error message, and the
// per-device GEMV workspace.
#include <cstdarg>
#include <cstdio>
#include <mutex>
#include <vector>

#include "sx8_host.h"

namespace sx8 {
namespace {
thread_local char g_msg[512] = "";

struct Workspace {
    float* partial = nullptr;
    uint32_t* counters = nullptr;
    int64_t partial_cap = 0;
    int64_t counter_cap = 0;
};
std::mutex g_ws_mutex;
std::vector<Workspace> g_ws;
}  // namespace

int32_t fail(int32_t code, const char* fmt, ...) {
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(g_msg, sizeof(g_msg), fmt, ap);
    va_end(ap);
    return code;
}

int32_t ok() {
    g_msg[0] = '\0';
    return SX8_OK;
}

int32_t check_launch(const char* what) {
    const hipError_t e = hipGetLastError();
    if (e != hipSuccess) return fail(SX8_ERR_HIP, "%s: launch failed: %s", what, hipGetErrorString(e));
    return ok();
}

int32_t gemv_workspace(int64_t partial_floats, int64_t n_counters, float** partial,
                       uint32_t** counters) {
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess) return fail(SX8_ERR_HIP, "hipGetDevice failed");
    std::lock_guard<std::mutex> lock(g_ws_mutex);
    if ((int)g_ws.size() <= dev) g_ws.resize(dev + 1);
    Workspace& w = g_ws[dev];
    if (w.partial_cap < partial_floats) {
        if (w.partial) (void)hipFree(w.partial);
        w.partial = nullptr;
        w.partial_cap = 0;
        const int64_t cap = partial_floats + (partial_floats >> 1) + 1024;
        if (hipMalloc(reinterpret_cast<void**>(&w.partial), cap * sizeof(float)) != hipSuccess)
            return fail(SX8_ERR_HIP, "hipMalloc of %lld GEMV partials failed", (long long)cap);
        w.partial_cap = cap;
    }
    if (w.counter_cap < n_counters) {
        if (w.counters) (void)hipFree(w.counters);
        w.counters = nullptr;
        w.counter_cap = 0;
        const int64_t cap = n_counters + (n_counters >> 1) + 256;
        if (hipMalloc(reinterpret_cast<void**>(&w.counters), cap * sizeof(uint32_t)) != hipSuccess)
            return fail(SX8_ERR_HIP, "hipMalloc of %lld GEMV counters failed", (long long)cap);
        // Synchronous clear: the counters start at zero and every launch leaves them there.
        if (hipMemset(w.counters, 0, cap * sizeof(uint32_t)) != hipSuccess)
            return fail(SX8_ERR_HIP, "hipMemset of GEMV counters failed");
        w.counter_cap = cap;
    }
    *partial = w.partial;
    *counters = w.counters;
    return SX8_OK;
}

}  // namespace sx8

extern "C" int32_t sx8_abi_version(void) { return SX8_ABI_VERSION; }

extern "C" const char* sx8_last_error(void) { return sx8::g_msg; }
