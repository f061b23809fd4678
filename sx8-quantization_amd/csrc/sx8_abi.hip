// sx8_abi.hip -- library-wide C-ABI plumbing: version, last-error message, and the
// per-device fallback workspace.
#include <cstdarg>
#include <cstdio>
#include <mutex>
#include <vector>

#include "sx8_host.h"

namespace sx8 {
namespace {
thread_local char g_msg[512] = "";

struct Workspace {
    void* ptr = nullptr;
    int64_t cap = 0;
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

int32_t device_workspace(int64_t bytes, void** ptr) {
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess) return fail(SX8_ERR_HIP, "hipGetDevice failed");
    std::lock_guard<std::mutex> lock(g_ws_mutex);
    if ((int)g_ws.size() <= dev) g_ws.resize(dev + 1);
    Workspace& w = g_ws[dev];
    if (w.cap < bytes) {
        if (w.ptr) {
            (void)hipDeviceSynchronize();   // earlier launches may still read it
            (void)hipFree(w.ptr);
        }
        w.ptr = nullptr;
        w.cap = 0;
        const int64_t cap = ((bytes + (bytes >> 1)) + 4095) & ~int64_t(4095);
        if (hipMalloc(&w.ptr, cap) != hipSuccess)
            return fail(SX8_ERR_HIP, "hipMalloc of %lld workspace bytes failed", (long long)cap);
        w.cap = cap;
    }
    *ptr = w.ptr;
    return SX8_OK;
}

}  // namespace sx8

extern "C" int32_t sx8_abi_version(void) { return SX8_ABI_VERSION; }

extern "C" const char* sx8_last_error(void) { return sx8::g_msg; }
