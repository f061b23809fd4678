// sx8_abi.hip -- library-wide C-ABI plumbing: version and last-error message.
#include <cstdarg>
#include <cstdio>

#include "sx8_host.h"

namespace sx8 {
namespace {
thread_local char g_msg[512] = "";

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

}  // namespace sx8

extern "C" int32_t sx8_abi_version(void) { return SX8_ABI_VERSION; }

extern "C" const char* sx8_last_error(void) { return sx8::g_msg; }
