// sx8_host.h -- host-side helpers shared by the C-ABI entry points: error reporting,
// argument checks and the per-device workspace used by the split-K GEMV.
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "sx8_hip.h"

namespace sx8 {

// Record a formatted message for sx8_last_error() on this thread and return `code`.
int32_t fail(int32_t code, const char* fmt, ...) __attribute__((format(printf, 2, 3)));

// Clear the thread's error message and return SX8_OK.
int32_t ok();

// Turn the result of the launches just made into a status code.
int32_t check_launch(const char* what);

inline bool aligned(const void* p, uintptr_t a) {
    return (reinterpret_cast<uintptr_t>(p) & (a - 1)) == 0;
}

inline hipStream_t as_stream(void* s) { return reinterpret_cast<hipStream_t>(s); }

// Device workspace for the split-K GEMV: `partial_floats` float32 partial sums and
// `n_counters` arrival counters that are zero between launches (each launch's last
// work-group resets the counters it used).  Grow-only, one per device, allocated
// with hipMalloc on first need; returns SX8_OK or SX8_ERR_HIP.
int32_t gemv_workspace(int64_t partial_floats, int64_t n_counters, float** partial,
                       uint32_t** counters);

}  // namespace sx8
