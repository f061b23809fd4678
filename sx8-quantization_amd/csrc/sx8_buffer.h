// sx8_buffer.h -- raw buffer resources for the S-X8 kernels' streaming loads (gfx950).
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

// Raw buffer resource over `bytes` bytes at p (gfx9 resource word 3 = raw 32-bit
// buffer).  A load whose offset lies at or past the end returns zero without touching
// memory; offsets are 32-bit, so callers keep every tensor they address this way
// below 2 GiB.
typedef __amdgpu_buffer_rsrc_t sx8_rsrc;
constexpr int kRsrcFlags = 0x00020000;

__device__ __forceinline__ sx8_rsrc make_rsrc(const void* p, int64_t bytes) {
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(p), (short)0,
                                             (int)min(bytes, (int64_t)0x7FFFFFFF), kRsrcFlags);
}
