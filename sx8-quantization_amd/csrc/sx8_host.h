// sx8_host.h -- host-side helpers shared by the C-ABI entry points: error reporting,
// argument checks and the Z / packed-X pass shared by the GEMV and the prefill GEMM.
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

// Z[m, kb, j] = scales[kb, j] * sum_t X[m, kb*32+t] * basis[kb, 32j+t] (reference tree
// order), reading only columns k < K of X (the rest count as zero).  hl = false: Z as f32
// (M, n_cb, 2); hl = true: each value stored as the fp16 pair sx8_split_hl(z), i.e.
// (Z0 hi, Z0 lo, Z1 hi, Z1 lo) per (m, kb), the prefill GEMM's PCA operand.  Same size.
// Z may be null (no Z).  xpack != null also writes the prefill GEMM's packed X:
// ceil(M / 32) * n_cb chunks of 2 KB (see k_compute_z).  Launch only; the caller
// validated the arguments.
int32_t compute_z(const uint16_t* X, int64_t M, int64_t ldx, int64_t K, const float* basis,
                  const float* scales, int64_t n_cb, void* Z, bool hl, uint16_t* xpack,
                  hipStream_t st);

// The same for n (0..kMaxZSets) basis sets in one pass over X (the matrices of a prefill
// group): Z[s] from basis[s] / scales[s].
constexpr int kMaxZSets = 4;
struct ZSets {
    const float* basis[kMaxZSets];
    const float* scales[kMaxZSets];
    float* Z[kMaxZSets];
    int n;
};
int32_t compute_z_sets(const uint16_t* X, int64_t M, int64_t ldx, int64_t K, const ZSets& zs,
                       int64_t n_cb, bool hl, uint16_t* xpack, hipStream_t st);

// compute_z_sets (split Z, packed X) with x = fp16(silu(g) * u) produced from two float32
// matrices with row stride ld (the arithmetic of sx8_dec_silu_mul).
int32_t compute_z_silu(const float* g, const float* u, int64_t M, int64_t ld, int64_t K,
                       const ZSets& zs, int64_t n_cb, uint16_t* xpack, hipStream_t st);

}  // namespace sx8
