// sx8_layout.hip -- load-time layout transform: S-X8 v4.3 split arrays (pkl / .sx8v43
// container order, n-major bid' = n * n_cb + kb) -> v4.4 kb-major device records
// (bid = kb * N + n): hdr (6 or 8 bytes: dmin | dmax | config | coeff | pad) and levels
// (24 bytes: levels_hi[16] | levels_lo[8]).
//
// Role of prepare_v44.to_v44 (scripts/prepare_v44.py:35-79), which the reference runs on
// the CPU with numpy at the first forward; here the container's record payload is copied
// to the device once and laid out there.  A byte permutation: no arithmetic.
//
// One thread per destination record, destination order (n fastest), so the 24-byte level
// records and the headers are written as contiguous runs; the source fields are read with
// byte loads (their offsets inside a container payload carry no alignment).
#include "sx8_host.h"

namespace {

constexpr int kThreads = 256;

template <int HB>
__global__ __launch_bounds__(kThreads) void k_v43_to_v44(
    const uint8_t* __restrict__ dmin, const uint8_t* __restrict__ dmax,
    const uint8_t* __restrict__ config, const uint8_t* __restrict__ coeff,
    const uint8_t* __restrict__ hi, const uint8_t* __restrict__ lo, int64_t N, int64_t n_cb,
    uint8_t* __restrict__ hdr, uint8_t* __restrict__ levels) {
    const int64_t bid = (int64_t)blockIdx.x * kThreads + threadIdx.x;
    if (bid >= N * n_cb) return;
    const int64_t kb = bid / N;
    const int64_t n = bid - kb * N;
    const int64_t s = n * n_cb + kb;
    const uint32_t h0 = (uint32_t)dmin[2 * s] | ((uint32_t)dmin[2 * s + 1] << 8) |
                        ((uint32_t)dmax[2 * s] << 16) | ((uint32_t)dmax[2 * s + 1] << 24);
    const uint32_t h1 = (uint32_t)config[s] | ((uint32_t)coeff[s] << 8);
    if constexpr (HB == 8) {
        *reinterpret_cast<uint2*>(hdr + bid * 8) = make_uint2(h0, h1);
    } else {
        uint16_t* o = reinterpret_cast<uint16_t*>(hdr + bid * 6);
        o[0] = (uint16_t)h0;
        o[1] = (uint16_t)(h0 >> 16);
        o[2] = (uint16_t)h1;
    }
    uint32_t w[6];
#pragma unroll
    for (int q = 0; q < 4; ++q) {
        const uint8_t* p = hi + 16 * s + 4 * q;
        w[q] = (uint32_t)p[0] | ((uint32_t)p[1] << 8) | ((uint32_t)p[2] << 16) | ((uint32_t)p[3] << 24);
    }
#pragma unroll
    for (int q = 0; q < 2; ++q) {
        const uint8_t* p = lo + 8 * s + 4 * q;
        w[4 + q] = (uint32_t)p[0] | ((uint32_t)p[1] << 8) | ((uint32_t)p[2] << 16) | ((uint32_t)p[3] << 24);
    }
    uint2* d = reinterpret_cast<uint2*>(levels + bid * 24);
    d[0] = make_uint2(w[0], w[1]);
    d[1] = make_uint2(w[2], w[3]);
    d[2] = make_uint2(w[4], w[5]);
}

}  // namespace

extern "C" int32_t sx8_v43_to_v44(const uint8_t* dmin, const uint8_t* dmax, const uint8_t* config,
                                  const uint8_t* coeff, const uint8_t* levels_hi,
                                  const uint8_t* levels_lo, int64_t out_f, int64_t n_cb,
                                  int32_t hdr_bytes, uint8_t* hdr, uint8_t* levels,
                                  void* stream) {
    using namespace sx8;
    if (!dmin || !dmax || !config || !coeff || !levels_hi || !levels_lo || !hdr || !levels)
        return fail(SX8_ERR_INVALID, "sx8_v43_to_v44: null pointer argument");
    if (hdr_bytes != 6 && hdr_bytes != 8)
        return fail(SX8_ERR_INVALID, "sx8_v43_to_v44: hdr_bytes must be 6 or 8, got %d", hdr_bytes);
    if (out_f <= 0 || n_cb <= 0 || out_f > ((int64_t)1 << 40) / n_cb)
        return fail(SX8_ERR_INVALID, "sx8_v43_to_v44: bad shape out_f=%lld n_cb=%lld",
                    (long long)out_f, (long long)n_cb);
    if (!aligned(hdr, hdr_bytes == 8 ? 8 : 2) || !aligned(levels, 8))
        return fail(SX8_ERR_INVALID, "sx8_v43_to_v44: misaligned output (hdr %d B, levels 8 B)",
                    hdr_bytes == 8 ? 8 : 2);
    const int64_t n_blk = out_f * n_cb;
    const int64_t grid = (n_blk + kThreads - 1) / kThreads;
    if (grid > 0x7FFFFFFF) return fail(SX8_ERR_UNSUPPORTED, "sx8_v43_to_v44: tensor too large");
    if (hdr_bytes == 8)
        hipLaunchKernelGGL(k_v43_to_v44<8>, dim3((unsigned)grid), dim3(kThreads), 0,
                           as_stream(stream), dmin, dmax, config, coeff, levels_hi, levels_lo,
                           out_f, n_cb, hdr, levels);
    else
        hipLaunchKernelGGL(k_v43_to_v44<6>, dim3((unsigned)grid), dim3(kThreads), 0,
                           as_stream(stream), dmin, dmax, config, coeff, levels_hi, levels_lo,
                           out_f, n_cb, hdr, levels);
    return check_launch("sx8_v43_to_v44");
}
