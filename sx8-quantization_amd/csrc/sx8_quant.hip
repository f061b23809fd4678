// sx8_quant.hip -- the deterministic half of the S-X8 v4.3 quantizer on the GPU: the V6
// encode of every 32-weight block (dmin, dmax, per-sub-block range strategy, 6-bit
// levels) and the level packing, written straight into the pkl / container split arrays.
//
// Role of v6_encode_6bit_gpu and pack_levels_6bit
// (scripts/quantize_qwen35_4b_sx8_v43_gpu.py:22-47, :148-167).  The PCA half (per-K-block
// bases from the residuals) stays a batched Gram / eigen decomposition in torch: it is a
// few hundred 32 x 32 problems per tensor.
//
// Arithmetic (binary32, every operation rounded, no contraction), per block:
//   dmin, dmax = min, max of the 32 weights; d = max(dmax - dmin, 1e-10); q = d / 4;
//   candidates (lo, hi) = (dmin, dmax), (dmin, dmin + q), (dmax - q, dmax),
//   (dmin + q, dmax - q); per 8-weight sub-block and candidate: step = max((hi - lo) / 63,
//   1e-10), lv = clamp(rint((x - lo) / step), 0, 63), rec = lo + step * lv, mse = (sum of
//   the eight (x - rec)^2 left to right) / 8; the first candidate with the strictly lowest
//   mse wins.  config = s0 | s1 << 2 | s2 << 4 | s3 << 6.
// Packing: qh[t >> 1] holds (lv >> 2) of weight t at bits 4 (t & 1); ql[t >> 2] holds
// (lv & 3) at bits 2 (3 - (t & 3)).
//
// One thread per block, n-major (bid = n * n_cb + kb): a wave reads 64 consecutive
// 64-byte row segments.  Columns past in_f are zero (the reference pads W with zeros).
#include "sx8_device.h"
#include "sx8_host.h"

namespace {

constexpr int kThreads = 256;

__global__ __launch_bounds__(kThreads) void k_v6_encode(
    const uint16_t* __restrict__ W, int64_t out_f, int64_t in_f, int64_t ld, int64_t n_cb,
    uint8_t* __restrict__ levels, uint16_t* __restrict__ dmin_out, uint16_t* __restrict__ dmax_out,
    uint8_t* __restrict__ config_out, uint8_t* __restrict__ hi_out, uint8_t* __restrict__ lo_out) {
#pragma clang fp contract(off)
    const int64_t bid = (int64_t)blockIdx.x * kThreads + threadIdx.x;
    if (bid >= out_f * n_cb) return;
    const int64_t n = bid / n_cb;
    const int64_t kb = bid - n * n_cb;
    const uint16_t* row = W + n * ld + kb * 32;
    float x[32];
    const bool full = (kb + 1) * 32 <= in_f && (reinterpret_cast<uintptr_t>(row) & 15) == 0;
    if (full) {
#pragma unroll
        for (int q4 = 0; q4 < 4; ++q4) {
            const uint4 v = reinterpret_cast<const uint4*>(row)[q4];
            const uint32_t w4[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
            for (int i = 0; i < 8; ++i) x[8 * q4 + i] = sx8_h2f(w4[i >> 1] >> (16 * (i & 1)));
        }
    } else {
#pragma unroll
        for (int t = 0; t < 32; ++t) x[t] = kb * 32 + t < in_f ? sx8_h2f(row[t]) : 0.f;
    }
    float mn = x[0], mx = x[0];
#pragma unroll
    for (int t = 1; t < 32; ++t) {
        mn = x[t] < mn ? x[t] : mn;
        mx = x[t] > mx ? x[t] : mx;
    }
    float d = mx - mn;
    d = d > 1e-10f ? d : 1e-10f;
    const float q = d / 4.0f;
    const float lo_c[4] = {mn, mn, mx - q, mn + q};
    const float hi_c[4] = {mx, mn + q, mx, mx - q};
    uint32_t cfg = 0;
    uint8_t lv_best[32];
#pragma unroll
    for (int sb = 0; sb < 4; ++sb) {
        float best = __builtin_inff();
        int s_best = 0;
        uint8_t lvb[8] = {0, 0, 0, 0, 0, 0, 0, 0};
#pragma unroll
        for (int c = 0; c < 4; ++c) {
            float step = (hi_c[c] - lo_c[c]) / 63.0f;
            step = step > 1e-10f ? step : 1e-10f;
            uint8_t lv[8];
            float acc = 0.f;
#pragma unroll
            for (int i = 0; i < 8; ++i) {
                float r = __builtin_rintf((x[8 * sb + i] - lo_c[c]) / step);
                r = r < 0.f ? 0.f : (r > 63.f ? 63.f : r);
                lv[i] = (uint8_t)(int)r;
                const float rec = lo_c[c] + step * r;
                const float e = x[8 * sb + i] - rec;
                acc = i == 0 ? e * e : acc + e * e;
            }
            const float mse = acc / 8.0f;
            if (mse < best) {
                best = mse;
                s_best = c;
#pragma unroll
                for (int i = 0; i < 8; ++i) lvb[i] = lv[i];
            }
        }
        cfg |= (uint32_t)s_best << (2 * sb);
#pragma unroll
        for (int i = 0; i < 8; ++i) lv_best[8 * sb + i] = lvb[i];
    }
    dmin_out[bid] = __builtin_bit_cast(uint16_t, (_Float16)mn);
    dmax_out[bid] = __builtin_bit_cast(uint16_t, (_Float16)mx);
    config_out[bid] = (uint8_t)cfg;
    uint32_t h[4] = {0, 0, 0, 0}, l[2] = {0, 0};
#pragma unroll
    for (int t = 0; t < 32; ++t) {
        h[t >> 3] |= (uint32_t)(lv_best[t] >> 2) << (4 * (t & 7));
        l[t >> 4] |= (uint32_t)(lv_best[t] & 3) << (8 * ((t >> 2) & 3) + 2 * (3 - (t & 3)));
    }
    uint8_t* ho = hi_out + bid * 16;
    uint8_t* lo = lo_out + bid * 8;
#pragma unroll
    for (int k = 0; k < 16; ++k) ho[k] = (uint8_t)(h[k >> 2] >> (8 * (k & 3)));
#pragma unroll
    for (int k = 0; k < 8; ++k) lo[k] = (uint8_t)(l[k >> 2] >> (8 * (k & 3)));
    if (levels) {
        uint8_t* lvo = levels + bid * 32;
#pragma unroll
        for (int t = 0; t < 32; ++t) lvo[t] = lv_best[t];
    }
}

}  // namespace

extern "C" int32_t sx8_v6_encode(const uint16_t* W, int64_t out_f, int64_t in_f, int64_t ld,
                                 uint8_t* levels, uint16_t* dmin, uint16_t* dmax, uint8_t* config,
                                 uint8_t* levels_hi, uint8_t* levels_lo, void* stream) {
    using namespace sx8;
    if (!W || !dmin || !dmax || !config || !levels_hi || !levels_lo)
        return fail(SX8_ERR_INVALID, "sx8_v6_encode: null pointer argument");
    if (out_f <= 0 || in_f <= 0 || ld < in_f)
        return fail(SX8_ERR_INVALID, "sx8_v6_encode: bad shape out_f=%lld in_f=%lld ld=%lld",
                    (long long)out_f, (long long)in_f, (long long)ld);
    if (!aligned(W, 2) || !aligned(dmin, 2) || !aligned(dmax, 2))
        return fail(SX8_ERR_INVALID, "sx8_v6_encode: misaligned pointer");
    const int64_t n_cb = (in_f + 31) / 32;
    const int64_t grid = (out_f * n_cb + kThreads - 1) / kThreads;
    if (grid > 0x7FFFFFFF) return fail(SX8_ERR_UNSUPPORTED, "sx8_v6_encode: tensor too large");
    hipLaunchKernelGGL(k_v6_encode, dim3((unsigned)grid), dim3(kThreads), 0, as_stream(stream), W,
                       out_f, in_f, ld, n_cb, levels, dmin, dmax, config, levels_hi, levels_lo);
    return check_launch("sx8_v6_encode");
}
