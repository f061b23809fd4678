// sx8_layout.hip -- load-time layout transforms and the GGUF-side decode:
//   * S-X8 v4.3 blocks in n-major order (bid' = n * n_cb + kb), as the pkl / .sx8v43
//     container's split arrays or as GGUF block_sx8 records (30 interleaved bytes) ->
//     v4.4 kb-major device records (bid = kb * N + n): hdr (6 or 8 bytes: dmin | dmax |
//     config | coeff | pad) and levels (24 bytes: levels_hi[16] | levels_lo[8]);
//   * llama.cpp's no-PCA float32 dequant of block_sx8 records ("R32-ggml"), for
//     comparing this engine with the reference's llama.cpp fork on the same GGUF.
//
// Role of prepare_v44.to_v44 (scripts/prepare_v44.py:35-79), which the reference runs on
// the CPU with numpy at the first forward; here the container's record payload is copied
// to the device once and laid out there.  A byte permutation: no arithmetic.
//
// One thread per destination record, destination order (n fastest), so the 24-byte level
// records and the headers are written as contiguous runs; the source fields are read with
// byte loads (their offsets inside a container payload carry no alignment).
#include "sx8_device.h"
#include "sx8_host.h"

namespace {

constexpr int kThreads = 256;

// Where the six block fields of n-major block s live: field f starts at p[f] + s * st[f]
// (f = dmin, dmax, config, coeff, levels_hi, levels_lo).  Split arrays (pkl, container):
// strides 2, 2, 1, 1, 16, 8; interleaved 30-byte block_sx8 records (GGUF): stride 30.
struct BlockFields {
    const uint8_t* p[6];
    int64_t st[6];
};

__device__ __forceinline__ uint32_t ld_u32(const uint8_t* __restrict__ q) {
    return (uint32_t)q[0] | ((uint32_t)q[1] << 8) | ((uint32_t)q[2] << 16) | ((uint32_t)q[3] << 24);
}

template <int HB>
__global__ __launch_bounds__(kThreads) void k_to_v44(const BlockFields f, int64_t N, int64_t n_cb,
                                                     uint8_t* __restrict__ hdr,
                                                     uint8_t* __restrict__ levels) {
    const int64_t bid = (int64_t)blockIdx.x * kThreads + threadIdx.x;
    if (bid >= N * n_cb) return;
    const int64_t kb = bid / N;
    const int64_t n = bid - kb * N;
    const int64_t s = n * n_cb + kb;
    const uint8_t* dmin = f.p[0] + s * f.st[0];
    const uint8_t* dmax = f.p[1] + s * f.st[1];
    const uint32_t h0 = (uint32_t)dmin[0] | ((uint32_t)dmin[1] << 8) | ((uint32_t)dmax[0] << 16) |
                        ((uint32_t)dmax[1] << 24);
    const uint32_t h1 = (uint32_t)f.p[2][s * f.st[2]] | ((uint32_t)f.p[3][s * f.st[3]] << 8);
    if constexpr (HB == 8) {
        *reinterpret_cast<uint2*>(hdr + bid * 8) = make_uint2(h0, h1);
    } else {
        uint16_t* o = reinterpret_cast<uint16_t*>(hdr + bid * 6);
        o[0] = (uint16_t)h0;
        o[1] = (uint16_t)(h0 >> 16);
        o[2] = (uint16_t)h1;
    }
    const uint8_t* hi = f.p[4] + s * f.st[4];
    const uint8_t* lo = f.p[5] + s * f.st[5];
    uint2* d = reinterpret_cast<uint2*>(levels + bid * 24);
    d[0] = make_uint2(ld_u32(hi), ld_u32(hi + 4));
    d[1] = make_uint2(ld_u32(hi + 8), ld_u32(hi + 12));
    d[2] = make_uint2(ld_u32(lo), ld_u32(lo + 4));
}

// llama.cpp's dequantize_row_sx8 (llama-cpp-sx8.patch:746-767): float32, no PCA (the
// coeff byte is ignored), branch-free strategy offsets rlo = lo + q (3[s=2] + [s=3]),
// rhi = hi - q (3[s=1] + [s=3]), step = (rhi - rlo) * 0.015873f floored at 1e-10f,
// w = rlo + step * lv.  kContract: the three a*b+c forms as single fused multiply-adds
// (a C compiler contracting them, e.g. GCC's default -ffp-contract=fast with FMA
// hardware); otherwise every operation rounds separately.  One thread per (block,
// sub-block) of interleaved 30-byte records in n-major order; 8 floats out.
template <bool kContract>
__global__ __launch_bounds__(kThreads) void k_dequant_ggml(const uint8_t* __restrict__ blocks,
                                                           int64_t n_blk, int64_t n_cb, int64_t in_f,
                                                           float* __restrict__ out) {
#pragma clang fp contract(off)
    const int64_t gid = (int64_t)blockIdx.x * kThreads + threadIdx.x;
    if (gid >= n_blk * 4) return;
    const int64_t b = gid >> 2;
    const int sb = (int)(gid & 3);
    const uint8_t* r = blocks + b * 30;
    const float lo_f = sx8_h2f((uint32_t)r[0] | ((uint32_t)r[1] << 8));
    const float hi_f = sx8_h2f((uint32_t)r[2] | ((uint32_t)r[3] << 8));
    const int s = (r[4] >> (2 * sb)) & 3;
    const float q = (hi_f - lo_f) * 0.25f;
    const float k1 = (float)(3 * (s == 2) + (s == 3));
    const float k2 = (float)(3 * (s == 1) + (s == 3));
    float rlo, rhi;
    if constexpr (kContract) {
        rlo = __builtin_fmaf(q, k1, lo_f);
        rhi = __builtin_fmaf(-q, k2, hi_f);
    } else {
        rlo = lo_f + q * k1;
        rhi = hi_f - q * k2;
    }
    float step = (rhi - rlo) * 0.015873f;
    if (step < 1e-10f) step = 1e-10f;
    const uint32_t H = ld_u32(r + 5 + 4 * sb);
    const uint32_t P = (uint32_t)r[21 + 2 * sb] | ((uint32_t)r[22 + 2 * sb] << 8);
    float w[8];
#pragma unroll
    for (int i = 0; i < 8; ++i) {
        const float lv = (float)sx8_level(H, P, i);
        w[i] = kContract ? __builtin_fmaf(step, lv, rlo) : rlo + step * lv;
    }
    const int64_t n = b / n_cb;
    const int64_t col = (b - n * n_cb) * 32 + 8 * sb;
    float* o = out + n * in_f + col;
    if (col + 8 <= in_f && ((reinterpret_cast<uintptr_t>(o) & 15) == 0)) {
        reinterpret_cast<float4*>(o)[0] = make_float4(w[0], w[1], w[2], w[3]);
        reinterpret_cast<float4*>(o)[1] = make_float4(w[4], w[5], w[6], w[7]);
    } else {
#pragma unroll
        for (int i = 0; i < 8; ++i)
            if (col + i < in_f) o[i] = w[i];
    }
}

int32_t launch_to_v44(const BlockFields& f, int64_t out_f, int64_t n_cb, int32_t hdr_bytes,
                      uint8_t* hdr, uint8_t* levels, void* stream, const char* who) {
    using namespace sx8;
    if (hdr_bytes != 6 && hdr_bytes != 8)
        return fail(SX8_ERR_INVALID, "%s: hdr_bytes must be 6 or 8, got %d", who, hdr_bytes);
    if (out_f <= 0 || n_cb <= 0 || out_f > ((int64_t)1 << 40) / n_cb)
        return fail(SX8_ERR_INVALID, "%s: bad shape out_f=%lld n_cb=%lld", who, (long long)out_f,
                    (long long)n_cb);
    if (!hdr || !levels) return fail(SX8_ERR_INVALID, "%s: null output", who);
    if (!aligned(hdr, hdr_bytes == 8 ? 8 : 2) || !aligned(levels, 8))
        return fail(SX8_ERR_INVALID, "%s: misaligned output (hdr %d B, levels 8 B)", who,
                    hdr_bytes == 8 ? 8 : 2);
    const int64_t grid = (out_f * n_cb + kThreads - 1) / kThreads;
    if (grid > 0x7FFFFFFF) return fail(SX8_ERR_UNSUPPORTED, "%s: tensor too large", who);
    if (hdr_bytes == 8)
        hipLaunchKernelGGL(k_to_v44<8>, dim3((unsigned)grid), dim3(kThreads), 0, as_stream(stream), f,
                           out_f, n_cb, hdr, levels);
    else
        hipLaunchKernelGGL(k_to_v44<6>, dim3((unsigned)grid), dim3(kThreads), 0, as_stream(stream), f,
                           out_f, n_cb, hdr, levels);
    return check_launch(who);
}

}  // namespace

extern "C" int32_t sx8_v43_to_v44(const uint8_t* dmin, const uint8_t* dmax, const uint8_t* config,
                                  const uint8_t* coeff, const uint8_t* levels_hi,
                                  const uint8_t* levels_lo, int64_t out_f, int64_t n_cb,
                                  int32_t hdr_bytes, uint8_t* hdr, uint8_t* levels,
                                  void* stream) {
    using namespace sx8;
    if (!dmin || !dmax || !config || !coeff || !levels_hi || !levels_lo)
        return fail(SX8_ERR_INVALID, "sx8_v43_to_v44: null pointer argument");
    const BlockFields f{{dmin, dmax, config, coeff, levels_hi, levels_lo}, {2, 2, 1, 1, 16, 8}};
    return launch_to_v44(f, out_f, n_cb, hdr_bytes, hdr, levels, stream, "sx8_v43_to_v44");
}

extern "C" int32_t sx8_blocks_to_v44(const uint8_t* blocks, int64_t out_f, int64_t n_cb,
                                     int32_t hdr_bytes, uint8_t* hdr, uint8_t* levels, void* stream) {
    using namespace sx8;
    if (!blocks) return fail(SX8_ERR_INVALID, "sx8_blocks_to_v44: null pointer argument");
    const BlockFields f{{blocks, blocks + 2, blocks + 4, blocks + 29, blocks + 5, blocks + 21},
                        {30, 30, 30, 30, 30, 30}};
    return launch_to_v44(f, out_f, n_cb, hdr_bytes, hdr, levels, stream, "sx8_blocks_to_v44");
}

extern "C" int32_t sx8_dequant_ggml_f32(const uint8_t* blocks, int64_t out_f, int64_t in_f,
                                        int64_t n_cb, int32_t contract, float* out, void* stream) {
    using namespace sx8;
    if (!blocks || !out) return fail(SX8_ERR_INVALID, "sx8_dequant_ggml_f32: null pointer argument");
    if (out_f <= 0 || in_f <= 0 || n_cb <= 0 || n_cb * 32 < in_f || (n_cb - 1) * 32 >= in_f)
        return fail(SX8_ERR_INVALID, "sx8_dequant_ggml_f32: bad shape out_f=%lld in_f=%lld n_cb=%lld",
                    (long long)out_f, (long long)in_f, (long long)n_cb);
    if (!aligned(out, 4)) return fail(SX8_ERR_INVALID, "sx8_dequant_ggml_f32: misaligned output");
    const int64_t n_blk = out_f * n_cb;
    const int64_t grid = (n_blk * 4 + kThreads - 1) / kThreads;
    if (grid > 0x7FFFFFFF) return fail(SX8_ERR_UNSUPPORTED, "sx8_dequant_ggml_f32: tensor too large");
    if (contract)
        hipLaunchKernelGGL(k_dequant_ggml<true>, dim3((unsigned)grid), dim3(kThreads), 0,
                           as_stream(stream), blocks, n_blk, n_cb, in_f, out);
    else
        hipLaunchKernelGGL(k_dequant_ggml<false>, dim3((unsigned)grid), dim3(kThreads), 0,
                           as_stream(stream), blocks, n_blk, n_cb, in_f, out);
    return check_launch("sx8_dequant_ggml_f32");
}
