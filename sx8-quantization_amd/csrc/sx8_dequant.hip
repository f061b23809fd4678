// sx8_dequant.hip -- canonical (R64, bit-exact) dequantization kernels:
//   * k_dequant_split: whole tensor from the pkl/container split arrays (n-major);
//     role of kernel_sx8_v43.decode_tensor_gpu_fast (scripts/kernel_sx8_v43.py:109-145).
//   * k_gather_v44: selected rows from the kb-major v4.4 layout; role of the embedding
//     gather sx8_embed_v44 (cuda/sx8_embed_v44.cu:21-94) and, with identity ids, of a
//     whole-tensor dequant from the v4.4 layout.
//
// Both give one thread per (row, block, sub-block): 8 weights, one 16-byte store.
// Threads are ordered sub-block fastest, then block along K, then row, so a wave
// writes 64 x 16 contiguous bytes of one output row.  The inputs are read with
// dword/short loads; these kernels move 30 B in and 64 B out per block, so the fp16
// write stream sets their speed.
#include "sx8_device.h"
#include "sx8_host.h"

namespace {

constexpr int kThreads = 256;

// Store 8 fp16 values for columns [col, col+8) of an output row.  Vector store when
// the row pitch allows it, element stores (and the in_f cut) otherwise.
__device__ __forceinline__ void store8(uint16_t* __restrict__ row, int64_t col, int64_t in_f,
                                       bool vec_ok, const uint32_t w[4]) {
    if (vec_ok && col + 8 <= in_f) {
        *reinterpret_cast<uint4*>(row + col) = make_uint4(w[0], w[1], w[2], w[3]);
    } else {
#pragma unroll
        for (int e = 0; e < 8; ++e)
            if (col + e < in_f) row[col + e] = (uint16_t)(w[e >> 1] >> (16 * (e & 1)));
    }
}

// basis (n_cb, 64) f32: b0 = [0, 32), b1 = [32, 64); load the sub-block's 8 + 8 values.
__device__ __forceinline__ void load_basis(const float* __restrict__ basis,
                                           const float* __restrict__ scales, int64_t kb, int sb,
                                           double b0[8], double b1[8], double& s0, double& s1) {
    const float4* p0 = reinterpret_cast<const float4*>(basis + kb * 64 + 8 * sb);
    const float4* p1 = reinterpret_cast<const float4*>(basis + kb * 64 + 32 + 8 * sb);
    const float4 a0 = p0[0], a1 = p0[1], c0 = p1[0], c1 = p1[1];
    b0[0] = a0.x; b0[1] = a0.y; b0[2] = a0.z; b0[3] = a0.w;
    b0[4] = a1.x; b0[5] = a1.y; b0[6] = a1.z; b0[7] = a1.w;
    b1[0] = c0.x; b1[1] = c0.y; b1[2] = c0.z; b1[3] = c0.w;
    b1[4] = c1.x; b1[5] = c1.y; b1[6] = c1.z; b1[7] = c1.w;
    const float2 sc = *reinterpret_cast<const float2*>(scales + kb * 2);
    s0 = sc.x;
    s1 = sc.y;
}

__global__ __launch_bounds__(kThreads) void k_dequant_split(
    const uint16_t* __restrict__ dmin, const uint16_t* __restrict__ dmax,
    const uint8_t* __restrict__ config, const uint8_t* __restrict__ coeff,
    const uint8_t* __restrict__ hi, const uint8_t* __restrict__ lo,
    const float* __restrict__ basis, const float* __restrict__ scales, int64_t n_blocks,
    int64_t n_cb, int64_t in_f, bool vec_ok, uint16_t* __restrict__ out) {
    const int64_t gid = (int64_t)blockIdx.x * kThreads + threadIdx.x;
    const int64_t bid = gid >> 2;
    const int sb = (int)(gid & 3);
    if (bid >= n_blocks) return;
    const int64_t n = bid / n_cb;
    const int64_t kb = bid - n * n_cb;
    double b0[8], b1[8], s0, s1;
    load_basis(basis, scales, kb, sb, b0, b1, s0, s1);
    const uint32_t H = *reinterpret_cast<const uint32_t*>(hi + bid * 16 + 4 * sb);
    const uint32_t P16 = *reinterpret_cast<const uint16_t*>(lo + bid * 8 + 2 * sb);
    uint32_t w[4];
    sx8_r64_subblock(sx8_h2f(dmin[bid]), sx8_h2f(dmax[bid]), config[bid], coeff[bid], sb, H, P16,
                     b0, b1, s0, s1, w);
    store8(out + n * in_f, kb * 32 + 8 * sb, in_f, vec_ok, w);
}

// ids == nullptr: row t of the output is row t of W.  Rows outside [0, N) are skipped.
template <int HB>
__global__ __launch_bounds__(kThreads) void k_gather_v44(
    const int64_t* __restrict__ ids, int64_t T, const uint8_t* __restrict__ hdr,
    const uint8_t* __restrict__ levels, const float* __restrict__ basis,
    const float* __restrict__ scales, int64_t K, int64_t N, int64_t n_cb, bool vec_ok,
    uint16_t* __restrict__ out) {
    const int64_t gid = (int64_t)blockIdx.x * kThreads + threadIdx.x;
    const int64_t per_row = n_cb * 4;
    const int64_t t = gid / per_row;
    if (t >= T) return;
    const int64_t r = gid - t * per_row;
    const int64_t kb = r >> 2;
    const int sb = (int)(r & 3);
    const int64_t row = ids ? ids[t] : t;
    if (row < 0 || row >= N) return;
    const int64_t bid = kb * N + row;
    uint32_t d0, d1, cfg, cf;
    sx8_load_hdr<HB>(hdr, bid, d0, d1, cfg, cf);
    const uint8_t* lv = levels + bid * 24;
    const uint32_t H = *reinterpret_cast<const uint32_t*>(lv + 4 * sb);
    const uint32_t Pw = *reinterpret_cast<const uint32_t*>(lv + 16 + 4 * (sb >> 1));
    const uint32_t P16 = (sb & 1) ? (Pw >> 16) : (Pw & 0xFFFFu);
    double b0[8], b1[8], s0, s1;
    load_basis(basis, scales, kb, sb, b0, b1, s0, s1);
    uint32_t w[4];
    sx8_r64_subblock(sx8_h2f(d0), sx8_h2f(d1), cfg, cf, sb, H, P16, b0, b1, s0, s1, w);
    store8(out + t * K, kb * 32 + 8 * sb, K, vec_ok, w);
}

}  // namespace

extern "C" int32_t sx8_dequant_f16(const uint16_t* dmin, const uint16_t* dmax,
                                   const uint8_t* config, const uint8_t* coeff,
                                   const uint8_t* levels_hi, const uint8_t* levels_lo,
                                   const float* basis, const float* scales, int64_t out_f,
                                   int64_t in_f, int64_t n_cb, uint16_t* out, void* stream) {
    using namespace sx8;
    if (!dmin || !dmax || !config || !coeff || !levels_hi || !levels_lo || !basis || !scales || !out)
        return fail(SX8_ERR_INVALID, "sx8_dequant_f16: null pointer argument");
    if (out_f <= 0 || in_f <= 0 || n_cb <= 0 || n_cb * 32 < in_f || (n_cb - 1) * 32 >= in_f)
        return fail(SX8_ERR_INVALID, "sx8_dequant_f16: bad shape out_f=%lld in_f=%lld n_cb=%lld",
                    (long long)out_f, (long long)in_f, (long long)n_cb);
    if (!aligned(levels_hi, 4) || !aligned(levels_lo, 2) || !aligned(basis, 16) ||
        !aligned(scales, 8) || !aligned(out, 2))
        return fail(SX8_ERR_INVALID, "sx8_dequant_f16: misaligned pointer");
    const int64_t n_blocks = out_f * n_cb;
    const bool vec_ok = aligned(out, 16) && (in_f % 8 == 0);
    const int64_t threads = n_blocks * 4;
    const int64_t grid = (threads + kThreads - 1) / kThreads;
    if (grid > 0x7FFFFFFF) return fail(SX8_ERR_UNSUPPORTED, "sx8_dequant_f16: tensor too large");
    hipLaunchKernelGGL(k_dequant_split, dim3((unsigned)grid), dim3(kThreads), 0, as_stream(stream),
                       dmin, dmax, config, coeff, levels_hi, levels_lo, basis, scales, n_blocks,
                       n_cb, in_f, vec_ok, out);
    return check_launch("sx8_dequant_f16");
}

extern "C" int32_t sx8_embed_gather(const int64_t* ids, int64_t T, const uint8_t* hdr,
                                    const uint8_t* levels, int32_t hdr_bytes,
                                    const float* basis, const float* scales, int64_t K,
                                    int64_t N, int64_t n_cb, uint16_t* out, void* stream) {
    using namespace sx8;
    if (!hdr || !levels || !basis || !scales || !out)
        return fail(SX8_ERR_INVALID, "sx8_embed_gather: null pointer argument");
    if (hdr_bytes != 6 && hdr_bytes != 8)
        return fail(SX8_ERR_INVALID, "sx8_embed_gather: hdr_bytes must be 6 or 8, got %d", hdr_bytes);
    if (!ids) T = N;
    if (T < 0 || K <= 0 || N <= 0 || n_cb <= 0 || n_cb * 32 < K || (n_cb - 1) * 32 >= K)
        return fail(SX8_ERR_INVALID, "sx8_embed_gather: bad shape T=%lld K=%lld N=%lld n_cb=%lld",
                    (long long)T, (long long)K, (long long)N, (long long)n_cb);
    if (!aligned(hdr, hdr_bytes == 8 ? 8 : 2) || !aligned(levels, 8) || !aligned(basis, 16) ||
        !aligned(scales, 8) || !aligned(out, 2) || (ids && !aligned(ids, 8)))
        return fail(SX8_ERR_INVALID, "sx8_embed_gather: misaligned pointer");
    if (T == 0) return ok();
    const bool vec_ok = aligned(out, 16) && (K % 8 == 0);
    const int64_t threads = T * n_cb * 4;
    const int64_t grid = (threads + kThreads - 1) / kThreads;
    if (grid > 0x7FFFFFFF) return fail(SX8_ERR_UNSUPPORTED, "sx8_embed_gather: too many rows");
    if (hdr_bytes == 8)
        hipLaunchKernelGGL(k_gather_v44<8>, dim3((unsigned)grid), dim3(kThreads), 0,
                           as_stream(stream), ids, T, hdr, levels, basis, scales, K, N, n_cb,
                           vec_ok, out);
    else
        hipLaunchKernelGGL(k_gather_v44<6>, dim3((unsigned)grid), dim3(kThreads), 0,
                           as_stream(stream), ids, T, hdr, levels, basis, scales, K, N, n_cb,
                           vec_ok, out);
    return check_launch("sx8_embed_gather");
}
