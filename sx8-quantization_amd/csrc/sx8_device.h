// sx8_device.h -- device-side building blocks shared by the S-X8 HIP kernels (gfx950).
//
// S-X8 v4.3 block (docs/SX8_FLASH_V4_3_SPEC.md:13-25 in the reference): 32 weights of
// one row in 30 bytes -- dmin fp16, dmax fp16, config u8 (4 x 2-bit range strategy),
// 16 B of high nibbles, 8 B of low quads, coeff u8 (two signed 4-bit PCA coefficients).
//
// Decode recipes of this library:
//   * R64 (sx8_r64_subblock, here): the canonical dequant of scripts/kernel_sx8_v43.py:
//     14-51 under Numba typing -- binary32 hi-lo, binary64 everywhere else, binary32
//     store, RNE to fp16.  The kernels that hand fp16 weights to a caller (full dequant,
//     embedding gather) use it, so those weights are bit-identical to the canonical
//     dequant.
//   * the prefill GEMM's MFMA operand (sx8_gemm.hip): the PCA-free core rlo + step*lv
//     with the reference's float32 range parameters (cuda/sx8_fused_wmma.cu:70-94), the
//     multiply-add rounded once to fp16; PCA is added through Z.  Not R64: it differs
//     from the R64 weights without PCA in the last fp16 bit on about 1e-4 of weights.
//   * the fp32 GEMV decode in sx8_gemv.hip, which only feeds an fp32 dot product.
//   The GEMV and GEMM products meet max|dY| / max|Y| <= 1e-3 against the float64 product
//   of the R64 weights (scripts/sx8_decode1_v3.py:131-133).
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

typedef _Float16 sx8_half8 __attribute__((ext_vector_type(8)));
typedef _Float16 sx8_half2 __attribute__((ext_vector_type(2)));
typedef float sx8_float4 __attribute__((ext_vector_type(4)));

// fp16 bit pattern (low 16 bits) -> float, exact.
__host__ __device__ __forceinline__ float sx8_h2f(uint32_t bits) {
    return (float)__builtin_bit_cast(_Float16, (uint16_t)(bits & 0xFFFFu));
}

// z as two fp16 values hi = fp16(z), lo = fp16(z - hi) packed hi | lo << 16 (hi + lo
// keeps ~22 significant bits of z).
__device__ __forceinline__ uint32_t sx8_split_hl(float z) {
    const _Float16 hi = (_Float16)z;
    const _Float16 lo = (_Float16)(z - (float)hi);
    return (uint32_t)__builtin_bit_cast(uint16_t, hi) |
           ((uint32_t)__builtin_bit_cast(uint16_t, lo) << 16);
}

__host__ __device__ __forceinline__ int sx8_sext4(uint32_t v) {
    return (int)((v & 0xFu) ^ 0x8u) - 8;      // 0..7 -> 0..7, 8..15 -> -8..-1
}

// 6-bit level of weight i (0..7) of a sub-block, from its 4 hi-nibble bytes H (weight i
// at bits 4i) and its 2 lo-quad bytes P (weight i at bits 8*(i>>2) + 6 - 2*(i&3)).
// This is kernel_sx8_v43.py:23-25 restricted to one sub-block.
__host__ __device__ __forceinline__ uint32_t sx8_level(uint32_t H, uint32_t P, int i) {
    uint32_t nib = (H >> (4 * i)) & 0xFu;
    uint32_t qua = (P >> (8 * (i >> 2) + 6 - 2 * (i & 3))) & 0x3u;
    return (nib << 2) | qua;
}

// R64 decode of one 8-weight sub-block `sb` of a block (host-callable too, so the CPU
// tests can run this exact function against the oracle).  lo_f/hi_f are the fp16
// endpoints widened to float, b0/b1 the sub-block's slice of the two PCA bases and
// s0/s1 the scales, all widened to double (exact).  Writes the 8 fp16 results as
// four packed dwords, weight 2j in the low half of out[j].
//
// Arithmetic (kernel_sx8_v43.py:28-51):
//   q    = (double)(hi_f - lo_f) * 0.25          binary32 subtract, exact scale
//   rlo, rhi by strategy s                        exact in binary64 (<= 43 bits)
//   step = (rhi - rlo) * 0.015873, floored at 1e-10 (NaN passes the floor)
//   w    = fma(step, lv, rlo)                     NVVM contracts this mul+add
//   w    = fma((1.0*c0)*s0, b0, w), then c1/s1/b1 (the products are exact)
//   out  = fp16(float(w))                          two RNE conversions
// kPca = false drops the two PCA terms (the "core" weights rlo + step*lv), used when
// the PCA term is applied at the GEMM output from a caller-supplied Z.
template <bool kPca = true>
__host__ __device__ __forceinline__ void sx8_r64_subblock(float lo_f, float hi_f, uint32_t cfg,
                                                 uint32_t coeff, int sb, uint32_t H,
                                                 uint32_t P, const double* b0,
                                                 const double* b1, double s0, double s1,
                                                 uint32_t out[4]) {
#pragma clang fp contract(off)
    const float d32 = hi_f - lo_f;
    const double q = (double)d32 * 0.25;
    const double lo64 = (double)lo_f, hi64 = (double)hi_f;
    const uint32_t s = (cfg >> (2 * sb)) & 3u;
    double rlo, rhi;
    if (s == 0u)      { rlo = lo64;     rhi = hi64; }
    else if (s == 1u) { rlo = lo64;     rhi = lo64 + q; }
    else if (s == 2u) { rlo = hi64 - q; rhi = hi64; }
    else              { rlo = lo64 + q; rhi = hi64 - q; }
    double step = (rhi - rlo) * 0.015873;
    if (step < 1e-10) step = 1e-10;
    const double p0 = (1.0 * (double)sx8_sext4(coeff)) * s0;
    const double p1 = (1.0 * (double)sx8_sext4(coeff >> 4)) * s1;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        float f[2];
#pragma unroll
        for (int e = 0; e < 2; ++e) {
            const int i = 2 * j + e;
            double w = __builtin_fma(step, (double)sx8_level(H, P, i), rlo);
            if constexpr (kPca) {
                w = __builtin_fma(p0, b0[i], w);
                w = __builtin_fma(p1, b1[i], w);
            }
            f[e] = (float)w;
        }
        sx8_half2 h;
        h.x = (_Float16)f[0];
        h.y = (_Float16)f[1];
        out[j] = __builtin_bit_cast(uint32_t, h);
    }
}

// Load helpers for the kb-major v4.4 header row of block `bid` (HB = 6 or 8 bytes):
// dmin fp16 | dmax fp16 | config | coeff (| pad).  6-byte rows are only 2-byte aligned.
template <int HB>
__device__ __forceinline__ void sx8_load_hdr(const uint8_t* __restrict__ hdr, int64_t bid,
                                             uint32_t& d0, uint32_t& d1, uint32_t& cfg,
                                             uint32_t& coeff) {
    if constexpr (HB == 8) {
        const uint2 v = *reinterpret_cast<const uint2*>(hdr + bid * 8);
        d0 = v.x & 0xFFFFu;
        d1 = v.x >> 16;
        cfg = v.y & 0xFFu;
        coeff = (v.y >> 8) & 0xFFu;
    } else {
        const uint16_t* h = reinterpret_cast<const uint16_t*>(hdr + bid * 6);
        d0 = h[0];
        d1 = h[1];
        const uint32_t cc = h[2];
        cfg = cc & 0xFFu;
        coeff = cc >> 8;
    }
}

// x = silu(g) * u = g * rcp(1 + e^-g) * u in float32 (v_exp_f32, v_rcp_f32: the reciprocal
// is within 1 ulp, where a correctly rounded division costs nine more instructions; x is
// rounded to fp16 afterwards, 13 bits coarser), the product rounded to float32 before any
// fp16 conversion: the pin keeps the compiler from folding it into the conversion (one
// v_fma_mixlo_f16, a single rounding), which it does in some kernels and not in others.
// Every producer of the MLP's fp16 input -- the SiLU launch, the GEMV table build, the pair
// GEMV's epilogue, the prefill pack pass and the prefill GEMM's gate/up epilogue -- goes
// through here, so they give the same bits.
__device__ __forceinline__ float sx8_silu_mul(float g, float u) {
    float x = g * __builtin_amdgcn_rcpf(1.0f + __expf(-g)) * u;
    asm volatile("" : "+v"(x));
    return x;
}

// v with lanes 0-31 and 32-63 swapped (v_permlane32_swap).
__device__ __forceinline__ float sx8_lane_swap32(float v) {
    const uint32_t u = __builtin_bit_cast(uint32_t, v);
    const auto sw = __builtin_amdgcn_permlane32_swap(u, u, false, false);
    return __builtin_bit_cast(float, (threadIdx.x & 32) ? sw[0] : sw[1]);
}

// The prefill GEMM's packed operands (packed X and Zhl, the layouts of
// sx8_gemm_prefill_packed) of one 32-value K block of one row, from a 32 x 32 MFMA output
// fragment's lane layout: lane 32 h + c holds the row's values t = 8 gq + 4 h + e (gq, e <
// 4) in v[4 gq + e].  x = fp16(v) (zeros for rows past the end) goes into the packed chunk
// (k-step st, lane 32 hf + c, 8 values X[c][16 hf + 8 st ..]), and Z0, Z1 of the block in
// the reference's tree order -- products x_t b_t, pairs (t, t + 16), then offsets 8, 4, 2,
// 1 (cuda/sx8_decode1_v3.cu:53-63) -- times the scales, as split fp16 hi / lo pairs (lane h
// = 0 stores).  Offsets 16 and 8 stay in the lane, offset 4 is one swap of lane halves, so
// every lane of the wave must take part.  Bit for bit what k_compute_z<true, true> writes
// from the fp16 row.  bl: the block's 64 basis values (both vectors), sc: its two scales;
// xdst: the (row group, K block) chunk; zdst: the row's Zhl entry of the block.
__device__ __forceinline__ void sx8_pack_fragment(const float (&v)[16], bool row_ok, int c, int h,
                                                  const float* bl, float2 sc, uint16_t* xdst, uint32_t* zdst) {
#pragma clang fp contract(off)
    uint32_t xw[8];
    float xf[16];
#pragma unroll
    for (int i = 0; i < 8; ++i) {
        const uint16_t lo = row_ok ? __builtin_bit_cast(uint16_t, (_Float16)v[2 * i]) : (uint16_t)0;
        const uint16_t hi = row_ok ? __builtin_bit_cast(uint16_t, (_Float16)v[2 * i + 1]) : (uint16_t)0;
        xw[i] = (uint32_t)lo | ((uint32_t)hi << 16);
        xf[2 * i] = sx8_h2f(lo);
        xf[2 * i + 1] = sx8_h2f(hi);
    }
#pragma unroll
    for (int gq = 0; gq < 4; ++gq)
        *reinterpret_cast<uint2*>(xdst + (gq & 1) * 512 + ((gq >> 1) * 32 + c) * 8 + 4 * h) =
            make_uint2(xw[2 * gq], xw[2 * gq + 1]);
    float z[2];
#pragma unroll
    for (int j = 0; j < 2; ++j) {
        const float4* b = reinterpret_cast<const float4*>(bl + 32 * j + 4 * h);
        float pr[16];
#pragma unroll
        for (int gq = 0; gq < 4; ++gq) {
            const float4 bb = b[2 * gq];
            pr[4 * gq] = xf[4 * gq] * bb.x;
            pr[4 * gq + 1] = xf[4 * gq + 1] * bb.y;
            pr[4 * gq + 2] = xf[4 * gq + 2] * bb.z;
            pr[4 * gq + 3] = xf[4 * gq + 3] * bb.w;
        }
        float p[4];
#pragma unroll
        for (int e = 0; e < 4; ++e) {
            const float t16 = pr[e] + pr[8 + e];          // t = 4 h + e, with t + 16
            const float u16 = pr[4 + e] + pr[12 + e];     // t + 8, with t + 24
            p[e] = t16 + u16;                             // offset 8
        }
#pragma unroll
        for (int e = 0; e < 4; ++e) p[e] = p[e] + sx8_lane_swap32(p[e]);   // offset 4 (h = 0: t = e)
        p[0] = p[0] + p[2];
        p[1] = p[1] + p[3];
        z[j] = (j ? sc.y : sc.x) * (p[0] + p[1]);
        // z rounded to float32 before its fp16 split, as in k_compute_z (see sx8_silu_mul)
        asm volatile("" : "+v"(z[j]));
    }
    if (row_ok && h == 0) *reinterpret_cast<uint2*>(zdst) = make_uint2(sx8_split_hl(z[0]), sx8_split_hl(z[1]));
}

