// sx8_decoder.hip -- the small per-token ops of the end-to-end decoder that sit between
// the S-X8 GEMVs: residual add + RMSNorm, q/k RMSNorm + RoPE + KV-cache write, decode
// attention over the cache, SiLU * up, greedy argmax.  (In the reference these are the
// Hugging Face Qwen modules driven by scripts/infer_sx8.py:109-173.)  Each is one launch
// that reads its position from device memory, so a whole decode step can be captured in
// a HIP graph and replayed.
#include "sx8_buffer.h"
#include "sx8_device.h"
#include "sx8_host.h"

namespace {

__device__ __forceinline__ float h2f(uint16_t h) { return (float)__builtin_bit_cast(_Float16, h); }
__device__ __forceinline__ uint16_t f2h(float f) { return __builtin_bit_cast(uint16_t, (_Float16)f); }

typedef uint32_t sx8_u32x4 __attribute__((ext_vector_type(4)));

// A read-only argument pinned in SGPRs through an empty asm, so that its loads keep their
// place in the program (a load from the argument itself may be moved past barriers to its
// first use), and cast back to the global address space: through the pinned (generic)
// pointer the loads would be flat loads, counted on the LDS counter as well, so that every
// LDS wait would also wait for them.  (The attribute applies to the device pass only.)
#if defined(__HIP_DEVICE_COMPILE__)
#define SX8_DEC_GLOBAL __attribute__((address_space(1)))
#else
#define SX8_DEC_GLOBAL
#endif
template <typename T>
__device__ __forceinline__ const T SX8_DEC_GLOBAL* pinned_global(const T* p) {
    asm volatile("" : "+s"(p));
    return (const T SX8_DEC_GLOBAL*)p;
}
__device__ __forceinline__ sx8_u32x4 ld_u32x4(const uint16_t SX8_DEC_GLOBAL* p) {
    return *reinterpret_cast<const sx8_u32x4 SX8_DEC_GLOBAL*>(p);
}

// Sum over a 256-thread block (wave64 shuffles, then 4 partials through LDS).
__device__ __forceinline__ float block_sum256(float v, float* red) {
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o, 64);
    const int w = threadIdx.x >> 6;
    __syncthreads();
    if ((threadIdx.x & 63) == 0) red[w] = v;
    __syncthreads();
    return red[0] + red[1] + red[2] + red[3];
}

__device__ __forceinline__ float block_max256(float v, float* red) {
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) v = fmaxf(v, __shfl_xor(v, o, 64));
    const int w = threadIdx.x >> 6;
    __syncthreads();
    if ((threadIdx.x & 63) == 0) red[w] = v;
    __syncthreads();
    return fmaxf(fmaxf(red[0], red[1]), fmaxf(red[2], red[3]));
}

// Row r: resid = (init ? fp16 init : resid) + (delta ? delta : 0) in f32; out = fp16(resid *
// rsqrt(mean(resid^2) + eps) * w).  Rows of up to 256 * kRmsPer values stay in registers
// (every load of the row is issued before the reduction); longer rows loop.  vec (H % 4 ==
// 0, 16-byte aligned f32 rows, 8-byte aligned fp16 rows): 4 consecutive values per load,
// rows of up to 256 * 4 * kRmsPer4 values.
constexpr int kRmsPer = 16, kRmsPer4 = 4;

__device__ __forceinline__ float4 h4f(uint2 v) {
    return make_float4(h2f((uint16_t)(v.x & 0xFFFFu)), h2f((uint16_t)(v.x >> 16)), h2f((uint16_t)(v.y & 0xFFFFu)),
                       h2f((uint16_t)(v.y >> 16)));
}

// The vec path's row arithmetic, shared with k_add_rmsnorm_pack so both give the same bits:
// thread t's values i = t + 256 u (float4 units) of h = (init ? fp16 init : resid) + delta
// (+ pending partial slices), zero past the row; their squares summed with explicit fmas in
// a fixed order; x = h * inv * w rounded to float32 (pinned) before its fp16 conversion.
// NP > 0: delta is the first K range of a split GEMM whose other NP ranges' partial products
// sit at parts + s * slice (same row-major layout); each element is delta + part 0 + ... +
// part NP-1 in that order (the split-K sum of the GEMM, bit for bit) before it is added.
// One form per (init, delta) pair, with every load of the row (all rounds u, the delta and
// its partial slices) issued before the first sum: a null-pointer test inside the round loop
// became a branch per round, after which the compiler waited for all of that round's loads
// before issuing the next round's, one memory round trip per round.
template <int NP, bool kInit, bool kDelta>
__device__ __forceinline__ void rms_row_load_t(float4 (&v)[kRmsPer4], uint2 (&wv)[kRmsPer4], const float* resid,
                                               const float* delta, const uint16_t* init, const uint16_t* w,
                                               const float* parts, int64_t slice, int64_t base, int H4, int t) {
    constexpr int kP = kDelta ? NP : 0;
    const float4* r4 = reinterpret_cast<const float4*>(resid + base);
    const float4* d4 = reinterpret_cast<const float4*>(delta + (kDelta ? base : 0));
    const uint2* i4 = reinterpret_cast<const uint2*>(init + (kInit ? base : 0));
    const uint2* w4 = reinterpret_cast<const uint2*>(w);
    uint2 hi[kInit ? kRmsPer4 : 1];
    float4 x0[kRmsPer4], dd[kDelta ? kRmsPer4 : 1], pv[kRmsPer4][kP > 0 ? kP : 1];
#pragma unroll
    for (int u = 0; u < kRmsPer4; ++u) {       // every load of the row before the reduction
        const int ic = min(t + 256 * u, H4 - 1);
        if constexpr (kInit) hi[u] = i4[ic];
        else x0[u] = r4[ic];
        if constexpr (kDelta) {
            dd[u] = d4[ic];
#pragma unroll
            for (int s2 = 0; s2 < kP; ++s2) pv[u][s2] = reinterpret_cast<const float4*>(parts + s2 * slice + base)[ic];
        }
        wv[u] = w4[ic];
    }
#pragma unroll
    for (int u = 0; u < kRmsPer4; ++u) {
        const int i = t + 256 * u;
        float4 x = kInit ? h4f(hi[u]) : x0[u];
        if constexpr (kDelta) {
            float4 d = dd[u];
#pragma unroll
            for (int s2 = 0; s2 < kP; ++s2)
                d = make_float4(d.x + pv[u][s2].x, d.y + pv[u][s2].y, d.z + pv[u][s2].z, d.w + pv[u][s2].w);
            x = make_float4(x.x + d.x, x.y + d.y, x.z + d.z, x.w + d.w);
        }
        v[u] = i < H4 ? x : make_float4(0.f, 0.f, 0.f, 0.f);
    }
}

template <int NP>
__device__ __forceinline__ void rms_row_load(float4 (&v)[kRmsPer4], uint2 (&wv)[kRmsPer4], const float* resid,
                                             const float* delta, const uint16_t* init, const uint16_t* w,
                                             const float* parts, int64_t slice, int64_t base, int H4, int t) {
    if (init) {
        if (delta) rms_row_load_t<NP, true, true>(v, wv, resid, delta, init, w, parts, slice, base, H4, t);
        else rms_row_load_t<NP, true, false>(v, wv, resid, delta, init, w, parts, slice, base, H4, t);
    } else {
        if (delta) rms_row_load_t<NP, false, true>(v, wv, resid, delta, init, w, parts, slice, base, H4, t);
        else rms_row_load_t<NP, false, false>(v, wv, resid, delta, init, w, parts, slice, base, H4, t);
    }
}

__device__ __forceinline__ float rms_row_ss(const float4 (&v)[kRmsPer4]) {
    float ss = 0.f;
#pragma unroll
    for (int u = 0; u < kRmsPer4; ++u) {
        ss = __builtin_fmaf(v[u].x, v[u].x, ss);
        ss = __builtin_fmaf(v[u].y, v[u].y, ss);
        ss = __builtin_fmaf(v[u].z, v[u].z, ss);
        ss = __builtin_fmaf(v[u].w, v[u].w, ss);
    }
    return ss;
}

__device__ __forceinline__ float rms_scale(float h, float inv, float w) {
    float y = h * inv * w;
    asm volatile("" : "+v"(y));
    return y;
}

// (the row's 4 wave sums, added in wave order after the shuffle tree, as block_sum256)
__device__ __forceinline__ float wave_sum64(float v) {
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o, 64);
    return v;
}

template <int NP = 0>
__global__ __launch_bounds__(256) void k_add_rmsnorm(float* __restrict__ resid, const float* __restrict__ delta,
                                                     const uint16_t* __restrict__ init,
                                                     const uint16_t* __restrict__ w,
                                                     uint16_t* __restrict__ out, int H, float eps, bool vec,
                                                     const float* __restrict__ parts = nullptr,
                                                     int64_t slice = 0) {
    __shared__ float red[4];
    const int64_t base = (int64_t)blockIdx.x * H;
    auto dsum = [&](int64_t e) {         // delta (plus its pending partial sums) at element e
        float dd = delta[e];
        if constexpr (NP > 0) {
            float pv[NP];
#pragma unroll
            for (int s2 = 0; s2 < NP; ++s2) pv[s2] = parts[s2 * slice + e];
#pragma unroll
            for (int s2 = 0; s2 < NP; ++s2) dd += pv[s2];
        }
        return dd;
    };
    if (vec && H <= 256 * 4 * kRmsPer4) {
        const int H4 = H >> 2;
        float4 v[kRmsPer4];
        uint2 wv[kRmsPer4];
        rms_row_load<NP>(v, wv, resid, delta, init, w, parts, slice, base, H4, threadIdx.x);
        const float inv = 1.0f / sqrtf(block_sum256(rms_row_ss(v), red) / (float)H + eps);
        float4* r4 = reinterpret_cast<float4*>(resid + base);
        uint2* o4 = reinterpret_cast<uint2*>(out + base);
#pragma unroll
        for (int u = 0; u < kRmsPer4; ++u) {
            const int i = threadIdx.x + 256 * u;
            if (i < H4) {
                r4[i] = v[u];
                const float4 wf = h4f(wv[u]);
                o4[i] = make_uint2((uint32_t)f2h(rms_scale(v[u].x, inv, wf.x)) | ((uint32_t)f2h(rms_scale(v[u].y, inv, wf.y)) << 16),
                                   (uint32_t)f2h(rms_scale(v[u].z, inv, wf.z)) | ((uint32_t)f2h(rms_scale(v[u].w, inv, wf.w)) << 16));
            }
        }
        return;
    }
    if (H <= 256 * kRmsPer) {
        float v[kRmsPer], wv[kRmsPer];
#pragma unroll
        for (int u = 0; u < kRmsPer; ++u) {
            const int i = threadIdx.x + 256 * u;
            const int ic = min(i, H - 1);
            float x = init ? h2f(init[base + ic]) : resid[base + ic];
            if (delta) x += dsum(base + ic);
            v[u] = i < H ? x : 0.f;
            wv[u] = h2f(w[ic]);
        }
        float ss = 0.f;
#pragma unroll
        for (int u = 0; u < kRmsPer; ++u) ss += v[u] * v[u];
        const float inv = 1.0f / sqrtf(block_sum256(ss, red) / (float)H + eps);
#pragma unroll
        for (int u = 0; u < kRmsPer; ++u) {
            const int i = threadIdx.x + 256 * u;
            if (i < H) {
                resid[base + i] = v[u];
                out[base + i] = f2h(v[u] * inv * wv[u]);
            }
        }
        return;
    }
    float ss = 0.f;
    for (int i = threadIdx.x; i < H; i += 256) {
        float x = init ? h2f(init[base + i]) : resid[base + i];
        if (delta) x += dsum(base + i);
        resid[base + i] = x;
        ss += x * x;
    }
    const float inv = 1.0f / sqrtf(block_sum256(ss, red) / (float)H + eps);
    for (int i = threadIdx.x; i < H; i += 256) out[base + i] = f2h(resid[base + i] * inv * h2f(w[i]));
}

// k_add_rmsnorm's vec path, bit for bit (rms_row_*), for two rows per 512-thread work-group,
// whose normalized rows go out as the prefill GEMM's packed operands of the NS matrices that
// multiply them (sx8_gemm_prefill_packed) instead of fp16 rows: x into the packed X (rows
// past M up to the next multiple of 32 pack zeros) and, per matrix, Z0 / Z1 of every K
// block of every row (the reference's tree order, split fp16 hi / lo) into its Zhl -- what
// the GEMM's own pass over the fp16 rows writes.  Phase 1: the rows' values, sums and
// stores, x kept in LDS; phase 2: thread d takes the dot products (matrix s, K block kb,
// vector j) numbered d, d + 512, ..., for both rows at once (one basis read for two rows).
// H % 32 == 0, H <= 4096.
constexpr int kPackRows = 2;
struct NormPack {
    const float* basis[4];
    const float* scales[4];
    uint32_t* Zhl[4];
    uint16_t* Xp;
    int n_cb;
};

template <int NP, int NS>
__global__ __launch_bounds__(256 * kPackRows) void k_add_rmsnorm_pack(float* __restrict__ resid,
                                                                     const float* __restrict__ delta,
                                                                     const uint16_t* __restrict__ init,
                                                                     const uint16_t* __restrict__ w, int M, int H,
                                                                     float eps, const float* __restrict__ parts,
                                                                     int64_t slice, const NormPack pk) {
    __shared__ float red[kPackRows][4];
    // x in LDS, K block kb at 36 kb (4 floats of padding per block): phase 2 reads 32
    // consecutive floats per lane with the K block varying across lanes, which at a
    // 32-float stride would put every lane's 16-byte reads on the same banks
    constexpr int kXsStride = 36;
    __shared__ __align__(16) float xs[kPackRows][256 * 4 * kRmsPer4 / 32 * kXsStride];
    const int rl = threadIdx.x >> 8, t = threadIdx.x & 255;
    const int row = blockIdx.x * kPackRows + rl;
    const int H4 = H >> 2;
    const int n_cb = pk.n_cb;
    const bool live = row < M;
    const int rowc = live ? row : M - 1;              // rows past M: loads of a valid row, unused
    const int64_t base = (int64_t)rowc * H;
    // the basis vector and scale of this thread's first dot product (phase 2), requested
    // ahead of the rows so their round trip overlaps phase 1
    const int nd = NS * n_cb * 2;
    auto dot_of = [&](int d, int& s, int& kb, int& j) {
        s = d / (2 * n_cb);
        const int rem = d - s * 2 * n_cb;
        kb = rem >> 1;
        j = rem & 1;
    };
    auto set_ptr = [&](auto const (&a)[4], int s) { return s == 0 ? a[0] : s == 1 ? a[1] : s == 2 ? a[2] : a[3]; };
    float4 b0[8];
    float sc0 = 0.f;
    {
        int s, kb, j;
        dot_of(min((int)threadIdx.x, nd - 1), s, kb, j);
        const float4* b4 = reinterpret_cast<const float4*>(set_ptr(pk.basis, s) + (int64_t)kb * 64 + 32 * j);
#pragma unroll
        for (int q = 0; q < 8; ++q) b0[q] = b4[q];
        sc0 = set_ptr(pk.scales, s)[2 * kb + j];
    }
    float4 v[kRmsPer4];
    uint2 wv[kRmsPer4];
    rms_row_load<NP>(v, wv, resid, delta, init, w, parts, slice, base, H4, t);
    const float ws = wave_sum64(rms_row_ss(v));
    if ((t & 63) == 0) red[rl][t >> 6] = ws;
    __syncthreads();
    const float inv = 1.0f / sqrtf((red[rl][0] + red[rl][1] + red[rl][2] + red[rl][3]) / (float)H + eps);
    const int G = row >> 5, r = row & 31;
    float4* r4 = reinterpret_cast<float4*>(resid + base);
#pragma unroll
    for (int u = 0; u < kRmsPer4; ++u) {
        const int i = t + 256 * u;
        if (i >= H4) continue;
        uint32_t lo = 0u, hi = 0u;
        if (live) {
            r4[i] = v[u];
            const float4 wf = h4f(wv[u]);
            lo = (uint32_t)f2h(rms_scale(v[u].x, inv, wf.x)) | ((uint32_t)f2h(rms_scale(v[u].y, inv, wf.y)) << 16);
            hi = (uint32_t)f2h(rms_scale(v[u].z, inv, wf.z)) | ((uint32_t)f2h(rms_scale(v[u].w, inv, wf.w)) << 16);
        }
        *reinterpret_cast<float4*>(&xs[rl][kXsStride * (i >> 3) + 4 * (i & 7)]) = h4f(make_uint2(lo, hi));
        // element 4 i of the row: K block kb, chunk (hf, st), offset 0 or 4 within it
        const int e0 = 4 * i, kb = e0 >> 5, tt = e0 & 31;
        *reinterpret_cast<uint2*>(pk.Xp + (((int64_t)G * n_cb + kb) * 2 + ((tt >> 3) & 1)) * 512 +
                                  ((tt >> 4) * 32 + r) * 8 + (tt & 7)) = make_uint2(lo, hi);
    }
    __syncthreads();
    {
#pragma clang fp contract(off)
    for (int d = threadIdx.x; d < nd; d += 256 * kPackRows) {
        int s, kb, j;
        dot_of(d, s, kb, j);
        uint32_t* zs = set_ptr(pk.Zhl, s);
        float b[32];
        float sc = sc0;
        if (d == (int)threadIdx.x) {                    // the prefetched first dot product
#pragma unroll
            for (int q = 0; q < 8; ++q) {
                b[4 * q] = b0[q].x; b[4 * q + 1] = b0[q].y; b[4 * q + 2] = b0[q].z; b[4 * q + 3] = b0[q].w;
            }
        } else {
            const float4* b4 = reinterpret_cast<const float4*>(set_ptr(pk.basis, s) + (int64_t)kb * 64 + 32 * j);
#pragma unroll
            for (int q = 0; q < 8; ++q) {
                const float4 bb = b4[q];
                b[4 * q] = bb.x; b[4 * q + 1] = bb.y; b[4 * q + 2] = bb.z; b[4 * q + 3] = bb.w;
            }
            sc = set_ptr(pk.scales, s)[2 * kb + j];
        }
#pragma unroll
        for (int rr = 0; rr < kPackRows; ++rr) {
            const int row2 = blockIdx.x * kPackRows + rr;
            if (row2 >= M) break;
            const float* x = &xs[rr][kXsStride * kb];
            float p[16];
#pragma unroll
            for (int q = 0; q < 16; ++q) p[q] = x[q] * b[q] + x[q + 16] * b[q + 16];
#pragma unroll
            for (int off = 8; off > 0; off >>= 1)
#pragma unroll
                for (int q = 0; q < off; ++q) p[q] = p[q] + p[q + off];
            float z = sc * p[0];
            asm volatile("" : "+v"(z));
            zs[((int64_t)row2 * n_cb + kb) * 2 + j] = sx8_split_hl(z);
        }
    }
    }
}

// Heads per 256-thread block: nh query heads, then nk key heads, then nk value heads, TPH =
// 64 ceil(hd / 128) threads per head (256 / TPH heads per block, blockIdx.x numbering head
// groups), thread d < hd / 2 owning the pair (d, d + hd / 2): q/k RMSNorm over the head,
// RoPE (rotate-half) at position *pos, q to q_out, k into k_cache and v into v_cache (both
// (nk, L, hd)).  A multi-row call takes kRopeRows tokens per block (blockIdx.y) and requests
// every row's inputs before the first norm: a block per (head, token) leaves tens of
// thousands of one-wave work-groups that each wait two memory round trips.
constexpr int kRopeRows = 4;

// A float32 result pinned before its fp16 conversion: the compiler would otherwise fold the
// last multiply or fma into the conversion (v_fma_mixlo_f16, one rounding instead of two)
// in some kernels and unrolled copies and not in others.
__device__ __forceinline__ float rope_pin(float x) {
    asm volatile("" : "+v"(x));
    return x;
}

// NP > 0: q_raw, k_raw, v_raw hold the first K range of a split GEMM whose other NP ranges'
// partial products sit at q_part / k_part / v_part + s * slice (same layout); every value
// read is raw + part 0 + ... + part NP-1 in that order (the split-K sum, bit for bit).
template <int NP = 0>
__global__ __launch_bounds__(256) void k_qk_rope_cache(const float* __restrict__ q_raw,
                                                       const float* __restrict__ k_raw,
                                                       const float* __restrict__ v_raw,
                                                       const uint16_t* __restrict__ qn,
                                                       const uint16_t* __restrict__ kn,
                                                       const float* __restrict__ cos_t,
                                                       const float* __restrict__ sin_t,
                                                       const int64_t* __restrict__ pos_p,
                                                       uint16_t* __restrict__ q_out,
                                                       uint16_t* __restrict__ k_cache,
                                                       uint16_t* __restrict__ v_cache, int nh,
                                                       int nk, int hd, int L, float eps, int rows,
                                                       const float* __restrict__ q_part = nullptr,
                                                       const float* __restrict__ k_part = nullptr,
                                                       const float* __restrict__ v_part = nullptr,
                                                       int64_t slice = 0) {
    __shared__ float red[kRopeRows][4][2];
    const int half = hd >> 1;
    const int tph = hd > 128 ? 128 : 64;
    const int lh = (int)threadIdx.x / tph, d = (int)threadIdx.x - lh * tph;
    const int b = (int)blockIdx.x * (256 / tph) + lh;
    const bool is_v = b >= nh + nk && b < nh + 2 * nk;
    const bool is_qk = b < nh + nk;
    const bool is_q = b < nh;
    const int h = is_q ? b : is_qk ? b - nh : b - nh - nk;
    const bool act = is_qk && d < half;
    const int y0 = (int)blockIdx.y * kRopeRows;
    const int64_t pos0 = *pos_p;
    // (1) every row's q/k pair (and its value-head elements) requested together, with the
    // pending partial sums of each value (NP > 0) behind them
    float x1[kRopeRows], x2[kRopeRows], va[kRopeRows], vb[kRopeRows];
    constexpr int kP = NP > 0 ? NP : 1;
    float p1[kRopeRows][kP], p2[kRopeRows][kP], pa[kRopeRows][kP], pb[kRopeRows][kP];
#pragma unroll
    for (int r = 0; r < kRopeRows; ++r) {
        const int y = min(y0 + r, rows - 1);
        const int64_t qko = (is_q ? (int64_t)y * nh * hd : (int64_t)y * nk * hd) + h * hd;
        const float* src = (is_q ? q_raw : k_raw) + qko;
        x1[r] = act ? src[d] : 0.f;
        x2[r] = act ? src[d + half] : 0.f;
        const int64_t vo = (int64_t)y * nk * hd + h * hd;
        const float* vs = v_raw + vo;
        va[r] = is_v && d < hd ? vs[d] : 0.f;
        vb[r] = is_v && d + tph < hd ? vs[d + tph] : 0.f;
        if constexpr (NP > 0) {
            const float* ps = (is_q ? q_part : k_part) + qko;
            const float* pv = v_part + vo;
#pragma unroll
            for (int s2 = 0; s2 < NP; ++s2) {
                p1[r][s2] = act ? ps[s2 * slice + d] : 0.f;
                p2[r][s2] = act ? ps[s2 * slice + d + half] : 0.f;
                pa[r][s2] = is_v && d < hd ? pv[s2 * slice + d] : 0.f;
                pb[r][s2] = is_v && d + tph < hd ? pv[s2 * slice + d + tph] : 0.f;
            }
        }
    }
    if constexpr (NP > 0) {
#pragma unroll
        for (int r = 0; r < kRopeRows; ++r)
#pragma unroll
            for (int s2 = 0; s2 < NP; ++s2) {
                x1[r] += p1[r][s2];
                x2[r] += p2[r][s2];
                va[r] += pa[r][s2];
                vb[r] += pb[r][s2];
            }
    }
    // (2) per row: RMSNorm, RoPE at *pos + y, stores (rows outside the cache write nothing)
#pragma unroll
    for (int r = 0; r < kRopeRows; ++r) {
        const int y = y0 + r;
        const int64_t pos = pos0 + y;
        const bool row_ok = y < rows && pos >= 0 && pos < L;
        if (row_ok && is_v) {
            uint16_t* vd = v_cache + ((int64_t)h * L + pos) * hd;
            if (d < hd) vd[d] = f2h(rope_pin(va[r]));
            if (d + tph < hd) vd[d + tph] = f2h(rope_pin(vb[r]));
            for (int e = d + 2 * tph; e < hd; e += tph) {
                const int64_t vo = (int64_t)y * nk * hd + h * hd + e;
                float ve = v_raw[vo];
                if constexpr (NP > 0) {
#pragma unroll
                    for (int s2 = 0; s2 < NP; ++s2) ve += v_part[s2 * slice + vo];
                }
                vd[e] = f2h(rope_pin(ve));
            }
        }
        // (explicit fmas here and in the rotation: which product the compiler would fuse
        // differs between kernels)
        float ss = __builtin_fmaf(x1[r], x1[r], x2[r] * x2[r]);
#pragma unroll
        for (int o = 32; o > 0; o >>= 1) ss += __shfl_xor(ss, o, 64);
        if (tph > 64) {                      // two waves per head (every thread reaches the barrier)
            if ((d & 63) == 0) red[r][lh][d >> 6] = ss;
            __syncthreads();
            ss = red[r][lh][0] + red[r][lh][1];
        }
        if (!act || !row_ok) continue;
        const uint16_t* nw = is_q ? qn : kn;
        const float inv = 1.0f / sqrtf(ss / (float)hd + eps);
        // round to fp16 after the norm, as the fp16 activations of the model do
        const float n1 = h2f(f2h(rope_pin(x1[r] * inv * h2f(nw[d]))));
        const float n2 = h2f(f2h(rope_pin(x2[r] * inv * h2f(nw[d + half]))));
        const float c = cos_t[pos * half + d], s = sin_t[pos * half + d];
        const float o1 = rope_pin(__builtin_fmaf(n1, c, -(n2 * s))), o2 = rope_pin(__builtin_fmaf(n2, c, n1 * s));
        if (is_q) {
            uint16_t* qo = q_out + (int64_t)y * nh * hd + h * hd;
            qo[d] = f2h(o1);
            qo[d + half] = f2h(o2);
        } else {
            uint16_t* kd = k_cache + ((int64_t)h * L + pos) * hd;
            kd[d] = f2h(o1);
            kd[d + half] = f2h(o2);
        }
    }
}

// Decode attention: one 256-thread block per query head over cache positions 0..*pos,
// caches (nk, L, hd).  Work-group b runs query head (b % 8) * (nh / 8) + b / 8, so the
// query heads sharing a KV head run on one XCD and share its L2 copy of the cache (for
// nh % 8 == 0).  Scores: a lane holds 8 consecutive dims of one position (one 16-byte
// load), the CH = hd / 8 lanes of a position reduce with shuffles.  Output: thread
// (position group, 8-dim chunk) accumulates its positions, the groups meet in LDS.
constexpr int kAttnMaxL = 4096;

template <int HD>
__global__ __launch_bounds__(256) void k_attn_decode(const uint16_t* __restrict__ q,
                                                     const uint16_t* __restrict__ k_cache,
                                                     const uint16_t* __restrict__ v_cache,
                                                     const int64_t* __restrict__ pos_p,
                                                     uint16_t* __restrict__ out, int nh, int nk,
                                                     int L, float scale) {
    constexpr int CH = HD / 8;             // 16-byte chunks per cache row
    constexpr int PG = 256 / CH;           // position groups of the output pass
    __shared__ float p[kAttnMaxL];
    __shared__ float red[4];
    __shared__ float acc[PG][HD + 4];
    const int b = blockIdx.x;
    const int h = (nh % 8 == 0) ? (b % 8) * (nh / 8) + b / 8 : b;
    const int kv = h / (nh / nk);
    const int64_t pos = *pos_p;
    const int n = (int)min(max(pos, (int64_t)0) + 1, (int64_t)L);   // positions 0..pos, inside the cache
    const int tid = threadIdx.x;
    const int c = tid % CH;
    float qv[8];
    {
        const sx8_u32x4 w = *reinterpret_cast<const sx8_u32x4*>(q + h * HD + 8 * c);
#pragma unroll
        for (int e = 0; e < 4; ++e) {
            qv[2 * e] = h2f(w[e] & 0xFFFFu);
            qv[2 * e + 1] = h2f(w[e] >> 16);
        }
    }
    const uint16_t* kc = k_cache + (int64_t)kv * L * HD;
    float m = -INFINITY;
    // kU positions per lane in flight: all loads of a round are issued before any is used
    constexpr int kU = 8;
    for (int j0 = tid / CH; j0 < n; j0 += kU * PG) {
        sx8_u32x4 w[kU];
#pragma unroll
        for (int u = 0; u < kU; ++u) {
            const int j = min(j0 + u * PG, n - 1);      // past the end: a valid row, result unused
            w[u] = *reinterpret_cast<const sx8_u32x4*>(kc + (int64_t)j * HD + 8 * c);
        }
#pragma unroll
        for (int u = 0; u < kU; ++u) {
            float s = 0.f;
#pragma unroll
            for (int e = 0; e < 4; ++e)
                s += qv[2 * e] * h2f(w[u][e] & 0xFFFFu) + qv[2 * e + 1] * h2f(w[u][e] >> 16);
#pragma unroll
            for (int o = CH / 2; o > 0; o >>= 1) s += __shfl_xor(s, o, 64);
            s *= scale;
            const int j = j0 + u * PG;
            if (j < n) {
                if (c == 0) p[j] = s;
                m = fmaxf(m, s);
            }
        }
    }
    m = block_max256(m, red);            // its barriers also publish p[]
    float sum = 0.f;
    for (int j = tid; j < n; j += 256) {
        const float e = __expf(p[j] - m);
        p[j] = e;
        sum += e;
    }
    sum = block_sum256(sum, red);
    const uint16_t* vc = v_cache + (int64_t)kv * L * HD;
    const int pg = tid / CH;
    float a[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
    for (int j0 = pg; j0 < n; j0 += kU * PG) {
        sx8_u32x4 w[kU];
#pragma unroll
        for (int u = 0; u < kU; ++u) {
            const int j = min(j0 + u * PG, n - 1);
            w[u] = *reinterpret_cast<const sx8_u32x4*>(vc + (int64_t)j * HD + 8 * c);
        }
#pragma unroll
        for (int u = 0; u < kU; ++u) {
            const int j = j0 + u * PG;
            const float pj = j < n ? p[j] : 0.f;
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                a[2 * e] += pj * h2f(w[u][e] & 0xFFFFu);
                a[2 * e + 1] += pj * h2f(w[u][e] >> 16);
            }
        }
    }
#pragma unroll
    for (int e = 0; e < 8; ++e) acc[pg][8 * c + e] = a[e];
    __syncthreads();
    if (tid < HD) {
        float t = 0.f;
        for (int g = 0; g < PG; ++g) t += acc[g][tid];
        out[h * HD + tid] = f2h(t / sum);
    }
}

// k_qk_rope_cache for HD = 128, bit for bit, with 16-byte accesses: 16 lanes per (row,
// head), unit u = y (nh + 2 nk) + b of the 16 per 256-thread work-group (b numbering q, then
// k, then v heads as k_qk_rope_cache does).  A q/k lane j holds dims 4 j .. 4 j + 3 and their
// RoPE partners 64 + 4 j .. (the pair k_qk_rope_cache's thread d owns, four at a time); its
// sum of squares follows k_qk_rope_cache's 64-lane butterfly exactly: dim bits 5, 4, 3, 2
// are lane bits 3, 2, 1, 0 (shuffles over lanes j ^ 8, ^ 4, ^ 2, ^ 1, per dim), bits 1 and 0
// the dim within the lane.  A v lane copies dims 8 j .. 8 j + 7.  Every load is issued
// unconditionally (clamped to a valid unit and table row) ahead of any arithmetic.  Needs
// 16-byte aligned rows, partial slices and caches, 8-byte aligned norm weights.
template <int NP = 0>
__global__ __launch_bounds__(256) void k_qk_rope128(const float* __restrict__ q_raw, const float* __restrict__ k_raw,
                                                    const float* __restrict__ v_raw,
                                                    const uint16_t* __restrict__ qn,
                                                    const uint16_t* __restrict__ kn,
                                                    const float* __restrict__ cos_t,
                                                    const float* __restrict__ sin_t,
                                                    const int64_t* __restrict__ pos_p,
                                                    uint16_t* __restrict__ q_out, uint16_t* __restrict__ k_cache,
                                                    uint16_t* __restrict__ v_cache, int nh, int nk, int hd, int L,
                                                    float eps, int rows, const float* __restrict__ q_part,
                                                    const float* __restrict__ k_part,
                                                    const float* __restrict__ v_part, int64_t slice) {
    constexpr int HD = 128, half = 64;
    const int NH = nh + 2 * nk;
    const int unit = (int)blockIdx.x * 16 + ((int)threadIdx.x >> 4), j = (int)threadIdx.x & 15;
    const bool live = unit < rows * NH;
    const int uc = min(unit, rows * NH - 1);
    const int y = uc / NH, b = uc - y * NH;
    const bool is_q = b < nh, is_v = b >= nh + nk;
    const int h = is_q ? b : is_v ? b - nh - nk : b - nh;
    const int width = is_q ? nh * HD : nk * HD;
    const int64_t ro = (int64_t)y * width + h * HD;                 // the unit's row in its source
    // (sources read through pinned_global and ordered by an empty asm below: a load from a
    // read-only argument may otherwise sink behind the branches to its first use)
    typedef const float SX8_DEC_GLOBAL* gf;
    const gf qg = pinned_global(q_raw), kg = pinned_global(k_raw), vg = pinned_global(v_raw);
    const gf qpg = pinned_global(q_part), kpg = pinned_global(k_part), vpg = pinned_global(v_part);
    const gf src = is_q ? qg : is_v ? vg : kg;
    const gf prt = is_q ? qpg : is_v ? vpg : kpg;
    const int e1 = is_v ? 8 * j : 4 * j, e2 = is_v ? 8 * j + 4 : half + 4 * j;
    const int64_t pos = *pos_p + y;
    const int pr = (int)min(max(pos, (int64_t)0), (int64_t)L - 1);
    const uint16_t SX8_DEC_GLOBAL* qng = pinned_global(qn);
    const uint16_t SX8_DEC_GLOBAL* kng = pinned_global(kn);
    const uint16_t SX8_DEC_GLOBAL* nw = is_q ? qng : kng;
    const float SX8_DEC_GLOBAL* ct = pinned_global(cos_t);
    const float SX8_DEC_GLOBAL* st = pinned_global(sin_t);
    typedef const float4 SX8_DEC_GLOBAL* gf4;
    typedef const uint2 SX8_DEC_GLOBAL* gu2;
    float4 x1 = *(gf4)(src + ro + e1);
    float4 x2 = *(gf4)(src + ro + e2);
    constexpr int kP = NP > 0 ? NP : 1;
    float4 p1[kP], p2[kP];
#pragma unroll
    for (int s2 = 0; s2 < NP; ++s2) {
        p1[s2] = *(gf4)(prt + s2 * slice + ro + e1);
        p2[s2] = *(gf4)(prt + s2 * slice + ro + e2);
    }
    const uint2 w1 = *(gu2)(nw + 4 * j);
    const uint2 w2 = *(gu2)(nw + half + 4 * j);
    const float4 cs = *(gf4)(ct + (int64_t)pr * half + 4 * j);
    const float4 sn = *(gf4)(st + (int64_t)pr * half + 4 * j);
    asm volatile("" ::: "memory");
#pragma unroll
    for (int s2 = 0; s2 < NP; ++s2) {
        x1 = make_float4(x1.x + p1[s2].x, x1.y + p1[s2].y, x1.z + p1[s2].z, x1.w + p1[s2].w);
        x2 = make_float4(x2.x + p2[s2].x, x2.y + p2[s2].y, x2.z + p2[s2].z, x2.w + p2[s2].w);
    }
    const float a1[4] = {x1.x, x1.y, x1.z, x1.w}, a2[4] = {x2.x, x2.y, x2.z, x2.w};
    float ssd[4];
#pragma unroll
    for (int e = 0; e < 4; ++e) ssd[e] = __builtin_fmaf(a1[e], a1[e], a2[e] * a2[e]);
#pragma unroll
    for (int o = 8; o > 0; o >>= 1)
#pragma unroll
        for (int e = 0; e < 4; ++e) ssd[e] += __shfl_xor(ssd[e], o, 16);
    const float ss = (ssd[0] + ssd[2]) + (ssd[1] + ssd[3]);
    // (every lane computes the q/k result, so that no load sinks behind a branch)
    const float inv = 1.0f / sqrtf(ss / (float)hd + eps);
    const float wf1[4] = {h2f((uint16_t)(w1.x & 0xFFFFu)), h2f((uint16_t)(w1.x >> 16)), h2f((uint16_t)(w1.y & 0xFFFFu)),
                          h2f((uint16_t)(w1.y >> 16))};
    const float wf2[4] = {h2f((uint16_t)(w2.x & 0xFFFFu)), h2f((uint16_t)(w2.x >> 16)), h2f((uint16_t)(w2.y & 0xFFFFu)),
                          h2f((uint16_t)(w2.y >> 16))};
    const float c4[4] = {cs.x, cs.y, cs.z, cs.w}, s4[4] = {sn.x, sn.y, sn.z, sn.w};
    uint16_t o1h[4], o2h[4];
#pragma unroll
    for (int e = 0; e < 4; ++e) {
        // round to fp16 after the norm, as the fp16 activations of the model do
        const float n1 = h2f(f2h(rope_pin(a1[e] * inv * wf1[e]))), n2 = h2f(f2h(rope_pin(a2[e] * inv * wf2[e])));
        const float c = c4[e], sv = s4[e];
        o1h[e] = f2h(rope_pin(__builtin_fmaf(n1, c, -(n2 * sv))));
        o2h[e] = f2h(rope_pin(__builtin_fmaf(n2, c, n1 * sv)));
    }
    const uint2 u1 = make_uint2((uint32_t)o1h[0] | ((uint32_t)o1h[1] << 16), (uint32_t)o1h[2] | ((uint32_t)o1h[3] << 16));
    const uint2 u2 = make_uint2((uint32_t)o2h[0] | ((uint32_t)o2h[1] << 16), (uint32_t)o2h[2] | ((uint32_t)o2h[3] << 16));
    // rows outside the cache write nothing
    if (!(live && pos >= 0 && pos < L)) return;
    if (is_v) {
        auto hp = [](float a, float b) {
            return (uint32_t)f2h(rope_pin(a)) | ((uint32_t)f2h(rope_pin(b)) << 16);
        };
        *reinterpret_cast<uint4*>(v_cache + ((int64_t)h * L + pos) * HD + 8 * j) =
            make_uint4(hp(x1.x, x1.y), hp(x1.z, x1.w), hp(x2.x, x2.y), hp(x2.z, x2.w));
        return;
    }
    uint16_t* dst = is_q ? q_out + (int64_t)y * nh * HD + h * HD : k_cache + ((int64_t)h * L + pos) * HD;
    *reinterpret_cast<uint2*>(dst + 4 * j) = u1;
    *reinterpret_cast<uint2*>(dst + half + 4 * j) = u2;
}

// Split decode attention, two launches.  k_attn_split: work-group (kv head, chunk) takes
// positions [chunk T, chunk T + T) of 0..*pos (T = ceil(n / kAttnChunks)) for all G query
// heads that share the KV head, so every cache row is read once.  Lane group pg (CH lanes,
// 8 dims each) streams positions pg, pg + PG, ... of the chunk with an online softmax: the
// K and V rows of kU positions are loaded together, then per head the running max m, sum
// l of exp(s - m) and acc = sum exp(s - m) v are rescaled and updated, so one pass over
// the cache suffices and no score array is kept.  The lane groups meet in LDS and the
// chunk's (m, l, acc[hd]) per head goes to the workspace.  k_attn_combine: per head and
// dim, out = sum_c e^(m_c - M) acc_c / sum_c e^(m_c - M) l_c over the chunks in order
// (deterministic; an empty chunk has m = -inf, l = 0 and weighs nothing).
// kAttnChunks x n_kv work-groups spread the cache reads where one work-group per query head
// (k_attn_decode) waits on the cache latency round after round.  The combine reads every
// chunk's partials, so fewer chunks shorten it; 36-layer decode at 513..767 positions,
// ms per token on one box: 8 chunks 1.589, 12 1.534, 16 1.534, 24 1.557, 32 1.569.  (A
// chunk count derived from *pos on the device was slower, 1.66: the combine's loads then
// wait for that read.)
constexpr int kAttnChunks = 16;
constexpr int64_t kAttnSplitMaxL = (int64_t)1 << 20;

// Inputs of the RoPE-fused form (kRope): the raw f32 projections and what
// k_qk_rope_cache takes; the work-group whose chunk holds *pos also writes that
// position's k and v into the caches.
struct RopeIn {
    const float* q_raw;      // (nh, HD)
    const float* k_raw;      // (nk, HD)
    const float* v_raw;      // (nk, HD)
    const uint16_t* qn;      // q RMSNorm weight (HD)
    const uint16_t* kn;      // k RMSNorm weight (HD)
    const float* cos_t;      // (L, HD / 2)
    const float* sin_t;
    uint16_t* k_out;         // k_cache, written at *pos
    uint16_t* v_out;         // v_cache
    float eps;
};

// Lane-group helpers.  A lane group is CH = HD / 8 consecutive lanes (16 for HD 128: one
// DPP row; 8 for HD 64: half a row), lane c holding dims 8c .. 8c + 7 of a head row.
template <int kCtrl>
__device__ __forceinline__ float dpp_f(float v) {
    return __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), kCtrl, 0xF, 0xF,
                                                                 false));
}

// Sum over the lanes of a lane group, the same value in every lane: DPP quad swaps, then
// the half-row mirror and (CH = 16) the row mirror -- VALU operations, no LDS round trips.
template <int CH>
__device__ __forceinline__ float group_sum(float v) {
    v += dpp_f<0xB1>(v);                              // quad_perm [1, 0, 3, 2]
    v += dpp_f<0x4E>(v);                              // quad_perm [2, 3, 0, 1]
    v += dpp_f<0x141>(v);                             // row_half_mirror
    if constexpr (CH == 16) v += dpp_f<0x140>(v);     // row_mirror
    return v;
}

// The value of lane c ^ (CH / 2) of the lane group (the RoPE partner of lane c).
template <int CH>
__device__ __forceinline__ float group_partner(float v) {
    if constexpr (CH == 16) return dpp_f<0x128>(v);   // row_ror:8 (= lane ^ 8 within the row)
    else return __shfl_xor(v, CH / 2, CH);
}

// One head row's inputs for RMSNorm + RoPE (8 values per lane): the row, the norm weight
// and the cos / sin entries at the table row, all requested together.
struct RopeRow {
    float4 a, b;
    sx8_u32x4 w;
    float4 c0, c1, s0, s1;
};

template <int HD>
__device__ __forceinline__ void rope_load(RopeRow& r, const float* __restrict__ src,
                                          const uint16_t* __restrict__ w, const float* __restrict__ cos_t,
                                          const float* __restrict__ sin_t, int64_t pos, int c) {
    constexpr int CH = HD / 8, half = HD / 2;
    r.a = *reinterpret_cast<const float4*>(src + 8 * c);
    r.b = *reinterpret_cast<const float4*>(src + 8 * c + 4);
    r.w = *reinterpret_cast<const sx8_u32x4*>(w + 8 * c);
    const int d0 = c < CH / 2 ? 8 * c : 8 * c - half;
    r.c0 = *reinterpret_cast<const float4*>(cos_t + pos * half + d0);
    r.c1 = *reinterpret_cast<const float4*>(cos_t + pos * half + d0 + 4);
    r.s0 = *reinterpret_cast<const float4*>(sin_t + pos * half + d0);
    r.s1 = *reinterpret_cast<const float4*>(sin_t + pos * half + d0 + 4);
}

// RMSNorm over the head row (sum of squares over the lane group), fp16 rounding, then
// rotate-half RoPE: dim d < HD / 2 pairs with d + HD / 2, i.e. lane c with c ^ (CH / 2).
// The results are fp16-rounded (as the caches and k_qk_rope_cache hold them), packed in
// pairs: o[e] = (dim 8c + 2e, dim 8c + 2e + 1).
template <int HD>
__device__ __forceinline__ void rope_apply(const RopeRow& r, int c, float eps, uint32_t o[4]) {
    constexpr int CH = HD / 8;
    const float x[8] = {r.a.x, r.a.y, r.a.z, r.a.w, r.b.x, r.b.y, r.b.z, r.b.w};
    const float cs[8] = {r.c0.x, r.c0.y, r.c0.z, r.c0.w, r.c1.x, r.c1.y, r.c1.z, r.c1.w};
    const float sn[8] = {r.s0.x, r.s0.y, r.s0.z, r.s0.w, r.s1.x, r.s1.y, r.s1.z, r.s1.w};
    float ss = 0.f;
#pragma unroll
    for (int e = 0; e < 8; ++e) ss += x[e] * x[e];
    ss = group_sum<CH>(ss);
    const float inv = 1.0f / sqrtf(ss / (float)HD + eps);
    const bool lo = c < CH / 2;
    float res[8];
#pragma unroll
    for (int e = 0; e < 8; ++e) {
        const float nv = h2f(f2h(x[e] * inv * h2f((uint16_t)(r.w[e >> 1] >> (16 * (e & 1))))));
        const float other = group_partner<CH>(nv);
        // first half: n1 c - n2 s; second half: n2 c + n1 s (own value is n2, partner n1)
        res[e] = lo ? nv * cs[e] - other * sn[e] : nv * cs[e] + other * sn[e];
    }
#pragma unroll
    for (int e = 0; e < 4; ++e) o[e] = (uint32_t)f2h(res[2 * e]) | ((uint32_t)f2h(res[2 * e + 1]) << 16);
}

template <int HD, int G, bool kRope = false>
__global__ __launch_bounds__(256) void k_attn_split(const uint16_t* __restrict__ q,
                                                    const uint16_t* __restrict__ k_cache,
                                                    const uint16_t* __restrict__ v_cache,
                                                    const int64_t* __restrict__ pos_p,
                                                    float* __restrict__ part, int L, float scale,
                                                    const RopeIn ri = RopeIn{}) {
    constexpr int CH = HD / 8;
    constexpr int PG = 256 / CH;
    constexpr int kU = 4;
    // kRope rows by wave: waves 0 .. kQw - 1 the G q rows (one lane group each), wave kQw the
    // new k row, wave kQw + 1 the new v row -- one pointer per wave, picked with scalar
    // selects (a per-lane pick of a kernel-argument field becomes a vector load of it)
    constexpr int kGpw = 64 / CH, kQw = (G + kGpw - 1) / kGpw;
    static_assert(!kRope || kQw + 2 <= 4, "k_attn_split: waves for the q, k and v rows");
    __shared__ float sm[PG][G], sl[PG][G];
    __shared__ float sacc[PG][G][HD + 4];
    __shared__ uint32_t rq[kRope ? G : 1][HD / 2], rk[HD / 2], rv[HD / 2];   // RoPE'd rows (fp16 pairs)
    const int kv = blockIdx.x / kAttnChunks, chunk = blockIdx.x % kAttnChunks;
    const int64_t pos = *pos_p;
    const int n = (int)min(max(pos, (int64_t)0) + 1, (int64_t)L);
    const int T = (n + kAttnChunks - 1) / kAttnChunks;
    const int jb = chunk * T, je = min(jb + T, n);
    const int tid = threadIdx.x, c = tid % CH, pg = tid / CH;
    // kRope: the new position's row (pos inside the cache and inside this chunk) comes from
    // LDS, not from the cache this launch is writing
    const bool own_new = kRope && pos >= 0 && pos < L && pos >= jb && pos < je;
    const int64_t pr = min(max(pos, (int64_t)0), (int64_t)L - 1);   // RoPE table row

    // (1) kRope: the inputs of this lane group's row -- q head kv G + pg in the q waves, the
    // new k row in wave kQw, the new v row in wave kQw + 1 (every lane group of a wave loads
    // its row; the idle ones repeat a valid one) -- requested first, without branches (rows
    // merged from branches would be register copies that wait for their loads)
    const int wv = __builtin_amdgcn_readfirstlane(tid >> 6);
    RopeRow rr;
    if constexpr (kRope) {
        const float* src = wv < kQw ? ri.q_raw + (int64_t)(kv * G + min(pg, G - 1)) * HD
                                    : (wv == kQw ? ri.k_raw : ri.v_raw) + (int64_t)kv * HD;
        rope_load<HD>(rr, src, wv < kQw ? ri.qn : ri.kn, ri.cos_t, ri.sin_t, pr, c);
    }
    // (2) then the chunk's first kU K and V rows of this lane group (past the chunk: a valid
    // row, its score is -inf), behind the row inputs: the memory counter retires loads in
    // order, so the RoPE math waits only for what was issued before these
    asm volatile("" ::: "memory");
    const uint16_t* kc = k_cache + (int64_t)kv * L * HD;
    const uint16_t* vc = v_cache + (int64_t)kv * L * HD;
    sx8_u32x4 kr[kU], vr[kU];
    auto load_rows = [&](int j0) {
#pragma unroll
        for (int u = 0; u < kU; ++u)
            kr[u] = *reinterpret_cast<const sx8_u32x4*>(kc + (int64_t)min(j0 + u * PG, je - 1) * HD + 8 * c);
#pragma unroll
        for (int u = 0; u < kU; ++u)
            vr[u] = *reinterpret_cast<const sx8_u32x4*>(vc + (int64_t)min(j0 + u * PG, je - 1) * HD + 8 * c);
    };
    load_rows(jb + pg);
    __builtin_amdgcn_sched_barrier(0);       // no RoPE math (which waits for its rows) above here

    // (3) kRope: norm + RoPE of the G q rows and the new k row in parallel (one lane group
    // each), the new rows into the caches (the chunk holding *pos), all of them into LDS
    uint32_t qv[G][4];
    sx8_u32x4 knew = sx8_u32x4{0u, 0u, 0u, 0u}, vnew = knew;
    if constexpr (kRope) {
        uint32_t o[4];
        rope_apply<HD>(rr, c, ri.eps, o);          // every lane group (the v row's result is unused)
        const bool first = pg == wv * kGpw;       // the first lane group of its wave
        if (wv < kQw) {
            if (pg < G)
#pragma unroll
                for (int e = 0; e < 4; ++e) rq[pg][4 * c + e] = o[e];
        } else if (wv == kQw && first && own_new) {
            const sx8_u32x4 w = sx8_u32x4{o[0], o[1], o[2], o[3]};
            *reinterpret_cast<sx8_u32x4*>(&rk[4 * c]) = w;
            *reinterpret_cast<sx8_u32x4*>(ri.k_out + ((int64_t)kv * L + pos) * HD + 8 * c) = w;
        } else if (wv == kQw + 1 && first && own_new) {
            const float f[8] = {rr.a.x, rr.a.y, rr.a.z, rr.a.w, rr.b.x, rr.b.y, rr.b.z, rr.b.w};
            sx8_u32x4 w;
#pragma unroll
            for (int e = 0; e < 4; ++e) w[e] = (uint32_t)f2h(f[2 * e]) | ((uint32_t)f2h(f[2 * e + 1]) << 16);
            *reinterpret_cast<sx8_u32x4*>(&rv[4 * c]) = w;
            *reinterpret_cast<sx8_u32x4*>(ri.v_out + ((int64_t)kv * L + pos) * HD + 8 * c) = w;
        }
        __syncthreads();
#pragma unroll
        for (int g = 0; g < G; ++g)
#pragma unroll
            for (int e = 0; e < 4; ++e) qv[g][e] = rq[g][4 * c + e];
        if (own_new) {
            knew = *reinterpret_cast<const sx8_u32x4*>(&rk[4 * c]);
            vnew = *reinterpret_cast<const sx8_u32x4*>(&rv[4 * c]);
        }
    } else {
#pragma unroll
        for (int g = 0; g < G; ++g) {
            const sx8_u32x4 x = *reinterpret_cast<const sx8_u32x4*>(q + (kv * G + g) * HD + 8 * c);
#pragma unroll
            for (int e = 0; e < 4; ++e) qv[g][e] = x[e];
        }
    }

    // (4) online softmax over the lane group's positions pg, pg + PG, ... of the chunk
    float m[G], l[G], a[G][8];
#pragma unroll
    for (int g = 0; g < G; ++g) {
        m[g] = -INFINITY;
        l[g] = 0.f;
#pragma unroll
        for (int e = 0; e < 8; ++e) a[g][e] = 0.f;
    }
    for (int j0 = jb + pg; j0 < je;) {
        float s[kU][G];
        float vf[kU][8];
#pragma unroll
        for (int u = 0; u < kU; ++u) {
            const bool is_new = own_new && min(j0 + u * PG, je - 1) == pos;
#pragma unroll
            for (int g = 0; g < G; ++g) {
                float sc = 0.f;
#pragma unroll
                for (int e = 0; e < 4; ++e) {
                    // (through a scalar: a bit_cast of a vector-element lvalue reads element 0)
                    const uint32_t kw = is_new ? knew[e] : kr[u][e];
                    sc = __builtin_amdgcn_fdot2(__builtin_bit_cast(sx8_half2, qv[g][e]),
                                                __builtin_bit_cast(sx8_half2, kw), sc, false);
                }
                sc = group_sum<CH>(sc);
                s[u][g] = j0 + u * PG < je ? sc * scale : -INFINITY;
            }
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                const uint32_t vw = is_new ? vnew[e] : vr[u][e];
                vf[u][2 * e] = h2f((uint16_t)(vw & 0xFFFFu));
                vf[u][2 * e + 1] = h2f((uint16_t)(vw >> 16));
            }
        }
#pragma unroll
        for (int g = 0; g < G; ++g) {
            float mx = m[g];
#pragma unroll
            for (int u = 0; u < kU; ++u) mx = fmaxf(mx, s[u][g]);       // finite: u = 0 is in the chunk
            const float alpha = __expf(m[g] - mx);                       // 0 on the first pass
            l[g] *= alpha;
#pragma unroll
            for (int e = 0; e < 8; ++e) a[g][e] *= alpha;
#pragma unroll
            for (int u = 0; u < kU; ++u) {
                const float pu = __expf(s[u][g] - mx);
                l[g] += pu;
#pragma unroll
                for (int e = 0; e < 8; ++e) a[g][e] += pu * vf[u][e];
            }
            m[g] = mx;
        }
        j0 += kU * PG;
        if (j0 < je) load_rows(j0);
    }
    if (c == 0)
#pragma unroll
        for (int g = 0; g < G; ++g) {
            sm[pg][g] = m[g];
            sl[pg][g] = l[g];
        }
#pragma unroll
    for (int g = 0; g < G; ++g)
#pragma unroll
        for (int e = 0; e < 8; ++e) sacc[pg][g][8 * c + e] = a[g][e];
    __syncthreads();
    for (int t = tid; t < G * HD; t += 256) {
        const int g = t / HD, d = t - g * HD;
        float M = -INFINITY;
#pragma unroll
        for (int i = 0; i < PG; ++i) M = fmaxf(M, sm[i][g]);
        float num = 0.f, den = 0.f;
        if (M != -INFINITY) {                  // a lane group without positions weighs e^-inf = 0
#pragma unroll
            for (int i = 0; i < PG; ++i) {
                const float wi = __expf(sm[i][g] - M);
                num += wi * sacc[i][g][d];
                den += wi * sl[i][g];
            }
        }
        float* ph = part + ((int64_t)(kv * G + g) * kAttnChunks + chunk) * (HD + 2);
        ph[2 + d] = num;
        if (d == 0) {
            ph[0] = M;
            ph[1] = den;
        }
    }
}

template <int HD>
__global__ __launch_bounds__(HD) void k_attn_combine(const float* __restrict__ part,
                                                     uint16_t* __restrict__ out) {
    const int h = blockIdx.x, d = threadIdx.x;
    const float* ph = part + (int64_t)h * kAttnChunks * (HD + 2);
    float mc[kAttnChunks], lc[kAttnChunks], ac[kAttnChunks];
#pragma unroll
    for (int c = 0; c < kAttnChunks; ++c) {      // every load of the head issued at once
        mc[c] = ph[c * (HD + 2)];
        lc[c] = ph[c * (HD + 2) + 1];
        ac[c] = ph[c * (HD + 2) + 2 + d];
    }
    float M = mc[0];                             // chunk 0 always holds position 0
#pragma unroll
    for (int c = 1; c < kAttnChunks; ++c) M = fmaxf(M, mc[c]);
    float num = 0.f, den = 0.f;
#pragma unroll
    for (int c = 0; c < kAttnChunks; ++c) {
        const float wc = __expf(mc[c] - M);      // empty chunk: e^-inf = 0, l = acc = 0
        num += wc * ac[c];
        den += wc * lc[c];
    }
    out[h * HD + d] = f2h(num / den);
}

// out = fp16(silu(g) * u), g and u f32
__global__ __launch_bounds__(256) void k_silu_mul(const float* __restrict__ g, const float* __restrict__ u,
                                                  uint16_t* __restrict__ out, int64_t n) {
    const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
    if (i >= n) return;
    const float x = g[i];
    out[i] = f2h(sx8_silu_mul(x, u[i]));
}

// tok = argmax(logits) (first index among equal maxima; NaN entries are skipped), *pos += 1.
// One 1024-thread block; 16-byte loads, eight per thread in flight (the scan is bound by
// the latency of one CU's loads, 4 B x n).
__device__ __forceinline__ void arg_better(float x, int64_t i, float& v, int64_t& idx) {
    if (x > v || (x == v && i < idx)) {
        v = x;
        idx = i;
    }
}

__global__ __launch_bounds__(1024) void k_argmax_advance(const float* __restrict__ logits, int64_t n,
                                                         int64_t* __restrict__ tok,
                                                         int64_t* __restrict__ pos) {
    __shared__ float bv[16];
    __shared__ int64_t bi[16];
    float v = -INFINITY;
    int64_t idx = INT64_MAX;
    constexpr int kU = 8;
    const int64_t n4 = (reinterpret_cast<uintptr_t>(logits) & 15) == 0 ? n / 4 : 0;
    const float4* l4 = reinterpret_cast<const float4*>(logits);
    for (int64_t b = threadIdx.x; b < n4; b += 1024 * kU) {
        float4 x[kU];
#pragma unroll
        for (int u = 0; u < kU; ++u) {
            const int64_t i4 = b + 1024 * u;
            x[u] = l4[i4 < n4 ? i4 : n4 - 1];
        }
#pragma unroll
        for (int u = 0; u < kU; ++u) {
            const int64_t i4 = b + 1024 * u;
            if (i4 < n4) {
                arg_better(x[u].x, 4 * i4, v, idx);
                arg_better(x[u].y, 4 * i4 + 1, v, idx);
                arg_better(x[u].z, 4 * i4 + 2, v, idx);
                arg_better(x[u].w, 4 * i4 + 3, v, idx);
            }
        }
    }
    for (int64_t i = 4 * n4 + threadIdx.x; i < n; i += 1024) arg_better(logits[i], i, v, idx);
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) {
        const float ov = __shfl_xor(v, o, 64);
        const int64_t oi = __shfl_xor(idx, o, 64);
        arg_better(ov, oi, v, idx);
    }
    if ((threadIdx.x & 63) == 0) { bv[threadIdx.x >> 6] = v; bi[threadIdx.x >> 6] = idx; }
    __syncthreads();
    if (threadIdx.x == 0) {
        for (int w = 1; w < 16; ++w) arg_better(bv[w], bi[w], v, idx);
        tok[0] = idx;
        pos[0] += 1;
    }
}

}  // namespace

// Causal attention of T prompt rows over the cache (prefill), on MFMA
// (v_mfma_f32_32x32x16_f16, fp32 accumulation).  Work-group = (32-row query tile, KV
// head), two sets of G waves (one for G = 8): wave g of set s takes query head kvh * G + g
// and the key blocks s, s + 2, s + 4, ... (two waves per SIMD, each with half of the
// tile's serial chain; the sets merge their softmax states at the end).  The G heads of a set share
// the staged K and V of its block.  A work-group may instead take GW of the G heads (G / GW
// work-groups per KV head and tile) in NS sets of GW waves, set s taking blocks s, s + NS,
// ... (the host uses GW = 2, NS = 4 when G = 4 and the plain grid is short of the CUs).  Per 32-key block a wave computes S^T = K Q^T: keys
// are the MFMA rows and the tile's 32 queries the columns, so lane l = 32 h + c owns query
// c (keys 8 g + 4 h + r of the block in accumulator 4 g + r) and the online softmax is
// lane-local (one exchange with lane l ^ 32 for the other 16 keys).  Then O^T += V^T P^T:
// the P^T operand of k-step st is the lane's own accumulators 8 st .. 8 st + 7 converted
// to fp16 (the k index order is free as long as both operands use it: slot t of half h is
// key 16 st + 8 (t / 4) + 4 h + t % 4), and V^T comes from LDS, where the staging writes
// each block transposed with that key order (key bits 2 and 3 swapped; two keys per
// 4-byte write), so a lane's 8 values are one 16-byte read.  K goes through LDS as well
// (one coalesced global read per set instead of one per wave).  Row i (position start +
// i) attends keys 0 .. start + i; keys >= start + T are never read.  Output (T, nh * HD)
// fp16.
constexpr int kApVRow = 40;      // halves per LDS row of V^T: 32 keys + 8 pad (conflict-free reads)
constexpr int kApKRow = 136;     // halves per LDS row of K: up to 128 + 8 pad (conflict-free reads)

__device__ __forceinline__ float lane_swap32(float v) { return sx8_lane_swap32(v); }

// Wave sets per work-group: two while 2 G waves (two per SIMD) keep their registers.
template <int G>
constexpr int ap_sets() { return G <= 4 ? 2 : 1; }

// Where the packed form of k_attn_prefill puts its output: the o projection's prefill-GEMM
// operands (the packed X and Zhl of sx8_gemm_prefill_packed) for that projection's PCA
// basis rows and scales; n_cb = nh * HD / 32.
struct ApPack {
    const float* basis;
    const float* scales;
    uint16_t* Xp;
    uint32_t* Zhl;
    int n_cb;
};

template <int HD, int GW, int NS>
struct ApLds {
    static constexpr int kK = 32 * kApKRow * 2;                 // bytes of one staged K block
    static constexpr int kV = HD * kApVRow * 2;                 // bytes of one staged V^T block
    static constexpr int kStage = 2 * NS * (kK + kV);           // [buffer][set]
    // merge: every set's (m, lsum) and the O^T fragments it does not own (NT - NT / NS of them)
    static constexpr int kMerge = NS > 1 ? NS * GW * 64 * (2 + 16 * (HD / 32 - HD / 32 / NS)) * 4 : 0;
    static constexpr int kBytes = kStage > kMerge ? kStage : kMerge;
};

// GW of the G query heads of a KV head per work-group (G / GW work-groups per KV head and
// query tile), NS sets of GW waves: set s takes key blocks s, s + NS, s + 2 NS, ...
// kPack: the output goes out as the o projection's packed GEMM operands (ApPack) instead.
template <int HD, int G, int GW, int NS, bool kPack = false>
__global__ __launch_bounds__(64 * GW * NS) void k_attn_prefill(const uint16_t* __restrict__ q,
                                                          const uint16_t* __restrict__ k_cache,
                                                          const uint16_t* __restrict__ v_cache,
                                                          uint16_t* __restrict__ out, int T, int start,
                                                          int nh, int L, float scale_log2, const ApPack pk) {
    typedef float f32x16 __attribute__((ext_vector_type(16)));
    typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
    using Lds = ApLds<HD, GW, NS>;
    static_assert(G % GW == 0 && NS >= 1 && NS <= 4, "k_attn_prefill: head split / sets");
    constexpr int KS = HD / 16;                 // k-steps of S^T over the head dimension
    constexpr int NT = HD / 32;                 // 32-row tiles of O^T
    constexpr int CPR = HD / 8;                 // 16-byte chunks per key row
    constexpr int ST = 64 * GW;                 // threads per set
    constexpr int KCH = 32 * CPR / ST;          // K chunks staged per thread and block
    static_assert(KCH >= 1 && KCH * ST == 32 * CPR, "K staging split");
    constexpr int VPT = (16 * CPR + ST - 1) / ST;   // V key-pair tasks per thread
    __shared__ __align__(16) unsigned char lds[Lds::kBytes];
    // (the wave index read as uniform, so that the set's block choices are scalar: a per-lane
    // condition on a load's offset would split the load into two under complementary masks)
    const int tid = threadIdx.x, lane = tid & 63, w = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int set = w / GW, g = w % GW, ts = tid % ST;
    const int c = lane & 31, h = lane >> 5;
    constexpr int R = G / GW;
    const int kvh = blockIdx.y / R, head = kvh * G + (blockIdx.y % R) * GW + g;
    const int q0 = blockIdx.x * 32, qi = q0 + c;
    const int ktot = start + T;                                 // keys in the cache
    const int nblk = (start + min(q0 + 32, T) + 31) / 32;       // key blocks this tile needs
    const int nstep = (nblk + NS - 1) / NS;
    auto kt = [&](int buf) { return reinterpret_cast<uint16_t*>(lds + (buf * NS + set) * Lds::kK); };
    auto vt = [&](int buf) {
        return reinterpret_cast<uint16_t*>(lds + 2 * NS * Lds::kK + (buf * NS + set) * Lds::kV);
    };
    const sx8_u32x4 zero4 = {0u, 0u, 0u, 0u};
    // The query and basis are read through pinned_global: a load from a read-only argument
    // is otherwise free to sink past the barriers to its first use, which would put it
    // behind the first staging instead of in flight during it.  Their loads are issued
    // unconditionally from clamped (valid) addresses and the values selected afterwards (a
    // load under a condition becomes a branch, after which the compiler can only wait for
    // every outstanding load).
    // The query tile of the work-group's GW heads: every set needs all of it, so with NS > 1
    // set s loads chunks s QC .. s QC + QC - 1 of its wave's head (QC = KS / NS) and the sets
    // exchange them through the free second staging buffer (kQLds, where they fit), instead
    // of every wave loading its head's whole tile from memory.
    const uint16_t SX8_DEC_GLOBAL* qg = pinned_global(q);
    constexpr bool kQLds = NS > 1 && KS % NS == 0 && GW * KS * 1024 <= NS * Lds::kK;
    constexpr int QC = kQLds ? KS / NS : KS;      // query chunks this wave loads
    sx8_u32x4 qb[KS], qpart[QC];
    {
        const uint16_t SX8_DEC_GLOBAL* qr = qg + ((int64_t)min(qi, T - 1) * nh + head) * HD + 8 * h;
        const int st0 = kQLds ? set * QC : 0;
#pragma unroll
        for (int i = 0; i < QC; ++i) qpart[i] = ld_u32x4(qr + 16 * (st0 + i));
    }
    // [g][st][lane] 16-byte chunks at the start of the second buffer's K blocks
    sx8_u32x4* const qlds = reinterpret_cast<sx8_u32x4*>(lds + NS * Lds::kK);
    // kPack: the basis rows and scales of the work-group's GW heads' K blocks (one float4
    // per thread), staged in LDS with the first key block
    constexpr int kPkF4 = kPack ? GW * NT * 16 : 1;
    static_assert(!kPack || kPkF4 <= 64 * GW * NS, "one basis float4 per thread");
    __shared__ float4 apb[kPkF4];
    __shared__ float2 aps[kPack ? GW * NT : 1];
    const int kbw = (head - g) * NT;                            // first K block of the work-group
    float4 bpre = make_float4(0.f, 0.f, 0.f, 0.f);
    float2 spre = make_float2(0.f, 0.f);
    if constexpr (kPack) {
        const float SX8_DEC_GLOBAL* bg = pinned_global(pk.basis) + (int64_t)kbw * 64;
        const float SX8_DEC_GLOBAL* sg = pinned_global(pk.scales) + (int64_t)kbw * 2;
        bpre = reinterpret_cast<const float4 SX8_DEC_GLOBAL*>(bg)[min(tid, kPkF4 - 1)];
        spre = reinterpret_cast<const float2 SX8_DEC_GLOBAL*>(sg)[min(tid, GW * NT - 1)];
    }
    // the keys the tile reads: the KV head's cached keys below min(ktot, 32 nblk), HD halves each
    // (the host keeps a head's cache, plus the blocks read past it, below 2 GiB)
    const int64_t kbytes = (int64_t)min(ktot, 32 * nblk) * HD * 2;
    const sx8_rsrc krs = make_rsrc(k_cache + (int64_t)kvh * L * HD, kbytes);
    const sx8_rsrc vrs = make_rsrc(v_cache + (int64_t)kvh * L * HD, kbytes);
    // Step j: set s computes block NS j + s from LDS buffer j & 1 and stages its block of
    // step j + 1 into the other buffer; its global loads run kPf steps ahead of the
    // staging (a ring of kPf register sets, the loop unrolled by kPf).  One barrier per
    // step.
    constexpr int kPf = 2;
    sx8_u32x4 kreg[kPf][KCH], vreg[kPf][2 * VPT];
    // Block kb through raw buffer loads over the keys the tile reads (krs / vrs): a block past
    // the tile's last (kb >= nblk) and keys past the cache lie past the buffer and load zeros
    // without touching memory.  Every load is issued unconditionally, with no condition on its
    // offset either (the compiler would split such a load in two behind a branch), so the wait
    // counts stay static and the set's next blocks stay in flight while it stages.
    auto load_blk = [&](sx8_u32x4 (&kr)[KCH], sx8_u32x4 (&vr)[2 * VPT], int kb) {
#pragma unroll
        for (int i = 0; i < KCH; ++i) {          // K: coalesced 16-byte chunks of whole rows
            const int ch = ts + i * ST;
            const int off = (kb * 32 + ch / CPR) * (HD * 2) + 16 * (ch % CPR);
            kr[i] = __builtin_bit_cast(sx8_u32x4, __builtin_amdgcn_raw_buffer_load_b128(krs, off, 0, 0));
        }
#pragma unroll
        for (int i = 0; i < VPT; ++i) {          // V: keys 2 kp, 2 kp + 1 at columns d0 .. d0 + 7
            const int tc = min(ts + i * ST, 16 * CPR - 1);   // (past the V tasks: loaded, not staged)
            const int kp = tc & 15, d0 = 8 * (tc >> 4);
            const int off = (kb * 32 + 2 * kp) * (HD * 2) + 2 * d0;
            vr[2 * i] = __builtin_bit_cast(sx8_u32x4, __builtin_amdgcn_raw_buffer_load_b128(vrs, off, 0, 0));
            vr[2 * i + 1] = __builtin_bit_cast(sx8_u32x4, __builtin_amdgcn_raw_buffer_load_b128(vrs, off + HD * 2, 0, 0));
        }
    };
    auto stage = [&](int buf, const sx8_u32x4 (&kr)[KCH], const sx8_u32x4 (&vr)[2 * VPT]) {
        uint16_t* kd = kt(buf);
        uint16_t* vd = vt(buf);
#pragma unroll
        for (int i = 0; i < KCH; ++i) {
            const int ch = ts + i * ST;
            *reinterpret_cast<sx8_u32x4*>(kd + (ch / CPR) * kApKRow + 8 * (ch % CPR)) = kr[i];
        }
#pragma unroll
        for (int i = 0; i < VPT; ++i) {
            const int t = ts + i * ST;
            if (t < 16 * CPR) {
                const int kp = t & 15, d0 = 8 * (t >> 4);
                const int kl = 2 * kp;
                const int col = (kl & ~12) | ((kl & 4) << 1) | ((kl & 8) >> 1);   // even; col + 1 is key kl + 1
                const uint32_t a[4] = {vr[2 * i].x, vr[2 * i].y, vr[2 * i].z, vr[2 * i].w};
                const uint32_t bb[4] = {vr[2 * i + 1].x, vr[2 * i + 1].y, vr[2 * i + 1].z, vr[2 * i + 1].w};
                // dim d0 + e of both keys: half e & 1 of word e / 2 of each, one v_perm_b32
                // (bytes 0-3 select from a, 4-7 from bb)
#pragma unroll
                for (int e = 0; e < 8; ++e)
                    *reinterpret_cast<uint32_t*>(vd + (d0 + e) * kApVRow + col) =
                        __builtin_amdgcn_perm(bb[e >> 1], a[e >> 1], (e & 1) ? 0x07060302u : 0x05040100u);
            }
        }
    };
    f32x16 o[NT];
#pragma unroll
    for (int n = 0; n < NT; ++n)
#pragma unroll
        for (int r = 0; r < 16; ++r) o[n][r] = 0.f;
    // running max m (log2 units) and sum; m is raised only when a block's max exceeds it by
    // more than kLazy (the wave then rescales together), so probabilities stay <= 2^kLazy
    constexpr float kLazy = 8.f;
    float m = -__builtin_inff(), lsum = 0.f;
    const int qpos = start + qi;
    auto body = [&](int j, sx8_u32x4 (&kr)[KCH], sx8_u32x4 (&vr)[2 * VPT]) {
        const int b = j & 1, kb = NS * j + set;
        if (kb + NS < nblk) stage(b ^ 1, kr, vr);
        load_blk(kr, vr, kb + NS * (1 + kPf));
        if (kb < nblk) {
            const uint16_t* kd = kt(b);
            const uint16_t* vd = vt(b);
            f32x16 sacc;
#pragma unroll
            for (int r = 0; r < 16; ++r) sacc[r] = 0.f;
#pragma unroll
            for (int st = 0; st < KS; ++st) {
                const sx8_u32x4 a = *reinterpret_cast<const sx8_u32x4*>(kd + c * kApKRow + 16 * st + 8 * h);
                sacc = __builtin_amdgcn_mfma_f32_32x32x16_f16(__builtin_bit_cast(f16x8, a),
                                                              __builtin_bit_cast(f16x8, qb[st]), sacc, 0, 0, 0);
            }
            // raw scores; the scale (> 0) is applied after the max, inside the exponent's fma.
            // Masking only where the block reaches past the tile's first query or the keys.
            if (kb * 32 + 31 > start + q0 || kb * 32 + 31 >= ktot) {
#pragma unroll
                for (int r = 0; r < 16; ++r) {
                    const int key = kb * 32 + 8 * (r >> 2) + 4 * h + (r & 3);
                    sacc[r] = key <= qpos && key < ktot ? sacc[r] : -__builtin_inff();
                }
            }
            float mx = sacc[0];
#pragma unroll
            for (int r = 1; r < 16; ++r) mx = fmaxf(mx, sacc[r]);
            mx = fmaxf(mx, lane_swap32(mx)) * scale_log2;
            // set 1 may meet a fully masked block first: it then keeps m = -inf (mx is -inf)
            if (__builtin_amdgcn_ballot_w64(mx > m + kLazy) != 0) {
                const float mn = fmaxf(m, mx);
                const float alpha = mn == -__builtin_inff() ? 1.f : __builtin_amdgcn_exp2f(m - mn);
                lsum *= alpha;
#pragma unroll
                for (int n = 0; n < NT; ++n)
#pragma unroll
                    for (int r = 0; r < 16; ++r) o[n][r] *= alpha;
                m = mn;
            }
            float ps = 0.f;
            const float nm = m == -__builtin_inff() ? 0.f : -m;   // m = -inf: every score is -inf
#pragma unroll
            for (int r = 0; r < 16; ++r) {
                const float pv = __builtin_amdgcn_exp2f(__builtin_fmaf(sacc[r], scale_log2, nm));
                sacc[r] = pv;
                ps += pv;
            }
            lsum += ps + lane_swap32(ps);
#pragma unroll
            for (int st = 0; st < 2; ++st) {
                f16x8 pb;
#pragma unroll
                for (int t = 0; t < 8; ++t) pb[t] = (_Float16)sacc[8 * st + t];
#pragma unroll
                for (int n = 0; n < NT; ++n) {
                    const sx8_u32x4 a = *reinterpret_cast<const sx8_u32x4*>(vd + (32 * n + c) * kApVRow + 16 * st + 8 * h);
                    o[n] = __builtin_amdgcn_mfma_f32_32x32x16_f16(__builtin_bit_cast(f16x8, a), pb, o[n], 0, 0, 0);
                }
            }
        }
        __syncthreads();      // step j + 1 staged; step j's buffers free for step j + 2
    };
    // ring slot i holds the set's blocks of steps i + 1, i + 1 + kPf, ...; step 0 is staged first
    // Only the query, block 0 and the first ring slot are requested before the first barrier:
    // the work-group's loads share one address path, and the barrier waits for the slowest
    // wave's block 0; the other slots are requested behind it.
    {
        sx8_u32x4 k0[KCH], v0[2 * VPT];
        load_blk(k0, v0, set);
        load_blk(kreg[0], vreg[0], NS + set);
        stage(0, k0, v0);                        // (a set past the tile's blocks: zeros, unused)
#pragma unroll
        for (int i = 0; i < QC; ++i) {
            const sx8_u32x4 v = qi < T ? qpart[i] : zero4;
            if constexpr (kQLds) qlds[(g * KS + set * QC + i) * 64 + lane] = v;
            else qb[i] = v;
        }
        if constexpr (kPack) {      // (threads past the end store the last entry's value again)
            apb[min(tid, kPkF4 - 1)] = bpre;
            aps[min(tid, GW * NT - 1)] = spre;
        }
        __syncthreads();
#pragma unroll
        for (int i = 1; i < kPf; ++i) load_blk(kreg[i], vreg[i], NS * (i + 1) + set);
        if constexpr (kQLds) {
#pragma unroll
            for (int st = 0; st < KS; ++st) qb[st] = qlds[(g * KS + st) * 64 + lane];
            __syncthreads();                     // the second buffer is free again for step 0
        }
    }
    // (whole rounds of kPf steps: a step past nstep only loads and passes its barrier, and
    // no step is skipped behind a branch that would end the loads' static wait counts)
    for (int j = 0; j < nstep; j += kPf) {
#pragma unroll
        for (int i = 0; i < kPf; ++i) body(j + i, kreg[i], vreg[i]);
    }
    // kPack: fragment n of the row (16 values, dims 32 n + 8 gq + 4 h + e) as packed operands;
    // every lane of the wave takes part (the Z tree swaps lane halves), rows past T pack zeros
    auto emit_packed = [&](int n, const float (&v)[16]) {
        const int kb = kbw + g * NT + n;
        sx8_pack_fragment(v, qi < T, c, h, reinterpret_cast<const float*>(apb) + (g * NT + n) * 64, aps[g * NT + n],
                         pk.Xp + ((int64_t)blockIdx.x * pk.n_cb + kb) * 1024,
                         pk.Zhl + ((int64_t)qi * pk.n_cb + kb) * 2);
    };
    auto emit = [&](int n, const float (&v)[16]) {
        if constexpr (kPack) {
            emit_packed(n, v);
        } else {
            uint16_t* orow = out + ((int64_t)qi * nh + head) * HD;
#pragma unroll
            for (int gq = 0; gq < 4; ++gq) {
                const uint32_t lo = (uint32_t)f2h(v[4 * gq]) | ((uint32_t)f2h(v[4 * gq + 1]) << 16);
                const uint32_t hi = (uint32_t)f2h(v[4 * gq + 2]) | ((uint32_t)f2h(v[4 * gq + 3]) << 16);
                *reinterpret_cast<uint2*>(orow + 32 * n + 8 * gq + 4 * h) = make_uint2(lo, hi);
            }
        }
    };
    if (NS == 1) {
        if (!kPack && qi >= T) return;
        const float inv = 1.0f / lsum;
#pragma unroll
        for (int n = 0; n < NT; ++n) {
            float v[16];
#pragma unroll
            for (int r = 0; r < 16; ++r) {
                v[r] = o[n][r] * inv;
                asm volatile("" : "+v"(v[r]));    // rounded to float32, then to fp16 (see below)
            }
            emit(n, v);
        }
        return;
    }
    // merge: set s finishes the fragments n = s, s + NS, ... of its wave's head.  Every set
    // hands its (m, lsum) and the O^T fragments it does not own to the others through LDS (the
    // staging buffers are free after the last barrier; lane-contiguous rows), then merges its
    // own fragments over all sets in set order -- the arithmetic one merging set would do --
    // so the epilogue work is spread over the NS sets
    static_assert(NT % NS == 0, "whole fragments per set");
    constexpr int NX = NT - NT / NS;                            // fragments a set hands over
    float* ml = reinterpret_cast<float*>(lds);                  // [set][g][m, lsum][64]
    float* ob = ml + NS * GW * 128;                             // [set][slot < NX][g][16][64]
    auto slot = [](int t, int n) { return n - n / NS - (n % NS > t ? 1 : 0); };   // n % NS != t
    ml[(set * GW + g) * 128 + lane] = m;
    ml[(set * GW + g) * 128 + 64 + lane] = lsum;
#pragma unroll
    for (int n = 0; n < NT; ++n) {
        if (n % NS == set) continue;
        float* dst = ob + ((set * NX + slot(set, n)) * GW + g) * 1024 + lane;
#pragma unroll
        for (int r = 0; r < 16; ++r) dst[r * 64] = o[n][r];
    }
    __syncthreads();
    if (!kPack && qi >= T) return;
    // set t's state weighs 2^(m_t - max m); an empty set (m = -inf) weighs nothing, and m is
    // finite in set 0, which owns block 0
    float ms[NS], ls[NS], f[NS];
#pragma unroll
    for (int t = 0; t < NS; ++t) {
        ms[t] = ml[(t * GW + g) * 128 + lane];
        ls[t] = ml[(t * GW + g) * 128 + 64 + lane];
    }
    float mm = ms[0];
#pragma unroll
    for (int t = 1; t < NS; ++t) mm = fmaxf(mm, ms[t]);
    f[0] = __builtin_amdgcn_exp2f(ms[0] - mm);
#pragma unroll
    for (int t = 1; t < NS; ++t) f[t] = ms[t] == -__builtin_inff() ? 0.f : __builtin_amdgcn_exp2f(ms[t] - mm);
    float den = ls[0] * f[0];
#pragma unroll
    for (int t = 1; t < NS; ++t) den += ls[t] * f[t];
    const float inv = 1.0f / den;
    float wgt[NS];
#pragma unroll
    for (int t = 0; t < NS; ++t) wgt[t] = f[t] * inv;
#pragma unroll
    for (int n = 0; n < NT; ++n) {
        if (n % NS != set) continue;
        float v[16];
#pragma unroll
        for (int r = 0; r < 16; ++r) {
            // set t's value: this wave's own accumulator for t = set, else the LDS copy
            // (slot 0 stands in for t = set, so the address stays inside the handed-over block)
            auto val = [&](int t) {
                const int sl = t == set ? 0 : slot(t, n);
                return t == set ? o[n][r] : ob[((t * NX + sl) * GW + g) * 1024 + r * 64 + lane];
            };
            // explicit fmas, and the float32 result pinned before its fp16 conversion: the
            // compiler would otherwise pick which product to fuse and fold the last one into
            // the conversion (v_fma_mixlo_f16), so the plain and packed outputs could differ
            float acc = val(0) * wgt[0];
#pragma unroll
            for (int t = 1; t < NS; ++t) acc = __builtin_fmaf(val(t), wgt[t], acc);
            asm volatile("" : "+v"(acc));
            v[r] = acc;
        }
        emit(n, v);
    }
}

namespace {

// Checks of the pending split-K sums a *_parts entry point takes: n_parts in 0 ..
// kMaxPendingParts, and with n_parts > 0 a 4-byte aligned parts pointer and a slice that
// covers `need` floats.
constexpr int kMaxPendingParts = 7;

int32_t check_parts(const char* what, const float* parts, int32_t n_parts, int64_t slice, int64_t need) {
    using namespace sx8;
    if (n_parts < 0 || n_parts > kMaxPendingParts)
        return fail(SX8_ERR_INVALID, "%s: n_parts must be 0..%d, got %d", what, kMaxPendingParts, n_parts);
    if (n_parts > 0 && (!parts || !aligned(parts, 4) || slice < need))
        return fail(SX8_ERR_INVALID, "%s: parts must be a 4-byte aligned pointer and slice >= %lld floats",
                    what, (long long)need);
    return SX8_OK;
}

// f(std::integral_constant<int, np>) for np = 0 .. kMaxPendingParts
template <class F>
void by_parts(int np, F&& f) {
    switch (np) {
        case 0: f(std::integral_constant<int, 0>{}); break;
        case 1: f(std::integral_constant<int, 1>{}); break;
        case 2: f(std::integral_constant<int, 2>{}); break;
        case 3: f(std::integral_constant<int, 3>{}); break;
        case 4: f(std::integral_constant<int, 4>{}); break;
        case 5: f(std::integral_constant<int, 5>{}); break;
        case 6: f(std::integral_constant<int, 6>{}); break;
        default: f(std::integral_constant<int, 7>{}); break;
    }
}

int32_t add_rmsnorm_impl(const char* what, float* resid, const float* delta, const uint16_t* init,
                         const uint16_t* w, uint16_t* out, int64_t M, int64_t H, float eps,
                         const float* parts, int32_t n_parts, int64_t slice, void* stream) {
    using namespace sx8;
    if (!resid || !w || !out) return fail(SX8_ERR_INVALID, "%s: null pointer", what);
    if (M <= 0 || H <= 0 || M > 0x7FFFFFFF || H > 0x7FFFFFFF) return fail(SX8_ERR_INVALID, "%s: bad shape", what);
    if (n_parts > 0 && !delta) return fail(SX8_ERR_INVALID, "%s: partial sums need delta", what);
    const int32_t rc = check_parts(what, parts, n_parts, slice, M * H);
    if (rc != SX8_OK) return rc;
    const bool vec = H % 4 == 0 && aligned(resid, 16) && (!delta || aligned(delta, 16)) &&
                     (!init || aligned(init, 8)) && aligned(w, 8) && aligned(out, 8) &&
                     (n_parts == 0 || (aligned(parts, 16) && slice % 4 == 0));
    by_parts(n_parts, [&](auto np) {
        hipLaunchKernelGGL((k_add_rmsnorm<decltype(np)::value>), dim3((unsigned)M), dim3(256), 0,
                           as_stream(stream), resid, delta, init, w, out, (int)H, eps, vec, parts, slice);
    });
    return check_launch(what);
}

}  // namespace

extern "C" int32_t sx8_dec_add_rmsnorm(float* resid, const float* delta, const uint16_t* init,
                                       const uint16_t* w, uint16_t* out, int64_t M, int64_t H,
                                       float eps, void* stream) {
    return add_rmsnorm_impl("sx8_dec_add_rmsnorm", resid, delta, init, w, out, M, H, eps, nullptr, 0, 0,
                            stream);
}

extern "C" int32_t sx8_dec_add_rmsnorm_parts(float* resid, const float* delta, const uint16_t* init,
                                             const uint16_t* w, uint16_t* out, int64_t M, int64_t H,
                                             float eps, const float* parts, int32_t n_parts, int64_t slice,
                                             void* stream) {
    return add_rmsnorm_impl("sx8_dec_add_rmsnorm_parts", resid, delta, init, w, out, M, H, eps, parts, n_parts,
                            slice, stream);
}

extern "C" int32_t sx8_dec_add_rmsnorm_packed(float* resid, const float* delta, const uint16_t* init,
                                              const uint16_t* w, int64_t M, int64_t H, float eps,
                                              const float* parts, int32_t n_parts, int64_t slice, int32_t n_mats,
                                              const float* const* bases, const float* const* scales,
                                              uint16_t* Xp, uint32_t* const* Zhl, void* stream) {
    using namespace sx8;
    const char* what = "sx8_dec_add_rmsnorm_packed";
    if (!resid || !w || !Xp || !bases || !scales || !Zhl) return fail(SX8_ERR_INVALID, "%s: null pointer", what);
    if (M <= 0 || H <= 0 || M > 0x7FFFFFFF - 64 || H % 32 != 0 || H > 256 * 4 * kRmsPer4)
        return fail(SX8_ERR_INVALID, "%s: bad shape (H a multiple of 32, at most %d)", what, 256 * 4 * kRmsPer4);
    if (n_mats < 1 || n_mats > 4) return fail(SX8_ERR_INVALID, "%s: n_mats must be 1..4, got %d", what, n_mats);
    if (n_parts > 0 && !delta) return fail(SX8_ERR_INVALID, "%s: partial sums need delta", what);
    int32_t rc = check_parts(what, parts, n_parts, slice, M * H);
    if (rc != SX8_OK) return rc;
    if (!aligned(resid, 16) || (delta && !aligned(delta, 16)) || (init && !aligned(init, 8)) || !aligned(w, 8) ||
        !aligned(Xp, 16) || (n_parts > 0 && (!aligned(parts, 16) || slice % 4 != 0)))
        return fail(SX8_ERR_INVALID, "%s: resid, delta, parts and Xp must be 16-byte aligned, init and w 8-byte "
                    "(slice a multiple of 4)", what);
    const int64_t n_cb = H / 32, Mp = (M + 31) / 32 * 32;
    if (Mp / 32 * n_cb * 2048 > 0x7FFFFFFF || M * n_cb * 8 > 0x7FFFFFFF)
        return fail(SX8_ERR_UNSUPPORTED, "%s: operands beyond 2 GiB", what);
    NormPack pk{};
    for (int i = 0; i < n_mats; ++i) {
        if (!bases[i] || !scales[i] || !Zhl[i]) return fail(SX8_ERR_INVALID, "%s: null pointer in matrix %d", what, i);
        if (!aligned(bases[i], 16) || !aligned(scales[i], 8) || !aligned(Zhl[i], 8))
            return fail(SX8_ERR_INVALID, "%s: misaligned basis, scales or Zhl of matrix %d", what, i);
        pk.basis[i] = bases[i];
        pk.scales[i] = scales[i];
        pk.Zhl[i] = Zhl[i];
    }
    pk.Xp = Xp;
    pk.n_cb = (int)n_cb;
    const dim3 grid((unsigned)(Mp / kPackRows));
    hipStream_t st = as_stream(stream);
    by_parts(n_parts, [&](auto np) {
        constexpr int NP = decltype(np)::value;
        switch (n_mats) {
            case 1: hipLaunchKernelGGL((k_add_rmsnorm_pack<NP, 1>), grid, dim3(256 * kPackRows), 0, st, resid, delta,
                                       init, w, (int)M, (int)H, eps, parts, slice, pk); break;
            case 2: hipLaunchKernelGGL((k_add_rmsnorm_pack<NP, 2>), grid, dim3(256 * kPackRows), 0, st, resid, delta,
                                       init, w, (int)M, (int)H, eps, parts, slice, pk); break;
            case 3: hipLaunchKernelGGL((k_add_rmsnorm_pack<NP, 3>), grid, dim3(256 * kPackRows), 0, st, resid, delta,
                                       init, w, (int)M, (int)H, eps, parts, slice, pk); break;
            default: hipLaunchKernelGGL((k_add_rmsnorm_pack<NP, 4>), grid, dim3(256 * kPackRows), 0, st, resid, delta,
                                        init, w, (int)M, (int)H, eps, parts, slice, pk); break;
        }
    });
    return check_launch(what);
}

namespace {

// k_qk_rope128 applies (head dim 128, its 16- and 8-byte accesses aligned); it gives
// k_qk_rope_cache's results bit for bit, so the choice does not change them.
bool rope128_ok(const float* q_raw, const float* k_raw, const float* v_raw, const uint16_t* q_norm,
                const uint16_t* k_norm, const float* cos_t, const float* sin_t, const uint16_t* q_out,
                const uint16_t* k_cache, const uint16_t* v_cache, const float* parts, int64_t slice, int32_t hd) {
    using namespace sx8;
    return hd == 128 && aligned(q_raw, 16) && aligned(k_raw, 16) && aligned(v_raw, 16) && aligned(cos_t, 16) &&
           aligned(sin_t, 16) && aligned(q_norm, 8) && aligned(k_norm, 8) && aligned(q_out, 8) &&
           aligned(k_cache, 16) && aligned(v_cache, 16) && (!parts || (aligned(parts, 16) && slice % 4 == 0));
}

}  // namespace

extern "C" int32_t sx8_dec_qk_rope_cache(const float* q_raw, const float* k_raw, const float* v_raw,
                                         const uint16_t* q_norm, const uint16_t* k_norm,
                                         const float* cos_t, const float* sin_t, const int64_t* pos,
                                         uint16_t* q_out, uint16_t* k_cache, uint16_t* v_cache,
                                         int32_t nh, int32_t nk, int32_t hd, int64_t L, float eps,
                                         void* stream) {
    using namespace sx8;
    if (!q_raw || !k_raw || !v_raw || !q_norm || !k_norm || !cos_t || !sin_t || !pos || !q_out ||
        !k_cache || !v_cache)
        return fail(SX8_ERR_INVALID, "sx8_dec_qk_rope_cache: null pointer");
    if (nh <= 0 || nk <= 0 || nh % nk || hd <= 0 || (hd & 1) || hd > 256 || L <= 0 || L > 0x7FFFFFFF)
        return fail(SX8_ERR_INVALID, "sx8_dec_qk_rope_cache: bad shape (hd even, <= 256)");
    if (rope128_ok(q_raw, k_raw, v_raw, q_norm, k_norm, cos_t, sin_t, q_out, k_cache, v_cache, nullptr, 0, hd)) {
        hipLaunchKernelGGL(k_qk_rope128<0>, dim3(((unsigned)(nh + 2 * nk) + 15) / 16), dim3(256), 0, as_stream(stream),
                           q_raw, k_raw, v_raw, q_norm, k_norm, cos_t, sin_t, pos, q_out, k_cache, v_cache, nh, nk,
                           hd, (int)L, eps, 1, nullptr, nullptr, nullptr, (int64_t)0);
        return check_launch("sx8_dec_qk_rope_cache");
    }
    const unsigned hpb = hd > 128 ? 2u : 4u;     // heads per 256-thread block
    hipLaunchKernelGGL(k_qk_rope_cache<0>, dim3(((unsigned)(nh + 2 * nk) + hpb - 1) / hpb), dim3(256), 0,
                       as_stream(stream), q_raw, k_raw, v_raw, q_norm, k_norm, cos_t, sin_t, pos,
                       q_out, k_cache, v_cache, nh, nk, hd, (int)L, eps, 1);
    return check_launch("sx8_dec_qk_rope_cache");
}

namespace {

int32_t rope_rows_impl(const char* what, const float* q_raw, const float* k_raw, const float* v_raw,
                       const uint16_t* q_norm, const uint16_t* k_norm, const float* cos_t, const float* sin_t,
                       const int64_t* pos, int64_t rows, uint16_t* q_out, uint16_t* k_cache, uint16_t* v_cache,
                       int32_t nh, int32_t nk, int32_t hd, int64_t L, float eps, const float* parts,
                       int32_t n_parts, int64_t slice, void* stream) {
    using namespace sx8;
    if (!q_raw || !k_raw || !v_raw || !q_norm || !k_norm || !cos_t || !sin_t || !pos || !q_out ||
        !k_cache || !v_cache)
        return fail(SX8_ERR_INVALID, "%s: null pointer", what);
    if (nh <= 0 || nk <= 0 || nh % nk || hd <= 0 || (hd & 1) || hd > 256 || L <= 0 || L > 0x7FFFFFFF ||
        rows <= 0 || rows > 65535)
        return fail(SX8_ERR_INVALID, "%s: bad shape (hd even, <= 256, rows 1..65535)", what);
    // the q/k/v group's partial slices: q block first, then k, then v (rows x width each)
    const int64_t qn = rows * nh * hd, kvn = rows * nk * hd;
    const int32_t rc = check_parts(what, parts, n_parts, slice, qn + 2 * kvn);
    if (rc != SX8_OK) return rc;
    const float* qp = n_parts ? parts : nullptr;
    const float* kp = n_parts ? parts + qn : nullptr;
    const float* vp = n_parts ? parts + qn + kvn : nullptr;
    if (rope128_ok(q_raw, k_raw, v_raw, q_norm, k_norm, cos_t, sin_t, q_out, k_cache, v_cache, parts, slice, hd) &&
        rows * (nh + 2 * nk) <= 0x7FFFFFFF - 16) {
        const unsigned nb = (unsigned)((rows * (nh + 2 * nk) + 15) / 16);
        by_parts(n_parts, [&](auto np) {
            hipLaunchKernelGGL((k_qk_rope128<decltype(np)::value>), dim3(nb), dim3(256), 0, as_stream(stream), q_raw,
                               k_raw, v_raw, q_norm, k_norm, cos_t, sin_t, pos, q_out, k_cache, v_cache, nh, nk, hd,
                               (int)L, eps, (int)rows, qp, kp, vp, slice);
        });
        return check_launch(what);
    }
    const unsigned hpb = hd > 128 ? 2u : 4u;     // heads per 256-thread block
    const unsigned yb = (unsigned)((rows + kRopeRows - 1) / kRopeRows);
    by_parts(n_parts, [&](auto np) {
        hipLaunchKernelGGL((k_qk_rope_cache<decltype(np)::value>), dim3(((unsigned)(nh + 2 * nk) + hpb - 1) / hpb, yb),
                           dim3(256), 0, as_stream(stream), q_raw, k_raw, v_raw, q_norm, k_norm, cos_t, sin_t,
                           pos, q_out, k_cache, v_cache, nh, nk, hd, (int)L, eps, (int)rows, qp, kp, vp, slice);
    });
    return check_launch(what);
}

}  // namespace

extern "C" int32_t sx8_dec_qk_rope_cache_rows(const float* q_raw, const float* k_raw, const float* v_raw,
                                              const uint16_t* q_norm, const uint16_t* k_norm,
                                              const float* cos_t, const float* sin_t, const int64_t* pos,
                                              int64_t rows, uint16_t* q_out, uint16_t* k_cache,
                                              uint16_t* v_cache, int32_t nh, int32_t nk, int32_t hd,
                                              int64_t L, float eps, void* stream) {
    return rope_rows_impl("sx8_dec_qk_rope_cache_rows", q_raw, k_raw, v_raw, q_norm, k_norm, cos_t, sin_t, pos,
                          rows, q_out, k_cache, v_cache, nh, nk, hd, L, eps, nullptr, 0, 0, stream);
}

extern "C" int32_t sx8_dec_qk_rope_cache_rows_parts(const float* q_raw, const float* k_raw, const float* v_raw,
                                                    const uint16_t* q_norm, const uint16_t* k_norm,
                                                    const float* cos_t, const float* sin_t, const int64_t* pos,
                                                    int64_t rows, uint16_t* q_out, uint16_t* k_cache,
                                                    uint16_t* v_cache, int32_t nh, int32_t nk, int32_t hd,
                                                    int64_t L, float eps, const float* parts, int32_t n_parts,
                                                    int64_t slice, void* stream) {
    return rope_rows_impl("sx8_dec_qk_rope_cache_rows_parts", q_raw, k_raw, v_raw, q_norm, k_norm, cos_t, sin_t,
                          pos, rows, q_out, k_cache, v_cache, nh, nk, hd, L, eps, parts, n_parts, slice, stream);
}

extern "C" int32_t sx8_dec_attn(const uint16_t* q, const uint16_t* k_cache, const uint16_t* v_cache,
                                const int64_t* pos, uint16_t* out, int32_t nh, int32_t nk, int32_t hd,
                                int64_t L, float scale, void* stream) {
    using namespace sx8;
    if (!q || !k_cache || !v_cache || !pos || !out) return fail(SX8_ERR_INVALID, "sx8_dec_attn: null pointer");
    if (nh <= 0 || nk <= 0 || nh % nk || (hd != 64 && hd != 128) || L <= 0 || L > kAttnMaxL)
        return fail(SX8_ERR_INVALID, "sx8_dec_attn: bad shape (hd 64 or 128, cache length <= %d)",
                    kAttnMaxL);
    if (!aligned(q, 16) || !aligned(k_cache, 16) || !aligned(v_cache, 16))
        return fail(SX8_ERR_INVALID, "sx8_dec_attn: q and caches must be 16-byte aligned");
    if (hd == 128)
        hipLaunchKernelGGL(k_attn_decode<128>, dim3((unsigned)nh), dim3(256), 0, as_stream(stream), q,
                           k_cache, v_cache, pos, out, nh, nk, (int)L, scale);
    else
        hipLaunchKernelGGL(k_attn_decode<64>, dim3((unsigned)nh), dim3(256), 0, as_stream(stream), q,
                           k_cache, v_cache, pos, out, nh, nk, (int)L, scale);
    return check_launch("sx8_dec_attn");
}

namespace {

// The prompt attention's kernel choice (shape checked by the caller).
template <bool kPack>
void launch_attn_prefill(const uint16_t* q, const uint16_t* k_cache, const uint16_t* v_cache, uint16_t* out,
                         int64_t T, int64_t start, int32_t nh, int32_t nk, int32_t hd, int64_t L, float scale,
                         const ApPack& pk, hipStream_t st) {
    const int G = nh / nk;
    const float sl2 = scale * 1.4426950408889634f;
    const dim3 grid((unsigned)((T + 31) / 32), (unsigned)nk);
#define SX8_AP(HD_, G_)                                                                                      \
    hipLaunchKernelGGL((k_attn_prefill<HD_, G_, G_, ap_sets<G_>(), kPack>), grid, dim3(64 * G_ * ap_sets<G_>()), \
                       0, st, q, k_cache, v_cache, out, (int)T, (int)start, nh, (int)L, sl2, pk)
    if (hd == 128) {
        if (G == 4 && (int64_t)grid.x * grid.y < 256) {
            // a grid short of one work-group per CU: two work-groups per KV head and tile (two
            // heads each) with four sets of two waves, so the longest (last) tiles' chain of key
            // blocks is half as long (T = 512: 18.3 -> 16.6 us).  Past that the heads share
            // the staging of four per work-group (T = 2048: 90 us against 117 for this form).
            hipLaunchKernelGGL((k_attn_prefill<128, 4, 2, 4, kPack>), dim3(grid.x, 2 * grid.y), dim3(512), 0, st, q,
                               k_cache, v_cache, out, (int)T, (int)start, nh, (int)L, sl2, pk);
        } else if (G == 4) SX8_AP(128, 4); else if (G == 1) SX8_AP(128, 1); else if (G == 2) SX8_AP(128, 2); else SX8_AP(128, 8);
    } else {
        if (G == 1) SX8_AP(64, 1); else if (G == 2) SX8_AP(64, 2); else SX8_AP(64, 4);
    }
#undef SX8_AP
}

int32_t check_attn_prefill(const char* what, const uint16_t* q, const uint16_t* k_cache, const uint16_t* v_cache,
                           int64_t T, int64_t start, int32_t nh, int32_t nk, int32_t hd, int64_t L) {
    using namespace sx8;
    if (!q || !k_cache || !v_cache) return fail(SX8_ERR_INVALID, "%s: null pointer", what);
    const int G = nk > 0 ? nh / nk : 0;
    if (nh <= 0 || nk <= 0 || nh % nk || (G != 1 && G != 2 && G != 4 && G != 8) || (hd != 64 && hd != 128) ||
        16 * G > hd || T <= 0 || start < 0 || L <= 0 || start + T > L || L * (int64_t)hd * 2 > 0x7FF00000 ||
        (T + 31) / 32 > 0x7FFFFFFF)
        return fail(SX8_ERR_INVALID, "%s: bad shape (nh / nk in {1, 2, 4, 8} with 16 nh / nk "
                    "<= hd, hd 64 or 128, 0 <= start, start + T <= L, a head's cache below 2 GiB)", what);
    if (!aligned(q, 16) || !aligned(k_cache, 16) || !aligned(v_cache, 16))
        return fail(SX8_ERR_INVALID, "%s: q and caches must be 16-byte aligned", what);
    return SX8_OK;
}

}  // namespace

extern "C" int32_t sx8_dec_attn_prefill(const uint16_t* q, const uint16_t* k_cache, const uint16_t* v_cache,
                                        uint16_t* out, int64_t T, int64_t start, int32_t nh, int32_t nk,
                                        int32_t hd, int64_t L, float scale, void* stream) {
    using namespace sx8;
    const char* what = "sx8_dec_attn_prefill";
    const int32_t rc = check_attn_prefill(what, q, k_cache, v_cache, T, start, nh, nk, hd, L);
    if (rc != SX8_OK) return rc;
    if (!out) return fail(SX8_ERR_INVALID, "%s: null pointer", what);
    if (!aligned(out, 8)) return fail(SX8_ERR_INVALID, "%s: out must be 8-byte aligned", what);
    launch_attn_prefill<false>(q, k_cache, v_cache, out, T, start, nh, nk, hd, L, scale, ApPack{},
                               as_stream(stream));
    return check_launch(what);
}

extern "C" int32_t sx8_dec_attn_prefill_packed(const uint16_t* q, const uint16_t* k_cache,
                                               const uint16_t* v_cache, int64_t T, int64_t start, int32_t nh,
                                               int32_t nk, int32_t hd, int64_t L, float scale,
                                               const float* basis, const float* scales, uint16_t* Xp,
                                               uint32_t* Zhl, void* stream) {
    using namespace sx8;
    const char* what = "sx8_dec_attn_prefill_packed";
    const int32_t rc = check_attn_prefill(what, q, k_cache, v_cache, T, start, nh, nk, hd, L);
    if (rc != SX8_OK) return rc;
    if (!basis || !scales || !Xp || !Zhl) return fail(SX8_ERR_INVALID, "%s: null pointer", what);
    if (!aligned(basis, 16) || !aligned(scales, 8) || !aligned(Xp, 16) || !aligned(Zhl, 16))
        return fail(SX8_ERR_INVALID, "%s: basis, Xp and Zhl must be 16-byte aligned, scales 8-byte", what);
    const int64_t n_cb = (int64_t)nh * hd / 32;
    if ((T + 31) / 32 * n_cb * 2048 > 0x7FFFFFFF || T * n_cb * 8 > 0x7FFFFFFF)
        return fail(SX8_ERR_UNSUPPORTED, "%s: operands beyond 2 GiB", what);
    const ApPack pk{basis, scales, Xp, Zhl, (int)n_cb};
    launch_attn_prefill<true>(q, k_cache, v_cache, nullptr, T, start, nh, nk, hd, L, scale, pk, as_stream(stream));
    return check_launch(what);
}

extern "C" int64_t sx8_dec_attn_workspace_bytes(int32_t nh, int32_t hd) {
    return nh > 0 && hd > 0 ? (int64_t)nh * kAttnChunks * (hd + 2) * (int64_t)sizeof(float) : 0;
}

extern "C" int32_t sx8_dec_attn_split(const uint16_t* q, const uint16_t* k_cache, const uint16_t* v_cache,
                                      const int64_t* pos, uint16_t* out, int32_t nh, int32_t nk,
                                      int32_t hd, int64_t L, float scale, void* workspace,
                                      int64_t workspace_bytes, void* stream) {
    using namespace sx8;
    if (!q || !k_cache || !v_cache || !pos || !out || !workspace)
        return fail(SX8_ERR_INVALID, "sx8_dec_attn_split: null pointer");
    const int G = nk > 0 ? nh / nk : 0;
    if (nh <= 0 || nk <= 0 || nh % nk || (G != 1 && G != 2 && G != 4 && G != 8) ||
        (hd != 64 && hd != 128) || L <= 0 || L > kAttnSplitMaxL)
        return fail(SX8_ERR_INVALID, "sx8_dec_attn_split: bad shape (nh / nk in {1, 2, 4, 8}, hd 64 or "
                                     "128, cache length <= %lld)", (long long)kAttnSplitMaxL);
    if (workspace_bytes < sx8_dec_attn_workspace_bytes(nh, hd) || !aligned(workspace, 16))
        return fail(SX8_ERR_INVALID, "sx8_dec_attn_split: workspace needs %lld bytes, 16-byte aligned",
                    (long long)sx8_dec_attn_workspace_bytes(nh, hd));
    if (!aligned(q, 16) || !aligned(k_cache, 16) || !aligned(v_cache, 16))
        return fail(SX8_ERR_INVALID, "sx8_dec_attn_split: q and caches must be 16-byte aligned");
    float* part = reinterpret_cast<float*>(workspace);
    const hipStream_t st = as_stream(stream);
    const dim3 grid((unsigned)(nk * kAttnChunks));
#define SX8_ATTN(HDV, GV)                                                                           \
    hipLaunchKernelGGL((k_attn_split<HDV, GV>), grid, dim3(256), 0, st, q, k_cache, v_cache, pos,  \
                       part, (int)L, scale)
    if (hd == 128) {
        if (G == 1) SX8_ATTN(128, 1); else if (G == 2) SX8_ATTN(128, 2); else if (G == 4) SX8_ATTN(128, 4); else SX8_ATTN(128, 8);
        hipLaunchKernelGGL(k_attn_combine<128>, dim3((unsigned)nh), dim3(128), 0, st, part, out);
    } else {
        if (G == 1) SX8_ATTN(64, 1); else if (G == 2) SX8_ATTN(64, 2); else if (G == 4) SX8_ATTN(64, 4); else SX8_ATTN(64, 8);
        hipLaunchKernelGGL(k_attn_combine<64>, dim3((unsigned)nh), dim3(64), 0, st, part, out);
    }
#undef SX8_ATTN
    return check_launch("sx8_dec_attn_split");
}

extern "C" int32_t sx8_dec_attn_rope(const float* q_raw, const float* k_raw, const float* v_raw,
                                     const uint16_t* q_norm, const uint16_t* k_norm, const float* cos_t,
                                     const float* sin_t, const int64_t* pos, uint16_t* k_cache,
                                     uint16_t* v_cache, uint16_t* out, int32_t nh, int32_t nk, int32_t hd,
                                     int64_t L, float scale, float eps, void* workspace,
                                     int64_t workspace_bytes, void* stream) {
    using namespace sx8;
    const char* what = "sx8_dec_attn_rope";
    if (!q_raw || !k_raw || !v_raw || !q_norm || !k_norm || !cos_t || !sin_t || !pos || !k_cache ||
        !v_cache || !out || !workspace)
        return fail(SX8_ERR_INVALID, "%s: null pointer", what);
    const int G = nk > 0 ? nh / nk : 0;
    if (nh <= 0 || nk <= 0 || nh % nk || (G != 1 && G != 2 && G != 4 && G != 8) ||
        (hd != 64 && hd != 128) || L <= 0 || L > kAttnSplitMaxL)
        return fail(SX8_ERR_INVALID, "%s: bad shape (nh / nk in {1, 2, 4, 8}, hd 64 or 128, cache length "
                                     "<= %lld)", what, (long long)kAttnSplitMaxL);
    if (workspace_bytes < sx8_dec_attn_workspace_bytes(nh, hd) || !aligned(workspace, 16))
        return fail(SX8_ERR_INVALID, "%s: workspace needs %lld bytes, 16-byte aligned", what,
                    (long long)sx8_dec_attn_workspace_bytes(nh, hd));
    if (!aligned(q_raw, 16) || !aligned(k_raw, 16) || !aligned(v_raw, 16) || !aligned(q_norm, 16) ||
        !aligned(k_norm, 16) || !aligned(k_cache, 16) || !aligned(v_cache, 16))
        return fail(SX8_ERR_INVALID, "%s: projections, norm weights and caches must be 16-byte aligned", what);
    RopeIn ri{q_raw, k_raw, v_raw, q_norm, k_norm, cos_t, sin_t, k_cache, v_cache, eps};
    float* part = reinterpret_cast<float*>(workspace);
    const hipStream_t st = as_stream(stream);
    const dim3 grid((unsigned)(nk * kAttnChunks));
#define SX8_ATTN(HDV, GV)                                                                               \
    hipLaunchKernelGGL((k_attn_split<HDV, GV, true>), grid, dim3(256), 0, st, nullptr, k_cache, v_cache, \
                       pos, part, (int)L, scale, ri)
    if (hd == 128) {
        if (G == 1) SX8_ATTN(128, 1); else if (G == 2) SX8_ATTN(128, 2); else if (G == 4) SX8_ATTN(128, 4); else SX8_ATTN(128, 8);
        hipLaunchKernelGGL(k_attn_combine<128>, dim3((unsigned)nh), dim3(128), 0, st, part, out);
    } else {
        if (G == 1) SX8_ATTN(64, 1); else if (G == 2) SX8_ATTN(64, 2); else if (G == 4) SX8_ATTN(64, 4); else SX8_ATTN(64, 8);
        hipLaunchKernelGGL(k_attn_combine<64>, dim3((unsigned)nh), dim3(64), 0, st, part, out);
    }
#undef SX8_ATTN
    return check_launch(what);
}

extern "C" int32_t sx8_dec_silu_mul(const float* g, const float* u, uint16_t* out, int64_t n, void* stream) {
    using namespace sx8;
    if (!g || !u || !out) return fail(SX8_ERR_INVALID, "sx8_dec_silu_mul: null pointer");
    if (n <= 0 || (n + 255) / 256 > 0x7FFFFFFF) return fail(SX8_ERR_INVALID, "sx8_dec_silu_mul: bad size");
    hipLaunchKernelGGL(k_silu_mul, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, as_stream(stream), g,
                       u, out, n);
    return check_launch("sx8_dec_silu_mul");
}

extern "C" int32_t sx8_dec_argmax_advance(const float* logits, int64_t n, int64_t* tok, int64_t* pos,
                                          void* stream) {
    using namespace sx8;
    if (!logits || !tok || !pos) return fail(SX8_ERR_INVALID, "sx8_dec_argmax_advance: null pointer");
    if (n <= 0) return fail(SX8_ERR_INVALID, "sx8_dec_argmax_advance: bad size");
    hipLaunchKernelGGL(k_argmax_advance, dim3(1), dim3(1024), 0, as_stream(stream), logits, n, tok, pos);
    return check_launch("sx8_dec_argmax_advance");
}
