// sx8_gemm.hip -- prefill GEMM Y (M, N) f32 = X (M, K) fp16 . W^T with W in S-X8 blocks.
//
// Reference roles: gemm_compact (cuda/sx8_gemm_compact.cu:55-194, CUDA-core FMAs with
// PCA applied through Z) and sx8_wmma_kernel / fused_forward (cuda/sx8_fused_wmma.cu:
// 11-154, WMMA 16x16x16 with per-weight PCA).  One kernel serves both: the weight
// tile is decoded with the canonical R64 recipe (bit-exact fp16, per-weight PCA) and
// fed to v_mfma_f32_16x16x32_f16 with float32 accumulation.
//
// Work decomposition (gfx950, wave64):
//   * a 256-thread work-group owns a kBM x 256 output tile; wave w owns 64 columns
//     (four groups of 16) for all kBM rows.
//   * K advances one S-X8 block (32 weights) per step.  For 16x16x32 MFMAs lane l holds
//     B-operand column l%16 and the 8 consecutive k of chunk l/16 -- exactly sub-block
//     sb = l/16 of that column's block.  Each lane therefore decodes its own operand
//     straight into registers (four sub-blocks per step, one per column group); the
//     weight tile never touches LDS and is decoded once per work-group.
//   * the X tile (kBM x 32 fp16) is staged in LDS (row pitch padded to 80 B) and read
//     as 16-byte A fragments, each reused by the four column groups.
//   * the LDS X tile is double-buffered; the B decode of step kb+1 overlaps the MFMAs
//     of step kb.
// Modes: kV44 (hdr/levels + basis/scales), kSplit (kb-major split arrays, the fused-WMMA
// contract), kCore (v4.4 without the PCA terms, for the caller-supplied-Z contract).
#include "sx8_device.h"
#include "sx8_host.h"

namespace {

constexpr int kBM = 128;
constexpr int kBN = 256;
constexpr int kThreads = 256;
constexpr int kXPitch = 40;  // fp16 per LDS row: 32 + 8 pad

enum { kV44 = 0, kSplit = 1, kCore = 2 };

struct SplitPtrs {
    const uint16_t* dmin;
    const uint16_t* dmax;
    const uint8_t* config;
    const uint8_t* coeff;
    const uint8_t* hi;
    const uint8_t* lo;
};

template <int MODE, int HB>
__device__ __forceinline__ void decode_operand(const uint8_t* __restrict__ hdr,
                                               const uint8_t* __restrict__ levels,
                                               const SplitPtrs& sp, int64_t bid, int sb,
                                               const double* b0, const double* b1, double s0,
                                               double s1, uint32_t w[4]) {
    uint32_t d0, d1, cfg, cf, H, P16;
    if constexpr (MODE == kSplit) {
        d0 = sp.dmin[bid];
        d1 = sp.dmax[bid];
        cfg = sp.config[bid];
        cf = sp.coeff[bid];
        H = *reinterpret_cast<const uint32_t*>(sp.hi + bid * 16 + 4 * sb);
        P16 = *reinterpret_cast<const uint16_t*>(sp.lo + bid * 8 + 2 * sb);
    } else {
        sx8_load_hdr<HB>(hdr, bid, d0, d1, cfg, cf);
        const uint8_t* lv = levels + bid * 24;
        H = *reinterpret_cast<const uint32_t*>(lv + 4 * sb);
        P16 = *reinterpret_cast<const uint16_t*>(lv + 16 + 2 * sb);
    }
    sx8_r64_subblock<MODE != kCore>(sx8_h2f(d0), sx8_h2f(d1), cfg, cf, sb, H, P16, b0, b1, s0, s1, w);
}

__device__ __forceinline__ void load_x_tile(const uint16_t* __restrict__ X, int M, int64_t ldx,
                                            int K, int m0, int kb, bool x_vec,
                                            uint16_t* __restrict__ xs) {
    for (int c = threadIdx.x; c < kBM * 4; c += kThreads) {
        const int row = c >> 2, ch = c & 3;
        const int m = m0 + row;
        const int k = kb * 32 + 8 * ch;
        uint4 v = make_uint4(0, 0, 0, 0);
        if (m < M) {
            const uint16_t* src = X + (int64_t)m * ldx + k;
            if (x_vec && k + 8 <= K) {
                v = *reinterpret_cast<const uint4*>(src);
            } else {
                uint32_t e[4] = {0, 0, 0, 0};
#pragma unroll
                for (int j = 0; j < 8; ++j)
                    if (k + j < K) e[j >> 1] |= (uint32_t)src[j] << (16 * (j & 1));
                v = make_uint4(e[0], e[1], e[2], e[3]);
            }
        }
        *reinterpret_cast<uint4*>(xs + row * kXPitch + 8 * ch) = v;
    }
}

template <int MODE, int HB>
__global__ __launch_bounds__(kThreads) void k_gemm(
    const uint16_t* __restrict__ X, int M, int64_t ldx, int K, const uint8_t* __restrict__ hdr,
    const uint8_t* __restrict__ levels, SplitPtrs sp, const float* __restrict__ basis,
    const float* __restrict__ scales, int N, int n_cb, bool x_vec, float* __restrict__ Y) {
    __shared__ __align__(16) uint16_t xs[2][kBM * kXPitch];
    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = tid >> 6;
    const int m0 = blockIdx.y * kBM;
    const int nw = blockIdx.x * kBN + wave * 64;
    const int c16 = lane & 15;
    const int sb = lane >> 4;

    sx8_float4 acc[kBM / 16][4];
#pragma unroll
    for (int r = 0; r < kBM / 16; ++r)
#pragma unroll
        for (int g = 0; g < 4; ++g) acc[r][g] = sx8_float4{0.f, 0.f, 0.f, 0.f};

    load_x_tile(X, M, ldx, K, m0, 0, x_vec, xs[0]);

    for (int kb = 0; kb < n_cb; ++kb) {
        // ---- decode this lane's B operands (4 column groups x 8 weights)
        double b0[8], b1[8], s0 = 0.0, s1 = 0.0;
        if constexpr (MODE != kCore) {
            const float4* p0 = reinterpret_cast<const float4*>(basis + (int64_t)kb * 64 + 8 * sb);
            const float4* p1 = reinterpret_cast<const float4*>(basis + (int64_t)kb * 64 + 32 + 8 * sb);
            const float4 a0 = p0[0], a1 = p0[1], c0 = p1[0], c1 = p1[1];
            b0[0] = a0.x; b0[1] = a0.y; b0[2] = a0.z; b0[3] = a0.w;
            b0[4] = a1.x; b0[5] = a1.y; b0[6] = a1.z; b0[7] = a1.w;
            b1[0] = c0.x; b1[1] = c0.y; b1[2] = c0.z; b1[3] = c0.w;
            b1[4] = c1.x; b1[5] = c1.y; b1[6] = c1.z; b1[7] = c1.w;
            s0 = scales[kb * 2];
            s1 = scales[kb * 2 + 1];
        } else {
#pragma unroll
            for (int i = 0; i < 8; ++i) b0[i] = b1[i] = 0.0;
        }
        sx8_half8 bop[4];
#pragma unroll
        for (int g = 0; g < 4; ++g) {
            const int n = nw + 16 * g + c16;
            uint32_t w[4] = {0, 0, 0, 0};
            if (n < N)
                decode_operand<MODE, HB>(hdr, levels, sp, (int64_t)kb * N + n, sb, b0, b1, s0, s1, w);
            bop[g] = __builtin_bit_cast(sx8_half8, make_uint4(w[0], w[1], w[2], w[3]));
        }

        // ---- X tile kb is in xs[kb & 1]; prefetch tile kb+1 into the other buffer
        __syncthreads();
        if (kb + 1 < n_cb) load_x_tile(X, M, ldx, K, m0, kb + 1, x_vec, xs[(kb + 1) & 1]);
        const uint16_t* xt = xs[kb & 1];
#pragma unroll
        for (int r = 0; r < kBM / 16; ++r) {
            const sx8_half8 a =
                *reinterpret_cast<const sx8_half8*>(xt + (16 * r + c16) * kXPitch + 8 * sb);
#pragma unroll
            for (int g = 0; g < 4; ++g)
                acc[r][g] = __builtin_amdgcn_mfma_f32_16x16x32_f16(a, bop[g], acc[r][g], 0, 0, 0);
        }
    }

    // ---- epilogue: lane holds column 16g + l%16, rows 16r + 4(l/16) + i
#pragma unroll
    for (int g = 0; g < 4; ++g) {
        const int n = nw + 16 * g + c16;
        if (n >= N) continue;
#pragma unroll
        for (int r = 0; r < kBM / 16; ++r)
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const int m = m0 + 16 * r + 4 * sb + i;
                if (m < M) Y[(int64_t)m * N + n] = acc[r][g][i];
            }
    }
}

// Output-side PCA: Y[m, n] += sum_kb c0(kb,n) Z[m,kb,0] + c1(kb,n) Z[m,kb,1].
// One thread per column, kRows rows per thread; coeff bytes read once per kb.
constexpr int kPcaRows = 8;

template <int HB>
__global__ __launch_bounds__(256) void k_pca_z(const float* __restrict__ Z, int M,
                                               const uint8_t* __restrict__ hdr, int N, int n_cb,
                                               float* __restrict__ Y) {
    const int n = blockIdx.x * 256 + threadIdx.x;
    const int m0 = blockIdx.y * kPcaRows;
    if (n >= N) return;
    float acc[kPcaRows];
#pragma unroll
    for (int i = 0; i < kPcaRows; ++i) acc[i] = 0.f;
    for (int kb = 0; kb < n_cb; ++kb) {
        const uint32_t cf = hdr[((int64_t)kb * N + n) * HB + 5];
        const float c0 = (float)sx8_sext4(cf), c1 = (float)sx8_sext4(cf >> 4);
#pragma unroll
        for (int i = 0; i < kPcaRows; ++i) {
            const int m = min(m0 + i, M - 1);
            const float2 z = *reinterpret_cast<const float2*>(Z + ((int64_t)m * n_cb + kb) * 2);
            acc[i] += c0 * z.x + c1 * z.y;
        }
    }
#pragma unroll
    for (int i = 0; i < kPcaRows; ++i)
        if (m0 + i < M) Y[(int64_t)(m0 + i) * N + n] += acc[i];
}

template <int MODE>
int32_t launch_gemm(const char* what, const uint16_t* X, int64_t M, int64_t ldx, int64_t K,
                    const uint8_t* hdr, const uint8_t* levels, int32_t hdr_bytes,
                    const SplitPtrs& sp, const float* basis, const float* scales, int64_t N,
                    int64_t n_cb, float* Y, void* stream) {
    using namespace sx8;
    if (M <= 0 || K <= 0 || N <= 0 || n_cb <= 0 || n_cb * 32 < K || (n_cb - 1) * 32 >= K ||
        ldx < K || M > 0x7FFFFFFF || N > 0x7FFFFFFF || n_cb > 0x7FFFFFFF / 64)
        return fail(SX8_ERR_INVALID, "%s: bad shape M=%lld K=%lld ldx=%lld N=%lld n_cb=%lld", what,
                    (long long)M, (long long)K, (long long)ldx, (long long)N, (long long)n_cb);
    if (!aligned(X, 2) || !aligned(Y, 4) || (basis && !aligned(basis, 16)) ||
        (scales && !aligned(scales, 8)))
        return fail(SX8_ERR_INVALID, "%s: misaligned pointer", what);
    const bool x_vec = aligned(X, 16) && (ldx % 8 == 0);
    const dim3 grid((unsigned)((N + kBN - 1) / kBN), (unsigned)((M + kBM - 1) / kBM));
    if (grid.y > 65535) return fail(SX8_ERR_UNSUPPORTED, "%s: M too large", what);
    const hipStream_t st = as_stream(stream);
    if (hdr_bytes == 8)
        hipLaunchKernelGGL((k_gemm<MODE, 8>), grid, dim3(kThreads), 0, st, X, (int)M, ldx, (int)K,
                           hdr, levels, sp, basis, scales, (int)N, (int)n_cb, x_vec, Y);
    else
        hipLaunchKernelGGL((k_gemm<MODE, 6>), grid, dim3(kThreads), 0, st, X, (int)M, ldx, (int)K,
                           hdr, levels, sp, basis, scales, (int)N, (int)n_cb, x_vec, Y);
    return check_launch(what);
}

}  // namespace

extern "C" int32_t sx8_gemm_prefill(const uint16_t* X, int64_t M, int64_t ldx, int64_t K,
                                    const uint8_t* hdr, const uint8_t* levels, int32_t hdr_bytes,
                                    const float* basis, const float* scales, int64_t N,
                                    int64_t n_cb, float* Y, void* stream) {
    using namespace sx8;
    if (!X || !hdr || !levels || !basis || !scales || !Y)
        return fail(SX8_ERR_INVALID, "sx8_gemm_prefill: null pointer");
    if (hdr_bytes != 6 && hdr_bytes != 8)
        return fail(SX8_ERR_INVALID, "sx8_gemm_prefill: hdr_bytes must be 6 or 8, got %d", hdr_bytes);
    if (!aligned(hdr, hdr_bytes == 8 ? 8 : 2) || !aligned(levels, 8))
        return fail(SX8_ERR_INVALID, "sx8_gemm_prefill: misaligned hdr/levels");
    return launch_gemm<kV44>("sx8_gemm_prefill", X, M, ldx, K, hdr, levels, hdr_bytes, SplitPtrs{},
                             basis, scales, N, n_cb, Y, stream);
}

extern "C" int32_t sx8_gemm_prefill_split(const uint16_t* X, int64_t M, int64_t ldx, int64_t K,
                                          const uint16_t* dmin, const uint16_t* dmax,
                                          const uint8_t* config, const uint8_t* coeff,
                                          const uint8_t* hi, const uint8_t* lo, const float* basis,
                                          const float* scales, int64_t N, int64_t n_cb, float* Y,
                                          void* stream) {
    using namespace sx8;
    if (!X || !dmin || !dmax || !config || !coeff || !hi || !lo || !basis || !scales || !Y)
        return fail(SX8_ERR_INVALID, "sx8_gemm_prefill_split: null pointer");
    if (!aligned(dmin, 2) || !aligned(dmax, 2) || !aligned(hi, 4) || !aligned(lo, 2))
        return fail(SX8_ERR_INVALID, "sx8_gemm_prefill_split: misaligned block arrays");
    const SplitPtrs sp{dmin, dmax, config, coeff, hi, lo};
    return launch_gemm<kSplit>("sx8_gemm_prefill_split", X, M, ldx, K, nullptr, nullptr, 6, sp,
                               basis, scales, N, n_cb, Y, stream);
}

extern "C" int32_t sx8_gemm_prefill_core(const uint16_t* X, int64_t M, int64_t ldx, int64_t K,
                                         const uint8_t* hdr, const uint8_t* levels,
                                         int32_t hdr_bytes, int64_t N, int64_t n_cb, float* Y,
                                         void* stream) {
    using namespace sx8;
    if (!X || !hdr || !levels || !Y) return fail(SX8_ERR_INVALID, "sx8_gemm_prefill_core: null pointer");
    if (hdr_bytes != 6 && hdr_bytes != 8)
        return fail(SX8_ERR_INVALID, "sx8_gemm_prefill_core: hdr_bytes must be 6 or 8, got %d", hdr_bytes);
    if (!aligned(hdr, hdr_bytes == 8 ? 8 : 2) || !aligned(levels, 8))
        return fail(SX8_ERR_INVALID, "sx8_gemm_prefill_core: misaligned hdr/levels");
    return launch_gemm<kCore>("sx8_gemm_prefill_core", X, M, ldx, K, hdr, levels, hdr_bytes,
                              SplitPtrs{}, nullptr, nullptr, N, n_cb, Y, stream);
}

extern "C" int32_t sx8_gemm_pca_z(const float* Z, int64_t M, const uint8_t* hdr, int32_t hdr_bytes,
                                  int64_t N, int64_t n_cb, float* Y, void* stream) {
    using namespace sx8;
    if (!Z || !hdr || !Y) return fail(SX8_ERR_INVALID, "sx8_gemm_pca_z: null pointer");
    if (hdr_bytes != 6 && hdr_bytes != 8)
        return fail(SX8_ERR_INVALID, "sx8_gemm_pca_z: hdr_bytes must be 6 or 8, got %d", hdr_bytes);
    if (M <= 0 || N <= 0 || n_cb <= 0 || M > 0x7FFFFFFF || N > 0x7FFFFFFF)
        return fail(SX8_ERR_INVALID, "sx8_gemm_pca_z: bad shape");
    if (!aligned(Z, 8) || !aligned(Y, 4)) return fail(SX8_ERR_INVALID, "sx8_gemm_pca_z: misaligned pointer");
    const dim3 grid((unsigned)((N + 255) / 256), (unsigned)((M + kPcaRows - 1) / kPcaRows));
    if (grid.y > 65535) return fail(SX8_ERR_UNSUPPORTED, "sx8_gemm_pca_z: M too large");
    if (hdr_bytes == 8)
        hipLaunchKernelGGL(k_pca_z<8>, grid, dim3(256), 0, as_stream(stream), Z, (int)M, hdr,
                           (int)N, (int)n_cb, Y);
    else
        hipLaunchKernelGGL(k_pca_z<6>, grid, dim3(256), 0, as_stream(stream), Z, (int)M, hdr,
                           (int)N, (int)n_cb, Y);
    return check_launch("sx8_gemm_pca_z");
}
