// sx8_gemv.hip -- PCA precompute (Z) and the M = 1 decode GEMV on the v4.4 layout.
//
// Reference roles: compute_z44 / compute_z44_batch (cuda/sx8_decode1_v3.cu:44-65,
// cuda/sx8_gemm_compact.cu:28-50) and decode1_v44_kernel (cuda/sx8_decode1_v3.cu:75-167)
// with its combined wrapper (:223-246).
//
// GEMV design (gfx950, HBM-bound):
//   * one lane per output column; a 256-thread work-group covers 64 consecutive
//     columns and a contiguous range of K blocks (kb); its four waves take every
//     fourth kb of that range.  In the kb-major layout a wave's loads for one kb are
//     64 consecutive 24-byte level records and 64 consecutive header records.
//   * the activation side of each kb (x pairs, per-sub-block sums of x, Z0/Z1) is
//     computed once per work-group into LDS and read back as wave-uniform broadcasts.
//   * the core dot sum_i x_i (rlo + step lv_i) is rewritten per 8-weight sub-block as
//     (rlo - 64 step) * Sx + step * sum_i x_i (64 + lv_i): the levels are spliced into
//     fp16 values 64 + lv (exponent 6, lv in mantissa bits 4..9) with two shifts and
//     two and-or's per pair of weights, and v_dot2_f32_f16 does two MACs per op.
//   * PCA is applied per block through Z (docs/SX8_FLASH_V4_3_SPEC.md:49-61).
//   * small-N shapes split K across work-groups; partial sums go to a workspace and
//     the last work-group to arrive for a column tile adds them in fixed order, so the
//     result is deterministic (the reference rejected atomicAdd split-K for that
//     reason).  The arrival counter is reset by that last work-group.
#include "sx8_device.h"
#include "sx8_host.h"

namespace {

constexpr int kWaves = 4;
constexpr int kThreads = 64 * kWaves;
constexpr int kCols = 64;
constexpr int kTargetGroups = 512;   // ~2 work-groups per CU on a 256-CU MI355X
constexpr int kMaxKbPerGroup = 320;  // bounds the LDS staging (96 B per kb)

struct KbInfo {
    uint32_t xp[16];  // (x[8sb+i], x[8sb+i+4]) as fp16 pairs, index 4*sb + i
    float sx[4];      // sum of the sub-block's 8 x values
    float z[2];       // Z0, Z1
    float pad[2];
};
static_assert(sizeof(KbInfo) == 96, "KbInfo layout");

// Z of one (row, kb, j) with the reference's warp tree: products x_t * b_t, then
// pairwise sums over lane offsets 16, 8, 4, 2, 1 (cuda/sx8_decode1_v3.cu:53-63),
// then scale * sum.
__device__ __forceinline__ float z_tree(const uint16_t* __restrict__ x,
                                        const float* __restrict__ b, float scale) {
#pragma clang fp contract(off)
    float p[32];
#pragma unroll
    for (int t = 0; t < 32; ++t) p[t] = sx8_h2f(x[t]) * b[t];
#pragma unroll
    for (int off = 16; off > 0; off >>= 1)
#pragma unroll
        for (int t = 0; t < off; ++t) p[t] = p[t] + p[t + off];
    return scale * p[0];
}

__global__ __launch_bounds__(256) void k_compute_z(const uint16_t* __restrict__ X, int64_t M,
                                                   int64_t ldx, const float* __restrict__ basis,
                                                   const float* __restrict__ scales, int64_t n_cb,
                                                   float* __restrict__ Z) {
    const int64_t gid = (int64_t)blockIdx.x * 256 + threadIdx.x;
    if (gid >= M * n_cb * 2) return;
    const int j = (int)(gid & 1);
    const int64_t mk = gid >> 1;
    const int64_t m = mk / n_cb;
    const int64_t kb = mk - m * n_cb;
    Z[gid] = z_tree(X + m * ldx + kb * 32, basis + kb * 64 + 32 * j, scales[kb * 2 + j]);
}

// Level pair i (weights i and i+4 of a sub-block) as two fp16 values 64 + lv.
// H: hi nibbles (weight w at bits 4w); P: lo quads spread so weights 0..3 sit in bits
// 0..7 and weights 4..7 in bits 16..23 (weight w at bit 6 - 2*(w&3) of its byte).
__device__ __forceinline__ uint32_t lv_pair(uint32_t H, uint32_t P, int i) {
    uint32_t hs, ps;
    if (i == 0)      { hs = H << 6; ps = P >> 2; }
    else if (i == 1) { hs = H << 2; ps = P; }
    else if (i == 2) { hs = H >> 2; ps = P << 2; }
    else             { hs = H >> 6; ps = P << 4; }
    return (hs & 0x03C003C0u) | (ps & 0x00300030u) | 0x54005400u;
}

__device__ __forceinline__ float dot2(uint32_t a, uint32_t b, float c) {
    return __builtin_amdgcn_fdot2(__builtin_bit_cast(sx8_half2, a),
                                  __builtin_bit_cast(sx8_half2, b), c, false);
}

template <int HB, bool kZGiven>
__global__ __launch_bounds__(kThreads) void k_gemv(
    const uint16_t* __restrict__ X, const uint8_t* __restrict__ hdr,
    const uint8_t* __restrict__ levels, const float* __restrict__ basis,
    const float* __restrict__ scales, const float* __restrict__ Zin, float* __restrict__ Zout,
    float* __restrict__ Y, float* __restrict__ partial, uint32_t* __restrict__ counters,
    int N, int n_cb, int kb_per) {
    extern __shared__ __align__(16) unsigned char smem[];
    KbInfo* info = reinterpret_cast<KbInfo*>(smem);
    float* red = reinterpret_cast<float*>(smem + sizeof(KbInfo) * kb_per);

    const int tile = blockIdx.x;
    const int split = blockIdx.y;
    const int S = gridDim.y;
    const int kb0 = split * kb_per;
    const int nkb = min(kb_per, n_cb - kb0);
    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = tid >> 6;

    // ---- stage the activation side of this work-group's kb range in LDS
    for (int u = tid; u < nkb * 4; u += kThreads) {
        const int kl = u >> 2, sb = u & 3;
        const uint4 xv = *reinterpret_cast<const uint4*>(X + (int64_t)(kb0 + kl) * 32 + 8 * sb);
        const uint32_t xw[4] = {xv.x, xv.y, xv.z, xv.w};
        float s = 0.f;
#pragma unroll
        for (int i = 0; i < 8; ++i) s += sx8_h2f(xw[i >> 1] >> (16 * (i & 1)));
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const uint32_t a = (xw[i >> 1] >> (16 * (i & 1))) & 0xFFFFu;             // x[i]
            const uint32_t b = (xw[(i + 4) >> 1] >> (16 * (i & 1))) & 0xFFFFu;       // x[i+4]
            info[kl].xp[4 * sb + i] = a | (b << 16);
        }
        info[kl].sx[sb] = s;
    }
    for (int u = tid; u < nkb * 2; u += kThreads) {
        const int kl = u >> 1, j = u & 1;
        const int kb = kb0 + kl;
        float z;
        if constexpr (kZGiven) {
            z = Zin[kb * 2 + j];
        } else {
            z = z_tree(X + (int64_t)kb * 32, basis + kb * 64 + 32 * j, scales[kb * 2 + j]);
            if (Zout && tile == 0) Zout[kb * 2 + j] = z;
        }
        info[kl].z[j] = z;
    }
    __syncthreads();

    // ---- stream this column tile's blocks
    const int n = tile * kCols + lane;
    const bool valid = n < N;
    const int64_t nn = valid ? n : N - 1;
    float acc = 0.f;
    for (int kl = wave; kl < nkb; kl += kWaves) {
        const int64_t bid = (int64_t)(kb0 + kl) * N + nn;
        uint32_t d0, d1, cfg, cf;
        sx8_load_hdr<HB>(hdr, bid, d0, d1, cfg, cf);
        const uint2* lp = reinterpret_cast<const uint2*>(levels + bid * 24);
        const uint2 v0 = lp[0], v1 = lp[1], v2 = lp[2];
        const uint32_t Hs[4] = {v0.x, v0.y, v1.x, v1.y};
        const uint32_t Pw[2] = {v2.x, v2.y};
        const KbInfo& ki = info[kl];

        const float lo = sx8_h2f(d0), hi = sx8_h2f(d1);
        const float q = (hi - lo) * 0.25f;
        acc += (float)sx8_sext4(cf) * ki.z[0] + (float)sx8_sext4(cf >> 4) * ki.z[1];
#pragma unroll
        for (int sb = 0; sb < 4; ++sb) {
            const uint32_t s = (cfg >> (2 * sb)) & 3u;
            const float k1 = (float)((0x1300u >> (4 * s)) & 0xFu);   // 0,0,3,1
            const float k2 = (float)((0x1030u >> (4 * s)) & 0xFu);   // 0,3,0,1
            const float rlo = lo + q * k1;
            const float rhi = hi - q * k2;
            float step = (rhi - rlo) * 0.015873f;
            if (step < 1e-10f) step = 1e-10f;
            const uint32_t P16 = (sb & 1) ? (Pw[sb >> 1] >> 16) : (Pw[sb >> 1] & 0xFFFFu);
            const uint32_t P = (P16 & 0xFFu) | ((P16 & 0xFF00u) << 8);
            float d = 0.f;
#pragma unroll
            for (int i = 0; i < 4; ++i) d = dot2(lv_pair(Hs[sb], P, i), ki.xp[4 * sb + i], d);
            acc += (rlo - 64.f * step) * ki.sx[sb] + step * d;
        }
    }

    // ---- reduce the four waves in a fixed order
    red[wave * 64 + lane] = acc;
    __syncthreads();
    if (wave != 0) return;
    const float total = ((red[lane] + red[64 + lane]) + red[128 + lane]) + red[192 + lane];
    if (S == 1) {
        if (valid) Y[n] = total;
        return;
    }
    if (valid) partial[(int64_t)split * N + n] = total;
    __threadfence();   // release this group's partials device-wide
    uint32_t prev = 0;
    if (lane == 0)
        prev = __hip_atomic_fetch_add(&counters[tile], 1u, __ATOMIC_ACQ_REL,
                                      __HIP_MEMORY_SCOPE_AGENT);
    prev = __shfl(prev, 0);
    if (prev != (uint32_t)(S - 1)) return;
    __threadfence();   // acquire the other groups' partials
    if (valid) {
        float t = 0.f;
        for (int s = 0; s < S; ++s)
            t += __hip_atomic_load(&partial[(int64_t)s * N + n], __ATOMIC_RELAXED,
                                   __HIP_MEMORY_SCOPE_AGENT);
        Y[n] = t;
    }
    if (lane == 0)
        __hip_atomic_store(&counters[tile], 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

template <int HB>
int32_t launch_gemv(const uint16_t* X, const uint8_t* hdr, const uint8_t* levels,
                    const float* basis, const float* scales, const float* Zin, float* Zout,
                    int N, int n_cb, float* Y, hipStream_t st) {
    using namespace sx8;
    const int tiles = (N + kCols - 1) / kCols;
    int S = 1;
    if (tiles < kTargetGroups) S = (kTargetGroups + tiles - 1) / tiles;
    S = std::min(S, std::max(1, n_cb / 8));                                // >= 8 kb per group
    S = std::max(S, (n_cb + kMaxKbPerGroup - 1) / kMaxKbPerGroup);         // LDS bound
    const int kb_per = (n_cb + S - 1) / S;
    S = (n_cb + kb_per - 1) / kb_per;
    float* partial = nullptr;
    uint32_t* counters = nullptr;
    if (S > 1) {
        const int32_t rc = gemv_workspace((int64_t)S * N, tiles, &partial, &counters);
        if (rc != SX8_OK) return rc;
    }
    const size_t smem = sizeof(KbInfo) * (size_t)kb_per + sizeof(float) * kThreads;
    const dim3 grid(tiles, S);
    if (Zin)
        hipLaunchKernelGGL((k_gemv<HB, true>), grid, dim3(kThreads), smem, st, X, hdr, levels,
                           basis, scales, Zin, Zout, Y, partial, counters, N, n_cb, kb_per);
    else
        hipLaunchKernelGGL((k_gemv<HB, false>), grid, dim3(kThreads), smem, st, X, hdr, levels,
                           basis, scales, Zin, Zout, Y, partial, counters, N, n_cb, kb_per);
    return check_launch("sx8_gemv");
}

}  // namespace

extern "C" int32_t sx8_compute_z(const uint16_t* X, int64_t M, int64_t ldx, const float* basis,
                                 const float* scales, int64_t n_cb, float* Z, void* stream) {
    using namespace sx8;
    if (!X || !basis || !scales || !Z) return fail(SX8_ERR_INVALID, "sx8_compute_z: null pointer");
    if (M <= 0 || n_cb <= 0 || ldx < n_cb * 32)
        return fail(SX8_ERR_INVALID, "sx8_compute_z: bad shape M=%lld ldx=%lld n_cb=%lld",
                    (long long)M, (long long)ldx, (long long)n_cb);
    if (!aligned(X, 2) || !aligned(basis, 4) || !aligned(scales, 4) || !aligned(Z, 4))
        return fail(SX8_ERR_INVALID, "sx8_compute_z: misaligned pointer");
    const int64_t threads = M * n_cb * 2;
    const int64_t grid = (threads + 255) / 256;
    if (grid > 0x7FFFFFFF) return fail(SX8_ERR_UNSUPPORTED, "sx8_compute_z: too large");
    hipLaunchKernelGGL(k_compute_z, dim3((unsigned)grid), dim3(256), 0, as_stream(stream), X, M,
                       ldx, basis, scales, n_cb, Z);
    return check_launch("sx8_compute_z");
}

extern "C" int32_t sx8_gemv(const uint16_t* X, const uint8_t* hdr, const uint8_t* levels,
                            int32_t hdr_bytes, const float* basis, const float* scales,
                            const float* Z_in, float* Z_out, int64_t N, int64_t n_cb, float* Y,
                            void* stream) {
    using namespace sx8;
    if (!X || !hdr || !levels || !Y) return fail(SX8_ERR_INVALID, "sx8_gemv: null pointer");
    if (!Z_in && (!basis || !scales))
        return fail(SX8_ERR_INVALID, "sx8_gemv: basis/scales required when Z_in is NULL");
    if (hdr_bytes != 6 && hdr_bytes != 8)
        return fail(SX8_ERR_INVALID, "sx8_gemv: hdr_bytes must be 6 or 8, got %d", hdr_bytes);
    if (N <= 0 || n_cb <= 0 || N > 0x7FFFFFFF / 2 || n_cb > 0x7FFFFFFF / 64)
        return fail(SX8_ERR_INVALID, "sx8_gemv: bad shape N=%lld n_cb=%lld", (long long)N,
                    (long long)n_cb);
    if (!aligned(X, 16) || !aligned(hdr, hdr_bytes == 8 ? 8 : 2) || !aligned(levels, 8) ||
        (basis && !aligned(basis, 4)) || (scales && !aligned(scales, 4)) ||
        (Z_in && !aligned(Z_in, 4)) || (Z_out && !aligned(Z_out, 4)) || !aligned(Y, 4))
        return fail(SX8_ERR_INVALID, "sx8_gemv: misaligned pointer (X needs 16-byte alignment)");
    if (hdr_bytes == 8)
        return launch_gemv<8>(X, hdr, levels, basis, scales, Z_in, Z_out, (int)N, (int)n_cb, Y,
                              as_stream(stream));
    return launch_gemv<6>(X, hdr, levels, basis, scales, Z_in, Z_out, (int)N, (int)n_cb, Y,
                          as_stream(stream));
}
