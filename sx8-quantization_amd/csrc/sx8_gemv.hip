// sx8_gemv.hip -- PCA precompute (Z) and the M = 1 decode GEMV on the v4.4 layout.
//
// Reference roles: compute_z44 / compute_z44_batch (cuda/sx8_decode1_v3.cu:44-65,
// cuda/sx8_gemm_compact.cu:28-50) and decode1_v44_kernel (cuda/sx8_decode1_v3.cu:75-167)
// with its wrappers decode1_v44 / decode1_v44_combined (:197-246).
//
// GEMV design (gfx950):
//   * k_gemv_panel streams the weights.  A 512-thread work-group owns a panel of CT
//     consecutive columns over the whole K; lane (c, j) = (column c, K slice j), so the
//     CT lanes of a slice read CT consecutive records of one kb row.  Slices are summed
//     in LDS in a fixed order: no device-scope fences or atomics, deterministic output.
//   * every block's decode needs the activation side of its kb (x pairs, sub-block sums
//     of x, splice biases, Z0/Z1): a 112-byte table entry per kb, built in LDS by each
//     work-group while its first weight loads are in flight (one launch).  When the
//     caller wants Z back (the combined entry point), k_kbinfo builds the table once
//     with the reference's summation tree -- Z bit-identical to compute_z44 -- and the
//     panel kernel copies it in.
//   * per 8-weight sub-block the core dot sum_i x_i (rlo + step lv_i) becomes
//     rlo * Sx + step * (sum x lv) with sum x lv from fp16 "splices" and
//     v_dot2_f32_f16 (see block_dot); PCA is applied per block through Z
//     (docs/SX8_FLASH_V4_3_SPEC.md:49-61).
//   * the K loop is software-pipelined (rotating record buffers, unconditional buffer
//     loads that read zeros past the end) and panels are renumbered per XCD (see
//     k_gemv_panel).
#include <algorithm>
#include <climits>
#include <type_traits>

#include "sx8_buffer.h"
#include "sx8_device.h"
#include "sx8_host.h"

namespace {

struct KbInfo {
    uint32_t xp[16];  // (x[8sb+i], x[8sb+i+4]) as fp16 pairs, index 4*sb + i
    float sx[4];      // sum of the sub-block's 8 x values (left to right)
    float nbias[4];   // -sum_i (x[8sb+i] + x[8sb+i+4]) * kSpliceBias[i] (see block_dot)
    float z[2];       // Z0, Z1
    float pad[2];
};
static_assert(sizeof(KbInfo) == 112, "KbInfo layout");

__device__ __forceinline__ float dot2(uint32_t a, uint32_t b, float c) {
    return __builtin_amdgcn_fdot2(__builtin_bit_cast(sx8_half2, a),
                                  __builtin_bit_cast(sx8_half2, b), c, false);
}

// Negated constant parts of block_dot's fp16 splices for weight pair i, as fp16 pairs:
// nibble splice (4096 for pairs 0, 2; 256 for pairs 1, 3) + quad splice (16, 64, 256,
// 1024), i.e. -4112, -320, -4352, -1280 (all exact in fp16).
constexpr uint32_t kNegSplice[4] = {0xEC04EC04u, 0xDD00DD00u, 0xEC40EC40u, 0xE500E500u};
constexpr uint32_t kOnePair = 0x3C003C00u;   // (1.0, 1.0)

// x pairs, sub-block sum and splice bias of one (kb, sb) from its 8 x values (fp16 pairs
// (x0,x1) (x2,x3) (x4,x5) (x6,x7) in xv): pair i = (x_i, x_{i+4}) by byte permutes, the
// sum and the bias -sum_i (x_i + x_{i+4}) * splice_i as v_dot2_f32_f16 chains (each
// product is exact in fp32).
__device__ __forceinline__ void fill_x_side(KbInfo& out, int sb, const uint4 xv) {
    const uint32_t p0 = __builtin_amdgcn_perm(xv.z, xv.x, 0x05040100u);
    const uint32_t p1 = __builtin_amdgcn_perm(xv.z, xv.x, 0x07060302u);
    const uint32_t p2 = __builtin_amdgcn_perm(xv.w, xv.y, 0x05040100u);
    const uint32_t p3 = __builtin_amdgcn_perm(xv.w, xv.y, 0x07060302u);
    *reinterpret_cast<uint4*>(out.xp + 4 * sb) = make_uint4(p0, p1, p2, p3);
    out.sx[sb] = dot2(xv.w, kOnePair, dot2(xv.z, kOnePair, dot2(xv.y, kOnePair,
                                                                 dot2(xv.x, kOnePair, 0.f))));
    out.nbias[sb] = dot2(p3, kNegSplice[3], dot2(p2, kNegSplice[2], dot2(p1, kNegSplice[1],
                                                                       dot2(p0, kNegSplice[0], 0.f))));
}

// Global-memory views: a pointer that went through an SGPR pin (see k_gemv_panel) is a
// generic pointer to the compiler, whose loads would be flat loads (counted on the LDS /
// scalar counter as well, so any wait for a scalar load would also wait for them).
// (The attribute applies to the device pass only; the host pass parses these bodies but
// never emits them.)
#if defined(__HIP_DEVICE_COMPILE__)
#define SX8_GLOBAL_AS __attribute__((address_space(1)))
#else
#define SX8_GLOBAL_AS
#endif
typedef const float4 SX8_GLOBAL_AS g_float4;
typedef const uint4 SX8_GLOBAL_AS g_uint4;
typedef const float SX8_GLOBAL_AS g_float;
typedef const uint16_t SX8_GLOBAL_AS g_u16;

template <typename T>
__device__ __forceinline__ const T SX8_GLOBAL_AS* to_global(const T* p) {
    return (const T SX8_GLOBAL_AS*)p;
}

constexpr int kPanelThreads = 512;
constexpr int kLdsMaxKb = 640;     // activation table staged in LDS up to this many K blocks

// Z of one (row, kb, j) follows the reference's warp tree: products x_t * b_t, then
// pairwise sums over lane offsets 16, 8, 4, 2, 1 (cuda/sx8_decode1_v3.cu:53-63), then
// scale * sum.
// One thread per (row m, kb): x read once as four 16-byte vectors (the row's tail past K
// is zero), then for every basis set s of `zs` both Z values (products and the reference
// tree in registers) -- one pass over X serves all matrices of a prefill group.
// Optional outputs: Z as f32 pairs or as split fp16 hi/lo pairs (hl), and the prefill
// GEMM's packed copy of X (Xp != nullptr): for each 32-row group G and block kb a 2 KB
// chunk [k-step st][MFMA lane l = 32 hf + r][8 values] holding X[32 G + r][32 kb + 16 hf +
// 8 st .. + 8], so the GEMM reads every A operand as one contiguous 1 KB wave load.  When
// packing, the grid covers the rows up to the next multiple of 32 (rows >= M pack zeros).
// kSilu: x is not read from X but produced from two float32 matrices (g, u with row
// stride ldx) as fp16(silu(g) * u) = fp16(g / (1 + exp(-g)) * u), the arithmetic of
// sx8_dec_silu_mul, so the prefill GEMM of the MLP's down projection takes the gate / up
// outputs directly.  The packing plain-x forms are held to 80 VGPRs (six waves per SIMD, no
// spills; 103 unbounded, four waves): the pass is latency-bound, and the larger grids (K =
// 9728, 2432 work-groups at M = 2048) run in fewer rounds (down at M = 2048 147.7 -> 145.2
// us per prefill call, A/B).
template <bool kZ, bool kPack, bool kSilu = false>
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(kSilu || !kPack ? 1 : 6, 8))) void k_compute_z(const uint16_t* __restrict__ X, int M,
                                                   int64_t ldx, int K, const sx8::ZSets zs,
                                                   int n_cb, bool x_vec, bool hl,
                                                   uint16_t* __restrict__ Xp,
                                                   const float* __restrict__ sg,
                                                   const float* __restrict__ su) {
#pragma clang fp contract(off)
    // 32-bit index arithmetic: the host keeps rows * n_cb below 2^31 (a 64-bit division
    // is a ~120-instruction sequence ahead of the first load)
    const int gid = (int)blockIdx.x * 256 + (int)threadIdx.x;
    const int rows = kPack ? (M + 31) / 32 * 32 : M;
    const int total = rows * n_cb;
    // packing: the row within its 32-row group runs fastest (whole 512-byte runs of packed
    // stores), so a work-group covers 8 (row group, kb) pairs and its basis rows are staged
    // once in LDS; otherwise kb runs fastest, which keeps every lane busy for the M = 1
    // callers
    __shared__ float4 bsh[kPack && kZ ? sx8::kMaxZSets : 1][8][16];
    // the X loads go out first, then the scales and the basis staging (global -> LDS ->
    // barrier), so the round trips overlap; threads past the end load a valid element and
    // stop after the barrier
    const bool live = gid < total;
    const int gq = live ? gid : total - 1;
    int m, kb;
    if constexpr (kPack) {
        const int rest = gq >> 5;
        const int grp = (int)((unsigned)rest / (unsigned)n_cb);
        kb = rest - grp * n_cb;
        m = grp * 32 + (gq & 31);
    } else {
        m = (int)((unsigned)gq / (unsigned)n_cb);
        kb = gq - m * n_cb;
    }
    const bool row_ok = m < M;
    const int kmax = row_ok ? min(32, K - kb * 32) : 0;
    // every set's two scales of this kb, requested with the X loads (the Z products below
    // would otherwise wait a round trip per set)
    // (sets past zs.n read set 0's rows, which a Z launch always has, so that no load sits
    // behind a branch; the set pointers are pinned in SGPRs, so a select between them is
    // not turned into a load from a selected argument address)
    float sc[sx8::kMaxZSets][2];
    auto set_ptr = [&](const float* const* a, int s) {
        const float* p = a[s];
        const float* p0 = a[0];
        asm volatile("" : "+s"(p), "+s"(p0));
        return to_global(s < zs.n ? p : p0);
    };
    auto load_scales = [&]() {
        if constexpr (kZ) {
#pragma unroll
            for (int s = 0; s < sx8::kMaxZSets; ++s) {
                const g_float* p = set_ptr(zs.scales, s) + kb * 2;
                sc[s][0] = p[0];
                sc[s][1] = p[1];
            }
        }
    };
    // the work-group's basis rows: 16 float4 per (set, kb) for its 8 kb, at most 512
    // float4, two per thread, both requested before either is written; a wave's 64
    // entries share one set (t >> 7)
    auto stage_basis = [&]() {
        if constexpr (kPack && kZ) {
            const int nrest = rows / 32 * n_cb;
            const int i = ((int)threadIdx.x >> 4) & 7, q = (int)threadIdx.x & 15;
            const int r = min((int)blockIdx.x * 8 + i, nrest - 1);
            const int row = (int)((unsigned)r % (unsigned)n_cb) * 64;
            const int s0 = (int)threadIdx.x >> 7, s1 = s0 + 2;
            const g_float* p0 = set_ptr(zs.basis, 0);
            const g_float* p1 = set_ptr(zs.basis, 1);
            const g_float* p2 = set_ptr(zs.basis, 2);
            const g_float* p3 = set_ptr(zs.basis, 3);
            const float4 v0 = reinterpret_cast<g_float4*>((s0 == 0 ? p0 : p1) + row)[q];
            const float4 v1 = reinterpret_cast<g_float4*>((s1 == 2 ? p2 : p3) + row)[q];
            if (s0 < zs.n) bsh[s0][i][q] = v0;
            if (s1 < zs.n) bsh[s1][i][q] = v1;
            __syncthreads();
        }
    };
    uint32_t xw[16];
    if constexpr (kSilu) {
        const int64_t off = (int64_t)min(m, M - 1) * ldx + kb * 32;
        float gv[32], uv[32];
        if (x_vec && kmax == 32) {
#pragma unroll
            for (int q = 0; q < 8; ++q) {
                const float4 a = reinterpret_cast<const float4*>(sg + off)[q];
                const float4 b = reinterpret_cast<const float4*>(su + off)[q];
                gv[4 * q] = a.x; gv[4 * q + 1] = a.y; gv[4 * q + 2] = a.z; gv[4 * q + 3] = a.w;
                uv[4 * q] = b.x; uv[4 * q + 1] = b.y; uv[4 * q + 2] = b.z; uv[4 * q + 3] = b.w;
            }
        } else {
#pragma unroll
            for (int t = 0; t < 32; ++t) {
                gv[t] = t < kmax ? sg[off + t] : 0.f;
                uv[t] = t < kmax ? su[off + t] : 0.f;
            }
        }
        load_scales();
        stage_basis();
#pragma unroll
        for (int t = 0; t < 16; ++t) {
            const float x0 = sx8_silu_mul(gv[2 * t], uv[2 * t]);
            const float x1 = sx8_silu_mul(gv[2 * t + 1], uv[2 * t + 1]);
            xw[t] = (uint32_t)__builtin_bit_cast(uint16_t, (_Float16)x0) |
                    ((uint32_t)__builtin_bit_cast(uint16_t, (_Float16)x1) << 16);
        }
    } else {
    const uint16_t* x = X + (int64_t)min(m, M - 1) * ldx + kb * 32;
    if (x_vec && kmax == 32) {
#pragma unroll
        for (int q = 0; q < 4; ++q) {
            const uint4 v = reinterpret_cast<const uint4*>(x)[q];
            xw[4 * q] = v.x; xw[4 * q + 1] = v.y; xw[4 * q + 2] = v.z; xw[4 * q + 3] = v.w;
        }
    } else {
#pragma unroll
        for (int t = 0; t < 16; ++t) {
            const uint32_t a = 2 * t < kmax ? x[2 * t] : 0u;
            const uint32_t b = 2 * t + 1 < kmax ? x[2 * t + 1] : 0u;
            xw[t] = a | (b << 16);
        }
    }
    load_scales();
    stage_basis();
    }
    if (!live) return;
    if constexpr (kPack) {
        const int G = m >> 5;
        const int r = m & 31;
#pragma unroll
        for (int hf = 0; hf < 2; ++hf)
#pragma unroll
            for (int st = 0; st < 2; ++st) {
                uint4* dst = reinterpret_cast<uint4*>(Xp + (((int64_t)G * n_cb + kb) * 2 + st) * 512 + (hf * 32 + r) * 8);
                const int q = 8 * hf + 4 * st;
                *dst = make_uint4(xw[q], xw[q + 1], xw[q + 2], xw[q + 3]);
            }
    }
    if constexpr (kZ) {
        if (!row_ok) return;
        const int64_t zi = (int64_t)m * n_cb + kb;
        auto xf = [&](int t) { return sx8_h2f(xw[t >> 1] >> (16 * (t & 1))); };
#pragma unroll
        for (int s = 0; s < sx8::kMaxZSets; ++s) {
            if (s >= zs.n) break;
            const float4* bv = kPack ? &bsh[s][threadIdx.x >> 5][0]
                                     : reinterpret_cast<const float4*>(zs.basis[s] + kb * 64);
            float z[2];
#pragma unroll
            for (int j = 0; j < 2; ++j) {
                // products x_t * b_t, then the tree: level 16 as each pair (t, t + 16)
                // arrives (float4 q and q + 4), then offsets 8, 4, 2, 1
                float p[16];
#pragma unroll
                for (int q = 0; q < 4; ++q) {
                    const float4 lo = bv[8 * j + q], hi = bv[8 * j + q + 4];
                    p[4 * q] = xf(4 * q) * lo.x + xf(4 * q + 16) * hi.x;
                    p[4 * q + 1] = xf(4 * q + 1) * lo.y + xf(4 * q + 17) * hi.y;
                    p[4 * q + 2] = xf(4 * q + 2) * lo.z + xf(4 * q + 18) * hi.z;
                    p[4 * q + 3] = xf(4 * q + 3) * lo.w + xf(4 * q + 19) * hi.w;
                }
#pragma unroll
                for (int off = 8; off > 0; off >>= 1)
#pragma unroll
                    for (int t = 0; t < off; ++t) p[t] = p[t] + p[t + off];
                z[j] = sc[s][j] * p[0];
            }
            float* Z = zs.Z[s];
            if (hl)
                *reinterpret_cast<uint2*>(Z + zi * 2) = make_uint2(sx8_split_hl(z[0]), sx8_split_hl(z[1]));
            else
                *reinterpret_cast<float2*>(Z + zi * 2) = make_float2(z[0], z[1]);
        }
    }
}

// Activation-side table, one 32-lane group per kb (8 kb per 256-thread block).
// Lane t: product x_t * b_jt for j = 0, 1 and the xor tree (bit-identical Z); lanes
// 0..3 build the x side of one sub-block each.  Used when the caller asks for Z back.
template <bool kZGiven>
__global__ __launch_bounds__(256) void k_kbinfo(const uint16_t* __restrict__ X,
                                                const float* __restrict__ basis,
                                                const float* __restrict__ scales,
                                                const float* __restrict__ Zin,
                                                float* __restrict__ Zout, int n_cb,
                                                KbInfo* __restrict__ table) {
#pragma clang fp contract(off)
    const int t = threadIdx.x & 31;
    const int kb = blockIdx.x * 8 + (threadIdx.x >> 5);
    const bool ok = kb < n_cb;                      // uniform across the 32-lane group
    const int kbc = ok ? kb : n_cb - 1;
    const uint16_t* x = X + (int64_t)kbc * 32;
    KbInfo& out = table[kbc];
    if constexpr (kZGiven) {
        if (ok && t < 2) out.z[t] = Zin[(int64_t)kb * 2 + t];
    } else {
        float p0 = sx8_h2f(x[t]) * basis[(int64_t)kbc * 64 + t];
        float p1 = sx8_h2f(x[t]) * basis[(int64_t)kbc * 64 + 32 + t];
#pragma unroll
        for (int off = 16; off > 0; off >>= 1) {
            p0 = p0 + __shfl_xor(p0, off, 32);
            p1 = p1 + __shfl_xor(p1, off, 32);
        }
        if (ok && t == 0) {
            const float z0 = scales[(int64_t)kb * 2] * p0;
            const float z1 = scales[(int64_t)kb * 2 + 1] * p1;
            out.z[0] = z0;
            out.z[1] = z1;
            if (Zout) {
                Zout[(int64_t)kb * 2] = z0;
                Zout[(int64_t)kb * 2 + 1] = z1;
            }
        }
    }
    if (!ok) return;
    if (t < 4) fill_x_side(out, t, *reinterpret_cast<const uint4*>(x + 8 * t));
    else if (t < 6) out.pad[t - 4] = 0.f;
}

// Loop-invariant masks and byte selectors held in VGPRs: on gfx9 a VOP3 instruction
// takes at most one scalar operand, so with the fp16 constants in SGPRs each splice
// below is a single v_and_or_b32 and each quad spread a single v_perm_b32.
struct SpliceK {
    uint32_t n_lo, n_hi, q0, q1, q2, q3, sel_even, sel_odd;
};

__device__ __forceinline__ SpliceK splice_consts() {
    SpliceK k{0x000F000Fu, 0x00F000F0u, 0x00C000C0u, 0x00300030u,
              0x000C000Cu, 0x00030003u, 0x0C010C00u, 0x0C030C02u};
    asm volatile("" : "+v"(k.n_lo), "+v"(k.n_hi), "+v"(k.q0), "+v"(k.q1));
    asm volatile("" : "+v"(k.q2), "+v"(k.q3), "+v"(k.sel_even), "+v"(k.sel_odd));
    return k;
}

// One block's raw records: lohi = dmin | dmax << 16, cc = config | coeff << 8, then the
// 16 hi-nibble bytes (a) and the 8 lo-quad bytes (b).
struct BlockRec {
    uint32_t lohi, cc;
    unsigned short cc16;   // 6-byte headers: cc as loaded, widened at its first use
    uint4 a;
    uint2 b;
};

// Records of block `bid` through buffer loads (header at bid * HB, levels at bid * 24);
// an offset past the end of a buffer reads zeros and moves no data.  The 6-byte header
// is read as a dword (possibly 2-byte aligned; buffer loads allow it) and a short.
template <int HB>
__device__ __forceinline__ void load_rec(BlockRec& o, sx8_rsrc hdr, sx8_rsrc lv, uint32_t bid) {
    if constexpr (HB == 8) {
        const uint2 h = __builtin_bit_cast(uint2, __builtin_amdgcn_raw_buffer_load_b64(hdr, bid * 8, 0, 0));
        o.lohi = h.x;
        o.cc = h.y;
    } else {
        o.lohi = __builtin_amdgcn_raw_buffer_load_b32(hdr, bid * 6, 0, 0);
        o.cc16 = __builtin_amdgcn_raw_buffer_load_b16(hdr, bid * 6 + 4, 0, 0);
    }
    o.a = __builtin_bit_cast(uint4, __builtin_amdgcn_raw_buffer_load_b128(lv, bid * 24, 0, 0));
    o.b = __builtin_bit_cast(uint2, __builtin_amdgcn_raw_buffer_load_b64(lv, bid * 24 + 16, 0, 0));
}

// fp32 contribution of one block (one column, one kb) to its output: PCA through Z,
// then per 8-weight sub-block rlo * Sx + step * sum_i x_i lv_i.
//
// sum_i x_i lv_i (lv = 4 nib + quad) comes from fp16 "splices": a field is or-ed into
// the mantissa of an fp16 constant whose last mantissa bit is worth the field's
// weight in lv, e.g. (H & 0x000F000F) | 0x6C006C00 = (4096 + 4 nib_0, 4096 + 4 nib_4)
// (exponent 12: ulp 4).  Nibble pairs use 4096/256/4096/256 (bits 0/4 of H and of
// H >> 8), quad pairs 16/64/256/1024 (bits 6/4/2/0 of each spread lo byte).  Eight
// v_dot2_f32_f16 per sub-block multiply the splices by x pairs into one fp32 sum t that
// starts at -sum x * constants (the table's nbias), leaving sum x lv.  Every spliced
// value is exact in fp16.
//
// Range parameters follow the reference's float32 form (cuda/sx8_decode1_v3.cu:108-117):
// rlo = lo + q k1[s] with q = (hi - lo) / 4, k1 = {0, 0, 3, 1}, and
// step = max(0.015873 (rhi - rlo), 1e-10) where rhi - rlo = (hi - lo) * {1, 1/4, 1/4, 1/2}.
// For hi > lo the floor never binds (an fp16 range is at least 2^-24, so step >= 2.4e-10)
// and step = m 2^e[s] with m = 0.015873 (hi - lo); for hi <= lo every sub-block's
// range is <= 0, so step = 1e-10 throughout (m = 1e-10, e = 0); NaN endpoints make rlo
// NaN as in the reference.  The four strategies are moved into the bytes of `sel` so
// that one v_perm_b32 per table looks k1 and e up for all sub-blocks at once.
__device__ __forceinline__ float block_dot_z(const BlockRec& o, const KbInfo& ki, float z0, float z1,
                                             const SpliceK& k) {
    const float lo = sx8_h2f(o.lohi), hi = sx8_h2f(o.lohi >> 16);
    const float d = hi - lo;
    const float q = d * 0.25f;
    const uint32_t cfg = o.cc & 0xFFu;
    uint32_t sel = (cfg << 6) | cfg;                  // strategy of sub-block sb -> bits 8sb
    sel = ((sel << 12) | sel) & 0x03030303u;
    const uint32_t k1b = __builtin_amdgcn_perm(0u, 0x01030000u, sel);                 // k1[s]
    const uint32_t eb = d > 0.f ? __builtin_amdgcn_perm(0u, 0xFFFEFE00u, sel) : 0u;  // e[s]
    const float m = d > 0.f ? d * 0.015873f : 1e-10f;
    const uint32_t cf = o.cc >> 8;
    float acc = (float)sx8_sext4(cf) * z0 + (float)sx8_sext4(cf >> 4) * z1;
    float T = 0.f;
    const uint32_t H[4] = {o.a.x, o.a.y, o.a.z, o.a.w};
#pragma unroll
    for (int sb = 0; sb < 4; ++sb) {
        const float rlo = __builtin_fmaf(q, (float)((k1b >> (8 * sb)) & 0xFFu), lo);
        const uint32_t h = H[sb];
        const uint32_t h8 = h >> 8;
        const uint32_t P = __builtin_amdgcn_perm(0u, (sb >> 1) ? o.b.y : o.b.x,
                                                 (sb & 1) ? k.sel_odd : k.sel_even);
        const uint32_t* xp = ki.xp + 4 * sb;
        float t = dot2((h & k.n_lo) | 0x6C006C00u, xp[0], ki.nbias[sb]);
        t = dot2((h & k.n_hi) | 0x5C005C00u, xp[1], t);
        t = dot2((h8 & k.n_lo) | 0x6C006C00u, xp[2], t);
        t = dot2((h8 & k.n_hi) | 0x5C005C00u, xp[3], t);
        t = dot2((P & k.q0) | 0x4C004C00u, xp[0], t);
        t = dot2((P & k.q1) | 0x54005400u, xp[1], t);
        t = dot2((P & k.q2) | 0x5C005C00u, xp[2], t);
        t = dot2((P & k.q3) | 0x64006400u, xp[3], t);
        acc = __builtin_fmaf(rlo, ki.sx[sb], acc);
        T += __builtin_ldexpf(t, __builtin_amdgcn_sbfe((int)eb, 8 * sb, 8));
    }
    return __builtin_fmaf(m, T, acc);
}

__device__ __forceinline__ float block_dot(const BlockRec& o, const KbInfo& ki, const SpliceK& k) {
    return block_dot_z(o, ki, ki.z[0], ki.z[1], k);
}

// v + (v of another lane), the lane picked by a DPP control (quad_perm, row mirrors).
template <int kCtrl>
__device__ __forceinline__ float dpp_add(float v) {
    return v + __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), kCtrl,
                                                                      0xF, 0xF, false));
}

// Table entries built inside the GEMV work-group: four threads per kb, thread q holding
// sub-block q's 8 x values and the matching 8 + 8 basis values.  Z is a quarter dot per
// thread summed over the four threads with two DPP exchanges (this Z is only used
// internally; the combined entry point's Z comes from k_kbinfo).
struct TabIn {
    uint4 x;
    float4 b0[2], b1[2];
    float s;
};

template <int kMode, bool kLoadX = true>
__device__ __forceinline__ void tab_load(TabIn& t, const g_u16* __restrict__ X,
                                         const g_float* __restrict__ basis,
                                         const g_float* __restrict__ scales,
                                         const g_float* __restrict__ Zin, int kb, int q) {
    if constexpr (kLoadX) t.x = *(const g_uint4*)(X + (int64_t)kb * 32 + 8 * q);
    if constexpr (kMode == 1) {
        const g_float4* b = (const g_float4*)(basis + (int64_t)kb * 64 + 8 * q);
        t.b0[0] = b[0];
        t.b0[1] = b[1];
        t.b1[0] = b[8];
        t.b1[1] = b[9];
        t.s = scales[2 * kb + (q & 1)];
    } else if constexpr (kMode == 4) {
        // Z from two partial sums per K block and basis (laid out [kb][slot][basis], in
        // the basis argument), then the scale: Z = (P0 + P1) * scale
        const int c = q & 1;
        t.s = (basis[(int64_t)kb * 4 + c] + basis[(int64_t)kb * 4 + 2 + c]) * scales[2 * kb + c];
    } else {
        t.s = Zin[2 * kb + (q & 1)];
    }
}

// Z value (q & 1) of the unit's K block from its x and basis quarters: each of the four
// threads of a kb dots its 8 x values with 8 + 8 basis values, two DPP exchanges sum the
// quarters, and t.s (the scale of basis q & 1) scales the sum.
__device__ __forceinline__ float tab_z(const TabIn& t, int q) {
    const uint32_t xw[4] = {t.x.x, t.x.y, t.x.z, t.x.w};
    const float* b0 = reinterpret_cast<const float*>(t.b0);
    const float* b1 = reinterpret_cast<const float*>(t.b1);
    float z0 = 0.f, z1 = 0.f;
#pragma unroll
    for (int i = 0; i < 8; ++i) {
        const float xf = sx8_h2f(xw[i >> 1] >> (16 * (i & 1)));
        z0 = __builtin_fmaf(xf, b0[i], z0);
        z1 = __builtin_fmaf(xf, b1[i], z1);
    }
    z0 = dpp_add<0xB1>(z0);      // + lane ^ 1
    z1 = dpp_add<0xB1>(z1);
    z0 = dpp_add<0x4E>(z0);      // + lane ^ 2
    z1 = dpp_add<0x4E>(z1);
    return t.s * ((q & 1) == 0 ? z0 : z1);
}

// Writes entry kb, or the spare entry past the table when !ok: no branch, so the compiler
// has no conditional block to sink the table loads into (below the weight records).
template <int kMode>
__device__ __forceinline__ void tab_store(KbInfo* info, const TabIn& t, int kb, int q, bool ok,
                                          int n_cb) {
    KbInfo& e = info[ok ? kb : n_cb];
    fill_x_side(e, q, t.x);
    e.z[q & 1] = kMode == 1 ? tab_z(t, q) : t.s;   // q = 2, 3 write the same values as q = 0, 1
}

// Input producers of the decoder's fused GEMVs: instead of reading x as fp16, every
// work-group computes it in its table build from the decoder state (K = n_cb * 32).
//   kXRms:  h = (init ? fp16 init : resid) + (delta ? delta : 0) in f32,
//           x = fp16(h * (1 / sqrt(sum(h^2) / K + eps)) * w); work-group 0 also stores h to
//           resid_out (the next residual; it must not alias resid or delta, which the other
//           work-groups are still reading).
//   kXSilu: x = fp16(silu(g) * u) = fp16(g / (1 + exp(-g)) * u).
constexpr int kXPlain = 0, kXRms = 1, kXSilu = 2;
struct XProd {
    const float* resid;
    const uint16_t* init;
    const float* delta;
    const uint16_t* w;
    float* resid_out;
    const float* g;
    const float* u;
    float eps;
    uint32_t* amax;   // kXRms, one matrix: per panel (max bits, first index of the max), or null
};

// Raw producer inputs of one table unit (kb, q): 8 consecutive elements 32 kb + 8 q.
// Loaded with buffer loads over resources whose size is zero for an absent input (init,
// resid or delta), so the loads are unconditional, read zeros for absent inputs and keep
// their issue order (the table inputs must all be requested before the weight records).
struct XRaw {
    float4 a0, a1;   // kXRms: resid, kXSilu: g
    float4 b0, b1;   // kXRms: delta, kXSilu: u
    uint4 h16;       // kXRms: init fp16
    uint4 w;         // kXRms: norm weight fp16
};

struct XRsrc {
    sx8_rsrc a, b, h16, w;
};

template <int kX>
__device__ __forceinline__ XRsrc xraw_rsrc(const XProd& xp, int K) {
    XRsrc r;
    if constexpr (kX == kXRms) {
        r.a = make_rsrc(xp.resid, xp.resid ? (int64_t)K * 4 : 0);
        r.b = make_rsrc(xp.delta, xp.delta ? (int64_t)K * 4 : 0);
        r.h16 = make_rsrc(xp.init, xp.init ? (int64_t)K * 2 : 0);
        r.w = make_rsrc(xp.w, (int64_t)K * 2);
    } else {
        r.a = make_rsrc(xp.g, (int64_t)K * 4);
        r.b = make_rsrc(xp.u, (int64_t)K * 4);
    }
    return r;
}

// The same from the preloaded argument slots (kPre): kXRms reads h = resid (no init, no
// delta) from the x slot and the norm weight from the header slot; kXSilu reads g from the
// x slot and u from g + K (the two vectors adjacent in memory).
template <int kX>
__device__ __forceinline__ XRsrc xraw_rsrc_pre(const void* xs, const void* hs, int K) {
    XRsrc r;
    if constexpr (kX == kXRms) {
        r.a = make_rsrc(xs, (int64_t)K * 4);
        r.b = make_rsrc(nullptr, 0);
        r.h16 = make_rsrc(nullptr, 0);
        r.w = make_rsrc(hs, (int64_t)K * 2);
    } else {
        r.a = make_rsrc(xs, (int64_t)K * 4);
        r.b = make_rsrc(static_cast<const float*>(xs) + K, (int64_t)K * 4);
    }
    return r;
}

__device__ __forceinline__ float4 ld_f4(sx8_rsrc r, uint32_t off) {
    return __builtin_bit_cast(float4, __builtin_amdgcn_raw_buffer_load_b128(r, off, 0, 0));
}

template <int kX, bool kPre = false>
__device__ __forceinline__ void xraw_load(XRaw& r, const XRsrc& rs, int kb, int q) {
    const uint32_t e = (uint32_t)(kb * 32 + 8 * q);
    r.a0 = ld_f4(rs.a, e * 4);
    r.a1 = ld_f4(rs.a, e * 4 + 16);
    if (kX == kXRms && kPre) {           // no delta, no init
        r.b0 = r.b1 = make_float4(0.f, 0.f, 0.f, 0.f);
        r.h16 = make_uint4(0u, 0u, 0u, 0u);
    } else {
        r.b0 = ld_f4(rs.b, e * 4);
        r.b1 = ld_f4(rs.b, e * 4 + 16);
        if constexpr (kX == kXRms)
            r.h16 = __builtin_bit_cast(uint4, __builtin_amdgcn_raw_buffer_load_b128(rs.h16, e * 2, 0, 0));
    }
    if constexpr (kX == kXRms)
        r.w = __builtin_bit_cast(uint4, __builtin_amdgcn_raw_buffer_load_b128(rs.w, e * 2, 0, 0));
}

__device__ __forceinline__ uint32_t pack_h2(float lo, float hi) {
    return (uint32_t)__builtin_bit_cast(uint16_t, (_Float16)lo) |
           ((uint32_t)__builtin_bit_cast(uint16_t, (_Float16)hi) << 16);
}

// Sum over a wave64 in a fixed order: DPP butterflies within each row of 16 lanes, then the
// four row sums (lanes 0, 16, 32, 48) in order.  Uniform result.
__device__ __forceinline__ float wave_sum(float v) {
    v = dpp_add<0xB1>(v);    // quad_perm [1, 0, 3, 2]
    v = dpp_add<0x4E>(v);    // quad_perm [2, 3, 0, 1]
    v = dpp_add<0x141>(v);   // row_half_mirror
    v = dpp_add<0x140>(v);   // row_mirror
    const float r0 = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), 0));
    const float r1 = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), 16));
    const float r2 = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), 32));
    const float r3 = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), 48));
    return ((r0 + r1) + r2) + r3;
}

// The 8 residual values h of a unit (kXRms): (init + resid) + delta, one of init and resid
// absent (zero), delta possibly absent (zero).
__device__ __forceinline__ void xraw_h(const XRaw& r, float h[8]) {
    const float a[8] = {r.a0.x, r.a0.y, r.a0.z, r.a0.w, r.a1.x, r.a1.y, r.a1.z, r.a1.w};
    const float d[8] = {r.b0.x, r.b0.y, r.b0.z, r.b0.w, r.b1.x, r.b1.y, r.b1.z, r.b1.w};
    const uint32_t hw[4] = {r.h16.x, r.h16.y, r.h16.z, r.h16.w};
#pragma unroll
    for (int i = 0; i < 8; ++i) h[i] = (sx8_h2f(hw[i >> 1] >> (16 * (i & 1))) + a[i]) + d[i];
}

// RMSNorm scale of the work-group's h (every unit within the TP passes): h per unit, the
// sum of h^2 over the work-group in a fixed order (so every work-group gets the same
// value), 1 / sqrt(mean + eps).  One s_barrier; the LDS-only wait leaves the records in
// flight.  red[0 .. 8) is used.
template <int TP>
__device__ __forceinline__ float rms_inv(const XRaw (&xr)[TP], float (&h)[TP][8], float* red, int n_units,
                                         int K, float eps, int tid) {
    float ss = 0.f;
#pragma unroll
    for (int p = 0; p < TP; ++p) {
        xraw_h(xr[p], h[p]);
        if (p * kPanelThreads + tid < n_units) {
#pragma unroll
            for (int i = 0; i < 8; ++i) ss = __builtin_fmaf(h[p][i], h[p][i], ss);
        }
    }
    ss = wave_sum(ss);
    if ((tid & 63) == 0) red[tid >> 6] = ss;
    __builtin_amdgcn_s_waitcnt(0xC07F);       // lgkmcnt(0): LDS only, records stay in flight
    asm volatile("s_barrier" ::: "memory");
    float tot = 0.f;
#pragma unroll
    for (int wv = 0; wv < kPanelThreads / 64; ++wv) tot += red[wv];
    return 1.0f / sqrtf(tot / (float)K + eps);
}

// x = fp16(h * inv * w) of one unit, as fp16 pairs
__device__ __forceinline__ uint4 rms_x(const float (&h)[8], const uint4 w, float inv) {
    const uint32_t ww[4] = {w.x, w.y, w.z, w.w};
    uint32_t xw[4];
#pragma unroll
    for (int i = 0; i < 4; ++i)
        xw[i] = pack_h2(h[2 * i] * inv * sx8_h2f(ww[i]), h[2 * i + 1] * inv * sx8_h2f(ww[i] >> 16));
    return make_uint4(xw[0], xw[1], xw[2], xw[3]);
}

// Table passes whose inputs are loaded before the weight records (the rest, for
// n_cb > kTabPasses * 128, load after them).
constexpr int kTabPassesShort = 1;   // n_cb <= 128
constexpr int kTabPassesLong = 3;    // n_cb <= 384

// M = 1 GEMV over column panels.  A 512-thread work-group owns CT consecutive columns
// over the whole K: lane tid = (slice j = tid / CT, column c = tid % CT), so for each kb
// the CT lanes of a slice read CT consecutive records, and slice j walks kb = j + r S
// (S = 512 / CT slices, rounds r < R = ceil(n_cb / S)); the 512 - S CT leftover lanes
// only take part in the table build and the reduction.  The host picks CT so that the
// grid is about one work-group per CU.  Slices meet in LDS and are summed in a fixed
// order: nothing leaves a work-group before the final store, so there are no
// device-scope fences or atomics and results are deterministic.
//
// Latency schedule: the table inputs go out first, then the records of the first NR
// rounds, then the table is built while they stream in.  The buffers form a ring: the
// one just decoded is refilled with the round NR ahead.  Loads are unconditional buffer
// loads; rounds and slices past
// the end of K have offsets past the end of the buffers and read zeros without memory
// traffic, and their contributions are masked, so the decode loop is straight-line code
// (exact memory-wait counts) with scheduling barriers keeping each refill ahead of the
// decode after it.
//
// kMode: 0 = copy the table k_kbinfo wrote into LDS; 1 = build it computing Z; 2 = build
// it with Z from Zin; 3 = read k_kbinfo's table from global memory (n_cb > kLdsMaxKb);
// 4 = build it with Z from two partial sums per K block (in the basis argument) and the
// scales (the down projection after k_gemv_pair).
// Work-groups go to the 8 XCDs round-robin by block index; panels are renumbered so each
// XCD gets a contiguous column range and neighbouring panels share cache lines in one L2.
// Weight matrices of one launch: every matrix multiplies the same x (same K); matrix m
// owns `panels` consecutive panels of the grid.
constexpr int kMaxGroup = 4;
struct GemvMat {
    const uint8_t* hdr;
    const uint8_t* levels;
    const float* basis;
    const float* scales;
    const float* Zin;
    float* Y;
    const float* add;   // Y = add + W x when set (may be Y itself: the residual updated in place)
    int N, panels;
};
struct GemvGroup {
    GemvMat m[kMaxGroup];
    int n_mats;
    int ct;   // panel width of a group launch (plan_panels)
};

// Panel width for a launch over `total` output columns: about one work-group per CU
// (ceil(total / 256) columns), two per CU past 64 columns, and 128 columns (4 slices, no
// idle lanes) past 65536, where that still leaves two or more work-groups per CU and
// halves the number of table builds (vocab-sized matrices; host and device share it).
// Measured on the 151936 x 2560 lm_head (timed regions of 50 back-to-back launches, same
// box): the RMSNorm + argmax-partials form 69.8-70.9 us against 72.4-72.7 us with 64
// columns (half the norms and partials), the plain GEMV 65.0-66.0 against 65.5-67.6 us;
// widths 96 and 160 (idle lanes) and 256 (too few work-groups) were slower than 64.
constexpr int kMaxPanelCt = 128;
static_assert(kPanelThreads % kMaxPanelCt == 0, "a 128-column panel has whole slices");
__host__ __device__ inline int panel_ct(int64_t total) {
    if (total > 65536) return kMaxPanelCt;
    int64_t ct = (total + 255) / 256;
    if (ct > 64) ct = (total + 511) / 512;
    return (int)(ct < 1 ? 1 : ct > 64 ? 64 : ct);
}

// Arguments: the fields a single-matrix launch needs first (hdr, levels, X, N, n_cb) lead,
// then its bases, scales and output; this file is built with the first 8 kernel arguments
// preloaded into SGPRs, so those arrive with the wave instead of after a scalar-memory
// round trip.  kOne (a single matrix) takes its fields and derives CT, S, R from them;
// a group (n_mats > 1) reads its matrices from `grp` and CT, S, R from the arguments.
// (Measured and rejected: building Z after the K loop, with the bases requested behind
// the first record rounds and each lane's coefficients kept for a PCA pass before the
// reduction -- 8% slower on the layer sweep; the epilogue it adds costs more than the
// prologue it shortens.)
// kPre: the producer's inputs sit in the argument slots that arrive preloaded (see
// xraw_rsrc_pre): a group's header slot is free (its matrices come from grp), so a
// grouped RMSNorm takes h and the norm weight from there; a single-matrix SiLU takes g
// (u = g + K).  kResY (single matrix): Y = Y + W x, the residual read from the preloaded
// output slot right after the first records are requested (not at the end, where a load
// would add a memory round trip to every work-group's finish).
template <int HB, int kMode, int NR, int TP, int kX = kXPlain, bool kOne = false, bool kPre = false,
          bool kResY = false>
__global__ __launch_bounds__(kPanelThreads) void k_gemv_panel(
    const uint8_t* __restrict__ hdr0, const uint8_t* __restrict__ lv0, const uint16_t* __restrict__ X,
    int N0, int n_cb, const float* __restrict__ bas0, const float* __restrict__ sca0,
    float* __restrict__ Y0, const GemvGroup grp,
    const KbInfo* __restrict__ table, const XProd xp) {
    extern __shared__ __align__(16) unsigned char smem[];
    float* red = reinterpret_cast<float*>(smem);                 // 2 x 512 floats
    KbInfo* info = reinterpret_cast<KbInfo*>(smem + sizeof(float) * 2 * kPanelThreads);
    const int tid = threadIdx.x;
    // The producer's inputs go out before anything else: with kPre they need no argument
    // load (a group's matrix fields are a memory round trip away).
    XRaw xr[kX == kXPlain ? 1 : TP];
    constexpr bool kBuild = kMode == 1 || kMode == 2 || kMode == 4;   // table built in-kernel
    if constexpr (kBuild && kX != kXPlain) {
        XRsrc xs;
        if constexpr (kPre) xs = xraw_rsrc_pre<kX>(X, hdr0, n_cb * 32);
        else xs = xraw_rsrc<kX>(xp, n_cb * 32);
#pragma unroll
        for (int p = 0; p < TP; ++p) {
            const int u = min(p * kPanelThreads + tid, n_cb * 4 - 1);
            xraw_load<kX, kPre>(xr[p], xs, u >> 2, u & 3);
        }
        asm volatile("" ::: "memory");
    }
    // panel number: XCD x (= blockIdx % 8) gets the contiguous range after the
    // sum_{y < x} ceil((G - y) / 8) panels of the XCDs before it (G = 8 q + r)
    const int xcd = blockIdx.x & 7;
    auto panel_of = [&](int G) { return (int)(blockIdx.x >> 3) + xcd * (G >> 3) + min(xcd, G & 7); };
    // a group's matrix for this panel; every field is read at a fixed kernel-argument
    // offset and picked with uniform selects, without branches, so the argument loads go
    // out together (no chain of dependent loads).  A group's grid is its panel count, so
    // the matrix is known before any division.
    int panel = 0, mi = 0;
    if constexpr (!kOne) {
        panel = panel_of((int)gridDim.x);
        const int nm = grp.n_mats;
        const int e0 = grp.m[0].panels, e1 = e0 + grp.m[1].panels, e2 = e1 + grp.m[2].panels;
        mi = (nm > 1 && panel >= e0) + (nm > 2 && panel >= e1) + (nm > 3 && panel >= e2);
        panel -= mi == 0 ? 0 : mi == 1 ? e0 : mi == 2 ? e1 : e2;
    }
    // field of the group's matrix mi: the four candidates are loaded (pinned in SGPRs, so
    // the compiler cannot turn the select into a load from a selected address) and picked
    auto pick = [&](auto field) {
        auto f0 = field(grp.m[0]), f1 = field(grp.m[1]), f2 = field(grp.m[2]), f3 = field(grp.m[3]);
        asm volatile("" : "+s"(f0), "+s"(f1), "+s"(f2), "+s"(f3));
        return mi == 0 ? f0 : mi == 1 ? f1 : mi == 2 ? f2 : f3;
    };
    const g_float* __restrict__ basis = to_global(kOne ? bas0 : pick([](const GemvMat& g) { return g.basis; }));
    const g_float* __restrict__ scales = to_global(kOne ? sca0 : pick([](const GemvMat& g) { return g.scales; }));
    // (a single matrix's Z arrives in the preloaded basis slot)
    const g_float* __restrict__ Zin = to_global(
        kMode != 2 ? nullptr : kOne ? bas0 : pick([](const GemvMat& g) { return g.Zin; }));
    // (X laundered through an empty asm: a load from the read-only argument itself could be
    // moved past the ordering point below, behind the divisions)
    const uint16_t* xa = X;
    asm volatile("" : "+s"(xa));
    const g_u16* __restrict__ Xg = to_global(xa);

    // The table inputs go out first, ahead of the panel geometry (integer divisions) and
    // the weight records: the table build gates the first decode, and its inputs depend
    // on nothing but the thread index and n_cb (6% on the layer sweep against issuing
    // them after the geometry).
    const int n_units = n_cb * 4;
    TabIn tin[TP];
    if constexpr (kBuild) {
#pragma unroll
        for (int p = 0; p < TP; ++p) {
            const int u = min(p * kPanelThreads + tid, n_units - 1);
            tab_load<kMode, kX == kXPlain>(tin[p], Xg, basis, scales, Zin, u >> 2, u & 3);
        }
    }
    // issue order = wait order (the memory counter retires loads in order): table
    // inputs, then round 0, 1, ...  (the clobber keeps the compiler from sinking a
    // table load below the geometry or the record loads, which would make the table
    // wait for them)
    asm volatile("" ::: "memory");
    __builtin_amdgcn_sched_barrier(0);

    // panel geometry: a single matrix derives it from N (as the host's plan_panels does; N
    // passes through an empty asm so that the divisions below cannot be hoisted above the
    // table loads), a group reads it with its matrix fields
    int n_one = N0;
    asm volatile("" : "+s"(n_one));
    const int CT = kOne ? panel_ct(n_one) : grp.ct;
    const int S = kPanelThreads / CT;
    const int R = (n_cb + S - 1) / S;
    const int j0 = tid / CT;
    const int c = tid - j0 * CT;
    // a single matrix's grid is its panel count (gridDim would be another argument load)
    if constexpr (kOne) panel = panel_of((N0 + CT - 1) / CT);
    const uint8_t* __restrict__ hdr = kOne ? hdr0 : pick([](const GemvMat& g) { return g.hdr; });
    const uint8_t* __restrict__ levels = kOne ? lv0 : pick([](const GemvMat& g) { return g.levels; });
    float* __restrict__ Y = kOne ? Y0 : pick([](const GemvMat& g) { return g.Y; });
    const int N = kOne ? N0 : pick([](const GemvMat& g) { return g.N; });
    const int n = panel * CT + c;
    const bool col_ok = n < N;
    const uint32_t nn = (uint32_t)min(n, N - 1);
    const bool lane_ok = j0 < S;
    const int j = lane_ok ? j0 : n_cb;           // leftover lanes: past the end of K
    const uint32_t n_blk = (uint32_t)n_cb * (uint32_t)N;
    const sx8_rsrc rh = make_rsrc(hdr, (int64_t)n_blk * HB);
    const sx8_rsrc rl = make_rsrc(levels, (int64_t)n_blk * 24);
    // block index of round r: (j + r S) N + nn < (n_cb + (NR + 1) S) N < 2^31 / 24
    // (checked by the host); leftover lanes stay at n_blk, the first block past the end
    const uint32_t bid0 = lane_ok ? (uint32_t)j * (uint32_t)N + nn : n_blk;
    const uint32_t dbid = lane_ok ? (uint32_t)S * (uint32_t)N : 0u;
    auto load = [&](BlockRec& o, int r) { load_rec<HB>(o, rh, rl, bid0 + (uint32_t)r * dbid); };

    // the first kNR0 rounds go out before the table build, the rest of the ring after it
    constexpr int kNR0 = NR < 2 ? NR : 2;
    BlockRec buf[NR];
#pragma unroll
    for (int i = 0; i < kNR0; ++i) {
        load(buf[i], i);
        __builtin_amdgcn_sched_barrier(0);
    }
    float yres = 0.f;                        // kResY: this column's residual, read early
    if constexpr (kResY) {
        if (tid < CT && col_ok) yres = *(const g_float*)(Y0 + n);
    }
    if constexpr (kMode == 0) {
        const uint4* src = reinterpret_cast<const uint4*>(table);
        uint4* dst = reinterpret_cast<uint4*>(info);
        for (int i = tid; i < n_cb * 7; i += kPanelThreads) dst[i] = src[i];
    } else if constexpr (kBuild) {
        if constexpr (kX == kXRms) {
            // every unit fits the TP passes (checked by the host): sum h^2 over the
            // work-group, then normalize; the sum's order is fixed, so every work-group
            // produces the same x
            float h[TP][8];
            const float inv = rms_inv<TP>(xr, h, red, n_units, n_cb * 32, xp.eps, tid);
            const bool writer = !kPre && blockIdx.x == 0 && xp.resid_out != nullptr;
#pragma unroll
            for (int p = 0; p < TP; ++p) {
                tin[p].x = rms_x(h[p], xr[p].w, inv);
                const int u = p * kPanelThreads + tid;
                if (writer && u < n_units) {
                    float4* ro = reinterpret_cast<float4*>(xp.resid_out + (int64_t)u * 8);
                    ro[0] = make_float4(h[p][0], h[p][1], h[p][2], h[p][3]);
                    ro[1] = make_float4(h[p][4], h[p][5], h[p][6], h[p][7]);
                }
            }
        } else if constexpr (kX == kXSilu) {
#pragma unroll
            for (int p = 0; p < TP; ++p) {
                const float g8[8] = {xr[p].a0.x, xr[p].a0.y, xr[p].a0.z, xr[p].a0.w,
                                     xr[p].a1.x, xr[p].a1.y, xr[p].a1.z, xr[p].a1.w};
                const float u8[8] = {xr[p].b0.x, xr[p].b0.y, xr[p].b0.z, xr[p].b0.w,
                                     xr[p].b1.x, xr[p].b1.y, xr[p].b1.z, xr[p].b1.w};
                uint32_t xw[4];
#pragma unroll
                for (int i = 0; i < 4; ++i)
                    xw[i] = pack_h2(sx8_silu_mul(g8[2 * i], u8[2 * i]), sx8_silu_mul(g8[2 * i + 1], u8[2 * i + 1]));
                tin[p].x = make_uint4(xw[0], xw[1], xw[2], xw[3]);
            }
        }
#pragma unroll
        for (int p = 0; p < TP; ++p) {
            const int u = p * kPanelThreads + tid;
            tab_store<kMode>(info, tin[p], min(u, n_units - 1) >> 2, u & 3, u < n_units, n_cb);
        }
        if constexpr (kX == kXPlain) {
            for (int u0 = TP * kPanelThreads; u0 < n_units; u0 += kPanelThreads) {
                const int u = min(u0 + tid, n_units - 1);
                tab_load<kMode>(tin[0], Xg, basis, scales, Zin, u >> 2, u & 3);
                tab_store<kMode>(info, tin[0], u >> 2, u & 3, u0 + tid < n_units, n_cb);
            }
        }
    }
    __syncthreads();
#pragma unroll
    for (int i = kNR0; i < NR; ++i) load(buf[i], i);

    const KbInfo* ti = kMode == 3 ? table : info;
    const SpliceK sk = splice_consts();
    float acc = 0.f;
    auto step = [&](const BlockRec& rec, int r) {
        // pin the record's first use here: nothing derived from it may be hoisted
        // above this point (that would wait for the loads of later rounds)
        BlockRec o = rec;
        if constexpr (HB == 8) {
            asm volatile("" : "+v"(o.lohi), "+v"(o.cc));
        } else {
            asm volatile("" : "+v"(o.lohi), "+v"(o.cc16));
            o.cc = o.cc16;
        }
        asm volatile("" : "+v"(o.a.x), "+v"(o.a.y), "+v"(o.a.z), "+v"(o.a.w), "+v"(o.b.x), "+v"(o.b.y));
        const int kb = j + r * S;
        const float v = block_dot(o, ti[min(kb, n_cb - 1)], sk);
        acc += (col_ok && kb < n_cb) ? v : 0.f;
    };
    int r = 0;
    for (; r + NR < R; r += NR) {
#pragma unroll
        for (int i = 0; i < NR; ++i) {
            step(buf[i], r + i);
            __builtin_amdgcn_sched_barrier(0);
            load(buf[i], r + NR + i);
            __builtin_amdgcn_sched_barrier(0);
        }
    }
#pragma unroll
    for (int i = 0; i < NR; ++i)
        if (r + i < R) step(buf[i], r + i);

    // slices -> columns in a fixed order.  CT <= 64 (S >= 8): thread t < 8 CT sums slices
    // g, g + 8, ... of column t % CT (g = t / CT), eight loads in flight at a time, then
    // thread c < CT sums the 8 partials of column c.  CT = kMaxPanelCt (S = 4, every lane a
    // slice): thread c sums its column's 4 slices in slice order (the same order the
    // two-step form gives with 4 groups of one slice each); red[kPanelThreads..) stays free.
    red[tid] = acc;
    __syncthreads();
    const bool wide = CT > 64;   // CT is kMaxPanelCt (the host plans no width in 65..127)
    if (!wide) {
        if (tid < 8 * CT) {
            float t = 0.f;
            int s = j0;
            for (; s + 56 < S; s += 64) {
                float v[8];
#pragma unroll
                for (int i = 0; i < 8; ++i) v[i] = red[(s + 8 * i) * CT + c];
#pragma unroll
                for (int i = 0; i < 8; ++i) t += v[i];
            }
            for (; s < S; s += 8) t += red[s * CT + c];
            red[kPanelThreads + tid] = t;
        }
        __syncthreads();
    }
    float yv = -INFINITY;
    if (tid < CT && col_ok) {
        float t = 0.f;
        if (wide) {
#pragma unroll
            for (int g = 0; g < kPanelThreads / kMaxPanelCt; ++g) t += red[g * kMaxPanelCt + tid];
        } else {
#pragma unroll
            for (int g = 0; g < 8; ++g) t += red[kPanelThreads + g * CT + tid];
        }
        // residual epilogue: h = resid + W x, each element read and written by this thread
        if constexpr (kResY) {
            t = yres + t;
        } else {
            const float* __restrict__ add = kOne ? grp.m[0].add : pick([](const GemvMat& g) { return g.add; });
            if (add) t = *(const g_float*)(add + n) + t;
        }
        *(float SX8_GLOBAL_AS*)(Y + n) = t;
        yv = t;
    }
    // argmax partials (lm_head): the panel's best column -- larger value, or equal value and
    // lower index, so the maxima of the panels give the first index of the overall maximum;
    // a NaN never wins -- from the CT columns of waves 0 (and 1 when CT > 64), wave 1's
    // best passed to wave 0 through LDS
    if constexpr (kX == kXRms && kOne) {
        if (xp.amax != nullptr) {   // the same for every thread of the work-group
            float v = -INFINITY;
            int idx = INT_MAX;
            if (tid < 128) {
                // a NaN logit never enters the butterfly: its lane starts empty (-inf,
                // INT_MAX) and takes its partners' values like any other
                const bool mine = tid < CT && col_ok && !__builtin_isnan(yv);
                v = mine ? yv : -INFINITY;
                idx = mine ? n : INT_MAX;
#pragma unroll
                for (int o = 32; o > 0; o >>= 1) {
                    const float ov = __shfl_xor(v, o);
                    const int oi = __shfl_xor(idx, o);
                    if (ov > v || (ov == v && oi < idx)) {
                        v = ov;
                        idx = oi;
                    }
                }
            }
            if (wide) {
                // the 128-column sums leave red[kPanelThreads..) unused
                if (tid == 64) {
                    red[kPanelThreads] = v;
                    red[kPanelThreads + 1] = __builtin_bit_cast(float, idx);
                }
                __syncthreads();
                if (tid == 0) {
                    const float ov = red[kPanelThreads];
                    const int oi = __builtin_bit_cast(int, red[kPanelThreads + 1]);
                    if (ov > v || (ov == v && oi < idx)) {
                        v = ov;
                        idx = oi;
                    }
                }
            }
            if (tid == 0) {
                xp.amax[2 * panel] = __builtin_bit_cast(uint32_t, v);
                xp.amax[2 * panel + 1] = (uint32_t)idx;
            }
        }
    }
}

// The argmax over the panel partials of a lm_head launch: *tok = first index of the
// maximum (INT64_MAX if no value compares, e.g. all NaN, as a scan of the logits gives),
// then *pos += 1.  One 256-thread work-group; each thread requests its kPer partials
// together before comparing (a loop that compares as it loads waits a memory round trip
// per partial).  The comparison -- larger value, or equal value and lower index; NaN never
// wins -- does not depend on the order, so any reduction tree gives the same token.
// Indices stay 32-bit (a panel's column, INT_MAX for none) until the store.
__global__ __launch_bounds__(256) void k_argmax_parts(const uint32_t* __restrict__ parts, int n_parts,
                                                      int64_t* __restrict__ tok, int64_t* __restrict__ pos) {
    constexpr int kThreads = 256, kPer = 10;
    __shared__ float bv[kThreads / 64];
    __shared__ int bi[kThreads / 64];
    auto better = [](float x, int i, float& v, int& idx) {
        if (x > v || (x == v && i < idx)) {
            v = x;
            idx = i;
        }
    };
    const uint2* p2 = reinterpret_cast<const uint2*>(parts);
    const int t = (int)threadIdx.x;
    float v = -INFINITY;
    int idx = INT_MAX;
    for (int base = 0; base < n_parts; base += kThreads * kPer) {
        uint2 w[kPer];
#pragma unroll
        for (int k = 0; k < kPer; ++k) w[k] = p2[min(base + k * kThreads + t, n_parts - 1)];
#pragma unroll
        for (int k = 0; k < kPer; ++k)
            if (base + k * kThreads + t < n_parts) better(__builtin_bit_cast(float, w[k].x), (int)w[k].y, v, idx);
    }
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) {
        const float ov = __shfl_xor(v, o, 64);
        const int oi = __shfl_xor(idx, o, 64);
        better(ov, oi, v, idx);
    }
    if ((t & 63) == 0) {
        bv[t >> 6] = v;
        bi[t >> 6] = idx;
    }
    __syncthreads();
    if (t == 0) {
        for (int w = 1; w < kThreads / 64; ++w) better(bv[w], bi[w], v, idx);
        tok[0] = idx == INT_MAX ? INT64_MAX : (int64_t)idx;
        pos[0] += 1;
    }
}

// Panel geometry: CT columns per panel (at most 64, or 128 past 65536 columns), from the
// group's total width: ceil(sum N / 256) gives about one work-group per CU; wider groups
// take two per CU (co-resident).  Three record buffers, two of them requested before the table build and
// the third right after it: more rounds ahead of the table lengthen the prologue, which is
// where a launch loses most of its time (measured slower on MI355X).
struct PanelPlan {
    int CT, S, R, TP;
    unsigned grid;
};

inline PanelPlan plan_panels(const int64_t* Ns, int n_mats, int n_cb) {
    int64_t total = 0;
    for (int i = 0; i < n_mats; ++i) total += Ns[i];
    PanelPlan p;
    p.CT = panel_ct(total);
    // a group rounds every matrix up to whole panels: widen the panels until the grid is
    // back within one (two) work-groups per CU -- one more work-group than CUs puts two on
    // one CU, and the launch waits for that CU (q/k/v 4096 + 1024 + 1024: CT 24 gives 257
    // panels, CT 25 gives 246)
    const int64_t cap = total > 64 * 256 ? 512 : 256;
    auto panels = [&](int ct) {
        int64_t g = 0;
        for (int i = 0; i < n_mats; ++i) g += (Ns[i] + ct - 1) / ct;
        return g;
    };
    while (p.CT < 64 && panels(p.CT) > cap) ++p.CT;
    p.S = kPanelThreads / p.CT;
    p.R = (n_cb + p.S - 1) / p.S;
    p.TP = n_cb <= 128 * kTabPassesShort ? kTabPassesShort : kTabPassesLong;
    p.grid = (unsigned)panels(p.CT);
    return p;
}

constexpr int kRing = 3;   // record buffers per lane (at most)
// Grids above this many work-groups (the vocab-sized matrices: many rounds of panels, each
// work-group's prologue amortized) run with two record buffers, which measured faster there.
constexpr unsigned kRing3MaxGrid = 1024;

// kPre / kResY: see k_gemv_panel.  A group (kPre, kXRms) passes h in the x slot and the
// norm weight in the header slot; a single matrix (kPre, kXSilu) passes g in the x slot.
template <int HB, int kMode, int kX = kXPlain, bool kPre = false, bool kResY = false>
void launch_panel(const PanelPlan& p, size_t smem, hipStream_t st, const uint16_t* X,
                  const GemvGroup& g, const KbInfo* table, int n_cb, const XProd& xp = XProd{}) {
    const dim3 grid(p.grid), block(kPanelThreads);
    const bool one = g.n_mats == 1;
    const GemvMat& m0 = g.m[0];
    // instantiated forms: kPre with kXRms only for groups, kPre with kXSilu and kResY only
    // for single matrices
    constexpr bool kAllowOne = !(kPre && kX == kXRms);
    constexpr bool kAllowGroup = !(kPre && kX == kXSilu) && !kResY;
    const uint8_t* h0 = (kPre && kX == kXRms) ? reinterpret_cast<const uint8_t*>(xp.w) : m0.hdr;
    // a single matrix with Z given (kMode 2) takes Z in the basis slot, which is preloaded
    const float* b0 = kMode == 2 ? m0.Zin : m0.basis;
    auto go = [&](auto nr, auto tp) {
        constexpr int NR = decltype(nr)::value, TP = decltype(tp)::value;
        if constexpr (kAllowOne) {
            if (one) {
                hipLaunchKernelGGL((k_gemv_panel<HB, kMode, NR, TP, kX, true, kPre, kResY>), grid, block, smem, st,
                                   h0, m0.levels, X, m0.N, n_cb, b0, m0.scales, m0.Y, g, table, xp);
                return;
            }
        }
        if constexpr (kAllowGroup)
            hipLaunchKernelGGL((k_gemv_panel<HB, kMode, NR, TP, kX, false, kPre, kResY>), grid, block, smem, st,
                               h0, m0.levels, X, m0.N, n_cb, m0.basis, m0.scales, m0.Y, g, table, xp);
    };
    auto by_ring = [&](auto tp) {
        if (p.grid <= kRing3MaxGrid)
            go(std::integral_constant<int, kRing>{}, tp);
        else
            go(std::integral_constant<int, 2>{}, tp);
    };
    if constexpr (kMode == 1 || kMode == 2 || kMode == 4) {
        if (p.TP == kTabPassesLong) {
            by_ring(std::integral_constant<int, kTabPassesLong>{});
            return;
        }
    }
    by_ring(std::integral_constant<int, kTabPassesShort>{});
}

// 32-bit buffer offsets: every block index a lane forms stays below 2^31 / 24.
inline bool offsets_fit(const PanelPlan& p, int64_t N, int64_t n_cb) {
    return (n_cb + (int64_t)(kRing + 1) * p.S) * N * 24 < ((int64_t)1 << 31);
}

inline size_t panel_smem(int n_cb, bool lds) {
    // table: n_cb entries + one spare entry for the build's idle threads
    return sizeof(float) * 2 * kPanelThreads + (lds ? sizeof(KbInfo) * (size_t)(n_cb + 1) : 0);
}

template <int HB>
int32_t launch_gemv(const uint16_t* X, const uint8_t* hdr, const uint8_t* levels,
                    const float* basis, const float* scales, const float* Zin, float* Zout,
                    int N, int n_cb, float* Y, KbInfo* table, hipStream_t st) {
    using namespace sx8;
    const int64_t N64 = N;
    const PanelPlan p = plan_panels(&N64, 1, n_cb);
    if (!offsets_fit(p, N, n_cb))
        return fail(SX8_ERR_UNSUPPORTED, "sx8_gemv: %lld x %lld blocks exceed 32-bit offsets",
                    (long long)N, (long long)n_cb);
    GemvGroup g{};
    g.n_mats = 1;
    g.ct = p.CT;
    g.m[0] = GemvMat{hdr, levels, basis, scales, Zin, Y, nullptr, N, (int)p.grid};
    const bool lds = n_cb <= kLdsMaxKb;
    const size_t smem = panel_smem(n_cb, lds);
    if (!Zout && lds) {   // single launch: the table is built inside every work-group
        if (Zin)
            launch_panel<HB, 2>(p, smem, st, X, g, table, n_cb);
        else
            launch_panel<HB, 1>(p, smem, st, X, g, table, n_cb);
        return check_launch("sx8_gemv");
    }
    const dim3 tgrid((n_cb + 7) / 8);
    if (Zin)
        hipLaunchKernelGGL(k_kbinfo<true>, tgrid, dim3(256), 0, st, X, basis, scales, Zin, Zout,
                           n_cb, table);
    else
        hipLaunchKernelGGL(k_kbinfo<false>, tgrid, dim3(256), 0, st, X, basis, scales, Zin, Zout,
                           n_cb, table);
    if (lds)
        launch_panel<HB, 0>(p, smem, st, X, g, table, n_cb);
    else
        launch_panel<HB, 3>(p, smem, st, X, g, table, n_cb);
    return check_launch("sx8_gemv");
}

// One launch over up to kMaxGroup matrices that share x; each work-group builds the table
// of its own matrix.  Z given (Zin) or computed must be the same for every matrix.
template <int HB>
int32_t launch_gemv_group(const uint16_t* X, int n_mats, const uint8_t* const* hdrs,
                          const uint8_t* const* levels, const float* const* bases,
                          const float* const* scales, const float* const* Zins,
                          const int64_t* Ns, int n_cb, float* const* Ys, hipStream_t st) {
    using namespace sx8;
    const PanelPlan p = plan_panels(Ns, n_mats, n_cb);
    GemvGroup g{};
    g.n_mats = n_mats;
    g.ct = p.CT;
    for (int i = 0; i < n_mats; ++i) {
        if (!offsets_fit(p, Ns[i], n_cb))
            return fail(SX8_ERR_UNSUPPORTED, "sx8_gemv_group: %lld x %lld blocks exceed 32-bit offsets",
                        (long long)Ns[i], (long long)n_cb);
        g.m[i] = GemvMat{hdrs[i], levels[i], bases ? bases[i] : nullptr,
                         scales ? scales[i] : nullptr, Zins ? Zins[i] : nullptr, Ys[i], nullptr,
                         (int)Ns[i], (int)((Ns[i] + p.CT - 1) / p.CT)};
    }
    const size_t smem = panel_smem(n_cb, true);
    if (Zins)
        launch_panel<HB, 2>(p, smem, st, X, g, nullptr, n_cb);
    else
        launch_panel<HB, 1>(p, smem, st, X, g, nullptr, n_cb);
    return check_launch("sx8_gemv_group");
}

}  // namespace

extern "C" int64_t sx8_gemv_workspace_bytes(int64_t n_cb) {
    return n_cb > 0 ? n_cb * (int64_t)sizeof(KbInfo) : 0;
}

int32_t sx8::compute_z_sets(const uint16_t* X, int64_t M, int64_t ldx, int64_t K, const ZSets& zs,
                           int64_t n_cb, bool hl, uint16_t* xpack, hipStream_t st) {
    const int64_t rows = xpack ? (M + 31) / 32 * 32 : M;
    if (rows * n_cb > 0x7FFFFFFF - 255 || K > n_cb * 32)
        return fail(SX8_ERR_UNSUPPORTED, "compute_z: %lld rows x %lld K blocks exceed 2^31", (long long)rows,
                    (long long)n_cb);
    const int64_t grid = (rows * n_cb + 255) / 256;
    const bool x_vec = aligned(X, 16) && ldx % 8 == 0;
    if (zs.n > 0 && xpack)
        hipLaunchKernelGGL((k_compute_z<true, true>), dim3((unsigned)grid), dim3(256), 0, st, X, (int)M, ldx,
                           (int)K, zs, (int)n_cb, x_vec, hl, xpack, nullptr, nullptr);
    else if (zs.n > 0)
        hipLaunchKernelGGL((k_compute_z<true, false>), dim3((unsigned)grid), dim3(256), 0, st, X, (int)M,
                           ldx, (int)K, zs, (int)n_cb, x_vec, hl, xpack, nullptr, nullptr);
    else if (xpack)
        hipLaunchKernelGGL((k_compute_z<false, true>), dim3((unsigned)grid), dim3(256), 0, st, X, (int)M,
                           ldx, (int)K, zs, (int)n_cb, x_vec, hl, xpack, nullptr, nullptr);
    return check_launch("compute_z");
}

int32_t sx8::compute_z_silu(const float* g, const float* u, int64_t M, int64_t ld, int64_t K,
                           const ZSets& zs, int64_t n_cb, uint16_t* xpack, hipStream_t st) {
    const int64_t rows = (M + 31) / 32 * 32;
    if (rows * n_cb > 0x7FFFFFFF - 255 || K > n_cb * 32)
        return fail(SX8_ERR_UNSUPPORTED, "compute_z: %lld rows x %lld K blocks exceed 2^31", (long long)rows,
                    (long long)n_cb);
    const int64_t grid = (rows * n_cb + 255) / 256;
    const bool vec = aligned(g, 16) && aligned(u, 16) && ld % 4 == 0;
    if (zs.n > 0)
        hipLaunchKernelGGL((k_compute_z<true, true, true>), dim3((unsigned)grid), dim3(256), 0, st, nullptr, (int)M,
                           ld, (int)K, zs, (int)n_cb, vec, true, xpack, g, u);
    else
        hipLaunchKernelGGL((k_compute_z<false, true, true>), dim3((unsigned)grid), dim3(256), 0, st, nullptr, (int)M,
                           ld, (int)K, zs, (int)n_cb, vec, true, xpack, g, u);
    return check_launch("compute_z");
}

int32_t sx8::compute_z(const uint16_t* X, int64_t M, int64_t ldx, int64_t K, const float* basis,
                       const float* scales, int64_t n_cb, void* Z, bool hl, uint16_t* xpack,
                       hipStream_t st) {
    ZSets zs{};
    if (Z) {
        zs.basis[0] = basis;
        zs.scales[0] = scales;
        zs.Z[0] = reinterpret_cast<float*>(Z);
        zs.n = 1;
    }
    return compute_z_sets(X, M, ldx, K, zs, n_cb, hl, xpack, st);
}

extern "C" int32_t sx8_compute_z(const uint16_t* X, int64_t M, int64_t ldx, const float* basis,
                                 const float* scales, int64_t n_cb, float* Z, void* stream) {
    using namespace sx8;
    if (!X || !basis || !scales || !Z) return fail(SX8_ERR_INVALID, "sx8_compute_z: null pointer");
    if (M <= 0 || n_cb <= 0 || ldx < n_cb * 32)
        return fail(SX8_ERR_INVALID, "sx8_compute_z: bad shape M=%lld ldx=%lld n_cb=%lld",
                    (long long)M, (long long)ldx, (long long)n_cb);
    if (!aligned(X, 2) || !aligned(basis, 16) || !aligned(scales, 4) || !aligned(Z, 8))
        return fail(SX8_ERR_INVALID, "sx8_compute_z: misaligned pointer (basis 16 B, Z 8 B)");
    return compute_z(X, M, ldx, n_cb * 32, basis, scales, n_cb, Z, false, nullptr, as_stream(stream));
}

extern "C" int32_t sx8_gemv(const uint16_t* X, const uint8_t* hdr, const uint8_t* levels,
                            int32_t hdr_bytes, const float* basis, const float* scales,
                            const float* Z_in, float* Z_out, int64_t N, int64_t n_cb, float* Y,
                            void* workspace, int64_t workspace_bytes, void* stream) {
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
    // the single-launch form builds its table in LDS; the Z-returning form and K beyond the
    // LDS table run k_kbinfo first and need the caller's workspace for its table
    const int64_t need = sx8_gemv_workspace_bytes(n_cb);
    const bool needs_ws = Z_out != nullptr || n_cb > kLdsMaxKb;
    KbInfo* table = reinterpret_cast<KbInfo*>(workspace);
    if (table && (workspace_bytes < need || !aligned(table, 16)))
        return fail(SX8_ERR_INVALID, "sx8_gemv: workspace needs %lld bytes, 16-byte aligned",
                    (long long)need);
    if (!table && needs_ws)
        return fail(SX8_ERR_INVALID,
                    "sx8_gemv: this call (Z_out given or n_cb > %d) needs a workspace of %lld bytes",
                    kLdsMaxKb, (long long)need);
    if (hdr_bytes == 8)
        return launch_gemv<8>(X, hdr, levels, basis, scales, Z_in, Z_out, (int)N, (int)n_cb, Y,
                              table, as_stream(stream));
    return launch_gemv<6>(X, hdr, levels, basis, scales, Z_in, Z_out, (int)N, (int)n_cb, Y, table,
                          as_stream(stream));
}

extern "C" int32_t sx8_gemv_group(const uint16_t* X, int32_t n_mats, const uint8_t* const* hdrs,
                                  const uint8_t* const* levels, int32_t hdr_bytes,
                                  const float* const* bases, const float* const* scales,
                                  const float* const* Z_in, const int64_t* Ns, int64_t n_cb,
                                  float* const* Ys, void* workspace, int64_t workspace_bytes,
                                  void* stream) {
    using namespace sx8;
    if (!X || !hdrs || !levels || !Ns || !Ys) return fail(SX8_ERR_INVALID, "sx8_gemv_group: null pointer");
    if (n_mats < 1 || n_mats > kMaxGroup)
        return fail(SX8_ERR_INVALID, "sx8_gemv_group: n_mats must be 1..%d, got %d", kMaxGroup, n_mats);
    if (!Z_in && (!bases || !scales))
        return fail(SX8_ERR_INVALID, "sx8_gemv_group: bases/scales required when Z_in is NULL");
    if (hdr_bytes != 6 && hdr_bytes != 8)
        return fail(SX8_ERR_INVALID, "sx8_gemv_group: hdr_bytes must be 6 or 8, got %d", hdr_bytes);
    if (n_cb <= 0 || n_cb > 0x7FFFFFFF / 64 || !aligned(X, 16))
        return fail(SX8_ERR_INVALID, "sx8_gemv_group: bad n_cb %lld or X not 16-byte aligned",
                    (long long)n_cb);
    for (int i = 0; i < n_mats; ++i) {
        const bool have_z = Z_in ? Z_in[i] != nullptr : (bases[i] && scales[i]);
        if (!hdrs[i] || !levels[i] || !Ys[i] || !have_z)
            return fail(SX8_ERR_INVALID, "sx8_gemv_group: null pointer in matrix %d", i);
        if (Ns[i] <= 0 || Ns[i] > 0x7FFFFFFF / 2)
            return fail(SX8_ERR_INVALID, "sx8_gemv_group: bad N %lld (matrix %d)", (long long)Ns[i], i);
        if (!aligned(hdrs[i], hdr_bytes == 8 ? 8 : 2) || !aligned(levels[i], 8) || !aligned(Ys[i], 4) ||
            (Z_in && !aligned(Z_in[i], 4)) ||
            (!Z_in && (!aligned(bases[i], 16) || !aligned(scales[i], 4))))
            return fail(SX8_ERR_INVALID, "sx8_gemv_group: misaligned pointer in matrix %d", i);
    }
    const hipStream_t st = as_stream(stream);
    if (n_cb > kLdsMaxKb) {   // table past LDS: one two-launch GEMV per matrix
        void* ws = workspace;
        if (!ws || workspace_bytes < sx8_gemv_workspace_bytes(n_cb) || !aligned(ws, 16))
            return fail(SX8_ERR_INVALID,
                        "sx8_gemv_group: n_cb > %d needs a 16-byte aligned workspace of %lld bytes",
                        kLdsMaxKb, (long long)sx8_gemv_workspace_bytes(n_cb));
        for (int i = 0; i < n_mats; ++i) {
            const float* b = Z_in ? nullptr : bases[i];
            const float* sc = Z_in ? nullptr : scales[i];
            const float* z = Z_in ? Z_in[i] : nullptr;
            const int32_t r = hdr_bytes == 8
                ? launch_gemv<8>(X, hdrs[i], levels[i], b, sc, z, nullptr, (int)Ns[i], (int)n_cb, Ys[i],
                                 reinterpret_cast<KbInfo*>(ws), st)
                : launch_gemv<6>(X, hdrs[i], levels[i], b, sc, z, nullptr, (int)Ns[i], (int)n_cb, Ys[i],
                                 reinterpret_cast<KbInfo*>(ws), st);
            if (r != SX8_OK) return r;
        }
        return SX8_OK;
    }
    if (hdr_bytes == 8)
        return launch_gemv_group<8>(X, n_mats, hdrs, levels, bases, scales, Z_in, Ns, (int)n_cb, Ys, st);
    return launch_gemv_group<6>(X, n_mats, hdrs, levels, bases, scales, Z_in, Ns, (int)n_cb, Ys, st);
}

// ------------------------------------------------------------------ fused decoder GEMVs

namespace {

// Argument checks shared by the fused entry points; fills the group (bases/scales form).
int32_t check_fused_group(const char* what, int32_t n_mats, const uint8_t* const* hdrs,
                          const uint8_t* const* levels, int32_t hdr_bytes, const float* const* bases,
                          const float* const* scales, const int64_t* Ns, int64_t n_cb,
                          float* const* Ys) {
    using namespace sx8;
    if (!hdrs || !levels || !bases || !scales || !Ns || !Ys) return fail(SX8_ERR_INVALID, "%s: null pointer", what);
    if (n_mats < 1 || n_mats > kMaxGroup)
        return fail(SX8_ERR_INVALID, "%s: n_mats must be 1..%d, got %d", what, kMaxGroup, n_mats);
    if (hdr_bytes != 6 && hdr_bytes != 8)
        return fail(SX8_ERR_INVALID, "%s: hdr_bytes must be 6 or 8, got %d", what, hdr_bytes);
    // every table unit is produced within the kTabPassesLong up-front passes
    if (n_cb <= 0 || n_cb * 4 > (int64_t)kTabPassesLong * kPanelThreads)
        return fail(SX8_ERR_UNSUPPORTED, "%s: n_cb %lld outside 1..%d", what, (long long)n_cb,
                    kTabPassesLong * kPanelThreads / 4);
    for (int i = 0; i < n_mats; ++i) {
        if (!hdrs[i] || !levels[i] || !Ys[i] || !bases[i] || !scales[i])
            return fail(SX8_ERR_INVALID, "%s: null pointer in matrix %d", what, i);
        if (Ns[i] <= 0 || Ns[i] > 0x7FFFFFFF / 2)
            return fail(SX8_ERR_INVALID, "%s: bad N %lld (matrix %d)", what, (long long)Ns[i], i);
        if (!aligned(hdrs[i], hdr_bytes == 8 ? 8 : 2) || !aligned(levels[i], 8) || !aligned(Ys[i], 4) ||
            !aligned(bases[i], 16) || !aligned(scales[i], 4))
            return fail(SX8_ERR_INVALID, "%s: misaligned pointer in matrix %d", what, i);
    }
    return SX8_OK;
}

template <int kX>
int32_t launch_fused(const char* what, const XProd& xp, int32_t n_mats, const uint8_t* const* hdrs,
                     const uint8_t* const* levels, int32_t hdr_bytes, const float* const* bases,
                     const float* const* scales, const int64_t* Ns, int64_t n_cb, float* const* Ys,
                     hipStream_t st, const uint16_t* X = nullptr, const float* const* adds = nullptr) {
    using namespace sx8;
    PanelPlan p = plan_panels(Ns, n_mats, (int)n_cb);
    GemvGroup g{};
    g.n_mats = n_mats;
    g.ct = p.CT;
    for (int i = 0; i < n_mats; ++i) {
        if (!offsets_fit(p, Ns[i], n_cb))
            return fail(SX8_ERR_UNSUPPORTED, "%s: %lld x %lld blocks exceed 32-bit offsets", what,
                        (long long)Ns[i], (long long)n_cb);
        g.m[i] = GemvMat{hdrs[i], levels[i], bases[i], scales[i], nullptr, Ys[i], adds ? adds[i] : nullptr,
                         (int)Ns[i], (int)((Ns[i] + p.CT - 1) / p.CT)};
    }
    const size_t smem = panel_smem((int)n_cb, true);
    const int64_t K = n_cb * 32;
    // preloaded producer inputs (see k_gemv_panel): a grouped RMSNorm of the residual alone,
    // or a single-matrix SiLU whose u follows g
    const bool pre = kX == kXRms ? (n_mats > 1 && xp.resid && !xp.init && !xp.delta && !xp.resid_out)
                     : kX == kXSilu ? (n_mats == 1 && xp.u == xp.g + K)
                                    : false;
    // the residual updated in place by a single matrix: read from the preloaded output slot
    // (kResY forms: plain x, or the preloaded SiLU; the others add through the descriptor)
    const bool resy = n_mats == 1 && adds && adds[0] == Ys[0] && (kX == kXPlain || (kX == kXSilu && pre));
    if (resy) g.m[0].add = nullptr;
    const uint16_t* xs = pre ? reinterpret_cast<const uint16_t*>(kX == kXRms ? xp.resid : xp.g) : X;
    auto run = [&](auto hb) {
        constexpr int HB = decltype(hb)::value;
        if constexpr (kX == kXRms) {
            if (pre) launch_panel<HB, 1, kX, true>(p, smem, st, xs, g, nullptr, (int)n_cb, xp);
            else launch_panel<HB, 1, kX>(p, smem, st, xs, g, nullptr, (int)n_cb, xp);
        } else if constexpr (kX == kXSilu) {
            if (pre && resy) launch_panel<HB, 1, kX, true, true>(p, smem, st, xs, g, nullptr, (int)n_cb, xp);
            else if (pre) launch_panel<HB, 1, kX, true>(p, smem, st, xs, g, nullptr, (int)n_cb, xp);
            else launch_panel<HB, 1, kX>(p, smem, st, xs, g, nullptr, (int)n_cb, xp);
        } else {
            if (resy) launch_panel<HB, 1, kX, false, true>(p, smem, st, xs, g, nullptr, (int)n_cb, xp);
            else launch_panel<HB, 1, kX>(p, smem, st, xs, g, nullptr, (int)n_cb, xp);
        }
    };
    if (hdr_bytes == 8)
        run(std::integral_constant<int, 8>{});
    else
        run(std::integral_constant<int, 6>{});
    return check_launch(what);
}

}  // namespace

extern "C" int32_t sx8_dec_gemv_rmsnorm(const float* resid, const uint16_t* init, const float* delta,
                                        const uint16_t* norm_w, float eps, float* resid_out,
                                        int32_t n_mats, const uint8_t* const* hdrs,
                                        const uint8_t* const* levels, int32_t hdr_bytes,
                                        const float* const* bases, const float* const* scales,
                                        const int64_t* Ns, int64_t n_cb, float* const* Ys,
                                        void* stream) {
    using namespace sx8;
    const char* what = "sx8_dec_gemv_rmsnorm";
    if ((!resid && !init) || !norm_w) return fail(SX8_ERR_INVALID, "%s: null pointer", what);
    if ((resid && !aligned(resid, 16)) || (init && !aligned(init, 16)) || (delta && !aligned(delta, 16)) ||
        !aligned(norm_w, 16) || (resid_out && !aligned(resid_out, 16)))
        return fail(SX8_ERR_INVALID, "%s: state vectors must be 16-byte aligned", what);
    if (resid_out && (resid_out == resid || resid_out == delta))
        return fail(SX8_ERR_INVALID, "%s: resid_out must not alias resid or delta", what);
    const int32_t rc = check_fused_group(what, n_mats, hdrs, levels, hdr_bytes, bases, scales, Ns, n_cb, Ys);
    if (rc != SX8_OK) return rc;
    XProd xp{};
    xp.resid = init ? nullptr : resid;
    xp.init = init;
    xp.delta = delta;
    xp.w = norm_w;
    xp.resid_out = resid_out;
    xp.eps = eps;
    return launch_fused<kXRms>(what, xp, n_mats, hdrs, levels, hdr_bytes, bases, scales, Ns, n_cb, Ys,
                               as_stream(stream));
}

extern "C" int64_t sx8_dec_argmax_parts_bytes(int64_t N, int64_t n_cb) {
    if (N <= 0 || n_cb <= 0) return -1;
    const int64_t N64 = N;
    return 8 * (int64_t)plan_panels(&N64, 1, (int)n_cb).grid;
}

extern "C" int32_t sx8_dec_gemv_rmsnorm_argmax(const float* resid, const uint16_t* norm_w, float eps,
                                               const uint8_t* hdr, const uint8_t* levels, int32_t hdr_bytes,
                                               const float* bases, const float* scales, int64_t N, int64_t n_cb,
                                               float* logits, void* parts, int64_t parts_bytes, int64_t* tok,
                                               int64_t* pos, void* stream) {
    using namespace sx8;
    const char* what = "sx8_dec_gemv_rmsnorm_argmax";
    if (!resid || !norm_w || !parts || !tok || !pos) return fail(SX8_ERR_INVALID, "%s: null pointer", what);
    if (!aligned(resid, 16) || !aligned(norm_w, 16) || !aligned(parts, 8))
        return fail(SX8_ERR_INVALID, "%s: resid and norm_w must be 16-byte aligned, parts 8-byte aligned", what);
    const int64_t need = sx8_dec_argmax_parts_bytes(N, n_cb);
    if (need < 0 || parts_bytes < need)
        return fail(SX8_ERR_INVALID, "%s: parts needs %lld bytes (sx8_dec_argmax_parts_bytes), got %lld", what,
                    (long long)need, (long long)parts_bytes);
    const uint8_t* const hdrs[1] = {hdr};
    const uint8_t* const lvls[1] = {levels};
    const float* const bas[1] = {bases};
    const float* const sca[1] = {scales};
    float* const ys[1] = {logits};
    const int32_t rc = check_fused_group(what, 1, hdrs, lvls, hdr_bytes, bas, sca, &N, n_cb, ys);
    if (rc != SX8_OK) return rc;
    XProd xp{};
    xp.resid = resid;
    xp.w = norm_w;
    xp.eps = eps;
    xp.amax = reinterpret_cast<uint32_t*>(parts);
    const int32_t r2 = launch_fused<kXRms>(what, xp, 1, hdrs, lvls, hdr_bytes, bas, sca, &N, n_cb, ys,
                                           as_stream(stream));
    if (r2 != SX8_OK) return r2;
    hipLaunchKernelGGL(k_argmax_parts, dim3(1), dim3(256), 0, as_stream(stream),
                       reinterpret_cast<const uint32_t*>(parts), (int)(need / 8), tok, pos);
    return check_launch(what);
}

extern "C" int32_t sx8_dec_gemv_silu(const float* g, const float* u, int32_t n_mats,
                                     const uint8_t* const* hdrs, const uint8_t* const* levels,
                                     int32_t hdr_bytes, const float* const* bases,
                                     const float* const* scales, const int64_t* Ns, int64_t n_cb,
                                     float* const* Ys, void* stream) {
    using namespace sx8;
    const char* what = "sx8_dec_gemv_silu";
    if (!g || !u) return fail(SX8_ERR_INVALID, "%s: null pointer", what);
    if (!aligned(g, 16) || !aligned(u, 16)) return fail(SX8_ERR_INVALID, "%s: g and u must be 16-byte aligned", what);
    const int32_t rc = check_fused_group(what, n_mats, hdrs, levels, hdr_bytes, bases, scales, Ns, n_cb, Ys);
    if (rc != SX8_OK) return rc;
    XProd xp{};
    xp.g = g;
    xp.u = u;
    return launch_fused<kXSilu>(what, xp, n_mats, hdrs, levels, hdr_bytes, bases, scales, Ns, n_cb, Ys,
                                as_stream(stream));
}

// Residual checks of the *_add entry points: adds[i] is either Ys[i] (updated in place: each
// element is read and written by the one thread that stores it) or a separate 4-byte
// aligned vector of Ns[i] floats that overlaps no output.  Any other overlap (a residual
// partly over its own output, or over another matrix's output) would let one work-group
// read an element another has already replaced, so it is refused.
static int32_t check_adds(const char* what, int32_t n_mats, const float* const* adds, float* const* Ys,
                          const int64_t* Ns) {
    using namespace sx8;
    if (!adds) return fail(SX8_ERR_INVALID, "%s: null pointer", what);
    auto overlap = [](const float* a, int64_t na, const float* b, int64_t nb) {
        return (uintptr_t)a < (uintptr_t)(b + nb) && (uintptr_t)b < (uintptr_t)(a + na);
    };
    for (int i = 0; i < n_mats; ++i) {
        if (!adds[i] || !aligned(adds[i], 4))
            return fail(SX8_ERR_INVALID, "%s: bad residual pointer (matrix %d)", what, i);
        for (int j = 0; j < n_mats; ++j) {
            if (j == i && adds[i] == Ys[i]) continue;
            if (overlap(adds[i], Ns[i], Ys[j], Ns[j]))
                return fail(SX8_ERR_INVALID, "%s: residual %d overlaps output %d (only adds[i] == Ys[i] may alias)",
                            what, i, j);
        }
    }
    return SX8_OK;
}

extern "C" int32_t sx8_dec_gemv_silu_add(const float* g, const float* u, int32_t n_mats,
                                         const uint8_t* const* hdrs, const uint8_t* const* levels,
                                         int32_t hdr_bytes, const float* const* bases,
                                         const float* const* scales, const int64_t* Ns, int64_t n_cb,
                                         const float* const* adds, float* const* Ys, void* stream) {
    using namespace sx8;
    const char* what = "sx8_dec_gemv_silu_add";
    if (!g || !u) return fail(SX8_ERR_INVALID, "%s: null pointer", what);
    if (!aligned(g, 16) || !aligned(u, 16)) return fail(SX8_ERR_INVALID, "%s: g and u must be 16-byte aligned", what);
    int32_t rc = check_fused_group(what, n_mats, hdrs, levels, hdr_bytes, bases, scales, Ns, n_cb, Ys);
    if (rc == SX8_OK) rc = check_adds(what, n_mats, adds, Ys, Ns);
    if (rc != SX8_OK) return rc;
    XProd xp{};
    xp.g = g;
    xp.u = u;
    return launch_fused<kXSilu>(what, xp, n_mats, hdrs, levels, hdr_bytes, bases, scales, Ns, n_cb, Ys,
                                as_stream(stream), nullptr, adds);
}

extern "C" int32_t sx8_dec_gemv_add(const uint16_t* x, int32_t n_mats, const uint8_t* const* hdrs,
                                    const uint8_t* const* levels, int32_t hdr_bytes, const float* const* bases,
                                    const float* const* scales, const int64_t* Ns, int64_t n_cb,
                                    const float* const* adds, float* const* Ys, void* stream) {
    using namespace sx8;
    const char* what = "sx8_dec_gemv_add";
    if (!x) return fail(SX8_ERR_INVALID, "%s: null pointer", what);
    if (!aligned(x, 16)) return fail(SX8_ERR_INVALID, "%s: x must be 16-byte aligned", what);
    int32_t rc = check_fused_group(what, n_mats, hdrs, levels, hdr_bytes, bases, scales, Ns, n_cb, Ys);
    if (rc == SX8_OK) rc = check_adds(what, n_mats, adds, Ys, Ns);
    if (rc != SX8_OK) return rc;
    return launch_fused<kXPlain>(what, XProd{}, n_mats, hdrs, levels, hdr_bytes, bases, scales, Ns, n_cb, Ys,
                                 as_stream(stream), x, adds);
}

// ------------------------------------------------------------------ gate / up pairs

namespace {

// k_gemv_pair: the decoder MLP's gate and up GEMVs over one RMSNorm'd input in a single
// launch, each work-group computing both for the same CTp columns (lanes alternate: even
// lanes gate, odd lanes up).  The epilogue emits m = fp16(silu(g) u) (the arithmetic of
// sx8_dec_silu_mul) and, for the down projection whose K blocks are these columns, the
// partial PCA sums P[kb][slot][c] = sum_j m_j basis_d[kb][c][j % 32] over the panel's
// columns j of block kb: with CTp >= 32 a block spans at most two panels, slot 0 comes
// from the panel holding the block's first column and slot 1 from the next one (zero when
// the block ends in the first).  The down GEMV then reads m and Z = (P0 + P1) scale
// (kMode 4) instead of g, u and its bases.
// Layout (checked by the host): the up matrix's headers, levels, bases and scales follow
// the gate matrix's in memory, so one pointer per field, preloaded, covers both; h and
// the norm weight are preloaded too.  Everything else is read late from PairArgs.
struct PairArgs {
    uint16_t* m;           // (N) fp16
    const float* bas_d;    // down bases (N / 32, 64)
    float* zp;             // (N / 32, 2, 2) partial sums
    float eps;
};

template <int HB, int NR, int TP>
__global__ __launch_bounds__(kPanelThreads) void k_gemv_pair(
    const uint8_t* __restrict__ hdr, const uint8_t* __restrict__ lv, const float* __restrict__ resid, int N,
    int n_cb, const uint16_t* __restrict__ nw, const float* __restrict__ bas, const float* __restrict__ sca,
    const PairArgs pa) {
    extern __shared__ __align__(16) unsigned char smem[];
    float* red = reinterpret_cast<float*>(smem);                 // 2 x 512 floats
    KbInfo* info = reinterpret_cast<KbInfo*>(smem + sizeof(float) * 2 * kPanelThreads);
    const int tid = threadIdx.x;
    const int n_units = n_cb * 4;
    // (1) h and the norm weight (preloaded pointers), then the bases of both matrices
    XRaw xr[TP];
    {
        const XRsrc xs = xraw_rsrc_pre<kXRms>(resid, nw, n_cb * 32);
#pragma unroll
        for (int p = 0; p < TP; ++p) {
            const int u = min(p * kPanelThreads + tid, n_units - 1);
            xraw_load<kXRms, true>(xr[p], xs, u >> 2, u & 3);
        }
    }
    asm volatile("" ::: "memory");
    TabIn tg[TP], tu[TP];
    const g_float* __restrict__ bg = to_global(bas);
    const g_float* __restrict__ sg = to_global(sca);
#pragma unroll
    for (int p = 0; p < TP; ++p) {
        const int u = min(p * kPanelThreads + tid, n_units - 1);
        tab_load<1, false>(tg[p], nullptr, bg, sg, nullptr, u >> 2, u & 3);
        tab_load<1, false>(tu[p], nullptr, bg + (int64_t)n_cb * 64, sg + (int64_t)n_cb * 2, nullptr, u >> 2, u & 3);
    }
    asm volatile("" ::: "memory");
    __builtin_amdgcn_sched_barrier(0);

    // (2) geometry: CTp = 32..64 column pairs per panel (N <= 16384), CT = 2 CTp lanes per
    // slice
    int n_one = N;
    asm volatile("" : "+s"(n_one));
    const int CTp = max((n_one + 255) / 256, 32), CT = 2 * CTp;
    const int S = kPanelThreads / CT, R = (n_cb + S - 1) / S;
    const int j0 = tid / CT, c = tid - j0 * CT;
    const int G = (n_one + CTp - 1) / CTp, xcd = blockIdx.x & 7;
    const int panel = (int)(blockIdx.x >> 3) + xcd * (G >> 3) + min(xcd, G & 7);
    const int mat = c & 1;                       // (epilogue mapping: thread tid)
    const int col = panel * CTp + (c >> 1);
    const bool col_ok = col < N;
    // K-loop mapping: the S CT active lanes spread evenly over the eight waves (lane i < A
    // of wave w is virtual lane w A + i = slice * CT + column), so no SIMD carries more
    // of them than another (S CT = 456 for CT = 76 would otherwise leave wave 7 with 8)
    const int nact = S * CT, A = (nact + 7) / 8;
    const int va = (tid >> 6) * A + (tid & 63);
    const bool lane_ok = (tid & 63) < A && va < nact;
    const int jv = va / CT, cv = va - jv * CT;
    const int matk = cv & 1;
    const int colk = panel * CTp + (cv >> 1);
    const bool col_okk = colk < N;
    const uint32_t nn = (uint32_t)min(colk, N - 1);
    const int j = lane_ok ? jv : n_cb;
    const uint32_t n_blk = (uint32_t)n_cb * (uint32_t)N;
    const sx8_rsrc rh = make_rsrc(hdr, (int64_t)n_blk * 2 * HB);
    const sx8_rsrc rl = make_rsrc(lv, (int64_t)n_blk * 2 * 24);
    const uint32_t bid0 = lane_ok ? (uint32_t)j * (uint32_t)N + nn + (matk ? n_blk : 0u) : 2 * n_blk;
    const uint32_t dbid = lane_ok ? (uint32_t)S * (uint32_t)N : 0u;
    auto load = [&](BlockRec& o, int r) { load_rec<HB>(o, rh, rl, bid0 + (uint32_t)r * dbid); };
    constexpr int kNR0 = NR < 2 ? NR : 2;
    BlockRec buf[NR];
#pragma unroll
    for (int i = 0; i < kNR0; ++i) {
        load(buf[i], i);
        __builtin_amdgcn_sched_barrier(0);
    }

    // (3) the table: x = RMSNorm(h), Z of the gate bases in z, of the up bases in pad
    {
        float h[TP][8];
        const float inv = rms_inv<TP>(xr, h, red, n_units, n_cb * 32, pa.eps, tid);
#pragma unroll
        for (int p = 0; p < TP; ++p) {
            const uint4 x = rms_x(h[p], xr[p].w, inv);
            tg[p].x = x;
            tu[p].x = x;
            const int u = p * kPanelThreads + tid;
            const int q = u & 3;
            KbInfo& e = info[u < n_units ? u >> 2 : n_cb];
            fill_x_side(e, q, x);
            e.z[q & 1] = tab_z(tg[p], q);
            e.pad[q & 1] = tab_z(tu[p], q);
        }
    }
    __syncthreads();
#pragma unroll
    for (int i = kNR0; i < NR; ++i) load(buf[i], i);
    // the down bases of this lane's column, for the epilogue: requested now (the argument
    // load behind pa.bas_d has arrived during the table build), used after the K loop
    float bd0 = 0.f, bd1 = 0.f;
    if (tid < CT && mat == 0 && col_ok) {
        const int kb = col >> 5, jj = col & 31;
        bd0 = pa.bas_d[(int64_t)kb * 64 + jj];
        bd1 = pa.bas_d[(int64_t)kb * 64 + 32 + jj];
    }

    // (4) the K loop (as k_gemv_panel), each lane with its matrix's Z pair
    const SpliceK sk = splice_consts();
    float acc = 0.f;
    auto step = [&](const BlockRec& rec, int r) {
        BlockRec o = rec;
        if constexpr (HB == 8) {
            asm volatile("" : "+v"(o.lohi), "+v"(o.cc));
        } else {
            asm volatile("" : "+v"(o.lohi), "+v"(o.cc16));
            o.cc = o.cc16;
        }
        asm volatile("" : "+v"(o.a.x), "+v"(o.a.y), "+v"(o.a.z), "+v"(o.a.w), "+v"(o.b.x), "+v"(o.b.y));
        const int kb = j + r * S;
        const KbInfo& ki = info[min(kb, n_cb - 1)];
        const float4 zz = *reinterpret_cast<const float4*>(&ki.z[0]);   // z[0], z[1], pad[0], pad[1]
        const float v = block_dot_z(o, ki, matk ? zz.z : zz.x, matk ? zz.w : zz.y, sk);
        acc += (col_okk && kb < n_cb) ? v : 0.f;
    };
    int r = 0;
    for (; r + NR < R; r += NR) {
#pragma unroll
        for (int i = 0; i < NR; ++i) {
            step(buf[i], r + i);
            __builtin_amdgcn_sched_barrier(0);
            load(buf[i], r + NR + i);
            __builtin_amdgcn_sched_barrier(0);
        }
    }
#pragma unroll
    for (int i = 0; i < NR; ++i)
        if (r + i < R) step(buf[i], r + i);

    // (5) slices -> lanes in a fixed order (NG partial groups: 4 when CT > 64), from the
    // virtual lanes' sums
    if (lane_ok) red[va] = acc;
    __syncthreads();
    const int NG = CT > 64 ? 4 : 8;
    if (tid < NG * CT) {
        float t = 0.f;
        int s = j0;
        for (; s + 7 * NG < S; s += 8 * NG) {
            float v[8];
#pragma unroll
            for (int i = 0; i < 8; ++i) v[i] = red[(s + NG * i) * CT + c];
#pragma unroll
            for (int i = 0; i < 8; ++i) t += v[i];
        }
        for (; s < S; s += NG) t += red[s * CT + c];
        red[kPanelThreads + tid] = t;
    }
    __syncthreads();
    float y = 0.f;
    if (tid < CT)
        for (int g = 0; g < NG; ++g) y += red[kPanelThreads + g * CT + tid];
    // lane pairs (2i, 2i + 1) = (gate, up) of column i sit in one wave (64 is even)
    const float yo = __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, y), 0xB1,
                                                                           0xF, 0xF, false));
    // (6) m and the down projection's contributions m_j basis_d[kb][c][j % 32]
    float* contrib = red;                  // [CTp][2] (the first half of red is free again)
    if (tid < CT && mat == 0) {
        float mv = 0.f;
        if (col_ok) {
            const uint16_t mh = __builtin_bit_cast(uint16_t, (_Float16)sx8_silu_mul(y, yo));
            *(uint16_t SX8_GLOBAL_AS*)(pa.m + col) = mh;
            mv = sx8_h2f(mh);
        }
        contrib[2 * (c >> 1)] = mv * bd0;
        contrib[2 * (c >> 1) + 1] = mv * bd1;
    }
    __syncthreads();
    // per (block, basis) 32 lanes, lane t holding column 32 kb + t's contribution (zero
    // outside the panel), summed by an xor tree (a fixed order)
    const int c0 = panel * CTp, c1 = min(c0 + CTp, N);
    if (c0 < c1) {
        const int kbf = c0 >> 5, kbl = (c1 - 1) >> 5;
        if (tid < 64 * (kbl - kbf + 1)) {             // whole 32-lane groups
            const int t = tid & 31, cc = (tid >> 5) & 1, kb = kbf + (tid >> 6);
            const int q = 32 * kb + t;
            float sum = q >= c0 && q < c1 ? contrib[2 * (q - c0) + cc] : 0.f;
#pragma unroll
            for (int off = 16; off > 0; off >>= 1) sum += __shfl_xor(sum, off, 32);
            if (t == 0) {
                const int slot = 32 * kb >= c0 ? 0 : 1;
                pa.zp[((int64_t)kb * 2 + slot) * 2 + cc] = sum;
                // the block ends in this panel: nobody else writes its slot 1
                if (slot == 0 && min(32 * kb + 32, N) <= c1) pa.zp[((int64_t)kb * 2 + 1) * 2 + cc] = 0.f;
            }
        }
    }
}

}  // namespace

extern "C" int32_t sx8_dec_gemv_rmsnorm_pair(const float* resid, const uint16_t* norm_w, float eps,
                                             const uint8_t* hdr, const uint8_t* levels, int32_t hdr_bytes,
                                             const float* bases, const float* scales, const uint8_t* up_hdr,
                                             const uint8_t* up_levels, const float* up_bases,
                                             const float* up_scales, int64_t N, int64_t n_cb,
                                             const float* down_bases, uint16_t* m, float* zp, void* stream) {
    using namespace sx8;
    const char* what = "sx8_dec_gemv_rmsnorm_pair";
    if (!resid || !norm_w || !hdr || !levels || !bases || !scales || !up_hdr || !up_levels || !up_bases ||
        !up_scales || !down_bases || !m || !zp)
        return fail(SX8_ERR_INVALID, "%s: null pointer", what);
    if (hdr_bytes != 6 && hdr_bytes != 8)
        return fail(SX8_ERR_INVALID, "%s: hdr_bytes must be 6 or 8, got %d", what, hdr_bytes);
    // panels of 32..64 column pairs (a K block of the down projection spans at most two);
    // N is the down projection's K, so its limit is sx8_dec_gemv_zp_add's n_cb limit x 32
    const int64_t n_max = (int64_t)kTabPassesLong * kPanelThreads / 4 * 32;
    if (N < 32 || N > n_max || N % 32)
        return fail(SX8_ERR_UNSUPPORTED, "%s: N must be a multiple of 32 in 32..%lld, got %lld", what,
                    (long long)n_max, (long long)N);
    if (n_cb <= 0 || n_cb * 4 > (int64_t)kTabPassesLong * kPanelThreads)
        return fail(SX8_ERR_UNSUPPORTED, "%s: n_cb %lld outside 1..%d", what, (long long)n_cb,
                    kTabPassesLong * kPanelThreads / 4);
    if (!aligned(resid, 16) || !aligned(norm_w, 16) || !aligned(hdr, hdr_bytes == 8 ? 8 : 2) ||
        !aligned(levels, 8) || !aligned(bases, 16) || !aligned(scales, 4) || !aligned(down_bases, 4) ||
        !aligned(m, 2) || !aligned(zp, 4))
        return fail(SX8_ERR_INVALID, "%s: misaligned pointer", what);
    const int64_t n_blk = N * n_cb;
    // the kernel reads both matrices through the gate's pointers (one buffer resource per
    // field): the up matrix's arrays must start where the gate's end
    if (up_hdr != hdr + n_blk * hdr_bytes || up_levels != levels + n_blk * 24 || up_bases != bases + n_cb * 64 ||
        up_scales != scales + n_cb * 2)
        return fail(SX8_ERR_INVALID,
                    "%s: the up matrix's headers, levels, bases and scales must follow the gate matrix's "
                    "in memory (one allocation per field holding both)", what);
    if ((n_cb + (int64_t)(kRing + 1) * kPanelThreads) * N * 24 * 2 >= ((int64_t)1 << 31))
        return fail(SX8_ERR_UNSUPPORTED, "%s: %lld x %lld blocks exceed 32-bit offsets", what, (long long)N,
                    (long long)n_cb);
    const int CTp = std::max((int)((N + 255) / 256), 32);
    const unsigned grid = (unsigned)((N + CTp - 1) / CTp);
    const int TP = n_cb <= 128 * kTabPassesShort ? kTabPassesShort : kTabPassesLong;
    const size_t smem = panel_smem((int)n_cb, true);
    const PairArgs pa{m, down_bases, zp, eps};
    const hipStream_t st = as_stream(stream);
    auto go = [&](auto hb, auto tp) {
        constexpr int HB = decltype(hb)::value, TPv = decltype(tp)::value;
        hipLaunchKernelGGL((k_gemv_pair<HB, kRing, TPv>), dim3(grid), dim3(kPanelThreads), smem, st, hdr, levels,
                           resid, (int)N, (int)n_cb, norm_w, bases, scales, pa);
    };
    auto by_tp = [&](auto hb) {
        if (TP == kTabPassesLong) go(hb, std::integral_constant<int, kTabPassesLong>{});
        else go(hb, std::integral_constant<int, kTabPassesShort>{});
    };
    if (hdr_bytes == 8) by_tp(std::integral_constant<int, 8>{});
    else by_tp(std::integral_constant<int, 6>{});
    return check_launch(what);
}

// The down projection after sx8_dec_gemv_rmsnorm_pair: Y = adds + W_down m with Z from the
// pair's partial sums (kMode 4); a residual updated in place (adds == Y) is read from the
// preloaded output slot.
extern "C" int32_t sx8_dec_gemv_zp_add(const uint16_t* m, const uint8_t* hdr, const uint8_t* levels,
                                       int32_t hdr_bytes, const float* zp, const float* scales, int64_t N,
                                       int64_t n_cb, const float* add, float* Y, void* stream) {
    using namespace sx8;
    const char* what = "sx8_dec_gemv_zp_add";
    if (!m || !hdr || !levels || !zp || !scales || !add || !Y) return fail(SX8_ERR_INVALID, "%s: null pointer", what);
    if (hdr_bytes != 6 && hdr_bytes != 8)
        return fail(SX8_ERR_INVALID, "%s: hdr_bytes must be 6 or 8, got %d", what, hdr_bytes);
    if (N <= 0 || N > 0x7FFFFFFF / 2) return fail(SX8_ERR_INVALID, "%s: bad N %lld", what, (long long)N);
    if (n_cb <= 0 || n_cb * 4 > (int64_t)kTabPassesLong * kPanelThreads)
        return fail(SX8_ERR_UNSUPPORTED, "%s: n_cb %lld outside 1..%d", what, (long long)n_cb,
                    kTabPassesLong * kPanelThreads / 4);
    if (!aligned(m, 16) || !aligned(hdr, hdr_bytes == 8 ? 8 : 2) || !aligned(levels, 8) || !aligned(zp, 4) ||
        !aligned(scales, 4) || !aligned(add, 4) || !aligned(Y, 4))
        return fail(SX8_ERR_INVALID, "%s: misaligned pointer", what);
    const int64_t N64 = N;
    const PanelPlan p = plan_panels(&N64, 1, (int)n_cb);
    if (!offsets_fit(p, N, n_cb))
        return fail(SX8_ERR_UNSUPPORTED, "%s: %lld x %lld blocks exceed 32-bit offsets", what, (long long)N,
                    (long long)n_cb);
    GemvGroup g{};
    g.n_mats = 1;
    g.ct = p.CT;
    const bool resy = add == Y;
    // the partial sums travel in the basis slot (kMode 4)
    g.m[0] = GemvMat{hdr, levels, zp, scales, nullptr, Y, resy ? nullptr : add, (int)N, (int)p.grid};
    const size_t smem = panel_smem((int)n_cb, true);
    const hipStream_t st = as_stream(stream);
    auto run = [&](auto hb) {
        constexpr int HB = decltype(hb)::value;
        if (resy) launch_panel<HB, 4, kXPlain, false, true>(p, smem, st, m, g, nullptr, (int)n_cb);
        else launch_panel<HB, 4, kXPlain>(p, smem, st, m, g, nullptr, (int)n_cb);
    };
    if (hdr_bytes == 8) run(std::integral_constant<int, 8>{});
    else run(std::integral_constant<int, 6>{});
    return check_launch(what);
}
