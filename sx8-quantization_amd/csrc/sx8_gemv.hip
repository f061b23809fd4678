// sx8_gemv.hip -- PCA precompute (Z) and the M = 1 decode GEMV on the v4.4 layout.
//
// Reference roles: compute_z44 / compute_z44_batch (cuda/sx8_decode1_v3.cu:44-65,
// cuda/sx8_gemm_compact.cu:28-50) and decode1_v44_kernel (cuda/sx8_decode1_v3.cu:75-167)
// with its wrappers decode1_v44 / decode1_v44_combined (:197-246).
//
// GEMV design (gfx950, HBM-bound):
//   * k_gemv_panel streams the weights.  A 512-thread work-group owns CT consecutive
//     columns over the whole K: lane (c, j) = (column c, K slice j), c fastest, so for
//     each kb the CT lanes of a slice read CT consecutive 24-byte level records and
//     header records (contiguous runs in the kb-major layout) and slice j walks
//     kb = j, j + S, ... (S = 512 / CT) four blocks per round.  Slices meet in LDS and
//     are summed in slice order: nothing leaves a work-group before the final store,
//     so there are no device-scope fences or atomics and results are deterministic.
//   * every block's decode needs the activation side of its kb (x pairs, sub-block
//     sums of x, splice biases, Z0/Z1): a 112-byte table entry per kb, built in LDS by
//     each work-group while its first weight loads are in flight (one launch).  When
//     the caller wants Z back (the combined entry point), k_kbinfo builds the table
//     once with the reference's summation tree -- Z bit-identical to compute_z44 --
//     and the panel kernel copies it in.
//   * per 8-weight sub-block the core dot sum_i x_i (rlo + step lv_i) becomes
//     rlo * Sx + step * (sum x lv) with sum x lv from fp16 "splices" and
//     v_dot2_f32_f16 (see block_dot); PCA is applied per block through Z
//     (docs/SX8_FLASH_V4_3_SPEC.md:49-61).
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

// Constant part of the fp16 splices of block_dot for weight pair i: nibble splice
// (4096 for pairs 0, 2; 256 for pairs 1, 3) + quad splice (16, 64, 256, 1024).
__device__ constexpr float kSpliceBias[4] = {4.f * 1024.f + 16.f, 4.f * 64.f + 64.f,
                                             4.f * 1024.f + 256.f, 4.f * 64.f + 1024.f};

// x pairs, sub-block sums and splice biases of one (kb, sb) from its 8 x values.
__device__ __forceinline__ void fill_x_side(KbInfo& out, int sb, const uint4 xv) {
#pragma clang fp contract(off)
    const uint32_t xw[4] = {xv.x, xv.y, xv.z, xv.w};
    float xf[8];
#pragma unroll
    for (int i = 0; i < 8; ++i) xf[i] = sx8_h2f(xw[i >> 1] >> (16 * (i & 1)));
    float s = 0.f, b = 0.f;
#pragma unroll
    for (int i = 0; i < 8; ++i) s += xf[i];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const uint32_t a = (xw[i >> 1] >> (16 * (i & 1))) & 0xFFFFu;            // x[i]
        const uint32_t c = (xw[(i + 4) >> 1] >> (16 * (i & 1))) & 0xFFFFu;      // x[i+4]
        out.xp[4 * sb + i] = a | (c << 16);
        b += (xf[i] + xf[i + 4]) * kSpliceBias[i];
    }
    out.sx[sb] = s;
    out.nbias[sb] = -b;
}

constexpr int kPanelThreads = 512;
constexpr int kUnroll = 4;
constexpr int kLdsMaxKb = 640;     // table staged in LDS up to 60 KB, read from L2 beyond

// Z of one (row, kb, j) with the reference's warp tree: products x_t * b_t, then
// pairwise sums over lane offsets 16, 8, 4, 2, 1 (cuda/sx8_decode1_v3.cu:53-63),
// then scale * sum.  One thread does the whole tree (used for M > 1 rows).
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

// Activation-side table, one 32-lane group per kb (8 kb per 256-thread block).
// Lane t: product x_t * b_jt for j = 0, 1 and the xor tree (bit-identical Z); lanes
// 0..15 build one x pair each, lanes 16..19 one sub-block sum each.
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

__device__ __forceinline__ float dot2(uint32_t a, uint32_t b, float c) {
    return __builtin_amdgcn_fdot2(__builtin_bit_cast(sx8_half2, a),
                                  __builtin_bit_cast(sx8_half2, b), c, false);
}

// fp32 contribution of one block (one column, one kb) to its output.
// PCA through Z, then per sub-block rlo * Sx + step * sum_i x_i lv_i, with
// rlo/rhi/step in the reference's float32 branchless form (cuda/sx8_decode1_v3.cu:
// 108-117) and sum_i x_i lv_i = 4 * sum x nib + sum x quad computed from fp16 splices:
// a nibble or quad is or-ed into the mantissa of an fp16 constant whose last mantissa
// bit is worth the field's weight, e.g. (H & 0x000F000F) | 0x64006400 holds
// (1024 + nib_0, 1024 + nib_4).  Pair i uses constants 1024/64/1024/64 for the
// nibbles (bits 0, 4, 8, 12 of H after an 8-bit shift for pairs 2-3) and 16/64/256/1024
// for the quads (bits 6, 4, 2, 0 of each spread lo byte); v_dot2_f32_f16 multiplies
// two splices by an x pair, and the constant offsets, weighted by x, are the
// per-sub-block `bias` of the activation table.  All spliced values are exact fp16.
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

// fp32 contribution of one block (one column, one kb) to its output: PCA through Z,
// then per 8-weight sub-block rlo * Sx + step * sum_i x_i lv_i.
//
// sum_i x_i lv_i (lv = 4 nib + quad) comes from fp16 "splices": a field is or-ed into
// the mantissa of an fp16 constant whose last mantissa bit is worth the field's
// weight in lv, e.g. (H & 0x000F000F) | 0x6C006C00 = (4096 + 4 nib_0, 4096 + 4 nib_4)
// (exponent 12: ulp 4).  Nibble pairs use 4096/256/4096/256 (bits 0/4 of H and of
// H >> 8), quad pairs 16/64/256/1024 (bits 6/4/2/0 of each spread lo byte).  Eight
// v_dot2_f32_f16 per sub-block multiply the splices by x pairs into one fp32 sum that
// starts at -sum x * constants (the table's nbias), leaving sum x lv.  Every spliced
// value is exact in fp16.
//
// Fast path (dmax >= dmin): rlo = lo + q * {0,0,3,1}[s], step = 0.015873 * (hi - lo)
// * {1, 1/4, 1/4, 1/2}[s] (the strategy range widths), both looked up with bfe on
// packed byte tables.  It matches the reference's float32 form (cuda/sx8_decode1_v3.cu:
// 108-117) to rounding, except that the 1e-10 step floor is not applied: the floor
// only binds when hi - lo < 1.3e-8, where it moves the block's contribution by at most
// 1e-10 * sum|x| * 63.  Blocks with hi < lo or NaN endpoints, where the floor changes
// the result, take block_dot_exact (see k_gemv_panel).
__device__ __forceinline__ float block_dot_fast(float lo, float hi, uint32_t cfg, uint32_t cf,
                                                const uint32_t H[4], const uint32_t Pw[2],
                                                const KbInfo& ki, const SpliceK& k) {
    const float d = hi - lo;
    const float q = d * 0.25f;
    const float cd = d * 0.015873f;
    float acc = (float)sx8_sext4(cf) * ki.z[0] + (float)sx8_sext4(cf >> 4) * ki.z[1];
#pragma unroll
    for (int sb = 0; sb < 4; ++sb) {
        const uint32_t sh = ((cfg >> (2 * sb)) & 3u) << 3;             // 8 * strategy
        const float k1 = (float)__builtin_amdgcn_ubfe(0x01030000u, sh, 8);   // 0,0,3,1
        const int e = __builtin_amdgcn_sbfe((int)0xFFFEFE00u, sh, 8);        // 0,-2,-2,-1
        const float rlo = lo + q * k1;
        const float step = __builtin_ldexpf(cd, e);
        const uint32_t h = H[sb];
        const uint32_t h8 = h >> 8;
        const uint32_t P = __builtin_amdgcn_perm(0u, Pw[sb >> 1], (sb & 1) ? k.sel_odd : k.sel_even);
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
        acc = __builtin_fmaf(step, t, acc);
    }
    return acc;
}

// Same contribution with the reference's float32 rlo/rhi/step and its 1e-10 floor
// (cuda/sx8_decode1_v3.cu:108-117), for waves holding a block with hi < lo or a NaN.
__device__ __forceinline__ float block_dot_exact(float lo, float hi, uint32_t cfg, uint32_t cf,
                                              const uint32_t H[4], const uint32_t Pw[2],
                                              const KbInfo& ki, const SpliceK& k) {
    const float q = (hi - lo) * 0.25f;
    float acc = (float)sx8_sext4(cf) * ki.z[0] + (float)sx8_sext4(cf >> 4) * ki.z[1];
#pragma unroll
    for (int sb = 0; sb < 4; ++sb) {
        const uint32_t s = (cfg >> (2 * sb)) & 3u;
        const float k1 = (float)((0x1300u >> (4 * s)) & 0xFu);   // 0,0,3,1
        const float k2 = (float)((0x1030u >> (4 * s)) & 0xFu);   // 0,3,0,1
        const float rlo = lo + q * k1;
        const float rhi = hi - q * k2;
        float step = (rhi - rlo) * 0.015873f;
        if (step < 1e-10f) step = 1e-10f;
        const uint32_t h = H[sb];
        const uint32_t h8 = h >> 8;
        const uint32_t P = __builtin_amdgcn_perm(0u, Pw[sb >> 1], (sb & 1) ? k.sel_odd : k.sel_even);
        const uint32_t* xp = ki.xp + 4 * sb;
        float t = dot2((h & k.n_lo) | 0x6C006C00u, xp[0], ki.nbias[sb]);
        t = dot2((h & k.n_hi) | 0x5C005C00u, xp[1], t);
        t = dot2((h8 & k.n_lo) | 0x6C006C00u, xp[2], t);
        t = dot2((h8 & k.n_hi) | 0x5C005C00u, xp[3], t);
        t = dot2((P & k.q0) | 0x4C004C00u, xp[0], t);
        t = dot2((P & k.q1) | 0x54005400u, xp[1], t);
        t = dot2((P & k.q2) | 0x5C005C00u, xp[2], t);
        t = dot2((P & k.q3) | 0x64006400u, xp[3], t);
        acc += rlo * ki.sx[sb] + step * t;
    }
    return acc;
}

// One kb's raw records for one column: hd = {dmin | dmax << 16, config | coeff << 8},
// lv = the 24 level bytes.
template <int HB>
__device__ __forceinline__ void load_block(const uint8_t* __restrict__ hdr,
                                           const uint8_t* __restrict__ levels, int64_t bid,
                                           uint32_t hd[2], uint2 lv[3]) {
    if constexpr (HB == 8) {
        const uint2 h = *reinterpret_cast<const uint2*>(hdr + bid * 8);
        hd[0] = h.x;
        hd[1] = h.y;
    } else {
        const uint16_t* h = reinterpret_cast<const uint16_t*>(hdr + bid * 6);
        hd[0] = h[0] | ((uint32_t)h[1] << 16);
        hd[1] = h[2];
    }
    const uint2* lp = reinterpret_cast<const uint2*>(levels + bid * 24);
    lv[0] = lp[0];
    lv[1] = lp[1];
    lv[2] = lp[2];
}

// Activation table for all n_cb blocks, built by one work-group in its LDS: the x side
// from one thread per (kb, sb), Z from one thread per (kb, j) (a left-to-right sum of
// the 32 products, or a copy of Zin).  Used by the panel GEMV when no Z output is
// requested; the entry point that must return Z runs k_kbinfo (reference tree) instead.
template <bool kZGiven>
__device__ __forceinline__ void stage_table(KbInfo* __restrict__ info,
                                            const uint16_t* __restrict__ X,
                                            const float* __restrict__ basis,
                                            const float* __restrict__ scales,
                                            const float* __restrict__ Zin, int n_cb) {
    const int tid = threadIdx.x;
    for (int u = tid; u < n_cb * 4; u += kPanelThreads)
        fill_x_side(info[u >> 2], u & 3,
                    *reinterpret_cast<const uint4*>(X + (int64_t)(u >> 2) * 32 + 8 * (u & 3)));
    for (int u = tid; u < n_cb * 2; u += kPanelThreads) {
        const int kb = u >> 1, jj = u & 1;
        float z;
        if constexpr (kZGiven) {
            z = Zin[u];
        } else {
            const uint4* xv = reinterpret_cast<const uint4*>(X + (int64_t)kb * 32);
            const float4* bv = reinterpret_cast<const float4*>(basis + (int64_t)kb * 64 + 32 * jj);
            float a = 0.f;
#pragma unroll
            for (int q = 0; q < 4; ++q) {
                const uint4 xx = xv[q];
                const float4 b0 = bv[2 * q], b1 = bv[2 * q + 1];
                a += sx8_h2f(xx.x) * b0.x + sx8_h2f(xx.x >> 16) * b0.y;
                a += sx8_h2f(xx.y) * b0.z + sx8_h2f(xx.y >> 16) * b0.w;
                a += sx8_h2f(xx.z) * b1.x + sx8_h2f(xx.z >> 16) * b1.y;
                a += sx8_h2f(xx.w) * b1.z + sx8_h2f(xx.w >> 16) * b1.w;
            }
            z = scales[u] * a;
        }
        info[kb].z[jj] = z;
    }
}

// kMode: 0 = read the table k_kbinfo wrote to global memory; 1 = build it in LDS
// computing Z; 2 = build it in LDS copying Zin.
template <int HB, int kMode>
__global__ __launch_bounds__(kPanelThreads) void k_gemv_panel(
    const uint16_t* __restrict__ X, const uint8_t* __restrict__ hdr,
    const uint8_t* __restrict__ levels, const float* __restrict__ basis,
    const float* __restrict__ scales, const float* __restrict__ Zin,
    const KbInfo* __restrict__ table, float* __restrict__ Y, int N, int n_cb, int ct_log2) {
    extern __shared__ __align__(16) unsigned char smem[];
    float* red = reinterpret_cast<float*>(smem);
    KbInfo* info = reinterpret_cast<KbInfo*>(smem + sizeof(float) * kPanelThreads);
    const int tid = threadIdx.x;
    const int CT = 1 << ct_log2;
    const int S = kPanelThreads >> ct_log2;
    const int c = tid & (CT - 1);
    const int j = tid >> ct_log2;
    const int n = blockIdx.x * CT + c;
    const bool valid = n < N;
    const int64_t nn = valid ? n : N - 1;

    // the first round of this lane's weight loads goes out before the table is built
    uint32_t hd[kUnroll][2];
    uint2 lv[kUnroll][3];
#pragma unroll
    for (int u = 0; u < kUnroll; ++u) {
        const int kb = j + u * S;
        if (kb < n_cb) load_block<HB>(hdr, levels, (int64_t)kb * N + nn, hd[u], lv[u]);
    }
    const KbInfo* ti = table;
    if constexpr (kMode == 0) {
        if (n_cb <= kLdsMaxKb) {
            const uint4* src = reinterpret_cast<const uint4*>(table);
            uint4* dst = reinterpret_cast<uint4*>(info);
            for (int i = tid; i < n_cb * 7; i += kPanelThreads) dst[i] = src[i];
            ti = info;
        }
    } else {
        stage_table<kMode == 2>(info, X, basis, scales, Zin, n_cb);
        ti = info;
    }
    __syncthreads();

    const SpliceK sk = splice_consts();
    float acc = 0.f;
    for (int kb0 = j;;) {
#pragma unroll
        for (int u = 0; u < kUnroll; ++u) {
            const int kb = kb0 + u * S;
            if (kb < n_cb) {
                const uint32_t H[4] = {lv[u][0].x, lv[u][0].y, lv[u][1].x, lv[u][1].y};
                const uint32_t Pw[2] = {lv[u][2].x, lv[u][2].y};
                const float lo = sx8_h2f(hd[u][0]), hi = sx8_h2f(hd[u][0] >> 16);
                const uint32_t cfg = hd[u][1] & 0xFFu, cf = (hd[u][1] >> 8) & 0xFFu;
                if (__builtin_amdgcn_ballot_w64(!(hi >= lo)) == 0)   // wave-uniform
                    acc += block_dot_fast(lo, hi, cfg, cf, H, Pw, ti[kb], sk);
                else
                    acc += block_dot_exact(lo, hi, cfg, cf, H, Pw, ti[kb], sk);
            }
        }
        kb0 += kUnroll * S;
        if (kb0 >= n_cb) break;
#pragma unroll
        for (int u = 0; u < kUnroll; ++u) {
            const int kb = kb0 + u * S;
            if (kb < n_cb) load_block<HB>(hdr, levels, (int64_t)kb * N + nn, hd[u], lv[u]);
        }
    }

    // slices -> columns: xor tree over the slices inside each wave (lanes c, c + CT,
    // ...), then the 8 wave sums in wave order; fixed order, so deterministic
    for (int off = CT; off < 64; off <<= 1) acc += __shfl_xor(acc, off);
    const int wave = tid >> 6;
    if ((tid & 63) < CT) red[wave * CT + c] = acc;
    __syncthreads();
    if (tid < CT && valid) {
        float t = 0.f;
#pragma unroll
        for (int w = 0; w < kPanelThreads / 64; ++w) t += red[w * CT + tid];
        Y[n] = t;
    }
}

// Panel width: the widest power of two <= 64 that still gives >= 256 work-groups (one
// per CU); wider panels amortise the per-work-group table build over more columns.
inline int panel_ct_log2(int N) {
    int lg = 6;
    while (lg > 2 && (N + (1 << lg) - 1) / (1 << lg) < 256) --lg;
    return lg;
}

template <int HB>
int32_t launch_gemv(const uint16_t* X, const uint8_t* hdr, const uint8_t* levels,
                    const float* basis, const float* scales, const float* Zin, float* Zout,
                    int N, int n_cb, float* Y, KbInfo* table, hipStream_t st) {
    using namespace sx8;
    const int lg = panel_ct_log2(N);
    const dim3 grid((N + (1 << lg) - 1) >> lg);
    const bool lds = n_cb <= kLdsMaxKb;
    const size_t smem = sizeof(float) * kPanelThreads + (lds ? sizeof(KbInfo) * (size_t)n_cb : 0);
    if (!Zout && lds) {   // single launch: the table is built inside every work-group
        if (Zin)
            hipLaunchKernelGGL((k_gemv_panel<HB, 2>), grid, dim3(kPanelThreads), smem, st, X, hdr,
                               levels, basis, scales, Zin, table, Y, N, n_cb, lg);
        else
            hipLaunchKernelGGL((k_gemv_panel<HB, 1>), grid, dim3(kPanelThreads), smem, st, X, hdr,
                               levels, basis, scales, Zin, table, Y, N, n_cb, lg);
        return check_launch("sx8_gemv");
    }
    const dim3 tgrid((n_cb + 7) / 8);
    if (Zin)
        hipLaunchKernelGGL(k_kbinfo<true>, tgrid, dim3(256), 0, st, X, basis, scales, Zin, Zout,
                           n_cb, table);
    else
        hipLaunchKernelGGL(k_kbinfo<false>, tgrid, dim3(256), 0, st, X, basis, scales, Zin, Zout,
                           n_cb, table);
    hipLaunchKernelGGL((k_gemv_panel<HB, 0>), grid, dim3(kPanelThreads), smem, st, X, hdr, levels,
                       basis, scales, Zin, table, Y, N, n_cb, lg);
    return check_launch("sx8_gemv");
}

}  // namespace

extern "C" int64_t sx8_gemv_workspace_bytes(int64_t n_cb) {
    return n_cb > 0 ? n_cb * (int64_t)sizeof(KbInfo) : 0;
}

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
    const int64_t need = sx8_gemv_workspace_bytes(n_cb);
    KbInfo* table = reinterpret_cast<KbInfo*>(workspace);
    if (table) {
        if (workspace_bytes < need || !aligned(table, 16))
            return fail(SX8_ERR_INVALID, "sx8_gemv: workspace needs %lld bytes, 16-byte aligned",
                        (long long)need);
    } else {
        void* ws = nullptr;
        const int32_t rc = device_workspace(need, &ws);
        if (rc != SX8_OK) return rc;
        table = reinterpret_cast<KbInfo*>(ws);
    }
    if (hdr_bytes == 8)
        return launch_gemv<8>(X, hdr, levels, basis, scales, Z_in, Z_out, (int)N, (int)n_cb, Y,
                              table, as_stream(stream));
    return launch_gemv<6>(X, hdr, levels, basis, scales, Z_in, Z_out, (int)N, (int)n_cb, Y, table,
                          as_stream(stream));
}
