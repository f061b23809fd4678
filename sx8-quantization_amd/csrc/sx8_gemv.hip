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
//   * the K loop is software-pipelined (rotating record buffers, unconditional clamped
//     loads) and panels are renumbered per XCD (see k_gemv_panel).
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
constexpr int kLdsMaxKb = 640;     // activation table staged in LDS up to this many K blocks

// Z of one (row, kb, j) follows the reference's warp tree: products x_t * b_t, then
// pairwise sums over lane offsets 16, 8, 4, 2, 1 (cuda/sx8_decode1_v3.cu:53-63), then
// scale * sum.
// One thread per (row m, kb): both Z values, x read once as four 16-byte vectors (the
// row's tail past K is zero), products and the reference tree in registers.
// Optional outputs: Z as f32 pairs or as split fp16 hi/lo pairs (hl), and the prefill
// GEMM's packed copy of X (Xp != nullptr): for each 32-row group G and block kb a 2 KB
// chunk [k-step st][MFMA lane l = 32 hf + r][8 values] holding X[32 G + r][32 kb + 16 hf +
// 8 st .. + 8], so the GEMM reads every A operand as one contiguous 1 KB wave load.  When
// packing, the grid covers the rows up to the next multiple of 32 (rows >= M pack zeros).
template <bool kZ, bool kPack>
__global__ __launch_bounds__(256) void k_compute_z(const uint16_t* __restrict__ X, int64_t M,
                                                   int64_t ldx, int64_t K,
                                                   const float* __restrict__ basis,
                                                   const float* __restrict__ scales, int64_t n_cb,
                                                   bool x_vec, bool hl, float* __restrict__ Z,
                                                   uint16_t* __restrict__ Xp) {
#pragma clang fp contract(off)
    const int64_t gid = (int64_t)blockIdx.x * 256 + threadIdx.x;
    const int64_t rows = kPack ? (M + 31) / 32 * 32 : M;
    if (gid >= rows * n_cb) return;
    // packing: the row within its 32-row group runs fastest, so a wave's packed stores
    // fill whole 512-byte runs; otherwise kb runs fastest (contiguous X reads, Z writes)
    int64_t m, kb;
    if constexpr (kPack) {
        const int64_t rest = gid >> 5;
        kb = rest % n_cb;
        m = (rest / n_cb) * 32 + (gid & 31);
    } else {
        m = gid / n_cb;
        kb = gid - m * n_cb;
    }
    const bool row_ok = m < M;
    const uint16_t* x = X + min(m, M - 1) * ldx + kb * 32;
    const int kmax = row_ok ? (int)min((int64_t)32, K - kb * 32) : 0;
    uint32_t xw[16];
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
    if constexpr (kPack) {
        const int64_t G = m >> 5;
        const int r = (int)(m & 31);
#pragma unroll
        for (int hf = 0; hf < 2; ++hf)
#pragma unroll
            for (int st = 0; st < 2; ++st) {
                uint4* dst = reinterpret_cast<uint4*>(Xp + ((G * n_cb + kb) * 2 + st) * 512 + (hf * 32 + r) * 8);
                const int q = 8 * hf + 4 * st;
                *dst = make_uint4(xw[q], xw[q + 1], xw[q + 2], xw[q + 3]);
            }
    }
    if constexpr (kZ) {
        if (!row_ok) return;
        const float4* bv = reinterpret_cast<const float4*>(basis + kb * 64);
        float z[2];
#pragma unroll
        for (int j = 0; j < 2; ++j) {
            float p[32];
#pragma unroll
            for (int q = 0; q < 8; ++q) {
                const float4 b = bv[8 * j + q];
                p[4 * q] = sx8_h2f(xw[2 * q]) * b.x;
                p[4 * q + 1] = sx8_h2f(xw[2 * q] >> 16) * b.y;
                p[4 * q + 2] = sx8_h2f(xw[2 * q + 1]) * b.z;
                p[4 * q + 3] = sx8_h2f(xw[2 * q + 1] >> 16) * b.w;
            }
#pragma unroll
            for (int off = 16; off > 0; off >>= 1)
#pragma unroll
                for (int t = 0; t < off; ++t) p[t] = p[t] + p[t + off];
            z[j] = scales[kb * 2 + j] * p[0];
        }
        const int64_t zi = m * n_cb + kb;
        if (hl)
            *reinterpret_cast<uint2*>(Z + zi * 2) = make_uint2(sx8_split_hl(z[0]), sx8_split_hl(z[1]));
        else
            *reinterpret_cast<float2*>(Z + zi * 2) = make_float2(z[0], z[1]);
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

__device__ __forceinline__ float dot2(uint32_t a, uint32_t b, float c) {
    return __builtin_amdgcn_fdot2(__builtin_bit_cast(sx8_half2, a),
                                  __builtin_bit_cast(sx8_half2, b), c, false);
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
    uint4 a;
    uint2 b;
};

typedef uint4 sx8_uint4_a8 __attribute__((aligned(8)));

template <int HB>
__device__ __forceinline__ void load_rec(BlockRec& o, const uint8_t* __restrict__ hdr,
                                         const uint8_t* __restrict__ levels, int64_t bid) {
    if constexpr (HB == 8) {
        const uint2 h = *reinterpret_cast<const uint2*>(hdr + bid * 8);
        o.lohi = h.x;
        o.cc = h.y;
    } else {
        const uint16_t* h = reinterpret_cast<const uint16_t*>(hdr + bid * 6);
        o.lohi = h[0] | ((uint32_t)h[1] << 16);
        o.cc = h[2];
    }
    o.a = *reinterpret_cast<const sx8_uint4_a8*>(levels + bid * 24);
    o.b = *reinterpret_cast<const uint2*>(levels + bid * 24 + 16);
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
__device__ __forceinline__ float block_dot(const BlockRec& o, const KbInfo& ki, const SpliceK& k) {
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
    float acc = (float)sx8_sext4(cf) * ki.z[0] + (float)sx8_sext4(cf >> 4) * ki.z[1];
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

// Table entries built inside the GEMV work-group: four threads per kb, thread q doing
// the x side of sub-block q and a quarter of both Z products (summed over the four
// threads with two xor shuffles; this Z is only used internally).
struct TabIn {
    uint4 x;
    float4 b0[2], b1[2];
    float s;
};

template <int kMode>
__device__ __forceinline__ void tab_load(TabIn& t, const uint16_t* __restrict__ X,
                                         const float* __restrict__ basis,
                                         const float* __restrict__ scales,
                                         const float* __restrict__ Zin, int kb, int q) {
    t.x = *reinterpret_cast<const uint4*>(X + (int64_t)kb * 32 + 8 * q);
    if constexpr (kMode == 1) {
        const float4* b = reinterpret_cast<const float4*>(basis + (int64_t)kb * 64 + 8 * q);
        t.b0[0] = b[0];
        t.b0[1] = b[1];
        t.b1[0] = b[8];
        t.b1[1] = b[9];
        t.s = scales[2 * kb + (q & 1)];
    } else {
        t.s = Zin[2 * kb + (q & 1)];
    }
}

template <int kMode>
__device__ __forceinline__ void tab_store(KbInfo* info, const TabIn& t, int kb, int q, bool ok) {
#pragma clang fp contract(off)
    float z = t.s;
    if constexpr (kMode == 1) {
        const uint32_t xw[4] = {t.x.x, t.x.y, t.x.z, t.x.w};
        const float* b0 = reinterpret_cast<const float*>(t.b0);
        const float* b1 = reinterpret_cast<const float*>(t.b1);
        float z0 = 0.f, z1 = 0.f;
#pragma unroll
        for (int i = 0; i < 8; ++i) {
            const float xf = sx8_h2f(xw[i >> 1] >> (16 * (i & 1)));
            z0 += xf * b0[i];
            z1 += xf * b1[i];
        }
        z0 += __shfl_xor(z0, 1);
        z1 += __shfl_xor(z1, 1);
        z0 += __shfl_xor(z0, 2);
        z1 += __shfl_xor(z1, 2);
        z = t.s * (q == 0 ? z0 : z1);
    }
    if (!ok) return;
    fill_x_side(info[kb], q, t.x);
    if (q < 2) info[kb].z[q] = z;
}

// M = 1 GEMV over column panels.  A 512-thread work-group owns CT = 2^ct_log2
// consecutive columns over the whole K: lane (c, j) = (column c, K slice j), c fastest,
// so for each kb the CT lanes of a slice read CT consecutive records, and slice j walks
// kb = j + r S (S = 512 / CT) for r < R = ceil(n_cb / S).  Slices meet in LDS and are
// summed in a fixed order: nothing leaves a work-group before the final store, so
// there are no device-scope fences or atomics and results are deterministic.
//
// Latency schedule: the table inputs go out first, then the records of rounds 0 .. D
// (D + 1 rotating buffers), then the table is built while they stream in.  In the main
// loop the buffer just consumed is refilled with round r + D + 1, so D + 1 rounds are
// in flight while one is decoded.  Every load is unconditional (indices clamped,
// contributions past the end masked): the loop body is straight-line code, which keeps
// the compiler's memory-wait counts exact, and scheduling barriers keep each refill
// ahead of the decode that follows it.
//
// kMode: 0 = copy the table k_kbinfo wrote into LDS; 1 = build it computing Z; 2 = build
// it with Z from Zin; 3 = read k_kbinfo's table from global memory (n_cb > kLdsMaxKb).  Work-groups go to the 8 XCDs round-robin by block index; panels
// are renumbered so each XCD gets a contiguous column range and neighbouring panels
// share their header cache lines in one L2.
template <int HB, int kMode, int D>
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
    const int G = gridDim.x, xcd = blockIdx.x & 7;
    int panel = blockIdx.x >> 3;
    for (int y = 0; y < xcd; ++y) panel += (G - y + 7) >> 3;
    const int n = panel * CT + c;
    const bool valid = n < N;
    const int64_t nn = valid ? n : N - 1;
    const int R = (n_cb + S - 1) / S;
    auto kbc = [&](int r) { return min(j + r * S, n_cb - 1); };
    auto bid = [&](int r) { return (int64_t)kbc(r) * N + nn; };

    const int n_units = n_cb * 4;
    TabIn tin;
    if constexpr (kMode == 1 || kMode == 2) {
        const int u = min(tid, n_units - 1);
        tab_load<kMode>(tin, X, basis, scales, Zin, u >> 2, u & 3);
    }
    BlockRec buf[D + 1];
#pragma unroll
    for (int i = 0; i <= D; ++i) load_rec<HB>(buf[i], hdr, levels, bid(i));
    if constexpr (kMode == 0) {
        const uint4* src = reinterpret_cast<const uint4*>(table);
        uint4* dst = reinterpret_cast<uint4*>(info);
        for (int i = tid; i < n_cb * 7; i += kPanelThreads) dst[i] = src[i];
    } else if constexpr (kMode == 1 || kMode == 2) {
        tab_store<kMode>(info, tin, min(tid, n_units - 1) >> 2, tid & 3, tid < n_units);
        for (int u0 = kPanelThreads; u0 < n_units; u0 += kPanelThreads) {
            const int u = min(u0 + tid, n_units - 1);
            tab_load<kMode>(tin, X, basis, scales, Zin, u >> 2, u & 3);
            tab_store<kMode>(info, tin, u >> 2, u & 3, u0 + tid < n_units);
        }
    }
    __syncthreads();

    const KbInfo* ti = kMode == 3 ? table : info;
    const SpliceK sk = splice_consts();
    float acc = 0.f;
    auto step = [&](const BlockRec& o, int r) {
        const float v = block_dot(o, ti[kbc(r)], sk);
        acc += (j + r * S < n_cb) ? v : 0.f;
    };
    int r = 0;
    for (; r + D < R; r += D + 1) {
#pragma unroll
        for (int i = 0; i <= D; ++i) {
            step(buf[i], r + i);
            __builtin_amdgcn_sched_barrier(0);
            load_rec<HB>(buf[i], hdr, levels, bid(r + i + D + 1));
            __builtin_amdgcn_sched_barrier(0);
        }
    }
#pragma unroll
    for (int i = 0; i < D; ++i)
        if (r + i < R) step(buf[i], r + i);

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

// Panel width: 16 columns (a slice reads 384 contiguous level bytes, three cache lines),
// 32 when that still leaves >= 256 work-groups and the K loop is short, 8 when 16 would
// leave fewer than 128 work-groups.
inline int panel_ct_log2(int N, int n_cb) {
    const int g16 = (N + 15) / 16;
    if (g16 < 128) return N >= 1024 ? 3 : 2;
    if ((N + 31) / 32 >= 256 && n_cb <= 96) return 5;
    return 4;
}

template <int HB, int kMode>
void launch_panel(int D, dim3 grid, size_t smem, hipStream_t st, const uint16_t* X,
                  const uint8_t* hdr, const uint8_t* levels, const float* basis,
                  const float* scales, const float* Zin, const KbInfo* table, float* Y, int N,
                  int n_cb, int lg) {
    if (D == 2)
        hipLaunchKernelGGL((k_gemv_panel<HB, kMode, 2>), grid, dim3(kPanelThreads), smem, st, X,
                           hdr, levels, basis, scales, Zin, table, Y, N, n_cb, lg);
    else
        hipLaunchKernelGGL((k_gemv_panel<HB, kMode, 1>), grid, dim3(kPanelThreads), smem, st, X,
                           hdr, levels, basis, scales, Zin, table, Y, N, n_cb, lg);
}

template <int HB>
int32_t launch_gemv(const uint16_t* X, const uint8_t* hdr, const uint8_t* levels,
                    const float* basis, const float* scales, const float* Zin, float* Zout,
                    int N, int n_cb, float* Y, KbInfo* table, hipStream_t st) {
    using namespace sx8;
    const int lg = panel_ct_log2(N, n_cb);
    const int S = kPanelThreads >> lg;
    const int R = (n_cb + S - 1) / S;
    const int D = R >= 6 ? 2 : 1;
    const dim3 grid((N + (1 << lg) - 1) >> lg);
    const bool lds = n_cb <= kLdsMaxKb;
    const size_t smem = sizeof(float) * kPanelThreads + (lds ? sizeof(KbInfo) * (size_t)n_cb : 0);
    if (!Zout && lds) {   // single launch: the table is built inside every work-group
        if (Zin)
            launch_panel<HB, 2>(D, grid, smem, st, X, hdr, levels, basis, scales, Zin, table, Y,
                                N, n_cb, lg);
        else
            launch_panel<HB, 1>(D, grid, smem, st, X, hdr, levels, basis, scales, Zin, table, Y,
                                N, n_cb, lg);
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
        launch_panel<HB, 0>(D, grid, smem, st, X, hdr, levels, basis, scales, Zin, table, Y, N,
                            n_cb, lg);
    else
        launch_panel<HB, 3>(D, grid, smem, st, X, hdr, levels, basis, scales, Zin, table, Y, N,
                            n_cb, lg);
    return check_launch("sx8_gemv");
}

}  // namespace

extern "C" int64_t sx8_gemv_workspace_bytes(int64_t n_cb) {
    return n_cb > 0 ? n_cb * (int64_t)sizeof(KbInfo) : 0;
}

int32_t sx8::compute_z(const uint16_t* X, int64_t M, int64_t ldx, int64_t K, const float* basis,
                       const float* scales, int64_t n_cb, void* Z, bool hl, uint16_t* xpack,
                       hipStream_t st) {
    const int64_t rows = xpack ? (M + 31) / 32 * 32 : M;
    const int64_t grid = (rows * n_cb + 255) / 256;
    if (grid > 0x7FFFFFFF) return fail(SX8_ERR_UNSUPPORTED, "compute_z: too large");
    const bool x_vec = aligned(X, 16) && ldx % 8 == 0;
    float* Zf = reinterpret_cast<float*>(Z);
    if (Z && xpack)
        hipLaunchKernelGGL((k_compute_z<true, true>), dim3((unsigned)grid), dim3(256), 0, st, X, M, ldx,
                           K, basis, scales, n_cb, x_vec, hl, Zf, xpack);
    else if (Z)
        hipLaunchKernelGGL((k_compute_z<true, false>), dim3((unsigned)grid), dim3(256), 0, st, X, M,
                           ldx, K, basis, scales, n_cb, x_vec, hl, Zf, xpack);
    else if (xpack)
        hipLaunchKernelGGL((k_compute_z<false, true>), dim3((unsigned)grid), dim3(256), 0, st, X, M,
                           ldx, K, basis, scales, n_cb, x_vec, hl, Zf, xpack);
    return check_launch("compute_z");
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
