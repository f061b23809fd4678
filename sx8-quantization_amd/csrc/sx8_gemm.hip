// sx8_gemm.hip -- prefill GEMM Y (M, N) f32 = X (M, K) fp16 . W^T with W in S-X8 blocks.
//
// Reference roles: gemm_compact (cuda/sx8_gemm_compact.cu:55-194, CUDA-core FMAs with
// PCA applied through Z) and sx8_wmma_kernel / fused_forward (cuda/sx8_fused_wmma.cu:
// 11-154, WMMA 16x16x16 with per-weight PCA).  One kernel serves every contract: the
// PCA-free core weights rlo + step*lv are decoded in float32 straight into MFMA B
// operands, and the PCA term sum_kb c0 Z0 + c1 Z1 rides along as extra MFMA k-steps
// (Z split into fp16 hi + lo parts, coefficients as exact fp16 integers).
//
// Work decomposition (gfx950, wave64, v_mfma_f32_32x32x16_f16):
//   * a 256-thread work-group owns a 128 x 128 output tile; wave w owns the 32 columns
//     [32w, 32w + 32) for all 128 rows (four 32 x 32 accumulators, 64 registers).
//   * K advances one S-X8 block (32 weights = two MFMA k-steps) per iteration.  For a
//     32x32x16 MFMA lane l holds the B values of column l % 32 for 8 consecutive k;
//     lane half s = l / 32 decodes sub-blocks 2s (k-step 0) and 2s + 1 (k-step 1) of
//     its column, so every weight of the tile is decoded exactly once per work-group.
//     The X tile keeps sub-blocks in the order 0, 2, 1, 3 to match.
//   * X tiles (128 x 32 fp16) and Z tiles (128 rows x 4 blocks x {Z0h, Z0l, Z1h, Z1l})
//     are double-buffered in LDS.  Global loads run two blocks ahead in two register
//     stages, so no iteration waits for a load it issued itself (each iteration ends
//     with a work-group barrier, and a one-block lead left every iteration waiting for a
//     full memory latency).
//   * every 4 K blocks (and after the last one) one PCA k-step per accumulator adds
//     Zhl (rows x 16) . C (16 x columns), C = the blocks' signed coefficient nibbles.
#include "sx8_device.h"
#include "sx8_host.h"

namespace {

constexpr int kBM = 128;
constexpr int kBN = 128;
constexpr int kThreads = 256;
constexpr int kXPitch = 40;   // fp16 per LDS row of an X tile: 32 + 8 pad (conflict-free b128 reads)
constexpr int kZPitch = 24;   // fp16 per LDS row of a Z tile: 16 + 8 pad

typedef float sx8_float16v __attribute__((ext_vector_type(16)));
typedef uint32_t sx8_u32x4 __attribute__((ext_vector_type(4)));

// Weight sources: the v4.4 layout (hdr + levels) or the kb-major split arrays.
struct WeightSrc {
    const uint8_t* hdr;
    const uint8_t* levels;
    const uint16_t* dmin;
    const uint16_t* dmax;
    const uint8_t* config;
    const uint8_t* coeff;
    const uint8_t* hi;
    const uint8_t* lo;
};

// The part of one block a lane needs, as loaded (no arithmetic on freshly loaded values,
// so prefetches stay in flight until use): v4.4 -> lohi = dmin | dmax << 16, cc = config |
// coeff << 8; split arrays -> lohi = dmin, hi16 = dmax, cc = config, cf = coeff.  Then the
// hi-nibble bytes of sub-blocks 2s, 2s + 1 and their four lo-quad bytes.
struct LaneRec {
    uint32_t lohi, hi16, cc, cf;
    uint2 h;
    uint32_t p;
};

// endpoints (dmin | dmax << 16) and config of a loaded record
template <bool kSplit>
__device__ __forceinline__ void rec_unpack(const LaneRec& r, uint32_t& lohi, uint32_t& cfg) {
    if constexpr (kSplit) {
        lohi = (r.lohi & 0xFFFFu) | (r.hi16 << 16);
        cfg = r.cc & 0xFFu;
    } else {
        lohi = r.lohi;
        cfg = r.cc & 0xFFu;
    }
}

// Core weights (rlo + step * lv, float32, then RNE to fp16) of one 8-weight sub-block in
// natural k order: out[j] = (w[2j], w[2j+1]).  H holds the sub-block's 8 nibbles (weight
// t at bits 4t), P its two quad bytes (weight t at bits 8(t >> 2) + 6 - 2(t & 3)).  The
// levels of the even and the odd weights are assembled as bytes and widened with
// v_cvt_f32_ubyte.
__device__ __forceinline__ sx8_half8 decode_sub(uint32_t H, uint32_t P, float rlo, float step) {
    const uint32_t x = __builtin_amdgcn_perm(0u, P, 0x01010000u);        // P0, P0, P1, P1
    const uint32_t qe = ((x >> 6) & 0x00030003u) | ((x >> 2) & 0x03000300u);   // q0 q2 q4 q6
    const uint32_t qo = ((x >> 4) & 0x00030003u) | (x & 0x03000300u);          // q1 q3 q5 q7
    const uint32_t le = ((H & 0x0F0F0F0Fu) << 2) | qe;                         // lv0 lv2 lv4 lv6
    const uint32_t lo = (((H >> 4) & 0x0F0F0F0Fu) << 2) | qo;                  // lv1 lv3 lv5 lv7
    sx8_half8 out;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        const float we = __builtin_fmaf(step, (float)((le >> (8 * j)) & 0xFFu), rlo);
        const float wo = __builtin_fmaf(step, (float)((lo >> (8 * j)) & 0xFFu), rlo);
        out[2 * j] = (_Float16)we;
        out[2 * j + 1] = (_Float16)wo;
    }
    return out;
}

// Range of sub-block sb: rlo = lo + q k1[s], step = max(0.015873 (rhi - rlo), 1e-10) in the
// reference's float32 form (cuda/sx8_fused_wmma.cu:70-94); the floor binds only for
// hi <= lo, where every sub-block's step is 1e-10.
__device__ __forceinline__ void sub_range(float lo, float d, float q, float m, uint32_t cfg, int sb,
                                          float& rlo, float& step) {
    const uint32_t s = (cfg >> (2 * sb)) & 3u;
    const float k1 = (float)((0x1300u >> (4 * s)) & 0xFu);        // 0, 0, 3, 1
    const int e = (int)((0x1220u >> (4 * s)) & 0xFu);             // 0, 2, 2, 1
    rlo = __builtin_fmaf(q, k1, lo);
    step = d > 0.f ? __builtin_ldexpf(m, -e) : 1e-10f;
}

// X tile of block kb into LDS: 128 rows x 4 sub-block chunks of 16 B, chunk of sub-block
// sb at position (sb & 1) * 2 + (sb >> 1).  kFast (X 16-byte aligned rows, K a multiple
// of 32): unconditional vector loads, rows >= M clamped to M - 1 (those output rows are
// never stored).  Otherwise rows >= M and columns >= K read as zero, element by element.
template <bool kFast>
__device__ __forceinline__ void load_x_chunks(const uint16_t* __restrict__ X, int M, int64_t ldx,
                                              int K, int m0, int kb, sx8_u32x4 v[2]) {
#pragma unroll
    for (int i = 0; i < 2; ++i) {
        const int c = threadIdx.x + i * kThreads;
        const int row = c >> 2, sb = c & 3;
        const int m = m0 + row;
        const int k = kb * 32 + 8 * sb;
        if constexpr (kFast) {
            v[i] = *reinterpret_cast<const sx8_u32x4*>(X + (int64_t)min(m, M - 1) * ldx + k);
        } else {
            uint32_t e[4] = {0, 0, 0, 0};
            if (m < M) {
                const uint16_t* src = X + (int64_t)m * ldx + k;
#pragma unroll
                for (int j = 0; j < 8; ++j)
                    if (k + j < K) e[j >> 1] |= (uint32_t)src[j] << (16 * (j & 1));
            }
            v[i] = sx8_u32x4{e[0], e[1], e[2], e[3]};
        }
    }
}

__device__ __forceinline__ void store_x_chunks(uint16_t* __restrict__ xs, const sx8_u32x4 v[2]) {
#pragma unroll
    for (int i = 0; i < 2; ++i) {
        const int c = threadIdx.x + i * kThreads;
        const int row = c >> 2, sb = c & 3;
        const int pos = ((sb & 1) << 1) | (sb >> 1);
        *reinterpret_cast<sx8_u32x4*>(xs + row * kXPitch + 8 * pos) = v[i];
    }
}

// One quarter (32 rows) of the Z tile of group g (blocks 4g .. 4g+3): thread t handles
// row 32 q + t / 8 and value e = t % 8 (block 4g + e / 2, basis e % 2).  Loaded from a
// clamped index; store_z_quarter zeroes rows >= M and blocks >= n_cb.  Z is split into
// fp16 hi + lo so the PCA k-step keeps ~22 bits.
__device__ __forceinline__ float load_z_quarter(const float* __restrict__ Z, int M, int n_cb, int m0,
                                                int g, int q) {
    const int m = min(m0 + 32 * q + (int)(threadIdx.x >> 3), M - 1);
    const int e = threadIdx.x & 7;
    const int kb = min(4 * g + (e >> 1), n_cb - 1);
    return Z[((int64_t)m * n_cb + kb) * 2 + (e & 1)];
}

__device__ __forceinline__ void store_z_quarter(uint16_t* __restrict__ zs, int M, int n_cb, int m0,
                                                int g, int q, float z) {
    const int row = 32 * q + (threadIdx.x >> 3);
    const int e = threadIdx.x & 7;
    if (m0 + row >= M || 4 * g + (e >> 1) >= n_cb) z = 0.f;
    const _Float16 h = (_Float16)z;
    const _Float16 l = (_Float16)(z - (float)h);
    const uint32_t v = (uint32_t)__builtin_bit_cast(uint16_t, h) |
                       ((uint32_t)__builtin_bit_cast(uint16_t, l) << 16);
    // value e -> k = 4 (e / 2) + 2 (e % 2): block-major, (Z0h, Z0l, Z1h, Z1l) per block
    *reinterpret_cast<uint32_t*>(zs + row * kZPitch + 4 * (e >> 1) + 2 * (e & 1)) = v;
}

// Work-group barrier for LDS hand-offs only: wait for this wave's LDS writes, then
// s_barrier.  __syncthreads() would also wait for every global load in flight (its
// release fence), which would undo the two-block load lead of the main loop.  The memory
// clobber keeps the compiler from moving LDS accesses across it.
__device__ __forceinline__ void lds_barrier() {
    asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
}

__device__ __forceinline__ uint32_t coeff_pair_f16(int c) {
    const uint32_t h = __builtin_bit_cast(uint16_t, (_Float16)(float)c);
    return h | (h << 16);
}

// Everything one K block needs from memory, loaded two iterations before its use: the X
// chunks of block kb (stored to LDS at the end of iteration kb - 1), this lane's weight
// record of block kb, and the Z-tile value stored at the end of iteration kb - 1.
struct Stage {
    sx8_u32x4 xv[2];
    LaneRec rec;
    float zq = 0.f;
};

// Buffer resources and per-lane byte offsets for the main loop's loads.  Everything that
// depends on the K block goes into the scalar offset of a buffer load, so the loop does no
// per-lane address arithmetic; loads past a buffer's end return zero.
typedef __amdgpu_buffer_rsrc_t sx8_rsrc;
constexpr int kRsrcFlags = 0x00020000;   // raw 32-bit buffer (gfx9 resource word 3)

__device__ __forceinline__ sx8_rsrc make_rsrc(const void* p, int64_t bytes) {
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(p), (short)0,
                                             (int)min(bytes, (int64_t)0x7FFFFFFF), kRsrcFlags);
}

struct LoopSrc {
    sx8_rsrc x, hdr, lv, z, dmin, dmax, cfg, cf, hi, lo;
    int x_off[2];      // X chunk i: row * ldx * 2 + 16 * sb
    int rec_off;       // nn (column) in blocks
    int z_off;         // Z value of quarter 0 of group 0
};

template <bool kSplit, int HB, bool kPca, bool kFast>
__device__ __forceinline__ void load_stage(Stage& st, const LoopSrc& ls,
                                           const uint16_t* __restrict__ X, int M, int64_t ldx,
                                           int K, int N, int n_cb, int m0, int s, int kb) {
    const int kc = min(kb, n_cb - 1);
    if constexpr (kFast) {
#pragma unroll
        for (int i = 0; i < 2; ++i)
            st.xv[i] = __builtin_bit_cast(sx8_u32x4,
                                          __builtin_amdgcn_raw_buffer_load_b128(ls.x, ls.x_off[i], kc * 64, 0));
    } else {
        load_x_chunks<false>(X, M, ldx, K, m0, kc, st.xv);
    }
    const int nn = ls.rec_off;
    const int rowb = kc * N;                       // first block of K row kc
    if constexpr (kSplit) {
        st.rec.lohi = __builtin_amdgcn_raw_buffer_load_b16(ls.dmin, nn * 2, rowb * 2, 0);
        st.rec.hi16 = __builtin_amdgcn_raw_buffer_load_b16(ls.dmax, nn * 2, rowb * 2, 0);
        st.rec.cc = __builtin_amdgcn_raw_buffer_load_b8(ls.cfg, nn, rowb, 0);
        st.rec.cf = __builtin_amdgcn_raw_buffer_load_b8(ls.cf, nn, rowb, 0);
        st.rec.h = __builtin_bit_cast(uint2, __builtin_amdgcn_raw_buffer_load_b64(ls.hi, nn * 16 + 8 * s, rowb * 16, 0));
        st.rec.p = __builtin_amdgcn_raw_buffer_load_b32(ls.lo, nn * 8 + 4 * s, rowb * 8, 0);
    } else {
        if constexpr (HB == 8) {
            const uint2 v = __builtin_bit_cast(uint2, __builtin_amdgcn_raw_buffer_load_b64(ls.hdr, nn * 8, rowb * 8, 0));
            st.rec.lohi = v.x;
            st.rec.cc = v.y;
        } else {
            st.rec.lohi = __builtin_amdgcn_raw_buffer_load_b32(ls.hdr, nn * 6, rowb * 6, 0);
            st.rec.cc = __builtin_amdgcn_raw_buffer_load_b16(ls.hdr, nn * 6 + 4, rowb * 6, 0);
        }
        st.rec.hi16 = st.rec.cf = 0;
        st.rec.h = __builtin_bit_cast(uint2, __builtin_amdgcn_raw_buffer_load_b64(ls.lv, nn * 24 + 8 * s, rowb * 24, 0));
        st.rec.p = __builtin_amdgcn_raw_buffer_load_b32(ls.lv, nn * 24 + 16 + 4 * s, rowb * 24, 0);
    }
    if constexpr (kPca) {
        const int i = max(kb - 1, 0);   // iteration whose end stores this value
        const int g = (i >> 2) + 1, q = i & 3;
        // value e of row 32 q + t / 8: Z[(m n_cb + 4 g + e / 2) * 2 + e % 2]; the whole offset
        // is in the vector part, so the buffer range check zeroes reads past the end
        st.zq = __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(
                                              ls.z, ls.z_off + (q * 32 * n_cb * 2 + g * 8) * 4, 0, 0));
    }
}

template <bool kSplit, int HB, bool kPca, bool kFast>
__global__ __launch_bounds__(kThreads) void k_gemm(const uint16_t* __restrict__ X, int M,
                                                   int64_t ldx, int K, WeightSrc w,
                                                   const float* __restrict__ Z, int N, int n_cb,
                                                   float* __restrict__ Y) {
    __shared__ __align__(16) uint16_t xs[2][kBM * kXPitch];
    __shared__ __align__(16) uint16_t zs[kPca ? 2 : 1][kPca ? kBM * kZPitch : 8];
    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = tid >> 6;
    const int c32 = lane & 31;
    const int s = lane >> 5;
    const int m0 = blockIdx.y * kBM;
    const int n = blockIdx.x * kBN + wave * 32 + c32;
    const bool n_ok = n < N;
    const int64_t nn = n_ok ? n : N - 1;

    sx8_float16v acc[kBM / 32];
#pragma unroll
    for (int r = 0; r < kBM / 32; ++r)
#pragma unroll
        for (int i = 0; i < 16; ++i) acc[r][i] = 0.f;

    LoopSrc ls;
    ls.x = make_rsrc(X, (int64_t)M * ldx * 2);
    const int64_t n_blk = (int64_t)N * n_cb;
    if constexpr (kSplit) {
        ls.dmin = make_rsrc(w.dmin, n_blk * 2);
        ls.dmax = make_rsrc(w.dmax, n_blk * 2);
        ls.cfg = make_rsrc(w.config, n_blk);
        ls.cf = make_rsrc(w.coeff, n_blk);
        ls.hi = make_rsrc(w.hi, n_blk * 16);
        ls.lo = make_rsrc(w.lo, n_blk * 8);
    } else {
        ls.hdr = make_rsrc(w.hdr, n_blk * HB);
        ls.lv = make_rsrc(w.levels, n_blk * 24);
    }
    if constexpr (kPca) ls.z = make_rsrc(Z, (int64_t)M * n_cb * 8);
#pragma unroll
    for (int i = 0; i < 2; ++i) {
        const int c = tid + i * kThreads;
        ls.x_off[i] = (int)((int64_t)(m0 + (c >> 2)) * ldx * 2) + 16 * (c & 3);
    }
    ls.rec_off = (int)nn;
    {
        const int e = tid & 7;
        ls.z_off = (int)(((int64_t)(m0 + (tid >> 3)) * n_cb * 2 + (e >> 1) * 2 + (e & 1)) * 4);
    }

    // prologue: stages of blocks 0 and 1 in flight, X tile 0 and the Z tile of group 0
    Stage S0, S1;
    load_stage<kSplit, HB, kPca, kFast>(S0, ls, X, M, ldx, K, N, n_cb, m0, s, 0);
    load_stage<kSplit, HB, kPca, kFast>(S1, ls, X, M, ldx, K, N, n_cb, m0, s, 1);
    if constexpr (kPca) {
#pragma unroll
        for (int q = 0; q < 4; ++q)
            store_z_quarter(zs[0], M, n_cb, m0, 0, q, load_z_quarter(Z, M, n_cb, m0, 0, q));
    }
    store_x_chunks(xs[0], S0.xv);
    __syncthreads();

    uint32_t cfa = 0, cfb = 0;
    // One K block: decode from `cur` (then refill it with block kb + 2), MFMAs on X tile
    // kb, PCA k-step at the end of a group, publish `nxt`'s X tile and Z value.
    auto body = [&](int kb, Stage& cur, const Stage& nxt) __attribute__((always_inline)) {
        uint32_t lohi, cfg;
        rec_unpack<kSplit>(cur.rec, lohi, cfg);
        const float lo = sx8_h2f(lohi), hi = sx8_h2f(lohi >> 16);
        const float d = hi - lo;
        const float q = d * 0.25f;
        const float mstep = d * 0.015873f;
        const bool live = kb < n_cb;
        sx8_half8 bop[2];
#pragma unroll
        for (int h = 0; h < 2; ++h) {
            float rlo, step;
            sub_range(lo, d, q, mstep, cfg, 2 * s + h, rlo, step);
            if (!live) rlo = step = 0.f;           // padding iteration: contributes zeros
            bop[h] = decode_sub(h ? cur.rec.h.y : cur.rec.h.x, h ? (cur.rec.p >> 16) : cur.rec.p,
                                rlo, step);
        }
        sx8_half8 cop;
        if constexpr (kPca) {
            // this lane's PCA k-step needs the coefficients of blocks 4g + 2s and 4g + 2s + 1
            // of its column: keep them as the group's blocks pass by (0 for absent blocks)
            const int j = kb & 3;
            const uint32_t cf = kSplit ? cur.rec.cf : (cur.rec.cc >> 8);
            if (live) {
                cfa = j == 2 * s ? cf : (j == 0 ? 0u : cfa);
                cfb = j == 2 * s + 1 ? cf : (j == 0 ? 0u : cfb);
            }
            const sx8_u32x4 cv = {coeff_pair_f16(sx8_sext4(cfa)), coeff_pair_f16(sx8_sext4(cfa >> 4)),
                                  coeff_pair_f16(sx8_sext4(cfb)), coeff_pair_f16(sx8_sext4(cfb >> 4))};
            cop = __builtin_bit_cast(sx8_half8, cv);
        }
        load_stage<kSplit, HB, kPca, kFast>(cur, ls, X, M, ldx, K, N, n_cb, m0, s, kb + 2);

        const uint16_t* xt = xs[kb & 1];
#pragma unroll
        for (int h = 0; h < 2; ++h)
#pragma unroll
            for (int r = 0; r < kBM / 32; ++r) {
                const sx8_half8 a = *reinterpret_cast<const sx8_half8*>(
                    xt + (32 * r + c32) * kXPitch + 8 * (2 * h + s));
                acc[r] = __builtin_amdgcn_mfma_f32_32x32x16_f16(a, bop[h], acc[r], 0, 0, 0);
            }
        if constexpr (kPca) {
            if (live && ((kb & 3) == 3 || kb == n_cb - 1)) {
                const uint16_t* zt = zs[(kb >> 2) & 1];
#pragma unroll
                for (int r = 0; r < kBM / 32; ++r) {
                    const sx8_half8 a = *reinterpret_cast<const sx8_half8*>(
                        zt + (32 * r + c32) * kZPitch + 8 * s);
                    acc[r] = __builtin_amdgcn_mfma_f32_32x32x16_f16(a, cop, acc[r], 0, 0, 0);
                }
            }
        }
        store_x_chunks(xs[(kb + 1) & 1], nxt.xv);
        if constexpr (kPca)
            store_z_quarter(zs[((kb >> 2) + 1) & 1], M, n_cb, m0, (kb >> 2) + 1, kb & 3, nxt.zq);
        lds_barrier();
    };
    for (int kb = 0; kb < n_cb; kb += 2) {
        body(kb, S0, S1);
        body(kb + 1, S1, S0);
    }

    // ---- epilogue: lane holds column n, rows 32r + (i % 4) + 4 s + 8 (i / 4)
    if (!n_ok) return;
#pragma unroll
    for (int r = 0; r < kBM / 32; ++r)
#pragma unroll
        for (int i = 0; i < 16; ++i) {
            const int m = m0 + 32 * r + (i & 3) + 4 * s + 8 * (i >> 2);
            if (m < M) Y[(int64_t)m * N + n] = acc[r][i];
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

int32_t check_shape(const char* what, int64_t M, int64_t ldx, int64_t K, int64_t N, int64_t n_cb) {
    using namespace sx8;
    if (M <= 0 || K <= 0 || N <= 0 || n_cb <= 0 || n_cb * 32 < K || (n_cb - 1) * 32 >= K ||
        ldx < K || M > 0x7FFFFFFF || N > 0x7FFFFFFF || n_cb > 0x7FFFFFFF / 64)
        return fail(SX8_ERR_INVALID, "%s: bad shape M=%lld K=%lld ldx=%lld N=%lld n_cb=%lld", what,
                    (long long)M, (long long)K, (long long)ldx, (long long)N, (long long)n_cb);
    if ((M + kBM - 1) / kBM > 65535) return fail(SX8_ERR_UNSUPPORTED, "%s: M too large", what);
    // the main loop addresses every operand with 32-bit buffer offsets
    if (M * ldx * 2 > 0x7FFFFFFF || N * n_cb * 24 > 0x7FFFFFFF || M * n_cb * 8 > 0x7FFFFFFF)
        return fail(SX8_ERR_UNSUPPORTED, "%s: operands beyond 2 GiB", what);
    return SX8_OK;
}

template <bool kSplit, bool kPca, int HB>
void launch_gemm_hb(dim3 grid, hipStream_t st, bool fast, const uint16_t* X, int64_t M,
                    int64_t ldx, int64_t K, const WeightSrc& w, const float* Z, int64_t N,
                    int64_t n_cb, float* Y) {
    if (fast)
        hipLaunchKernelGGL((k_gemm<kSplit, HB, kPca, true>), grid, dim3(kThreads), 0, st, X,
                           (int)M, ldx, (int)K, w, Z, (int)N, (int)n_cb, Y);
    else
        hipLaunchKernelGGL((k_gemm<kSplit, HB, kPca, false>), grid, dim3(kThreads), 0, st, X,
                           (int)M, ldx, (int)K, w, Z, (int)N, (int)n_cb, Y);
}

template <bool kSplit, bool kPca>
int32_t launch_gemm(const char* what, const uint16_t* X, int64_t M, int64_t ldx, int64_t K,
                    const WeightSrc& w, int32_t hdr_bytes, const float* Z, int64_t N, int64_t n_cb,
                    float* Y, hipStream_t st) {
    using namespace sx8;
    const bool fast = aligned(X, 16) && (ldx % 8 == 0) && (K % 32 == 0);
    const dim3 grid((unsigned)((N + kBN - 1) / kBN), (unsigned)((M + kBM - 1) / kBM));
    if (hdr_bytes == 8)
        launch_gemm_hb<kSplit, kPca, 8>(grid, st, fast, X, M, ldx, K, w, Z, N, n_cb, Y);
    else
        launch_gemm_hb<kSplit, kPca, 6>(grid, st, fast, X, M, ldx, K, w, Z, N, n_cb, Y);
    return check_launch(what);
}

// Z (M, n_cb, 2) f32 for the contracts that pass basis/scales, in the library's
// per-device workspace (columns k >= K of a ragged last block count as zero).
int32_t z_from_basis(const uint16_t* X, int64_t M, int64_t ldx, int64_t K, const float* basis,
                     const float* scales, int64_t n_cb, hipStream_t st, const float** Zp) {
    using namespace sx8;
    void* ws = nullptr;
    const int32_t rc = device_workspace(M * n_cb * 2 * (int64_t)sizeof(float), &ws);
    if (rc != SX8_OK) return rc;
    float* Zw = reinterpret_cast<float*>(ws);
    const int32_t zr = compute_z(X, M, ldx, K, basis, scales, n_cb, Zw, st);
    if (zr != SX8_OK) return zr;
    *Zp = Zw;
    return SX8_OK;
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
    if (!aligned(hdr, hdr_bytes == 8 ? 8 : 2) || !aligned(levels, 8) || !aligned(X, 2) ||
        !aligned(Y, 4) || !aligned(basis, 16) || !aligned(scales, 8))
        return fail(SX8_ERR_INVALID, "sx8_gemm_prefill: misaligned pointer");
    int32_t rc = check_shape("sx8_gemm_prefill", M, ldx, K, N, n_cb);
    if (rc != SX8_OK) return rc;
    const hipStream_t st = as_stream(stream);
    const float* Z = nullptr;
    rc = z_from_basis(X, M, ldx, K, basis, scales, n_cb, st, &Z);
    if (rc != SX8_OK) return rc;
    WeightSrc w{};
    w.hdr = hdr;
    w.levels = levels;
    return launch_gemm<false, true>("sx8_gemm_prefill", X, M, ldx, K, w, hdr_bytes, Z, N, n_cb, Y,
                                    st);
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
    if (!aligned(dmin, 2) || !aligned(dmax, 2) || !aligned(hi, 8) || !aligned(lo, 4) ||
        !aligned(X, 2) || !aligned(Y, 4) || !aligned(basis, 16) || !aligned(scales, 8))
        return fail(SX8_ERR_INVALID, "sx8_gemm_prefill_split: misaligned pointer");
    int32_t rc = check_shape("sx8_gemm_prefill_split", M, ldx, K, N, n_cb);
    if (rc != SX8_OK) return rc;
    const hipStream_t st = as_stream(stream);
    const float* Z = nullptr;
    rc = z_from_basis(X, M, ldx, K, basis, scales, n_cb, st, &Z);
    if (rc != SX8_OK) return rc;
    WeightSrc w{};
    w.dmin = dmin;
    w.dmax = dmax;
    w.config = config;
    w.coeff = coeff;
    w.hi = hi;
    w.lo = lo;
    return launch_gemm<true, true>("sx8_gemm_prefill_split", X, M, ldx, K, w, 6, Z, N, n_cb, Y, st);
}

extern "C" int32_t sx8_gemm_prefill_z(const uint16_t* X, int64_t M, int64_t ldx, int64_t K,
                                      const uint8_t* hdr, const uint8_t* levels, int32_t hdr_bytes,
                                      const float* Z, int64_t N, int64_t n_cb, float* Y,
                                      void* stream) {
    using namespace sx8;
    if (!X || !hdr || !levels || !Z || !Y)
        return fail(SX8_ERR_INVALID, "sx8_gemm_prefill_z: null pointer");
    if (hdr_bytes != 6 && hdr_bytes != 8)
        return fail(SX8_ERR_INVALID, "sx8_gemm_prefill_z: hdr_bytes must be 6 or 8, got %d", hdr_bytes);
    if (!aligned(hdr, hdr_bytes == 8 ? 8 : 2) || !aligned(levels, 8) || !aligned(X, 2) ||
        !aligned(Y, 4) || !aligned(Z, 4))
        return fail(SX8_ERR_INVALID, "sx8_gemm_prefill_z: misaligned pointer");
    const int32_t rc = check_shape("sx8_gemm_prefill_z", M, ldx, K, N, n_cb);
    if (rc != SX8_OK) return rc;
    WeightSrc w{};
    w.hdr = hdr;
    w.levels = levels;
    return launch_gemm<false, true>("sx8_gemm_prefill_z", X, M, ldx, K, w, hdr_bytes, Z, N, n_cb,
                                    Y, as_stream(stream));
}

extern "C" int32_t sx8_gemm_prefill_core(const uint16_t* X, int64_t M, int64_t ldx, int64_t K,
                                         const uint8_t* hdr, const uint8_t* levels,
                                         int32_t hdr_bytes, int64_t N, int64_t n_cb, float* Y,
                                         void* stream) {
    using namespace sx8;
    if (!X || !hdr || !levels || !Y) return fail(SX8_ERR_INVALID, "sx8_gemm_prefill_core: null pointer");
    if (hdr_bytes != 6 && hdr_bytes != 8)
        return fail(SX8_ERR_INVALID, "sx8_gemm_prefill_core: hdr_bytes must be 6 or 8, got %d", hdr_bytes);
    if (!aligned(hdr, hdr_bytes == 8 ? 8 : 2) || !aligned(levels, 8) || !aligned(X, 2) ||
        !aligned(Y, 4))
        return fail(SX8_ERR_INVALID, "sx8_gemm_prefill_core: misaligned hdr/levels");
    const int32_t rc = check_shape("sx8_gemm_prefill_core", M, ldx, K, N, n_cb);
    if (rc != SX8_OK) return rc;
    WeightSrc w{};
    w.hdr = hdr;
    w.levels = levels;
    return launch_gemm<false, false>("sx8_gemm_prefill_core", X, M, ldx, K, w, hdr_bytes, nullptr,
                                     N, n_cb, Y, as_stream(stream));
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
