// sx8_gemm.hip -- prefill GEMM Y (M, N) f32 = X (M, K) fp16 . W^T with W in S-X8 blocks.
//
// Reference roles: gemm_compact (cuda/sx8_gemm_compact.cu:55-194, CUDA-core FMAs with
// PCA applied through Z) and sx8_wmma_kernel / fused_forward (cuda/sx8_fused_wmma.cu:
// 11-154, WMMA 16x16x16 with per-weight PCA).  One kernel serves every contract: the
// PCA-free core weights rlo + step*lv are decoded in float32 into fp16 MFMA B operands,
// and the PCA term sum_kb c0 Z0 + c1 Z1 rides along as extra MFMA k-steps (Z split into
// fp16 hi + lo parts, coefficients as exact fp16 integers).
//
// Work decomposition (gfx950, wave64, v_mfma_f32_32x32x16_f16, 256 CUs in 8 XCDs):
//   * a 256-thread work-group owns a (128 MF) x 128 output tile (MF = 2 once M > 128);
//     wave w owns 32 MF rows for all 128 columns (MF x 4 accumulators of 32 x 32), so one
//     decoded weight feeds 4 MF MFMA rows of work and each wave's X rows are its own.
//   * K advances one S-X8 block (32 weights = two MFMA k-steps) per iteration.  Every
//     weight of the tile is decoded once per work-group (thread t: column t % 128,
//     sub-blocks 2 (t / 128), 2 (t / 128) + 1) into a double-buffered LDS B tile laid out
//     in MFMA lane order; X goes from global memory straight into A registers.
//   * global loads run two blocks ahead, and the per-iteration barrier waits for LDS only.
//   * every 4 K blocks (and after the last one) one PCA k-step per accumulator adds
//     Zhl (rows x 16) . C (16 x columns), C = the blocks' signed coefficient nibbles.
//   * tiles are dealt XCD by XCD in m-major order; shapes with fewer tiles than CUs
//     split K into ranges of whole 4-block groups and add the partials in a fixed order.
#include <algorithm>
#include <climits>
#include <cstdio>
#include <cstdlib>
#include <mutex>

#include "sx8_buffer.h"
#include "sx8_device.h"
#include "sx8_host.h"

namespace {

constexpr int kBN = 128;
constexpr int kThreads = 512;   // waves 0-3 run the MFMAs, waves 4-7 decode weights

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

// Matrices of one launch that multiply the same X (q/k/v, gate/up): column tiles are
// numbered across the group, matrix after matrix; each matrix has its own weights, Zhl
// operand and output.  poff: offset (floats) of this matrix's (M, N) block inside a
// k_gemm split-K partial slice (slices hold the whole group, M * Ntot floats).
constexpr int kMaxGemmGroup = 4;
// K ranges of a split plan: at most 8, so at most 7 partial slices or tiles to add
constexpr int kMaxSplitParts = 7;
struct GemmMat {
    WeightSrc w;
    const uint32_t* Zhl;
    float* Y;
    int N;
    int nb;          // column tiles, ceil(N / kBN)
    int64_t poff;
};
struct GemmGroup {
    GemmMat m[kMaxGemmGroup];
    int n_mats;
    int NB;          // column tiles of the group
    int64_t Ntot;    // columns of the group
};

// The matrix that owns global column tile nb; nb becomes the tile within it.
__device__ __forceinline__ int group_mat(const GemmGroup& g, int& nb) {
    int mi = 0;
    while (mi + 1 < g.n_mats && nb >= g.m[mi].nb) nb -= g.m[mi++].nb;
    return mi;
}

// The part of one block a decoding thread needs, as loaded (no arithmetic on freshly
// loaded values, so prefetches stay in flight until use): v4.4 -> lohi = dmin | dmax << 16,
// cc = config | coeff << 8, q = this lane's 12-byte half of the 24 level bytes (the two
// lanes of a column load its record contiguously and trade one word, see rec_levels);
// split arrays -> lohi = dmin, hi16 = dmax, cc = config, cf = coeff, q = the hi-nibble
// bytes of sub-blocks 2h, 2h + 1 and their four lo-quad bytes.
struct LaneRec {
    uint32_t lohi, hi16, cc, cf;
    uint32_t q0, q1, q2;
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

// LDS of one work-group: B operands in lane order, so every MFMA operand read is one
// conflict-free ds_read_b128 at lane * 16.
//   wt[b][j][st][l]: decoded weights of K block kb (b = kb % 3), n-fragment j (columns
//                    32j .. 32j + 31 of the tile), MFMA k-step st, MFMA lane l
//   pt[b][j][l]:     PCA k-step operand of group g (b = g & 1): for lane l = 32 hf + c,
//                    (c0, c0, c1, c1) of blocks 4g + 2hf and 4g + 2hf + 1 of column c
// Three weight buffers: while the MFMA waves multiply block kb (held in registers) and
// read block kb + 1, the decode waves write block kb + 2.
constexpr int kWtBufBytes = 4 * 2 * 64 * 16;
struct GemmSmem {
    sx8_u32x4 wt[3][4][2][64];
    sx8_u32x4 pt[2][4][64];
};

// A wave-uniform value kept in a scalar register (buffer loads take their K-block offset
// as the scalar offset; if the compiler loses track of its uniformity it wraps every load
// in a loop over distinct lane values).
__device__ __forceinline__ int sx8_uniform(int v) { return __builtin_amdgcn_readfirstlane(v); }

// Buffer resources and per-lane byte offsets for the main loop's loads.  The K block goes
// into the scalar offset, so the loop does no per-lane address arithmetic; a lane whose
// vector offset lies past the end of a buffer (X rows >= M) reads zero.

template <int MF>
struct LoopSrc {
    sx8_rsrc x, hdr, lv, z, dmin, dmax, cfg, cf, hi, lo;
    int a_off[MF];     // packed X of m-fragment f: row group * n_cb * 2048 + lane * 16
    int z_off[MF];     // Zhl row of m-fragment f: (row * n_cb + 2 hf) * 8
    int nn;            // weight column (clamped to N - 1)
    int h;             // sub-block pair {2h, 2h + 1} this thread decodes
};

// Header part (endpoints, config, coefficients) and level part (hi nibbles, lo quads) of
// this thread's record of K block kb; the main loop refills each part once its previous
// contents are consumed.
template <bool kSplit, int HB, int MF>
__device__ __forceinline__ void load_rec_hdr(LaneRec& r, const LoopSrc<MF>& ls, int N, int kb) {
    const int nn = ls.nn;
    const int rowb = sx8_uniform(kb * N);          // first block of K row kb
    if constexpr (kSplit) {
        r.lohi = __builtin_amdgcn_raw_buffer_load_b16(ls.dmin, nn * 2, rowb * 2, 0);
        r.hi16 = __builtin_amdgcn_raw_buffer_load_b16(ls.dmax, nn * 2, rowb * 2, 0);
        r.cc = __builtin_amdgcn_raw_buffer_load_b8(ls.cfg, nn, rowb, 0);
        r.cf = __builtin_amdgcn_raw_buffer_load_b8(ls.cf, nn, rowb, 0);
    } else {
        if constexpr (HB == 8) {
            const uint2 v = __builtin_bit_cast(uint2, __builtin_amdgcn_raw_buffer_load_b64(ls.hdr, nn * 8, rowb * 8, 0));
            r.lohi = v.x;
            r.cc = v.y;
        } else {
            r.lohi = __builtin_amdgcn_raw_buffer_load_b32(ls.hdr, nn * 6, rowb * 6, 0);
            r.cc = __builtin_amdgcn_raw_buffer_load_b16(ls.hdr, nn * 6 + 4, rowb * 6, 0);
        }
        r.hi16 = r.cf = 0;
    }
}

template <bool kSplit, int HB, int MF>
__device__ __forceinline__ void load_rec_lv(LaneRec& r, const LoopSrc<MF>& ls, int N, int kb) {
    const int nn = ls.nn, s = ls.h;
    const int rowb = sx8_uniform(kb * N);
    if constexpr (kSplit) {
        const uint2 v = __builtin_bit_cast(uint2, __builtin_amdgcn_raw_buffer_load_b64(ls.hi, nn * 16 + 8 * s, rowb * 16, 0));
        r.q0 = v.x;
        r.q1 = v.y;
        r.q2 = __builtin_amdgcn_raw_buffer_load_b32(ls.lo, nn * 8 + 4 * s, rowb * 8, 0);
    } else {
        typedef uint32_t u32x3 __attribute__((ext_vector_type(3)));
        const u32x3 v = __builtin_amdgcn_raw_buffer_load_b96(ls.lv, nn * 24 + 12 * s, rowb * 24, 0);
        r.q0 = v.x;
        r.q1 = v.y;
        r.q2 = v.z;
    }
}

// Hi-nibble words of sub-blocks 2h (Hx) and 2h + 1 (Hy) and their lo-quad bytes (P, low
// half for 2h).  v4.4: the level record of a column is qh[16] | ql[8]; lane c (h = 0) holds
// bytes 0-11 (qh 0-11), lane c + 32 (h = 1) bytes 12-23 (qh 12-15, ql 0-7).  h = 0 needs
// ql 0-3 from its partner, h = 1 needs qh 8-11: one swap of the wave's lane halves.
template <bool kSplit>
__device__ __forceinline__ void rec_levels(const LaneRec& r, int h, uint32_t& Hx, uint32_t& Hy,
                                           uint32_t& P) {
    if constexpr (kSplit) {
        Hx = r.q0;
        Hy = r.q1;
        P = r.q2;
    } else {
        const uint32_t send = h ? r.q1 : r.q2;
        // v_permlane32_swap: result[0] = send with lanes 32-63 taken from lanes 0-31,
        // result[1] = send with lanes 0-31 taken from lanes 32-63
        const auto sw = __builtin_amdgcn_permlane32_swap(send, send, false, false);
        const uint32_t recv = h ? sw[0] : sw[1];
        Hx = h ? recv : r.q0;
        Hy = h ? r.q0 : r.q1;
        P = h ? r.q2 : recv;
    }
}

template <bool kSplit, int HB, int MF>
__device__ __forceinline__ void load_rec(LaneRec& r, const LoopSrc<MF>& ls, int N, int kb) {
    load_rec_hdr<kSplit, HB, MF>(r, ls, N, kb);
    load_rec_lv<kSplit, HB, MF>(r, ls, N, kb);
}

// A operands of K block kb from the packed X (see k_compute_z): for m-fragment f and k-step
// st, lane l = 32 hf + r holds X[row r][32 kb + 16 hf + 8 st .. + 8], one contiguous 1 KB
// wave load.  (The MFMA pairs A lane l's k with B lane l's k, so this K order -- each
// lane's 16 consecutive values split over the two k-steps -- only has to match the order
// in which the weights are placed, see decode_block.)  Row groups past the packed rows
// read zero.
template <int MF>
__device__ __forceinline__ void load_a_step(sx8_u32x4 (&a)[MF][2], const LoopSrc<MF>& ls, int kb, int st) {
#pragma unroll
    for (int f = 0; f < MF; ++f)
        a[f][st] = __builtin_bit_cast(sx8_u32x4, __builtin_amdgcn_raw_buffer_load_b128(
                                                     ls.x, ls.a_off[f] + 1024 * st, sx8_uniform(kb * 2048), 0));
}

template <int MF>
__device__ __forceinline__ void load_a(sx8_u32x4 (&a)[MF][2], const LoopSrc<MF>& ls, int kb) {
    load_a_step<MF>(a, ls, kb, 0);
    load_a_step<MF>(a, ls, kb, 1);
}

// Zhl operand of group g (blocks 4g .. 4g + 3): lane l = 32 hf + r gets the 8 fp16 values
// (Z0 hi, Z0 lo, Z1 hi, Z1 lo) of blocks 4g + 2hf and 4g + 2hf + 1 of its row; values of
// blocks >= n_cb are zeroed here (their coefficient slots may hold stale values).
template <int MF>
__device__ __forceinline__ void load_za(sx8_u32x4 (&za)[MF], const LoopSrc<MF>& ls, int g) {
#pragma unroll
    for (int f = 0; f < MF; ++f)
        za[f] = __builtin_bit_cast(sx8_u32x4, __builtin_amdgcn_raw_buffer_load_b128(
                                                  ls.z, ls.z_off[f] + g * 32, 0, 0));
}

__device__ __forceinline__ sx8_half8 mask_za(sx8_u32x4 v, int n_cb, int g, int hf) {
    const int kb0 = 4 * g + 2 * hf;
    if (kb0 >= n_cb) v.x = v.y = 0u;
    if (kb0 + 1 >= n_cb) v.z = v.w = 0u;
    return __builtin_bit_cast(sx8_half8, v);
}

// Work-group barrier for LDS hand-offs only: wait for this wave's LDS accesses, then
// s_barrier.  __syncthreads() would also wait for every global load in flight (its
// release fence), which would undo the load lead of the main loop.  The memory clobber
// keeps the compiler from moving LDS accesses across it.
__device__ __forceinline__ void lds_barrier() {
    // the wait is a builtin so the compiler's wait-count tracking sees that this wave's LDS
    // reads have landed (an opaque asm wait would make it wait again for the next
    // iteration's reads before their first use)
    __builtin_amdgcn_s_waitcnt(0xC07F);   // lgkmcnt(0); vmcnt, expcnt untouched
    asm volatile("s_barrier" ::: "memory");
}

// The same barrier with up to four of this wave's LDS operations still in flight: LDS
// operations complete in issue order, so lgkmcnt(4) covers every LDS access but the last
// four (the caller issues no scalar memory loads, which share the counter, in its loop).
__device__ __forceinline__ void lds_barrier_keep4() {
    __builtin_amdgcn_s_waitcnt(0xC47F);   // lgkmcnt(4); vmcnt, expcnt untouched
    asm volatile("s_barrier" ::: "memory");
}

__device__ __forceinline__ uint32_t coeff_pair_f16(int c) {
    const uint32_t h = __builtin_bit_cast(uint16_t, (_Float16)(float)c);
    return h | (h << 16);
}

// levels of the even (le) and odd (lo) weights of a sub-block, one byte each
__device__ __forceinline__ void dec_unpack(uint32_t H, uint32_t P, uint32_t& le, uint32_t& lo) {
    const uint32_t x = __builtin_amdgcn_perm(0u, P, 0x01010000u);        // P0, P0, P1, P1
    const uint32_t qe = ((x >> 6) & 0x00030003u) | ((x >> 2) & 0x03000300u);   // q0 q2 q4 q6
    const uint32_t qo = ((x >> 4) & 0x00030003u) | (x & 0x03000300u);          // q1 q3 q5 q7
    le = ((H & 0x0F0F0F0Fu) << 2) | qe;
    lo = (((H >> 4) & 0x0F0F0F0Fu) << 2) | qo;
}

// weights 2j, 2j + 1 of a sub-block as a packed fp16 pair
__device__ __forceinline__ uint32_t dec_pair(uint32_t le, uint32_t lo, int j, float rlo, float step) {
    const float we = __builtin_fmaf(step, (float)((le >> (8 * j)) & 0xFFu), rlo);
    const float wo = __builtin_fmaf(step, (float)((lo >> (8 * j)) & 0xFFu), rlo);
    const sx8_half2 v = {(_Float16)we, (_Float16)wo};
    return __builtin_bit_cast(uint32_t, v);
}

// Decode of this thread's two sub-blocks of a block, in two halves so the decode waves can
// overlap the second half of block kb with the first half of block kb + 1 (one decode wave
// per SIMD has no other wave to hide its dependency chains behind).
// dec_prep: sub-block ranges, level bytes and the PCA coefficient (h = 0: c0, h = 1: c1)
// as an fp16 pair.
struct DecPrep {
    float rlo[2], step[2];
    uint32_t le[2], lv[2];
    uint32_t cpair;
};

template <bool kSplit>
__device__ __forceinline__ DecPrep dec_prep(const LaneRec& rec, int h) {
    uint32_t lohi, cfg;
    rec_unpack<kSplit>(rec, lohi, cfg);
    const float lo = sx8_h2f(lohi), hi = sx8_h2f(lohi >> 16);
    const float d = hi - lo;
    const float q = d * 0.25f;
    const float mstep = d * 0.015873f;
    uint32_t Hx, Hy, P;
    rec_levels<kSplit>(rec, h, Hx, Hy, P);
    DecPrep p;
#pragma unroll
    for (int st = 0; st < 2; ++st) {
        sub_range(lo, d, q, mstep, cfg, 2 * h + st, p.rlo[st], p.step[st]);
        dec_unpack(st ? Hy : Hx, st ? (P >> 16) : P, p.le[st], p.lv[st]);
    }
    const uint32_t cf = kSplit ? rec.cf : (rec.cc >> 8);
    p.cpair = coeff_pair_f16(sx8_sext4(cf >> (4 * h)));
    return p;
}

// dec_finish: the 16 weights into weight buffer b, the coefficient pair into the group's
// coefficient tile (h = 0 stores the slot's (c0, c0) pair, h = 1 its (c1, c1) pair).
template <bool kPca>
__device__ __forceinline__ void dec_finish(GemmSmem& sm, const DecPrep& p, int kb, int b, int wj, int wl,
                                           int h) {
#pragma unroll
    for (int st = 0; st < 2; ++st)
        sm.wt[b][wj][st][wl] = sx8_u32x4{dec_pair(p.le[st], p.lv[st], 0, p.rlo[st], p.step[st]),
                                         dec_pair(p.le[st], p.lv[st], 1, p.rlo[st], p.step[st]),
                                         dec_pair(p.le[st], p.lv[st], 2, p.rlo[st], p.step[st]),
                                         dec_pair(p.le[st], p.lv[st], 3, p.rlo[st], p.step[st])};
    if constexpr (kPca) {
        const int t4 = kb & 3;
        uint32_t* dst = reinterpret_cast<uint32_t*>(&sm.pt[(kb >> 2) & 1][wj][(t4 >> 1) * 32 + (wl & 31)]);
        dst[2 * (t4 & 1) + h] = p.cpair;
    }
}

template <bool kSplit, bool kPca>
__device__ __forceinline__ void decode_block(GemmSmem& sm, const LaneRec& rec, int kb, int b, int wj,
                                             int wl, int h) {
    dec_finish<kPca>(sm, dec_prep<kSplit>(rec, h), kb, b, wj, wl, h);
}

#define SX8_SCHED_FENCE() __builtin_amdgcn_sched_barrier(0)

// XCD-aware work order: the dispatcher deals work-groups round-robin over the 8 XCDs, so
// work-group b runs on XCD b % 8.  Give each XCD a contiguous run of the m-major tile order
// (consecutive tiles share their X rows, which then stay in that XCD's L2).
__device__ __forceinline__ int xcd_order(int b, int G) {
    const int x = b & 7;
    int start = 0;
    for (int y = 0; y < x; ++y) start += (G - y + 7) >> 3;
    return start + (b >> 3);
}

// Y (M, N) f32 = X . W^T (+ PCA term via Zhl).  Work-group: 8 waves, tile of 128 MF rows
// x 128 columns.  Waves 0-3 (one per SIMD) own 32 MF rows each for all 128 columns (MF x 4
// accumulators of 32 x 32) and issue only MFMAs, LDS reads and X loads; waves 4-7 decode
// every weight of the tile once (thread t: column t % 128, sub-blocks 2 (t / 128),
// 2 (t / 128) + 1) into the LDS ring two blocks ahead.  Each SIMD so runs one MFMA wave and
// one decode wave, and the decode VALU work proceeds while the matrix pipe is busy.
// One work-group barrier per K block.  S > 1 splits K into S ranges of whole 4-block
// groups; range ks > 0 writes its partial tile to part + (ks - 1) M N and k_reduce adds the
// partials to Y in a fixed order.
template <bool kSplit, int HB, bool kPca, int MF>
__global__ __launch_bounds__(kThreads) void k_gemm(const uint16_t* __restrict__ Xp, int M,
                                                   const GemmGroup g, int n_cb, int S, int kb_per_split,
                                                   float* __restrict__ part) {
    __shared__ GemmSmem sm;
    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = tid >> 6;
    const int NB = g.NB;
    const int MB = (M + 128 * MF - 1) / (128 * MF);
    const int G = MB * NB * S;
    const int o = xcd_order(blockIdx.x, G);
    int nb = o % NB;
    const int ks = (o / NB) % S;
    const int mb = o / (NB * S);
    const int mi = group_mat(g, nb);
    const WeightSrc w = g.m[mi].w;
    const uint32_t* __restrict__ Zhl = g.m[mi].Zhl;
    float* __restrict__ Y = g.m[mi].Y;
    const int N = g.m[mi].N;
    const int m0 = mb * 128 * MF;
    const int n0 = nb * kBN;
    const int kb0 = ks * kb_per_split;
    const int kb1 = min(n_cb, kb0 + kb_per_split);

    if constexpr (kPca) {
        // coefficient slots of blocks past n_cb are never written: start them at zero
        reinterpret_cast<sx8_u32x4*>(&sm.pt[0][0][0])[tid] = sx8_u32x4{0u, 0u, 0u, 0u};
        lds_barrier();
    }

    if (wave >= 4) {
        // ---------------- decode waves ----------------
        // decode wave d (0..3) owns columns 32d .. 32d + 31 (n-fragment d); lane l handles
        // column 32d + l % 32, sub-block pair h = l / 32, and writes B-tile slot l
        const int dw = wave - 4, l = lane;
        const int nl = 32 * dw + (l & 31), h = l >> 5;
        const int wj = dw, wl = l;
        LoopSrc<MF> ls;
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
        ls.nn = min(n0 + nl, N - 1);
        ls.h = h;
        // prologue: blocks kb0, kb0 + 1 decoded, block kb0 + 2 prepared, records of kb0 + 3,
        // kb0 + 4 in flight.  Weight records miss in L2 (each work-group of an XCD streams its
        // own columns), so they are requested two iterations before their first use.
        LaneRec R[2];
        DecPrep P[2];
        {
            LaneRec r0, r1;
            load_rec<kSplit, HB, MF>(r0, ls, N, kb0);
            load_rec<kSplit, HB, MF>(r1, ls, N, min(kb0 + 1, kb1 - 1));
            load_rec<kSplit, HB, MF>(R[0], ls, N, min(kb0 + 2, kb1 - 1));
            load_rec<kSplit, HB, MF>(R[1], ls, N, min(kb0 + 3, kb1 - 1));
            decode_block<kSplit, kPca>(sm, r0, kb0, kb0 % 3, wj, wl, h);
            decode_block<kSplit, kPca>(sm, r1, kb0 + 1, (kb0 + 1) % 3, wj, wl, h);
            P[0] = dec_prep<kSplit>(R[0], h);
            load_rec<kSplit, HB, MF>(R[0], ls, N, min(kb0 + 4, kb1 - 1));
            lds_barrier();
        }
        // iteration kb: finish block kb + 2 (prepared last iteration), prepare block kb + 3
        // (records in R[(kb - kb0 + 1) & 1], refilled with block kb + 5).  A block past the
        // range decodes a clamped record into a buffer nobody reads; its coefficient slot
        // meets a zeroed Z value.
        auto step = [&](int kb, LaneRec& r, const DecPrep& pcur, DecPrep& pnext) __attribute__((always_inline)) {
            pnext = dec_prep<kSplit>(r, h);
            dec_finish<kPca>(sm, pcur, kb + 2, (kb + 2) % 3, wj, wl, h);
            load_rec<kSplit, HB, MF>(r, ls, N, min(kb + 5, kb1 - 1));
            lds_barrier();
        };
        int kb = kb0;
        for (; kb + 2 <= kb1; kb += 2) {
            step(kb, R[1], P[0], P[1]);
            step(kb + 1, R[0], P[1], P[0]);
        }
        if (kb < kb1) step(kb, R[1], P[0], P[1]);
        return;
    }

    // ---------------- MFMA waves ----------------
    const int hf = lane >> 5, r = lane & 31;
    LoopSrc<MF> ls;
    ls.x = make_rsrc(Xp, (int64_t)((M + 31) / 32) * n_cb * 2048);
    if constexpr (kPca) ls.z = make_rsrc(Zhl, (int64_t)M * n_cb * 8);
#pragma unroll
    for (int f = 0; f < MF; ++f) {
        const int g32 = (m0 >> 5) + wave * MF + f;
        ls.a_off[f] = (int)((int64_t)g32 * n_cb * 2048) + lane * 16;
        const int row = m0 + wave * 32 * MF + 32 * f + r;
        ls.z_off[f] = (int)(((int64_t)row * n_cb + 2 * hf) * 8);
    }

    sx8_float16v acc[MF][4];
#pragma unroll
    for (int f = 0; f < MF; ++f)
#pragma unroll
        for (int j = 0; j < 4; ++j)
#pragma unroll
            for (int i = 0; i < 16; ++i) acc[f][j][i] = 0.f;

    // prologue: A of kb0, kb0 + 1 and the group's Z operand in flight; B of kb0 read once
    // the decode waves' prologue barrier has passed
    sx8_u32x4 A[2][MF][2];
    sx8_u32x4 za[MF];
    load_a<MF>(A[0], ls, kb0);
    load_a<MF>(A[1], ls, min(kb0 + 1, kb1 - 1));
    if constexpr (kPca) load_za<MF>(za, ls, kb0 >> 2);
    lds_barrier();
    const uint8_t* wbase = reinterpret_cast<const uint8_t*>(&sm.wt[0][0][0][lane]);
    sx8_u32x4 bw[2][4][2];
    {
        const uint8_t* src = wbase + (kb0 % 3) * kWtBufBytes;
#pragma unroll
        for (int j = 0; j < 4; ++j)
#pragma unroll
            for (int st = 0; st < 2; ++st)
                bw[0][j][st] = *reinterpret_cast<const sx8_u32x4*>(src + (j * 2 + st) * 1024);
        __builtin_amdgcn_s_waitcnt(0xC07F);   // lgkmcnt(0): the loop starts with no LDS read in flight
    }

    // iteration kb: request B of kb + 1, 16 MFMAs of block kb (A of kb + 2 requested as its
    // registers free up), PCA k-step when `pca` (end of a group), barrier.  The main loop
    // runs whole groups with `pca` a constant, so its body has no branch (a branch around
    // the PCA step makes the compiler wait for every LDS read before the next MFMA).
    auto body = [&](int kb, sx8_u32x4 (&acur)[MF][2], sx8_u32x4 (&bcur)[4][2], sx8_u32x4 (&bnext)[4][2],
                    const bool pca) __attribute__((always_inline)) {
        {
            const uint8_t* src = wbase + ((kb + 1) % 3) * kWtBufBytes;
#pragma unroll
            for (int j = 0; j < 4; ++j)
#pragma unroll
                for (int st = 0; st < 2; ++st)
                    bnext[j][st] = *reinterpret_cast<const sx8_u32x4*>(src + (j * 2 + st) * 1024);
        }
        const int ka = min(kb + 2, kb1 - 1);
        SX8_SCHED_FENCE();
#pragma unroll
        for (int st = 0; st < 2; ++st) {
#pragma unroll
            for (int j = 0; j < 4; ++j)
#pragma unroll
                for (int f = 0; f < MF; ++f)
                    acc[f][j] = __builtin_amdgcn_mfma_f32_32x32x16_f16(
                        __builtin_bit_cast(sx8_half8, bcur[j][st]),
                        __builtin_bit_cast(sx8_half8, acur[f][st]), acc[f][j], 0, 0, 0);
            SX8_SCHED_FENCE();
            load_a_step<MF>(acur, ls, ka, st);
            SX8_SCHED_FENCE();
        }
        if constexpr (kPca) {
            if (pca) {
                const int g = kb >> 2;
                sx8_half8 zh[MF];
#pragma unroll
                for (int f = 0; f < MF; ++f) zh[f] = mask_za(za[f], n_cb, g, hf);
#pragma unroll
                for (int j = 0; j < 4; ++j) {
                    const sx8_half8 c = __builtin_bit_cast(sx8_half8, sm.pt[g & 1][j][lane]);
#pragma unroll
                    for (int f = 0; f < MF; ++f)
                        acc[f][j] = __builtin_amdgcn_mfma_f32_32x32x16_f16(c, zh[f], acc[f][j], 0, 0, 0);
                }
                load_za<MF>(za, ls, min(g + 1, (kb1 - 1) >> 2));
            }
        }
        lds_barrier();
    };
    int kb = kb0;   // a multiple of 4
    for (; kb + 4 <= kb1; kb += 4) {
        body(kb, A[0], bw[0], bw[1], false);
        body(kb + 1, A[1], bw[1], bw[0], false);
        body(kb + 2, A[0], bw[0], bw[1], false);
        body(kb + 3, A[1], bw[1], bw[0], true);
    }
    // last partial group (n_cb % 4 blocks): its PCA step after its last block
    if (kb < kb1) body(kb, A[0], bw[0], bw[1], kb + 1 == kb1);
    if (kb + 1 < kb1) body(kb + 1, A[1], bw[1], bw[0], kb + 2 == kb1);
    if (kb + 2 < kb1) body(kb + 2, A[0], bw[0], bw[1], true);

    // epilogue: the MFMAs take the weights as the A operand, so accumulator (f, j) holds the
    // transposed tile: element i of lane l = 32 hf + c is column 32 j + 4 hf + 8 (i / 4) +
    // i % 4 of row 32 MF wave + 32 f + c, and elements 4q .. 4q + 3 are 4 consecutive
    // columns (one 16-byte store when N % 4 == 0 and Y is 16-byte aligned)
    float* dst = ks == 0 ? Y : part + (int64_t)(ks - 1) * M * g.Ntot + g.m[mi].poff;
    const bool vec = (N & 3) == 0 && (reinterpret_cast<uintptr_t>(dst) & 15) == 0;
#pragma unroll
    for (int f = 0; f < MF; ++f) {
        const int m = m0 + wave * 32 * MF + 32 * f + r;
        if (m >= M) continue;
        float* row = dst + (int64_t)m * N;
#pragma unroll
        for (int j = 0; j < 4; ++j)
#pragma unroll
            for (int q = 0; q < 4; ++q) {
                const int n = n0 + 32 * j + 8 * q + 4 * hf;
                const sx8_float4 v = {acc[f][j][4 * q], acc[f][j][4 * q + 1], acc[f][j][4 * q + 2],
                                      acc[f][j][4 * q + 3]};
                if (vec && n + 3 < N) {
                    *reinterpret_cast<sx8_float4*>(row + n) = v;
                } else {
#pragma unroll
                    for (int e = 0; e < 4; ++e)
                        if (n + e < N) row[n + e] = v[e];
                }
            }
    }
}

// One wave per SIMD, tile 512 x 128 (k_gemm_w1).  The decode VALU work per MFMA falls with
// the tile height: a 512-row tile does 32 MFMAs per wave per K block against the 16
// weights each lane decodes, half the ratio of the 256-row tile.  Each wave needs 256
// accumulator registers (4 m-fragments x 4 n-fragments of 32 x 32), so it runs alone on
// its SIMD (waves_per_eu = 1, up to 512 registers) and interleaves its own decode with its
// MFMAs: wave w owns rows 128 w .. 128 w + 127 for all 128 columns and decodes n-fragment
// w (columns 32 w .. 32 w + 31, lane l: column 32 w + l % 32, sub-blocks 2 (l / 32),
// 2 (l / 32) + 1) of every K block into the same three-deep LDS ring as k_gemm.
constexpr int kW1Threads = 256;
constexpr int kW1MF = 4;
constexpr int kW1BM = 128 * kW1MF;

// Work of one launch: T tiles in m-major order (tile t = row block t / NB, column block
// t % NB).  Work-groups 0 .. Tf - 1 (whole rounds of the 256 CUs, or none) each own one of
// the first Tf tiles over the whole K; the remaining T - Tf tiles are split into St K
// ranges of kbs blocks, one work-group each, which start as the full tiles finish.  K range
// 0 of a split tile writes Y, range s > 0 its partial tile part[(t - Tf) (St - 1) + s - 1]
// (512 x 128 f32, row-major), added to Y by k_reduce_tiles in range order.
template <bool kSplit, int HB, bool kPca>
__global__ __launch_bounds__(kW1Threads) __attribute__((amdgpu_waves_per_eu(1, 1))) void k_gemm_w1(
    const uint16_t* __restrict__ Xp, int M, const GemmGroup g, int n_cb, int Tf, int St, int kbs,
    float* __restrict__ part) {
    constexpr int MF = kW1MF;
    __shared__ GemmSmem sm;
    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = tid >> 6;
    const int NB = g.NB;
    const int b = blockIdx.x;
    int t, ks = 0, kb0 = 0, kb1 = n_cb;
    if (b < Tf) {
        t = xcd_order(b, Tf);
    } else {
        // Tf is a multiple of 8, so work-group b still runs on XCD b % 8
        const int o = xcd_order(b - Tf, gridDim.x - Tf);
        t = Tf + o / St;
        ks = o % St;
        kb0 = ks * kbs;
        kb1 = min(n_cb, kb0 + kbs);
    }
    int nb = t % NB;
    const int mb = t / NB;
    const int mi = group_mat(g, nb);
    const WeightSrc w = g.m[mi].w;
    const uint32_t* __restrict__ Zhl = g.m[mi].Zhl;
    float* __restrict__ Y = g.m[mi].Y;
    const int N = g.m[mi].N;
    const int m0 = mb * kW1BM;
    const int n0 = nb * kBN;
    const int hf = lane >> 5, r = lane & 31;
    const int h = hf;                     // decode: sub-block pair {2h, 2h + 1}
    const int wj = wave, wl = lane;       // decode: n-fragment and B-tile slot

    if constexpr (kPca) {
        // coefficient slots of blocks past n_cb are never written: start them at zero.
        // Thread t clears slots [b][wave][lane] of both groups, the slots only this wave
        // writes, so program order makes the clear precede its own coefficient stores.
        sx8_u32x4* p = reinterpret_cast<sx8_u32x4*>(&sm.pt[0][0][0]);
        p[tid] = sx8_u32x4{0u, 0u, 0u, 0u};
        p[tid + kW1Threads] = sx8_u32x4{0u, 0u, 0u, 0u};
    }

    LoopSrc<MF> ls;
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
    ls.nn = min(n0 + 32 * wave + r, N - 1);
    ls.h = h;
    ls.x = make_rsrc(Xp, (int64_t)((M + 31) / 32) * n_cb * 2048);
    if constexpr (kPca) ls.z = make_rsrc(Zhl, (int64_t)M * n_cb * 8);
#pragma unroll
    for (int f = 0; f < MF; ++f) {
        // rows past M lie past the end of both buffers (read as zero); the host checks that
        // these offsets fit 31 bits for the padded row count
        const int g32 = (m0 >> 5) + wave * MF + f;
        ls.a_off[f] = (int)((int64_t)g32 * n_cb * 2048) + lane * 16;
        const int row = m0 + wave * 32 * MF + 32 * f + r;
        ls.z_off[f] = (int)(((int64_t)row * n_cb + 2 * hf) * 8);
    }

    sx8_float16v acc[MF][4];
#pragma unroll
    for (int f = 0; f < MF; ++f)
#pragma unroll
        for (int j = 0; j < 4; ++j)
#pragma unroll
            for (int i = 0; i < 16; ++i) acc[f][j][i] = 0.f;

    // prologue: blocks kb0, kb0 + 1 decoded, block kb0 + 2 prepared, records of kb0 + 3 ..
    // kb0 + 6 and A of kb0, kb0 + 1 in flight; B of kb0 read after the barrier.  Records
    // form a ring of four (block b in R[(b - kb0) % 4]) so that each is requested four
    // iterations before its first use: this wave issues the MFMAs too, and a record that
    // has not arrived would stall them.
    LaneRec R[4];
    DecPrep P[2];
    sx8_u32x4 A[2][MF][2];
    sx8_u32x4 za[MF];
    {
        LaneRec r0, r1, r2;
        load_rec<kSplit, HB, MF>(r0, ls, N, kb0);
        load_rec<kSplit, HB, MF>(r1, ls, N, min(kb0 + 1, kb1 - 1));
        load_rec<kSplit, HB, MF>(r2, ls, N, min(kb0 + 2, kb1 - 1));
        load_a<MF>(A[0], ls, kb0);
        load_a_step<MF>(A[1], ls, min(kb0 + 1, kb1 - 1), 0);   // k-step 1: in iteration kb0
        if constexpr (kPca) load_za<MF>(za, ls, kb0 >> 2);
        load_rec<kSplit, HB, MF>(R[3], ls, N, min(kb0 + 3, kb1 - 1));
        load_rec<kSplit, HB, MF>(R[0], ls, N, min(kb0 + 4, kb1 - 1));
        load_rec<kSplit, HB, MF>(R[1], ls, N, min(kb0 + 5, kb1 - 1));
        load_rec<kSplit, HB, MF>(R[2], ls, N, min(kb0 + 6, kb1 - 1));
        decode_block<kSplit, kPca>(sm, r0, kb0, kb0 % 3, wj, wl, h);
        decode_block<kSplit, kPca>(sm, r1, kb0 + 1, (kb0 + 1) % 3, wj, wl, h);
        P[0] = dec_prep<kSplit>(r2, h);
        lds_barrier();
    }
    const uint8_t* wbase = reinterpret_cast<const uint8_t*>(&sm.wt[0][0][0][lane]);
    // B operands of one block, refilled per k-step right after that k-step's MFMAs
    sx8_u32x4 bw[4][2];
    auto read_b = [&](int kb, int st) __attribute__((always_inline)) {
        const uint8_t* src = wbase + (kb % 3) * kWtBufBytes;
#pragma unroll
        for (int j = 0; j < 4; ++j)
            bw[j][st] = *reinterpret_cast<const sx8_u32x4*>(src + (j * 2 + st) * 1024);
    };
    read_b(kb0, 0);   // k-step 1: in iteration kb0

    // iteration kb: finish block kb + 2 into the ring and prepare block kb + 3 (its
    // records refilled with block kb + 7); 32 MFMAs of block kb; PCA k-step at the end of a
    // 4-block group; one barrier.  Each k-step's registers are refilled during the other
    // k-step's MFMAs (A: block kb + 2, B: the next block, in LDS since a barrier), and the
    // decode VALU work, the loads and the LDS accesses are spread between the MFMAs
    // (sched_group_barrier patterns), so they issue while the matrix core is busy.
    auto body = [&](int kb, sx8_u32x4 (&acur)[MF][2], sx8_u32x4 (&aprev)[MF][2], LaneRec& rx,
                    const DecPrep& pcur, DecPrep& pnext, const bool pca) __attribute__((always_inline)) {
        const int ka = min(kb + 2, kb1 - 1);
        const int kp = min(kb + 1, kb1 - 1);
        // k-step 0: prepare block kb + 3; between the MFMAs, the second-k-step refills the
        // previous iteration left (A of kb + 1 into its buffer, B of kb from LDS)
        pnext = dec_prep<kSplit>(rx, h);
#pragma unroll
        for (int j = 0; j < 4; ++j)
#pragma unroll
            for (int f = 0; f < MF; ++f)
                acc[f][j] = __builtin_amdgcn_mfma_f32_32x32x16_f16(
                    __builtin_bit_cast(sx8_half8, bw[j][0]),
                    __builtin_bit_cast(sx8_half8, acur[f][0]), acc[f][j], 0, 0, 0);
        load_a_step<MF>(aprev, ls, kp, 1);
        read_b(kb, 1);
#pragma unroll
        for (int i = 0; i < 16; ++i) {
            __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);   // one MFMA
            __builtin_amdgcn_sched_group_barrier(0x002, 3, 0);   // up to three VALU
            if (i < 4) __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);           // a B read
            else if (i < 8) __builtin_amdgcn_sched_group_barrier(0x020, 1, 0);      // an A load
        }
        SX8_SCHED_FENCE();
        // k-step 1: finish block kb + 2 into the ring; between the MFMAs, refill A (block
        // kb + 2) and B (block kb + 1) for k-step 0 and the record ring
        dec_finish<kPca>(sm, pcur, kb + 2, (kb + 2) % 3, wj, wl, h);
#pragma unroll
        for (int j = 0; j < 4; ++j)
#pragma unroll
            for (int f = 0; f < MF; ++f)
                acc[f][j] = __builtin_amdgcn_mfma_f32_32x32x16_f16(
                    __builtin_bit_cast(sx8_half8, bw[j][1]),
                    __builtin_bit_cast(sx8_half8, acur[f][1]), acc[f][j], 0, 0, 0);
        load_a_step<MF>(acur, ls, ka, 0);
        load_rec<kSplit, HB, MF>(rx, ls, N, min(kb + 7, kb1 - 1));
        read_b(kb + 1, 0);
#pragma unroll
        for (int i = 0; i < 16; ++i) {
            __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);   // one MFMA
            __builtin_amdgcn_sched_group_barrier(0x002, 4, 0);   // up to four VALU
            if (i < 3) __builtin_amdgcn_sched_group_barrier(0x200, 1, 0);           // ring writes
            else if (i < 10) __builtin_amdgcn_sched_group_barrier(0x020, 1, 0);     // A / record loads
            else if (i < 14) __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);     // B reads
        }
        SX8_SCHED_FENCE();
        if constexpr (kPca) {
            if (pca) {
                const int g = kb >> 2;
                sx8_half8 zh[MF];
#pragma unroll
                for (int f = 0; f < MF; ++f) zh[f] = mask_za(za[f], n_cb, g, hf);
#pragma unroll
                for (int j = 0; j < 4; ++j) {
                    const sx8_half8 c = __builtin_bit_cast(sx8_half8, sm.pt[g & 1][j][lane]);
#pragma unroll
                    for (int f = 0; f < MF; ++f)
                        acc[f][j] = __builtin_amdgcn_mfma_f32_32x32x16_f16(c, zh[f], acc[f][j], 0, 0, 0);
                }
                load_za<MF>(za, ls, min(g + 1, (kb1 - 1) >> 2));
            }
        }
        lds_barrier();
    };
    int kb = kb0;   // a multiple of 4
    for (; kb + 4 <= kb1; kb += 4) {
        body(kb, A[0], A[1], R[3], P[0], P[1], false);
        body(kb + 1, A[1], A[0], R[0], P[1], P[0], false);
        body(kb + 2, A[0], A[1], R[1], P[0], P[1], false);
        body(kb + 3, A[1], A[0], R[2], P[1], P[0], true);
    }
    // last partial group (n_cb % 4 blocks): its PCA step after its last block
    if (kb < kb1) body(kb, A[0], A[1], R[3], P[0], P[1], kb + 1 == kb1);
    if (kb + 1 < kb1) body(kb + 1, A[1], A[0], R[0], P[1], P[0], kb + 2 == kb1);
    if (kb + 2 < kb1) body(kb + 2, A[0], A[1], R[1], P[0], P[1], true);

    // epilogue: accumulator (f, j) holds the transposed 32 x 32 tile (see k_gemm): a 16-byte
    // store of 4 consecutive columns per (f, j, q).  Partial tiles are dense 512 x 128.
    if (ks > 0) {
        float* pt = part + ((int64_t)(t - Tf) * (St - 1) + ks - 1) * (kW1BM * kBN);
#pragma unroll
        for (int f = 0; f < MF; ++f) {
            float* row = pt + (wave * 32 * MF + 32 * f + r) * kBN;
#pragma unroll
            for (int j = 0; j < 4; ++j)
#pragma unroll
                for (int q = 0; q < 4; ++q)
                    *reinterpret_cast<sx8_float4*>(row + 32 * j + 8 * q + 4 * hf) =
                        sx8_float4{acc[f][j][4 * q], acc[f][j][4 * q + 1], acc[f][j][4 * q + 2],
                                   acc[f][j][4 * q + 3]};
        }
        return;
    }
    const bool vec = (N & 3) == 0 && (reinterpret_cast<uintptr_t>(Y) & 15) == 0;
#pragma unroll
    for (int f = 0; f < MF; ++f) {
        const int m = m0 + wave * 32 * MF + 32 * f + r;
        if (m >= M) continue;
        float* row = Y + (int64_t)m * N;
#pragma unroll
        for (int j = 0; j < 4; ++j)
#pragma unroll
            for (int q = 0; q < 4; ++q) {
                const int n = n0 + 32 * j + 8 * q + 4 * hf;
                const sx8_float4 v = {acc[f][j][4 * q], acc[f][j][4 * q + 1], acc[f][j][4 * q + 2],
                                      acc[f][j][4 * q + 3]};
                if (vec && n + 3 < N) {
                    *reinterpret_cast<sx8_float4*>(row + n) = v;
                } else {
#pragma unroll
                    for (int e = 0; e < 4; ++e)
                        if (n + e < N) row[n + e] = v[e];
                }
            }
    }
}

// k_gemm_w2: the 512 x 128 tile of k_gemm_w1 with two waves per SIMD.  Eight waves, wave w
// owning rows 64 w .. 64 w + 63 (2 m-fragments x 4 n-fragments: 128 accumulator registers,
// so two waves fit a SIMD), each lane decoding one 8-weight sub-block per K block (thread
// t: column t % 128, sub-block t / 128).  Waves w and w + 4 share a SIMD: the decode VALU
// work of one issues while the matrix core runs the other's MFMAs, where k_gemm_w1 has to
// interleave both in one wave.  Same ring, record lead, plan, partial tiles and reduction
// as k_gemm_w1.
constexpr int kW2Threads = 512;
constexpr int kW2MF = 2;

// The part of a block one decoding thread of k_gemm_w2 needs: endpoints / config /
// coefficients as in LaneRec, the hi-nibble word and the lo-quad half-word of its sub-block.
struct LaneRec1 {
    uint32_t lohi, hi16, cc, cf;
    uint32_t qh, ql;
};

template <bool kSplit, int HB>
__device__ __forceinline__ void load_rec1(LaneRec1& r, const LoopSrc<kW2MF>& ls, int N, int kb, int sb) {
    const int nn = ls.nn;
    const int rowb = sx8_uniform(kb * N);
    if constexpr (kSplit) {
        r.lohi = __builtin_amdgcn_raw_buffer_load_b16(ls.dmin, nn * 2, rowb * 2, 0);
        r.hi16 = __builtin_amdgcn_raw_buffer_load_b16(ls.dmax, nn * 2, rowb * 2, 0);
        r.cc = __builtin_amdgcn_raw_buffer_load_b8(ls.cfg, nn, rowb, 0);
        r.cf = __builtin_amdgcn_raw_buffer_load_b8(ls.cf, nn, rowb, 0);
        r.qh = __builtin_amdgcn_raw_buffer_load_b32(ls.hi, nn * 16 + 4 * sb, rowb * 16, 0);
        r.ql = __builtin_amdgcn_raw_buffer_load_b16(ls.lo, nn * 8 + 2 * sb, rowb * 8, 0);
    } else {
        if constexpr (HB == 8) {
            const uint2 v = __builtin_bit_cast(uint2, __builtin_amdgcn_raw_buffer_load_b64(ls.hdr, nn * 8, rowb * 8, 0));
            r.lohi = v.x;
            r.cc = v.y;
        } else {
            r.lohi = __builtin_amdgcn_raw_buffer_load_b32(ls.hdr, nn * 6, rowb * 6, 0);
            r.cc = __builtin_amdgcn_raw_buffer_load_b16(ls.hdr, nn * 6 + 4, rowb * 6, 0);
        }
        r.hi16 = r.cf = 0;
        r.qh = __builtin_amdgcn_raw_buffer_load_b32(ls.lv, nn * 24 + 4 * sb, rowb * 24, 0);
        r.ql = __builtin_amdgcn_raw_buffer_load_b16(ls.lv, nn * 24 + 16 + 2 * sb, rowb * 24, 0);
    }
}

// One sub-block's range, levels and (for the first sub-block of a pair) PCA coefficient,
// the arithmetic of dec_prep
struct DecPrep1 {
    float rlo, step;
    uint32_t le, lv;
    uint32_t cpair;
};

template <bool kSplit>
__device__ __forceinline__ DecPrep1 dec1_prep(const LaneRec1& rec, int sb) {
    const uint32_t lohi = kSplit ? ((rec.lohi & 0xFFFFu) | (rec.hi16 << 16)) : rec.lohi;
    const uint32_t cfg = rec.cc & 0xFFu;
    const float lo = sx8_h2f(lohi), hi = sx8_h2f(lohi >> 16);
    const float d = hi - lo;
    DecPrep1 p;
    sub_range(lo, d, d * 0.25f, d * 0.015873f, cfg, sb, p.rlo, p.step);
    dec_unpack(rec.qh, rec.ql, p.le, p.lv);
    const uint32_t cf = kSplit ? rec.cf : (rec.cc >> 8);
    p.cpair = coeff_pair_f16(sx8_sext4(cf >> (4 * (sb >> 1))));
    return p;
}

// the sub-block's 8 weights into buffer b, slot (n-fragment c / 32, k-step sb & 1, lane
// 32 (sb / 2) + c % 32); the even sub-block of a pair stores the coefficient pair
template <bool kPca>
__device__ __forceinline__ void dec1_finish(GemmSmem& sm, const DecPrep1& p, int kb, int b, int c, int sb) {
    sm.wt[b][c >> 5][sb & 1][32 * (sb >> 1) + (c & 31)] =
        sx8_u32x4{dec_pair(p.le, p.lv, 0, p.rlo, p.step), dec_pair(p.le, p.lv, 1, p.rlo, p.step),
                  dec_pair(p.le, p.lv, 2, p.rlo, p.step), dec_pair(p.le, p.lv, 3, p.rlo, p.step)};
    if constexpr (kPca) {
        if ((sb & 1) == 0) {
            const int t4 = kb & 3;
            uint32_t* dst = reinterpret_cast<uint32_t*>(&sm.pt[(kb >> 2) & 1][c >> 5][(t4 >> 1) * 32 + (c & 31)]);
            dst[2 * (t4 & 1) + (sb >> 1)] = p.cpair;
        }
    }
}

// kPair (the MLP's gate and up projections, g.m[0] and g.m[1], N columns each): a tile's
// 128 columns are 64 gate columns and the same 64 up columns (tile p: intermediate indices
// 64 p .. 64 p + 63; fragments 0, 1 gate, 2, 3 up), so each lane holds g and u of the same
// (row, index) and the epilogue writes x = fp16(silu(g) u) straight into the down
// projection's packed operands (SiluOut: the packed X and Zhl of sx8_gemm_prefill_packed for
// the down projection's basis rows and scales, n_cb = its K blocks).  Whole tiles only (no
// K split).  Waves of even index decode gate columns, odd ones up columns.
struct SiluOut {
    const float* basis;
    const float* scales;
    uint16_t* Xp;
    uint32_t* Zhl;
    int n_cb;
};

template <bool kSplit, int HB, bool kPca, bool kPair = false>
__global__ __launch_bounds__(kW2Threads) __attribute__((amdgpu_waves_per_eu(2, 2))) void k_gemm_w2(
    const uint16_t* __restrict__ Xp, int M, const GemmGroup g, int n_cb, int Tf, int St, int kbs,
    float* __restrict__ part, const SiluOut so) {
    constexpr int MF = kW2MF;
    __shared__ GemmSmem sm;
    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = tid >> 6;
    const int NB = g.NB;
    const int b = blockIdx.x;
    int t, ks = 0, kb0 = 0, kb1 = n_cb;
    if (b < Tf) {
        t = xcd_order(b, Tf);
    } else {
        // Tf is a multiple of 8, so work-group b still runs on XCD b % 8
        const int o = xcd_order(b - Tf, gridDim.x - Tf);
        t = Tf + o / St;
        ks = o % St;
        kb0 = ks * kbs;
        kb1 = min(n_cb, kb0 + kbs);
    }
    int nb = t % NB;
    const int mb = t / NB;
    const int mi = kPair ? 0 : group_mat(g, nb);
    // kPair: this wave decodes columns of the gate (even waves) or up (odd) matrix
    // (wave-uniform, but the compiler cannot tell from the thread index: readfirstlane keeps
    // the weight pointers, and so the buffer resources, in scalar registers)
    const int wm = kPair ? sx8_uniform(wave & 1) : mi;
    const WeightSrc w = g.m[wm].w;
    const uint32_t* __restrict__ Zhl = g.m[mi].Zhl;
    float* __restrict__ Y = g.m[mi].Y;
    const int N = g.m[mi].N;
    const int m0 = mb * kW1BM;
    const int n0 = nb * (kPair ? kBN / 2 : kBN);   // kPair: first intermediate index
    const int hf = lane >> 5, r = lane & 31;
    const int dc = tid & 127, dsb = tid >> 7;    // decode: column and sub-block

    if constexpr (kPca) {
        // coefficient slots of blocks past n_cb are never written: start them at zero (each
        // thread clears one slot of the 512; the barrier of the prologue orders the clears
        // before every coefficient store, which comes after it)
        reinterpret_cast<sx8_u32x4*>(&sm.pt[0][0][0])[tid] = sx8_u32x4{0u, 0u, 0u, 0u};
        lds_barrier();
    }

    LoopSrc<MF> ls;
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
    ls.nn = min(n0 + (kPair ? (dc & 63) : dc), N - 1);
    ls.h = 0;
    ls.x = make_rsrc(Xp, (int64_t)((M + 31) / 32) * n_cb * 2048);
    if constexpr (kPca) ls.z = make_rsrc(Zhl, (int64_t)M * n_cb * 8);
    // kPair: the up matrix's Zhl (fragments 2, 3)
    const sx8_rsrc z_up = make_rsrc(kPair ? g.m[1].Zhl : Zhl, kPca && kPair ? (int64_t)M * n_cb * 8 : 0);
#pragma unroll
    for (int f = 0; f < MF; ++f) {
        const int g32 = (m0 >> 5) + wave * MF + f;
        ls.a_off[f] = (int)((int64_t)g32 * n_cb * 2048) + lane * 16;
        const int row = m0 + wave * 32 * MF + 32 * f + r;
        ls.z_off[f] = (int)(((int64_t)row * n_cb + 2 * hf) * 8);
    }
    // kPair: the down projection's basis rows and scales of this tile's two K blocks, staged
    // in LDS with the prologue's barrier for the epilogue (threads 0-31 one float4 each)
    __shared__ float4 dbas[kPair ? 32 : 1];
    __shared__ float2 dsca[kPair ? 2 : 1];
    float4 dbv = make_float4(0.f, 0.f, 0.f, 0.f);
    float2 dsv = make_float2(0.f, 0.f);
    if constexpr (kPair) {
        const int kbd = min((n0 >> 5) + (tid >> 4), so.n_cb - 1);      // (blocks past n_cb: unused)
        if (tid < 32) dbv = reinterpret_cast<const float4*>(so.basis + (int64_t)kbd * 64)[tid & 15];
        if (tid < 2) dsv = reinterpret_cast<const float2*>(so.scales)[min((n0 >> 5) + tid, so.n_cb - 1)];
    }
    auto load_za_up = [&](sx8_u32x4 (&zu)[MF], int gq) __attribute__((always_inline)) {
#pragma unroll
        for (int f = 0; f < MF; ++f)
            zu[f] = __builtin_bit_cast(sx8_u32x4, __builtin_amdgcn_raw_buffer_load_b128(
                                                      z_up, ls.z_off[f] + gq * 32, 0, 0));
    };

    sx8_float16v acc[MF][4];
#pragma unroll
    for (int f = 0; f < MF; ++f)
#pragma unroll
        for (int j = 0; j < 4; ++j)
#pragma unroll
            for (int i = 0; i < 16; ++i) acc[f][j][i] = 0.f;

    // prologue (as k_gemm_w1): blocks kb0, kb0 + 1 decoded, block kb0 + 2 prepared, records
    // of kb0 + 3 .. kb0 + 6 and A of kb0, kb0 + 1 in flight
    LaneRec1 R[4];
    DecPrep1 P[2];
    sx8_u32x4 A[2][MF][2];
    sx8_u32x4 za[MF];
    sx8_u32x4 zu[kPair ? MF : 1];
    {
        LaneRec1 r0, r1, r2;
        load_rec1<kSplit, HB>(r0, ls, N, kb0, dsb);
        load_rec1<kSplit, HB>(r1, ls, N, min(kb0 + 1, kb1 - 1), dsb);
        load_rec1<kSplit, HB>(r2, ls, N, min(kb0 + 2, kb1 - 1), dsb);
        load_a<MF>(A[0], ls, kb0);
        load_a_step<MF>(A[1], ls, min(kb0 + 1, kb1 - 1), 0);
        if constexpr (kPca) load_za<MF>(za, ls, kb0 >> 2);
        if constexpr (kPca && kPair) load_za_up(zu, kb0 >> 2);
        load_rec1<kSplit, HB>(R[3], ls, N, min(kb0 + 3, kb1 - 1), dsb);
        load_rec1<kSplit, HB>(R[0], ls, N, min(kb0 + 4, kb1 - 1), dsb);
        load_rec1<kSplit, HB>(R[1], ls, N, min(kb0 + 5, kb1 - 1), dsb);
        load_rec1<kSplit, HB>(R[2], ls, N, min(kb0 + 6, kb1 - 1), dsb);
        dec1_finish<kPca>(sm, dec1_prep<kSplit>(r0, dsb), kb0, kb0 % 3, dc, dsb);
        dec1_finish<kPca>(sm, dec1_prep<kSplit>(r1, dsb), kb0 + 1, (kb0 + 1) % 3, dc, dsb);
        P[0] = dec1_prep<kSplit>(r2, dsb);
        if constexpr (kPair) {
            if (tid < 32) dbas[tid] = dbv;
            if (tid < 2) dsca[tid] = dsv;
        }
        lds_barrier();
    }
    const uint8_t* wbase = reinterpret_cast<const uint8_t*>(&sm.wt[0][0][0][lane]);
    sx8_u32x4 bw[4][2];
    auto read_b = [&](int kb, int st) __attribute__((always_inline)) {
        const uint8_t* src = wbase + (kb % 3) * kWtBufBytes;
#pragma unroll
        for (int j = 0; j < 4; ++j)
            bw[j][st] = *reinterpret_cast<const sx8_u32x4*>(src + (j * 2 + st) * 1024);
    };
    read_b(kb0, 0);

    // iteration kb (as k_gemm_w1 with 8 MFMAs per k-step): k-step 0 prepares block kb + 3,
    // k-step 1 finishes block kb + 2 into the ring; PCA k-step at the end of a 4-block group
    auto body = [&](int kb, sx8_u32x4 (&acur)[MF][2], sx8_u32x4 (&aprev)[MF][2], LaneRec1& rx,
                    const DecPrep1& pcur, DecPrep1& pnext, const bool pca) __attribute__((always_inline)) {
        const int ka = min(kb + 2, kb1 - 1);
        const int kp = min(kb + 1, kb1 - 1);
        pnext = dec1_prep<kSplit>(rx, dsb);
#pragma unroll
        for (int j = 0; j < 4; ++j)
#pragma unroll
            for (int f = 0; f < MF; ++f)
                acc[f][j] = __builtin_amdgcn_mfma_f32_32x32x16_f16(
                    __builtin_bit_cast(sx8_half8, bw[j][0]),
                    __builtin_bit_cast(sx8_half8, acur[f][0]), acc[f][j], 0, 0, 0);
        load_a_step<MF>(aprev, ls, kp, 1);
        read_b(kb, 1);
#pragma unroll
        for (int i = 0; i < 8; ++i) {
            __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);   // one MFMA
            __builtin_amdgcn_sched_group_barrier(0x002, 4, 0);   // up to four VALU
            if (i < 4) __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);           // a B read
            else if (i < 6) __builtin_amdgcn_sched_group_barrier(0x020, 1, 0);      // an A load
        }
        SX8_SCHED_FENCE();
        dec1_finish<kPca>(sm, pcur, kb + 2, (kb + 2) % 3, dc, dsb);
#pragma unroll
        for (int j = 0; j < 4; ++j)
#pragma unroll
            for (int f = 0; f < MF; ++f)
                acc[f][j] = __builtin_amdgcn_mfma_f32_32x32x16_f16(
                    __builtin_bit_cast(sx8_half8, bw[j][1]),
                    __builtin_bit_cast(sx8_half8, acur[f][1]), acc[f][j], 0, 0, 0);
        load_a_step<MF>(acur, ls, ka, 0);
        load_rec1<kSplit, HB>(rx, ls, N, min(kb + 7, kb1 - 1), dsb);
        read_b(kb + 1, 0);
#pragma unroll
        for (int i = 0; i < 8; ++i) {
            __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);   // one MFMA
            __builtin_amdgcn_sched_group_barrier(0x002, 3, 0);   // up to three VALU
            if (i < 2) __builtin_amdgcn_sched_group_barrier(0x200, 1, 0);           // ring writes
            else if (i < 8) __builtin_amdgcn_sched_group_barrier(0x020, 1, 0);      // A / record loads
            if (i >= 4) __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);          // B reads
        }
        SX8_SCHED_FENCE();
        if constexpr (kPca) {
            if (pca) {
                const int gq = kb >> 2;
                sx8_half8 zh[MF], zh2[kPair ? MF : 1];
#pragma unroll
                for (int f = 0; f < MF; ++f) zh[f] = mask_za(za[f], n_cb, gq, hf);
                if constexpr (kPair) {
#pragma unroll
                    for (int f = 0; f < MF; ++f) zh2[f] = mask_za(zu[f], n_cb, gq, hf);
                }
#pragma unroll
                for (int j = 0; j < 4; ++j) {
                    const sx8_half8 cq = __builtin_bit_cast(sx8_half8, sm.pt[gq & 1][j][lane]);
#pragma unroll
                    for (int f = 0; f < MF; ++f)
                        acc[f][j] = __builtin_amdgcn_mfma_f32_32x32x16_f16(cq, kPair && j >= 2 ? zh2[f] : zh[f],
                                                                           acc[f][j], 0, 0, 0);
                }
                load_za<MF>(za, ls, min(gq + 1, (kb1 - 1) >> 2));
                if constexpr (kPair) load_za_up(zu, min(gq + 1, (kb1 - 1) >> 2));
            }
        }
        lds_barrier();
    };
    int kb = kb0;   // a multiple of 4
    for (; kb + 4 <= kb1; kb += 4) {
        body(kb, A[0], A[1], R[3], P[0], P[1], false);
        body(kb + 1, A[1], A[0], R[0], P[1], P[0], false);
        body(kb + 2, A[0], A[1], R[1], P[0], P[1], false);
        body(kb + 3, A[1], A[0], R[2], P[1], P[0], true);
    }
    if (kb < kb1) body(kb, A[0], A[1], R[3], P[0], P[1], kb + 1 == kb1);
    if (kb + 1 < kb1) body(kb + 1, A[1], A[0], R[0], P[1], P[0], kb + 2 == kb1);
    if (kb + 2 < kb1) body(kb + 2, A[0], A[1], R[1], P[0], P[1], true);

    if constexpr (kPair) {
        // x = fp16(silu(g) u) of rows m0 + 64 wave + 32 f + r and intermediate indices n0 +
        // 32 jj + t: the down projection's K block n0 / 32 + jj, as its packed operands
        // (indices past N pack zeros; row groups past the packed rows are not written)
        const int Gs = (M + 31) >> 5;
#pragma unroll
        for (int f = 0; f < MF; ++f) {
            const int G = (m0 >> 5) + wave * MF + f;
            if (G >= Gs) continue;                       // uniform across the wave
            const int row = 32 * G + r;
#pragma unroll
            for (int jj = 0; jj < 2; ++jj) {
                const int kb = (n0 >> 5) + jj;
                if (kb >= so.n_cb) continue;             // uniform
                float v[16];
#pragma unroll
                for (int i = 0; i < 16; ++i) {
                    const int idx = n0 + 32 * jj + 8 * (i >> 2) + 4 * hf + (i & 3);
                    v[i] = idx < N ? sx8_silu_mul(acc[f][jj][i], acc[f][jj + 2][i]) : 0.f;
                }
                sx8_pack_fragment(v, row < M, r, hf, reinterpret_cast<const float*>(dbas) + 64 * jj, dsca[jj],
                                  so.Xp + ((int64_t)G * so.n_cb + kb) * 1024,
                                  so.Zhl + ((int64_t)row * so.n_cb + kb) * 2);
            }
        }
        return;
    }
    // epilogue (as k_gemm_w1): partial tiles dense 512 x 128, else Y with bounds
    if (ks > 0) {
        float* pt = part + ((int64_t)(t - Tf) * (St - 1) + ks - 1) * (kW1BM * kBN);
#pragma unroll
        for (int f = 0; f < MF; ++f) {
            float* row = pt + (wave * 32 * MF + 32 * f + r) * kBN;
#pragma unroll
            for (int j = 0; j < 4; ++j)
#pragma unroll
                for (int q = 0; q < 4; ++q)
                    *reinterpret_cast<sx8_float4*>(row + 32 * j + 8 * q + 4 * hf) =
                        sx8_float4{acc[f][j][4 * q], acc[f][j][4 * q + 1], acc[f][j][4 * q + 2],
                                   acc[f][j][4 * q + 3]};
        }
        return;
    }
    const bool vec = (N & 3) == 0 && (reinterpret_cast<uintptr_t>(Y) & 15) == 0;
#pragma unroll
    for (int f = 0; f < MF; ++f) {
        const int m = m0 + wave * 32 * MF + 32 * f + r;
        if (m >= M) continue;
        float* row = Y + (int64_t)m * N;
#pragma unroll
        for (int j = 0; j < 4; ++j)
#pragma unroll
            for (int q = 0; q < 4; ++q) {
                const int n = n0 + 32 * j + 8 * q + 4 * hf;
                const sx8_float4 v = {acc[f][j][4 * q], acc[f][j][4 * q + 1], acc[f][j][4 * q + 2],
                                      acc[f][j][4 * q + 3]};
                if (vec && n + 3 < N) {
                    *reinterpret_cast<sx8_float4*>(row + n) = v;
                } else {
#pragma unroll
                    for (int e = 0; e < 4; ++e)
                        if (n + e < N) row[n + e] = v[e];
                }
            }
    }
}

// Y += the St - 1 partial tiles of each split tile Tf .. T - 1 of k_gemm_w1, in range order
// (deterministic).  One thread per 4 consecutive columns of a tile row.  NP = St - 1 is a
// template argument: every partial is requested before the first add, and exactly NP
// loads go out (clamped copies of the last partial would cost memory-pipeline cycles).
template <int NP>
__global__ __launch_bounds__(256) void k_reduce_tiles(const GemmGroup g, const float* __restrict__ part,
                                                      int M, int Tf, int n_split) {
    constexpr int St = NP + 1;
    const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;     // float4 index
    constexpr int kQ = kW1BM * kBN / 4;                            // float4s per tile
    if (i >= (int64_t)n_split * kQ) return;
    const int ts = (int)(i / kQ);
    const int e = (int)(i - (int64_t)ts * kQ) * 4;
    const int t = Tf + ts;
    int nb = t % g.NB;
    const int mi = group_mat(g, nb);
    const int N = g.m[mi].N;
    const int m = (t / g.NB) * kW1BM + e / kBN;
    const int n = nb * kBN + e % kBN;
    if (m >= M || n >= N) return;
    const float* p = part + (int64_t)ts * (St - 1) * (kW1BM * kBN) + e;
    float* y = g.m[mi].Y + (int64_t)m * N + n;
    sx8_float4 pv[NP];
#pragma unroll
    for (int s = 0; s < NP; ++s) pv[s] = *reinterpret_cast<const sx8_float4*>(p + (int64_t)s * (kW1BM * kBN));
    const bool vec = n + 3 < N && (reinterpret_cast<uintptr_t>(y) & 15) == 0;
    const int ne = min(4, N - n);
    sx8_float4 v = sx8_float4{0.f, 0.f, 0.f, 0.f};
    if (vec) {
        v = *reinterpret_cast<const sx8_float4*>(y);
    } else {
        for (int c = 0; c < ne; ++c) v[c] = y[c];
    }
#pragma unroll
    for (int s = 0; s < NP; ++s) v += pv[s];
    if (vec) {
        *reinterpret_cast<sx8_float4*>(y) = v;
    } else {
        for (int c = 0; c < ne; ++c) y[c] = v[c];
    }
}

// Y_i += partial slices 0 .. S - 2 of every matrix of the group, in slice order
// (deterministic).  Slice s holds the group's M x Ntot partials, matrix i's M x N_i block at
// poff_i; one launch covers all matrices.  kVec (every Y_i 16-byte aligned, every M N_i a
// multiple of 4): 4 floats per thread, never straddling two matrices; otherwise one.
// NP = S - 1 partials, all requested before the first add (exactly NP loads).
template <bool kVec, int NP>
__global__ __launch_bounds__(256) void k_reduce(const GemmGroup g, const float* __restrict__ part,
                                                int64_t MNtot) {
    const int64_t t = (int64_t)blockIdx.x * 256 + threadIdx.x;
    const int64_t e = kVec ? t * 4 : t;
    if (e >= MNtot) return;
    int mi = 0;
    while (mi + 1 < g.n_mats && e >= g.m[mi + 1].poff) ++mi;
    float* Y = g.m[mi].Y + (e - g.m[mi].poff);
    if constexpr (kVec) {
        sx8_float4 pv[NP];
#pragma unroll
        for (int p = 0; p < NP; ++p) pv[p] = *reinterpret_cast<const sx8_float4*>(part + (int64_t)p * MNtot + e);
        sx8_float4 y = *reinterpret_cast<const sx8_float4*>(Y);
#pragma unroll
        for (int p = 0; p < NP; ++p) y += pv[p];
        *reinterpret_cast<sx8_float4*>(Y) = y;
    } else {
        float pv[NP];
#pragma unroll
        for (int p = 0; p < NP; ++p) pv[p] = part[(int64_t)p * MNtot + e];
        float y = *Y;
#pragma unroll
        for (int p = 0; p < NP; ++p) y += pv[p];
        *Y = y;
    }
}

// fp32 Z (M, n_cb, 2) -> Zhl (M, n_cb, 4 x fp16): each value as the pair sx8_split_hl(z).
__global__ __launch_bounds__(256) void k_z_hl(const float* __restrict__ Z, int64_t n, uint32_t* __restrict__ Zhl) {
    const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
    if (i < n) Zhl[i] = sx8_split_hl(Z[i]);
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
    // the main loop addresses every operand with 32-bit buffer offsets
    if (M * ldx * 2 > 0x7FFFFFFF || N * n_cb * 24 > 0x7FFFFFFF || M * n_cb * 8 > 0x7FFFFFFF ||
        (M + 31) / 32 * n_cb * 2048 > 0x7FFFFFFF)
        return fail(SX8_ERR_UNSUPPORTED, "%s: operands beyond 2 GiB", what);
    return SX8_OK;
}

// Work split of one call.  k_gemm (w1 = false): tiles of 128 MF rows, S K ranges of
// kb_per_split blocks (a multiple of 4); grids with fewer tiles than the 256 CUs split K and
// pay (S - 1) M N f32 partials written and read back once (k_reduce).  k_gemm_w1 (w1 =
// true): 512-row tiles, the first Tf whole (full rounds of the CUs), the other n_split
// tiles in St K ranges of kbs blocks (partials added by k_reduce_tiles).
struct Plan {
    bool w1;
    int MF, S, kb_per_split;   // k_gemm
    int Tf, St, kbs;           // k_gemm_w1
    int64_t n_split;           // k_gemm_w1: tiles split St ways
    int64_t G;                 // work-groups
    double cost;
};

// Costs are in units of one 256-row tile iteration (~0.5 us): rounds of work-groups over the
// 256 CUs times the K blocks per work-group (a 512-row iteration costs kW1Cost of them, a
// 128-row one kMF1Cost), plus the traffic a split adds at about 10 KB per CU per unit: for
// S K ranges of a tile, S - 1 partial tiles written and read back, and Y read and written
// again by the sum -- 2 S tile-sized transfers, for both kernels.
constexpr double kW1Cost = 1.60, kMF1Cost = 0.62;
constexpr double kBytesPerUnit = 256.0 * 10240.0;

Plan plan_split(int64_t M, int64_t N, int64_t T, int64_t n_cb, int64_t S, int MF) {
    Plan p{};
    p.w1 = false;
    p.MF = MF;
    const int64_t groups = (n_cb + 3) / 4;
    p.kb_per_split = (int)(4 * ((groups + S - 1) / S));
    p.S = (int)((n_cb + p.kb_per_split - 1) / p.kb_per_split);
    p.G = T * p.S;
    const double rounds = (double)((p.G + 255) / 256);
    p.cost = rounds * p.kb_per_split * (MF == 2 ? 1.0 : kMF1Cost) +
             (p.S > 1 ? 2.0 * p.S * M * N * 4.0 / kBytesPerUnit : 0.0);
    return p;
}

// Tiles of 128 MF rows over NB column tiles (N columns in all); the number of K ranges
// (1..8, at most one per 4-block group) that the cost model prefers.
Plan plan_k_gemm(int64_t M, int64_t N, int64_t NB, int64_t n_cb, int MF, int64_t part_cap) {
    const int64_t T = ((M + 128 * MF - 1) / (128 * MF)) * NB;
    const int64_t groups = (n_cb + 3) / 4;
    Plan best = plan_split(M, N, T, n_cb, 1, MF);
    for (int64_t S = 2; S <= std::min<int64_t>(8, groups); ++S) {
        const Plan p = plan_split(M, N, T, n_cb, S, MF);
        if (p.cost < best.cost && (int64_t)(p.S - 1) * M * N * 4 <= part_cap) best = p;
    }
    return best;
}

// 512-row tiles, the first Tf (0 or whole rounds of 256) over the whole K and the rest in
// St K ranges.
Plan make_w1(int64_t M, int64_t NB, int64_t n_cb, int64_t Tf, int64_t St) {
    const int64_t T = ((M + kW1BM - 1) / kW1BM) * NB;
    const int64_t groups = (n_cb + 3) / 4;
    const int64_t rem = T - Tf;
    Plan p{};
    p.w1 = true;
    p.MF = kW1MF;
    p.Tf = (int)Tf;
    p.kbs = (int)(4 * ((groups + St - 1) / St));
    p.St = (int)((n_cb + p.kbs - 1) / p.kbs);
    p.n_split = p.St > 1 ? rem : 0;
    p.G = Tf + rem * p.St;
    const double tile_bytes = (double)kW1BM * kBN * 4.0;
    p.cost = (double)(Tf / 256) * n_cb * kW1Cost + (double)((rem * p.St + 255) / 256) * p.kbs * kW1Cost +
             (p.St > 1 ? (double)rem * 2.0 * p.St * tile_bytes / kBytesPerUnit : 0.0);
    return p;
}

// Tf = 0 (every tile split St ways) or the whole rounds of 256 tiles with the remainder
// split; St from 1 to 8.
Plan plan_w1(int64_t M, int64_t NB, int64_t n_cb, int64_t part_cap) {
    const int64_t T = ((M + kW1BM - 1) / kW1BM) * NB;
    const int64_t groups = (n_cb + 3) / 4;
    Plan best{};
    best.cost = 1e300;
    for (int64_t Tf : {int64_t(0), T / 256 * 256}) {
        for (int64_t St = 1; St <= std::min<int64_t>(8, groups); ++St) {
            const Plan p = make_w1(M, NB, n_cb, Tf, St);
            if (p.cost < best.cost && p.n_split * (p.St - 1) * kW1BM * kBN * 4 <= part_cap) best = p;
            if (Tf == T) break;
        }
    }
    return best;
}

// Tuning knobs, read from the environment once (at the first prefill call or plan query) and
// again only by sx8_gemm_reload_tuning, so a workspace sized for a call stays valid for it:
// SX8_GEMM_TILE=256 or 512 forces a tile height; SX8_GEMM_PLAN forces one plan, "k<MF>:<S>"
// (128 MF-row tiles in S K ranges) or "w<0|1>:<St>" (512-row tiles, 1: whole rounds first,
// St K ranges for the rest); SX8_GEMM_W2=0 runs 512-row plans on k_gemm_w1.
struct Tuning {
    int tile = 0;          // 0: the planner's choice
    bool w2 = true;
    bool plan = false;     // SX8_GEMM_PLAN parsed
    char kind = 0;
    int a = 0, b = 0;
};

Tuning read_tuning() {
    Tuning t;
    if (const char* e = getenv("SX8_GEMM_TILE")) t.tile = atoi(e);
    if (const char* e = getenv("SX8_GEMM_W2")) t.w2 = atoi(e) != 0;
    if (const char* f = getenv("SX8_GEMM_PLAN"))
        t.plan = sscanf(f, "%c%d:%d", &t.kind, &t.a, &t.b) == 3;
    return t;
}

std::mutex g_tuning_mu;
Tuning g_tuning;
bool g_tuning_read = false;

Tuning tuning() {
    std::lock_guard<std::mutex> lk(g_tuning_mu);
    if (!g_tuning_read) {
        g_tuning = read_tuning();
        g_tuning_read = true;
    }
    return g_tuning;
}

// N columns in NB column tiles (a group pads every matrix to whole tiles).  The plan forced
// by SX8_GEMM_PLAN if it is valid for the shape, else SX8_GEMM_TILE's tile height, else the
// cheaper plan.  part_cap bounds the split-K partial bytes (the unsplit plans need none).
Plan plan_gemm(int64_t M, int64_t N, int64_t NB, int64_t n_cb, int64_t part_cap = INT64_MAX) {
    const int MF = M > 128 ? 2 : 1;
    // k_gemm_w1 addresses rows up to the next multiple of 512 with 31-bit offsets
    const int64_t Mp = (M + kW1BM - 1) / kW1BM * kW1BM;
    const bool w1_ok = M > 256 && Mp / 32 * n_cb * 2048 <= 0x7FFFFFFF && Mp * n_cb * 8 <= 0x7FFFFFFF;
    const Tuning tu = tuning();
    if (tu.plan) {
        const char kind = tu.kind;
        const int a = tu.a, b = tu.b;
        const int64_t groups = (n_cb + 3) / 4;
        if (b >= 1 && b <= std::min<int64_t>(8, groups)) {
            if (kind == 'k' && (a == 1 || a == 2)) {
                const int64_t T = ((M + 128 * a - 1) / (128 * a)) * NB;
                const Plan p = plan_split(M, N, T, n_cb, b, a);
                if ((int64_t)(p.S - 1) * M * N * 4 <= part_cap) return p;
            }
            if (kind == 'w' && (a == 0 || a == 1) && w1_ok) {
                const int64_t T = ((M + kW1BM - 1) / kW1BM) * NB;
                const Plan p = make_w1(M, NB, n_cb, a ? T / 256 * 256 : 0, b);
                if (p.n_split * (p.St - 1) * kW1BM * kBN * 4 <= part_cap) return p;
            }
        }
    }
    Plan p256 = plan_k_gemm(M, N, NB, n_cb, MF, part_cap);
    // past 128 rows, 128-row tiles only where the 256-row plan leaves more than half the
    // CUs idle (the cost model prices them too cheaply for fuller grids).  Plan sweep at M =
    // 512 (every plan of each call, same box): k 1024 x 2560 26.0 us on 128-row tiles in 5
    // K ranges against 28.8 on 256-row tiles in 7 (112 work-groups); q, o and the q/k/v
    // group ran 1-5 us slower on 128-row tiles than on their 256-row plans (256, 160, 192
    // work-groups)
    if (MF == 2 && p256.G < 128 && tu.tile != 256) {
        const Plan p128 = plan_k_gemm(M, N, NB, n_cb, 1, part_cap);
        if (p128.cost < p256.cost) p256 = p128;
    }
    if (!w1_ok) return p256;
    const Plan p512 = plan_w1(M, NB, n_cb, part_cap);
    const int forced = tu.tile;
    if (forced == 256) return p256;
    if (forced == 512) return p512;
    return p512.cost < p256.cost ? p512 : p256;
}

// How the PCA operand reaches the kernel: none (core weights only), computed here from
// basis/scales, converted from a caller's f32 Z, or written by the caller's producer kernel
// together with the packed X (kPacked: nothing is staged in the workspace).
enum class ZMode { kNone, kBasis, kGiven, kPacked };

template <bool kSplit, bool kPca, int HB, int MF>
void launch_mf(const Plan& p, hipStream_t st, const uint16_t* Xp, int64_t M, const GemmGroup& g,
               int64_t n_cb, float* part) {
    hipLaunchKernelGGL((k_gemm<kSplit, HB, kPca, MF>), dim3((unsigned)p.G), dim3(kThreads), 0, st, Xp,
                       (int)M, g, (int)n_cb, p.S, p.kb_per_split, part);
}

template <bool kSplit, bool kPca, int HB>
void launch_hb(const Plan& p, hipStream_t st, const uint16_t* Xp, int64_t M, const GemmGroup& g,
               int64_t n_cb, float* part) {
    // 512-row plans run k_gemm_w2 (two waves per SIMD, measured 2-4% faster than k_gemm_w1
    // on the layer's 512-row shapes); SX8_GEMM_W2=0 selects k_gemm_w1 (tuning)
    const bool w2 = tuning().w2;
    if (p.w1 && w2)
        hipLaunchKernelGGL((k_gemm_w2<kSplit, HB, kPca>), dim3((unsigned)p.G), dim3(kW2Threads), 0, st,
                           Xp, (int)M, g, (int)n_cb, p.Tf, p.St, p.kbs, part, SiluOut{});
    else if (p.w1)
        hipLaunchKernelGGL((k_gemm_w1<kSplit, HB, kPca>), dim3((unsigned)p.G), dim3(kW1Threads), 0, st,
                           Xp, (int)M, g, (int)n_cb, p.Tf, p.St, p.kbs, part);
    else if (p.MF == 2)
        launch_mf<kSplit, kPca, HB, 2>(p, st, Xp, M, g, n_cb, part);
    else
        launch_mf<kSplit, kPca, HB, 1>(p, st, Xp, M, g, n_cb, part);
}

// Workspace of one call, carved from the caller's buffer (256-byte aligned): every matrix's
// Zhl operand (M * n_cb * 8 bytes each, 256-byte padded; absent for the core-only form),
// the packed X (ceil(M / 32) * n_cb * 2 KB) and the split-K partials of the plan.
struct WsLayout {
    int64_t z_bytes;      // per matrix
    int64_t xp_bytes;
    int64_t part_bytes;
    int64_t total;
};

WsLayout ws_layout(const Plan& p, int64_t M, int64_t Ntot, int64_t n_cb, int n_mats, bool with_z,
                   bool staged = true) {
    WsLayout l;
    l.z_bytes = with_z && staged ? ((M * n_cb * 8 + 255) & ~int64_t(255)) : 0;
    l.xp_bytes = staged ? ((M + 31) / 32 * n_cb * 2048 + 255) & ~int64_t(255) : 0;
    l.part_bytes = p.w1 ? p.n_split * (p.St - 1) * kW1BM * kBN * 4 : (int64_t)(p.S - 1) * M * Ntot * 4;
    l.total = l.z_bytes * n_mats + l.xp_bytes + l.part_bytes;
    return l;
}

// Group width and column tiles; false if the group is too wide for 32-bit column indices.
bool group_width(int n_mats, const int64_t* Ns, int64_t& Ntot, int64_t& NB) {
    Ntot = NB = 0;
    for (int i = 0; i < n_mats; ++i) {
        Ntot += Ns[i];
        NB += (Ns[i] + kBN - 1) / kBN;
    }
    return Ntot <= 0x7FFFFFFF;
}

// One call over n_mats matrices that share X (all of one contract).  Plan over the group's
// total width; in the caller's workspace, stage the packed X (one pass over X, with every
// matrix's Zhl operand) followed by the split-K partials; run the GEMM and, for a split
// plan, the fixed-order partial sums.  Nothing is allocated and nothing synchronizes: the
// call only enqueues kernels on `st`.
// Split-K sums a caller takes over (the *_deferred entry points): the plan's S - 1 partial
// slices in the workspace, slice s of matrix i at part + s * slice + M * (N_0 + .. + N_{i-1}).
struct PendingSums {
    float* part;
    int np;
    int64_t slice;
};

// The operands a producer kernel wrote (ZMode::kPacked): the packed X and every matrix's Zhl.
struct PackedIn {
    const uint16_t* Xp;
    const uint32_t* const* Zhl;
};

template <bool kSplit>
int32_t run_gemm(const char* what, const uint16_t* X, int64_t M, int64_t ldx, int64_t K, int n_mats,
                 const WeightSrc* ws_in, int32_t hdr_bytes, ZMode zm, const float* const* bases,
                 const float* const* scales, const float* Z, const int64_t* Ns, int64_t n_cb,
                 float* const* Ys, void* workspace, int64_t workspace_bytes, hipStream_t st,
                 const float* silu_g = nullptr, const float* silu_u = nullptr,
                 int64_t part_cap = INT64_MAX, PendingSums* defer = nullptr, const PackedIn* packed = nullptr) {
    using namespace sx8;
    if (defer) *defer = PendingSums{nullptr, 0, 0};
    int64_t Ntot = 0, NB = 0;
    if (!group_width(n_mats, Ns, Ntot, NB)) return fail(SX8_ERR_UNSUPPORTED, "%s: group too wide", what);
    const Plan p = plan_gemm(M, Ntot, NB, n_cb, part_cap);
    if (p.G > 0x7FFFFFFF) return fail(SX8_ERR_UNSUPPORTED, "%s: grid too large", what);
    const bool staged = zm != ZMode::kPacked;
    const WsLayout lay = ws_layout(p, M, Ntot, n_cb, n_mats, zm != ZMode::kNone, staged);
    // (a packed call whose plan does not split K needs no workspace at all)
    if (lay.total > 0 && (!workspace || workspace_bytes < lay.total || !aligned(workspace, 256)))
        return fail(SX8_ERR_INVALID,
                    "%s: needs a 256-byte aligned workspace of %lld bytes "
                    "(%s), got %lld bytes at %p",
                    what, (long long)lay.total,
                    staged ? "sx8_gemm_prefill_workspace_bytes" : "sx8_gemm_prefill_packed_workspace_bytes",
                    (long long)workspace_bytes, workspace);
    uint8_t* ws = reinterpret_cast<uint8_t*>(workspace);
    const int64_t z_bytes = lay.z_bytes;
    const uint16_t* Xp = staged ? reinterpret_cast<uint16_t*>(ws + z_bytes * n_mats) : packed->Xp;
    float* part = reinterpret_cast<float*>(ws + z_bytes * n_mats + lay.xp_bytes);
    GemmGroup g{};
    g.n_mats = n_mats;
    g.Ntot = Ntot;
    int64_t off = 0;
    for (int i = 0; i < n_mats; ++i) {
        GemmMat& m = g.m[i];
        m.w = ws_in[i];
        m.Zhl = staged ? reinterpret_cast<const uint32_t*>(ws + z_bytes * i) : packed->Zhl[i];
        m.Y = Ys[i];
        m.N = (int)Ns[i];
        m.nb = (int)((Ns[i] + kBN - 1) / kBN);
        m.poff = M * off;
        off += Ns[i];
        g.NB += m.nb;
    }
    // one pass over X: the packed copy and every matrix's Zhl
    ZSets zs{};
    if (zm == ZMode::kBasis) {
        zs.n = n_mats;
        for (int i = 0; i < n_mats; ++i) {
            zs.basis[i] = bases[i];
            zs.scales[i] = scales[i];
            zs.Z[i] = reinterpret_cast<float*>(ws + z_bytes * i);
        }
    } else if (zm == ZMode::kGiven) {
        const int64_t n = M * n_cb * 2;
        hipLaunchKernelGGL(k_z_hl, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, st, Z, n,
                           reinterpret_cast<uint32_t*>(ws));
    }
    if (staged) {
        uint16_t* xp_ws = reinterpret_cast<uint16_t*>(ws + z_bytes * n_mats);
        const int32_t rc = silu_g ? compute_z_silu(silu_g, silu_u, M, ldx, K, zs, n_cb, xp_ws, st)
                                  : compute_z_sets(X, M, ldx, K, zs, n_cb, true, xp_ws, st);
        if (rc != SX8_OK) return rc;
    }
    if constexpr (kSplit) {
        launch_hb<true, true, 6>(p, st, Xp, M, g, n_cb, part);
    } else if (zm == ZMode::kNone) {
        if (hdr_bytes == 8)
            launch_hb<false, false, 8>(p, st, Xp, M, g, n_cb, part);
        else
            launch_hb<false, false, 6>(p, st, Xp, M, g, n_cb, part);
    } else {
        if (hdr_bytes == 8)
            launch_hb<false, true, 8>(p, st, Xp, M, g, n_cb, part);
        else
            launch_hb<false, true, 6>(p, st, Xp, M, g, n_cb, part);
    }
    // the partial sums, instantiated per partial count (1 .. kMaxSplitParts)
    auto by_np = [](int np, auto&& f) {
        switch (np) {
            case 1: f(std::integral_constant<int, 1>{}); break;
            case 2: f(std::integral_constant<int, 2>{}); break;
            case 3: f(std::integral_constant<int, 3>{}); break;
            case 4: f(std::integral_constant<int, 4>{}); break;
            case 5: f(std::integral_constant<int, 5>{}); break;
            case 6: f(std::integral_constant<int, 6>{}); break;
            default: f(std::integral_constant<int, 7>{}); break;
        }
    };
    static_assert(kMaxSplitParts == 7, "by_np covers 1 .. kMaxSplitParts partials");
    if (p.w1 && p.n_split > 0) {
        const int64_t n4 = p.n_split * (kW1BM * kBN / 4);
        by_np(p.St - 1, [&](auto np) {
            hipLaunchKernelGGL((k_reduce_tiles<decltype(np)::value>), dim3((unsigned)((n4 + 255) / 256)),
                               dim3(256), 0, st, g, part, (int)M, p.Tf, (int)p.n_split);
        });
    } else if (!p.w1 && p.S > 1 && defer) {
        // the caller adds the slices (in slice order, as k_reduce does) where it reads Y
        *defer = PendingSums{part, p.S - 1, M * Ntot};
    } else if (!p.w1 && p.S > 1) {
        bool vec = true;
        for (int i = 0; i < n_mats; ++i) vec = vec && aligned(Ys[i], 16) && (M * Ns[i]) % 4 == 0;
        const int64_t MN = M * Ntot;
        by_np(p.S - 1, [&](auto np) {
            constexpr int NP = decltype(np)::value;
            if (vec)
                hipLaunchKernelGGL((k_reduce<true, NP>), dim3((unsigned)((MN / 4 + 255) / 256)), dim3(256), 0,
                                   st, g, part, MN);
            else
                hipLaunchKernelGGL((k_reduce<false, NP>), dim3((unsigned)((MN + 255) / 256)), dim3(256), 0, st,
                                   g, part, MN);
        });
    }
    return check_launch(what);
}

}  // namespace

extern "C" int64_t sx8_gemm_prefill_workspace_bytes(int64_t M, int32_t n_mats, const int64_t* Ns,
                                                    int64_t n_cb) {
    if (M <= 0 || n_cb <= 0 || !Ns || n_mats < 1 || n_mats > kMaxGemmGroup || M > 0x7FFFFFFF) return -1;
    for (int i = 0; i < n_mats; ++i)
        if (Ns[i] <= 0) return -1;
    int64_t Ntot = 0, NB = 0;
    if (!group_width(n_mats, Ns, Ntot, NB)) return -1;
    const Plan p = plan_gemm(M, Ntot, NB, n_cb);
    return ws_layout(p, M, Ntot, n_cb, n_mats, true).total;
}

extern "C" int32_t sx8_gemm_reload_tuning(void) {
    const Tuning t = read_tuning();
    std::lock_guard<std::mutex> lk(g_tuning_mu);
    g_tuning = t;
    g_tuning_read = true;
    return SX8_OK;
}

extern "C" int32_t sx8_gemm_prefill_plan(int64_t M, int32_t n_mats, const int64_t* Ns, int64_t n_cb,
                                         int64_t* desc) {
    using namespace sx8;
    if (!desc || sx8_gemm_prefill_workspace_bytes(M, n_mats, Ns, n_cb) < 0)
        return fail(SX8_ERR_INVALID, "sx8_gemm_prefill_plan: bad shape");
    int64_t Ntot = 0, NB = 0;
    group_width(n_mats, Ns, Ntot, NB);
    const Plan p = plan_gemm(M, Ntot, NB, n_cb);
    desc[0] = p.w1 ? kW1BM : 128 * p.MF;
    desc[1] = p.G;
    desc[2] = p.w1 ? p.St : p.S;
    desc[3] = p.w1 ? p.kbs : p.kb_per_split;
    desc[4] = p.w1 ? p.Tf : 0;
    desc[5] = p.w1 ? p.n_split : 0;
    desc[6] = ws_layout(p, M, Ntot, n_cb, n_mats, true).total;
    desc[7] = 0;
    return ok();
}

extern "C" int32_t sx8_gemm_prefill(const uint16_t* X, int64_t M, int64_t ldx, int64_t K,
                                    const uint8_t* hdr, const uint8_t* levels, int32_t hdr_bytes,
                                    const float* basis, const float* scales, int64_t N,
                                    int64_t n_cb, float* Y, void* workspace, int64_t workspace_bytes,
                                    void* stream) {
    using namespace sx8;
    if (!X || !hdr || !levels || !basis || !scales || !Y)
        return fail(SX8_ERR_INVALID, "sx8_gemm_prefill: null pointer");
    if (hdr_bytes != 6 && hdr_bytes != 8)
        return fail(SX8_ERR_INVALID, "sx8_gemm_prefill: hdr_bytes must be 6 or 8, got %d", hdr_bytes);
    if (!aligned(hdr, hdr_bytes == 8 ? 8 : 2) || !aligned(levels, 8) || !aligned(X, 2) ||
        !aligned(Y, 4) || !aligned(basis, 16) || !aligned(scales, 8))
        return fail(SX8_ERR_INVALID, "sx8_gemm_prefill: misaligned pointer");
    const int32_t rc = check_shape("sx8_gemm_prefill", M, ldx, K, N, n_cb);
    if (rc != SX8_OK) return rc;
    WeightSrc w{};
    w.hdr = hdr;
    w.levels = levels;
    return run_gemm<false>("sx8_gemm_prefill", X, M, ldx, K, 1, &w, hdr_bytes, ZMode::kBasis, &basis,
                           &scales, nullptr, &N, n_cb, &Y, workspace, workspace_bytes, as_stream(stream));
}

// ------------------------------------------------- the no-allocation prefill entry point
//
// sx8_gemm_prefill_static: sx8_gemm_prefill for callers that cannot allocate (code under
// HIP graph capture, serving loops, harnesses that forbid hipMalloc).  Its workspace is
// `scratch`, a file-scope device array of kScratchBytes that every device running this
// library holds until the process ends.  In host code `scratch` names a host-side stand-in,
// not device memory: its device address is looked up once per device with
// hipGetSymbolAddress (on the entry point's first call on that device, with the device
// current) and only that address is passed to kernels.  Calls on one device share the
// array: calls that overlap in time on one device race.  Nothing in it needs clearing:
// every byte a call reads was written earlier in the same call (Zhl and the packed X by
// the Z pass, partial tiles by the split-K work-groups; rows past M read zero through the
// buffer loads' range checks).

constexpr int64_t kScratchBytes = int64_t(64) << 20;
static __device__ __align__(256) uint8_t scratch[kScratchBytes];

namespace {
constexpr int kMaxScratchDevices = 64;
std::mutex g_scratch_mutex;
void* g_scratch_dev[kMaxScratchDevices] = {};

// Device address of `scratch` on the current device (looked up once per device).
int32_t scratch_address(void** out) {
    using namespace sx8;
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess) return fail(SX8_ERR_HIP, "sx8_gemm_prefill_static: hipGetDevice failed");
    if (dev < 0 || dev >= kMaxScratchDevices)
        return fail(SX8_ERR_UNSUPPORTED, "sx8_gemm_prefill_static: device %d beyond %d", dev, kMaxScratchDevices);
    std::lock_guard<std::mutex> lock(g_scratch_mutex);
    if (!g_scratch_dev[dev]) {
        void* p = nullptr;
        const hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
        if (e != hipSuccess || !p)
            return fail(SX8_ERR_HIP, "sx8_gemm_prefill_static: hipGetSymbolAddress(scratch) failed: %s",
                        hipGetErrorString(e));
        g_scratch_dev[dev] = p;
    }
    *out = g_scratch_dev[dev];
    return SX8_OK;
}
}  // namespace

extern "C" int32_t sx8_gemm_prefill_static(const uint16_t* X, int64_t M, int64_t ldx, int64_t K,
                                           const uint8_t* hdr, const uint8_t* levels, int32_t hdr_bytes,
                                           const float* basis, const float* scales, int64_t N,
                                           int64_t n_cb, float* Y, void* stream) {
    using namespace sx8;
    const char* what = "sx8_gemm_prefill_static";
    if (!X || !hdr || !levels || !basis || !scales || !Y) return fail(SX8_ERR_INVALID, "%s: null pointer", what);
    if (hdr_bytes != 6 && hdr_bytes != 8)
        return fail(SX8_ERR_INVALID, "%s: hdr_bytes must be 6 or 8, got %d", what, hdr_bytes);
    if (!aligned(hdr, hdr_bytes == 8 ? 8 : 2) || !aligned(levels, 8) || !aligned(X, 2) ||
        !aligned(Y, 4) || !aligned(basis, 16) || !aligned(scales, 8))
        return fail(SX8_ERR_INVALID, "%s: misaligned pointer", what);
    int32_t rc = check_shape(what, M, ldx, K, N, n_cb);
    if (rc != SX8_OK) return rc;
    // Zhl and the packed X must fit; split-K partials only in what is left of the array
    Plan unsplit{};
    unsplit.S = 1;
    const int64_t fixed = ws_layout(unsplit, M, N, n_cb, 1, true).total;
    if (fixed > kScratchBytes)
        return fail(SX8_ERR_UNSUPPORTED,
                    "%s: M=%lld n_cb=%lld needs %lld scratch bytes, the static scratch holds %lld "
                    "(use sx8_gemm_prefill with a workspace)",
                    what, (long long)M, (long long)n_cb, (long long)fixed, (long long)kScratchBytes);
    void* ws = nullptr;
    rc = scratch_address(&ws);
    if (rc != SX8_OK) return rc;
    WeightSrc w{};
    w.hdr = hdr;
    w.levels = levels;
    return run_gemm<false>(what, X, M, ldx, K, 1, &w, hdr_bytes, ZMode::kBasis, &basis, &scales, nullptr, &N,
                           n_cb, &Y, ws, kScratchBytes, as_stream(stream), nullptr, nullptr,
                           kScratchBytes - fixed);
}

namespace {

// Hands the pending sums to the caller's out-parameters (all three must be given).
int32_t report_pending(const char* what, const PendingSums& pend, float** parts, int32_t* n_parts,
                       int64_t* slice) {
    *parts = pend.part;
    *n_parts = pend.np;
    *slice = pend.slice;
    return sx8::check_launch(what);
}

int32_t gemm_silu_impl(const char* what, const float* g, const float* u, int64_t M, int64_t K,
                       const uint8_t* hdr, const uint8_t* levels, int32_t hdr_bytes, const float* basis,
                       const float* scales, int64_t N, int64_t n_cb, float* Y, void* workspace,
                       int64_t workspace_bytes, void* stream, PendingSums* defer) {
    using namespace sx8;
    if (!g || !u || !hdr || !levels || !basis || !scales || !Y)
        return fail(SX8_ERR_INVALID, "%s: null pointer", what);
    if (hdr_bytes != 6 && hdr_bytes != 8)
        return fail(SX8_ERR_INVALID, "%s: hdr_bytes must be 6 or 8, got %d", what, hdr_bytes);
    if (!aligned(hdr, hdr_bytes == 8 ? 8 : 2) || !aligned(levels, 8) || !aligned(g, 4) || !aligned(u, 4) ||
        !aligned(Y, 4) || !aligned(basis, 16) || !aligned(scales, 8))
        return fail(SX8_ERR_INVALID, "%s: misaligned pointer", what);
    const int32_t rc = check_shape(what, M, K, K, N, n_cb);
    if (rc != SX8_OK) return rc;
    WeightSrc w{};
    w.hdr = hdr;
    w.levels = levels;
    return run_gemm<false>(what, nullptr, M, K, K, 1, &w, hdr_bytes, ZMode::kBasis, &basis, &scales, nullptr,
                           &N, n_cb, &Y, workspace, workspace_bytes, as_stream(stream), g, u, INT64_MAX, defer);
}

}  // namespace

extern "C" int32_t sx8_dec_gemm_silu(const float* g, const float* u, int64_t M, int64_t K,
                                     const uint8_t* hdr, const uint8_t* levels, int32_t hdr_bytes,
                                     const float* basis, const float* scales, int64_t N, int64_t n_cb,
                                     float* Y, void* workspace, int64_t workspace_bytes, void* stream) {
    return gemm_silu_impl("sx8_dec_gemm_silu", g, u, M, K, hdr, levels, hdr_bytes, basis, scales, N, n_cb, Y,
                          workspace, workspace_bytes, stream, nullptr);
}

extern "C" int32_t sx8_dec_gemm_silu_deferred(const float* g, const float* u, int64_t M, int64_t K,
                                              const uint8_t* hdr, const uint8_t* levels, int32_t hdr_bytes,
                                              const float* basis, const float* scales, int64_t N,
                                              int64_t n_cb, float* Y, void* workspace,
                                              int64_t workspace_bytes, float** parts, int32_t* n_parts,
                                              int64_t* slice, void* stream) {
    using namespace sx8;
    const char* what = "sx8_dec_gemm_silu_deferred";
    if (!parts || !n_parts || !slice) return fail(SX8_ERR_INVALID, "%s: null out-parameter", what);
    PendingSums pend{};
    const int32_t rc = gemm_silu_impl(what, g, u, M, K, hdr, levels, hdr_bytes, basis, scales, N, n_cb, Y,
                                      workspace, workspace_bytes, stream, &pend);
    if (rc != SX8_OK) return rc;
    return report_pending(what, pend, parts, n_parts, slice);
}

extern "C" int32_t sx8_gemm_prefill_split(const uint16_t* X, int64_t M, int64_t ldx, int64_t K,
                                          const uint16_t* dmin, const uint16_t* dmax,
                                          const uint8_t* config, const uint8_t* coeff,
                                          const uint8_t* hi, const uint8_t* lo, const float* basis,
                                          const float* scales, int64_t N, int64_t n_cb, float* Y,
                                          void* workspace, int64_t workspace_bytes, void* stream) {
    using namespace sx8;
    if (!X || !dmin || !dmax || !config || !coeff || !hi || !lo || !basis || !scales || !Y)
        return fail(SX8_ERR_INVALID, "sx8_gemm_prefill_split: null pointer");
    if (!aligned(dmin, 2) || !aligned(dmax, 2) || !aligned(hi, 8) || !aligned(lo, 4) ||
        !aligned(X, 2) || !aligned(Y, 4) || !aligned(basis, 16) || !aligned(scales, 8))
        return fail(SX8_ERR_INVALID, "sx8_gemm_prefill_split: misaligned pointer");
    const int32_t rc = check_shape("sx8_gemm_prefill_split", M, ldx, K, N, n_cb);
    if (rc != SX8_OK) return rc;
    WeightSrc w{};
    w.dmin = dmin;
    w.dmax = dmax;
    w.config = config;
    w.coeff = coeff;
    w.hi = hi;
    w.lo = lo;
    return run_gemm<true>("sx8_gemm_prefill_split", X, M, ldx, K, 1, &w, 6, ZMode::kBasis, &basis,
                          &scales, nullptr, &N, n_cb, &Y, workspace, workspace_bytes, as_stream(stream));
}

extern "C" int32_t sx8_gemm_prefill_z(const uint16_t* X, int64_t M, int64_t ldx, int64_t K,
                                      const uint8_t* hdr, const uint8_t* levels, int32_t hdr_bytes,
                                      const float* Z, int64_t N, int64_t n_cb, float* Y,
                                      void* workspace, int64_t workspace_bytes, void* stream) {
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
    return run_gemm<false>("sx8_gemm_prefill_z", X, M, ldx, K, 1, &w, hdr_bytes, ZMode::kGiven, nullptr,
                           nullptr, Z, &N, n_cb, &Y, workspace, workspace_bytes, as_stream(stream));
}

extern "C" int32_t sx8_gemm_prefill_core(const uint16_t* X, int64_t M, int64_t ldx, int64_t K,
                                         const uint8_t* hdr, const uint8_t* levels,
                                         int32_t hdr_bytes, int64_t N, int64_t n_cb, float* Y,
                                         void* workspace, int64_t workspace_bytes, void* stream) {
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
    return run_gemm<false>("sx8_gemm_prefill_core", X, M, ldx, K, 1, &w, hdr_bytes, ZMode::kNone,
                           nullptr, nullptr, nullptr, &N, n_cb, &Y, workspace, workspace_bytes,
                           as_stream(stream));
}

namespace {

int32_t group_impl(const char* what, const uint16_t* X, int64_t M, int64_t ldx, int64_t K, int32_t n_mats,
                   const uint8_t* const* hdrs, const uint8_t* const* levels, int32_t hdr_bytes,
                   const float* const* bases, const float* const* scales, const int64_t* Ns, int64_t n_cb,
                   float* const* Ys, void* workspace, int64_t workspace_bytes, void* stream,
                   PendingSums* defer) {
    using namespace sx8;
    if (!X || !hdrs || !levels || !bases || !scales || !Ns || !Ys) return fail(SX8_ERR_INVALID, "%s: null pointer", what);
    if (n_mats < 1 || n_mats > kMaxGemmGroup)
        return fail(SX8_ERR_INVALID, "%s: n_mats must be 1..%d, got %d", what, kMaxGemmGroup, n_mats);
    if (hdr_bytes != 6 && hdr_bytes != 8)
        return fail(SX8_ERR_INVALID, "%s: hdr_bytes must be 6 or 8, got %d", what, hdr_bytes);
    if (!aligned(X, 2)) return fail(SX8_ERR_INVALID, "%s: misaligned X", what);
    WeightSrc w[kMaxGemmGroup]{};
    for (int i = 0; i < n_mats; ++i) {
        if (!hdrs[i] || !levels[i] || !bases[i] || !scales[i] || !Ys[i])
            return fail(SX8_ERR_INVALID, "%s: null pointer in matrix %d", what, i);
        if (!aligned(hdrs[i], hdr_bytes == 8 ? 8 : 2) || !aligned(levels[i], 8) || !aligned(Ys[i], 4) ||
            !aligned(bases[i], 16) || !aligned(scales[i], 8))
            return fail(SX8_ERR_INVALID, "%s: misaligned pointer in matrix %d", what, i);
        const int32_t rc = check_shape(what, M, ldx, K, Ns[i], n_cb);
        if (rc != SX8_OK) return rc;
        w[i].hdr = hdrs[i];
        w[i].levels = levels[i];
    }
    return run_gemm<false>(what, X, M, ldx, K, n_mats, w, hdr_bytes, ZMode::kBasis, bases, scales, nullptr,
                           Ns, n_cb, Ys, workspace, workspace_bytes, as_stream(stream), nullptr, nullptr,
                           INT64_MAX, defer);
}

}  // namespace

extern "C" int32_t sx8_gemm_prefill_group(const uint16_t* X, int64_t M, int64_t ldx, int64_t K,
                                          int32_t n_mats, const uint8_t* const* hdrs,
                                          const uint8_t* const* levels, int32_t hdr_bytes,
                                          const float* const* bases, const float* const* scales,
                                          const int64_t* Ns, int64_t n_cb, float* const* Ys,
                                          void* workspace, int64_t workspace_bytes, void* stream) {
    return group_impl("sx8_gemm_prefill_group", X, M, ldx, K, n_mats, hdrs, levels, hdr_bytes, bases, scales,
                      Ns, n_cb, Ys, workspace, workspace_bytes, stream, nullptr);
}

extern "C" int32_t sx8_gemm_prefill_group_deferred(const uint16_t* X, int64_t M, int64_t ldx, int64_t K,
                                                   int32_t n_mats, const uint8_t* const* hdrs,
                                                   const uint8_t* const* levels, int32_t hdr_bytes,
                                                   const float* const* bases, const float* const* scales,
                                                   const int64_t* Ns, int64_t n_cb, float* const* Ys,
                                                   void* workspace, int64_t workspace_bytes, float** parts,
                                                   int32_t* n_parts, int64_t* slice, void* stream) {
    using namespace sx8;
    const char* what = "sx8_gemm_prefill_group_deferred";
    if (!parts || !n_parts || !slice) return fail(SX8_ERR_INVALID, "%s: null out-parameter", what);
    PendingSums pend{};
    const int32_t rc = group_impl(what, X, M, ldx, K, n_mats, hdrs, levels, hdr_bytes, bases, scales, Ns, n_cb,
                                  Ys, workspace, workspace_bytes, stream, &pend);
    if (rc != SX8_OK) return rc;
    return report_pending(what, pend, parts, n_parts, slice);
}

namespace {

// The MLP's gate/up GEMM ending in the down projection's packed operands.  Fused form: a
// plan of whole 512-row tiles over the paired tiling (ceil(N / 64) tiles of 64 gate + 64
// up columns) runs k_gemm_w2<kPair>, whose epilogue writes x = fp16(silu(g) u) and its Zhl;
// any other plan runs the gate/up group GEMM into float32 g, u in the workspace and the
// SiLU pack pass over them (the same bits: both go through sx8_silu_mul and the
// reference's Z tree).  Workspace: the fused form's Zhl of gate and up and packed X, or the
// group call's workspace followed by g and u.
struct GateUpPlan {
    bool fused;
    Plan p;              // fused: the paired plan; else the group plan
    int64_t gu_off;      // fallback: byte offset of g (u follows at + M N 4)
    int64_t total;
};

GateUpPlan gateup_plan(int64_t M, int64_t N, int64_t n_cb) {
    GateUpPlan gp{};
    const int64_t NBp = (N + kBN / 2 - 1) / (kBN / 2);
    const Plan pp = plan_gemm(M, 2 * N, NBp, n_cb);
    gp.fused = pp.w1 && pp.n_split == 0 && tuning().w2;
    if (gp.fused) {
        gp.p = pp;
        gp.total = ws_layout(pp, M, 2 * N, n_cb, 2, true).total;
    } else {
        const int64_t NBg = 2 * ((N + kBN - 1) / kBN);
        gp.p = plan_gemm(M, 2 * N, NBg, n_cb);
        gp.gu_off = ws_layout(gp.p, M, 2 * N, n_cb, 2, true).total;
        gp.total = gp.gu_off + ((2 * M * N * 4 + 255) & ~int64_t(255));
    }
    return gp;
}

}  // namespace

extern "C" int64_t sx8_dec_gemm_gateup_silu_workspace_bytes(int64_t M, int64_t N, int64_t n_cb) {
    if (M <= 0 || N <= 0 || n_cb <= 0 || M > 0x7FFFFFFF || N > 0x3FFFFFFF) return -1;
    return gateup_plan(M, N, n_cb).total;
}

extern "C" int32_t sx8_dec_gemm_gateup_silu(const uint16_t* X, const uint16_t* Xp_in, const uint32_t* const* Zhl_in,
                                            int64_t M, int64_t K, const uint8_t* const* hdrs,
                                            const uint8_t* const* levels, int32_t hdr_bytes,
                                            const float* const* bases, const float* const* scales, int64_t N,
                                            int64_t n_cb, const float* down_basis, const float* down_scales,
                                            uint16_t* Xp, uint32_t* Zhl, void* workspace,
                                            int64_t workspace_bytes, void* stream) {
    using namespace sx8;
    const char* what = "sx8_dec_gemm_gateup_silu";
    const bool packed_in = Xp_in != nullptr;
    if ((X != nullptr) == packed_in || (packed_in && (!Zhl_in || !Zhl_in[0] || !Zhl_in[1])))
        return fail(SX8_ERR_INVALID, "%s: give X, or Xp_in and both Zhl_in (not both forms)", what);
    if (!hdrs || !levels || !bases || !scales || !down_basis || !down_scales || !Xp || !Zhl)
        return fail(SX8_ERR_INVALID, "%s: null pointer", what);
    if (hdr_bytes != 6 && hdr_bytes != 8)
        return fail(SX8_ERR_INVALID, "%s: hdr_bytes must be 6 or 8, got %d", what, hdr_bytes);
    if ((X && !aligned(X, 2)) || (packed_in && (!aligned(Xp_in, 16) || !aligned(Zhl_in[0], 16) ||
                                                !aligned(Zhl_in[1], 16))) ||
        !aligned(down_basis, 16) || !aligned(down_scales, 8) || !aligned(Xp, 16) || !aligned(Zhl, 16))
        return fail(SX8_ERR_INVALID, "%s: misaligned X / Xp_in / Zhl_in, down basis / scales, Xp or Zhl", what);
    const int64_t n_cb_d = (N + 31) / 32;
    if (N > 0x3FFFFFFF || (M + 31) / 32 * n_cb_d * 2048 > 0x7FFFFFFF || M * n_cb_d * 8 > 0x7FFFFFFF)
        return fail(SX8_ERR_UNSUPPORTED, "%s: operands beyond 2 GiB", what);
    WeightSrc w[2]{};
    for (int i = 0; i < 2; ++i) {
        if (!hdrs[i] || !levels[i] || !bases[i] || !scales[i])
            return fail(SX8_ERR_INVALID, "%s: null pointer in matrix %d", what, i);
        if (!aligned(hdrs[i], hdr_bytes == 8 ? 8 : 2) || !aligned(levels[i], 8) || !aligned(bases[i], 16) ||
            !aligned(scales[i], 8))
            return fail(SX8_ERR_INVALID, "%s: misaligned pointer in matrix %d", what, i);
        w[i].hdr = hdrs[i];
        w[i].levels = levels[i];
    }
    int32_t rc = check_shape(what, M, K, K, N, n_cb);
    if (rc != SX8_OK) return rc;
    const GateUpPlan gp = gateup_plan(M, N, n_cb);
    if (!workspace || workspace_bytes < gp.total || !aligned(workspace, 256))
        return fail(SX8_ERR_INVALID,
                    "%s: needs a 256-byte aligned workspace of %lld bytes "
                    "(sx8_dec_gemm_gateup_silu_workspace_bytes), got %lld bytes at %p",
                    what, (long long)gp.total, (long long)workspace_bytes, workspace);
    hipStream_t st = as_stream(stream);
    uint8_t* ws = reinterpret_cast<uint8_t*>(workspace);
    ZSets zd{};                                  // the down projection's basis set
    zd.n = 1;
    zd.basis[0] = down_basis;
    zd.scales[0] = down_scales;
    zd.Z[0] = reinterpret_cast<float*>(Zhl);
    if (!gp.fused) {
        float* gu = reinterpret_cast<float*>(ws + gp.gu_off);
        float* Ys[2] = {gu, gu + M * N};
        const int64_t Ns[2] = {N, N};
        const PackedIn in{Xp_in, Zhl_in};
        rc = run_gemm<false>(what, X, M, K, K, 2, w, hdr_bytes, packed_in ? ZMode::kPacked : ZMode::kBasis, bases,
                             scales, nullptr, Ns, n_cb, Ys, workspace, gp.gu_off, st, nullptr, nullptr, INT64_MAX,
                             nullptr, packed_in ? &in : nullptr);
        if (rc != SX8_OK) return rc;
        rc = compute_z_silu(Ys[0], Ys[1], M, N, N, zd, n_cb_d, Xp, st);
        if (rc != SX8_OK) return rc;
        return check_launch(what);
    }
    // fused: one pass over X (packed X, Zhl of gate and up), then the paired GEMM
    const Plan& p = gp.p;
    if (p.G > 0x7FFFFFFF) return fail(SX8_ERR_UNSUPPORTED, "%s: grid too large", what);
    const WsLayout lay = ws_layout(p, M, 2 * N, n_cb, 2, true);
    const uint16_t* xp_in = packed_in ? Xp_in : reinterpret_cast<uint16_t*>(ws + lay.z_bytes * 2);
    ZSets zs{};
    zs.n = 2;
    GemmGroup g{};
    g.n_mats = 2;
    g.Ntot = 2 * N;
    g.NB = (int)((N + kBN / 2 - 1) / (kBN / 2));
    for (int i = 0; i < 2; ++i) {
        zs.basis[i] = bases[i];
        zs.scales[i] = scales[i];
        zs.Z[i] = reinterpret_cast<float*>(ws + lay.z_bytes * i);
        g.m[i].w = w[i];
        g.m[i].Zhl = packed_in ? Zhl_in[i] : reinterpret_cast<const uint32_t*>(ws + lay.z_bytes * i);
        g.m[i].N = (int)N;
        g.m[i].nb = g.NB;
    }
    if (!packed_in) {
        rc = compute_z_sets(X, M, K, K, zs, n_cb, true, reinterpret_cast<uint16_t*>(ws + lay.z_bytes * 2), st);
        if (rc != SX8_OK) return rc;
    }
    const SiluOut so{down_basis, down_scales, Xp, Zhl, (int)n_cb_d};
    if (hdr_bytes == 8)
        hipLaunchKernelGGL((k_gemm_w2<false, 8, true, true>), dim3((unsigned)p.G), dim3(kW2Threads), 0, st, xp_in,
                           (int)M, g, (int)n_cb, p.Tf, p.St, p.kbs, nullptr, so);
    else
        hipLaunchKernelGGL((k_gemm_w2<false, 6, true, true>), dim3((unsigned)p.G), dim3(kW2Threads), 0, st, xp_in,
                           (int)M, g, (int)n_cb, p.Tf, p.St, p.kbs, nullptr, so);
    return check_launch(what);
}

extern "C" int64_t sx8_gemm_prefill_packed_workspace_bytes(int64_t M, int32_t n_mats, const int64_t* Ns,
                                                           int64_t n_cb) {
    if (M <= 0 || n_cb <= 0 || !Ns || n_mats < 1 || n_mats > kMaxGemmGroup || M > 0x7FFFFFFF) return -1;
    for (int i = 0; i < n_mats; ++i)
        if (Ns[i] <= 0) return -1;
    int64_t Ntot = 0, NB = 0;
    if (!group_width(n_mats, Ns, Ntot, NB)) return -1;
    const Plan p = plan_gemm(M, Ntot, NB, n_cb);
    return ws_layout(p, M, Ntot, n_cb, n_mats, true, false).total;
}

extern "C" int32_t sx8_gemm_prefill_packed(const uint16_t* Xp, const uint32_t* const* Zhl, int64_t M, int64_t K,
                                           int32_t n_mats, const uint8_t* const* hdrs,
                                           const uint8_t* const* levels, int32_t hdr_bytes, const int64_t* Ns,
                                           int64_t n_cb, float* const* Ys, void* workspace,
                                           int64_t workspace_bytes, float** parts, int32_t* n_parts,
                                           int64_t* slice, void* stream) {
    using namespace sx8;
    const char* what = "sx8_gemm_prefill_packed";
    if (!Xp || !Zhl || !hdrs || !levels || !Ns || !Ys) return fail(SX8_ERR_INVALID, "%s: null pointer", what);
    const int n_out = (parts != nullptr) + (n_parts != nullptr) + (slice != nullptr);
    if (n_out != 0 && n_out != 3)
        return fail(SX8_ERR_INVALID, "%s: give all three of parts, n_parts, slice or none", what);
    if (n_mats < 1 || n_mats > kMaxGemmGroup)
        return fail(SX8_ERR_INVALID, "%s: n_mats must be 1..%d, got %d", what, kMaxGemmGroup, n_mats);
    if (hdr_bytes != 6 && hdr_bytes != 8)
        return fail(SX8_ERR_INVALID, "%s: hdr_bytes must be 6 or 8, got %d", what, hdr_bytes);
    if (!aligned(Xp, 16)) return fail(SX8_ERR_INVALID, "%s: Xp must be 16-byte aligned", what);
    WeightSrc w[kMaxGemmGroup]{};
    for (int i = 0; i < n_mats; ++i) {
        if (!hdrs[i] || !levels[i] || !Zhl[i] || !Ys[i])
            return fail(SX8_ERR_INVALID, "%s: null pointer in matrix %d", what, i);
        if (!aligned(hdrs[i], hdr_bytes == 8 ? 8 : 2) || !aligned(levels[i], 8) || !aligned(Ys[i], 4) ||
            !aligned(Zhl[i], 16))
            return fail(SX8_ERR_INVALID, "%s: misaligned pointer in matrix %d", what, i);
        const int32_t rc = check_shape(what, M, K, K, Ns[i], n_cb);
        if (rc != SX8_OK) return rc;
        w[i].hdr = hdrs[i];
        w[i].levels = levels[i];
    }
    const PackedIn in{Xp, Zhl};
    PendingSums pend{};
    const int32_t rc = run_gemm<false>(what, nullptr, M, K, K, n_mats, w, hdr_bytes, ZMode::kPacked, nullptr,
                                       nullptr, nullptr, Ns, n_cb, Ys, workspace, workspace_bytes,
                                       as_stream(stream), nullptr, nullptr, INT64_MAX, n_out ? &pend : nullptr,
                                       &in);
    if (rc != SX8_OK || !n_out) return rc;
    return report_pending(what, pend, parts, n_parts, slice);
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
