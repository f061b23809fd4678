/*
 * sx8_hip.h -- C ABI of libsx8_hip.so, the MI355X (gfx950) implementation of the
 * S-X8 v4.3 weight-dequantization hot path.
 *
 * Conventions
 *   - Every pointer is a device pointer on the current HIP device unless stated.
 *   - fp16 tensors are passed as uint16_t bit patterns; no HIP or torch types appear
 *     in the signatures except the stream, passed as an opaque void* (a hipStream_t;
 *     NULL means the legacy default stream).
 *   - Every entry point enqueues work on `stream`, never synchronises the device, never
 *     allocates device memory, and returns SX8_OK or an error code; sx8_last_error() then
 *     holds a message.  Scratch memory comes from the caller (`workspace`, sized by the
 *     matching *_workspace_bytes query), so every call can be captured into a HIP graph
 *     and calls on different streams never share scratch.
 *   - Argument checks (null pointers, sizes, hdr_bytes, alignment) happen on the
 *     host before any launch, so an invalid call never reaches the GPU.
 *
 * Block layouts (reference paths are relative to the reference repository):
 *   split arrays, pkl/container order ("n-major", bid = n*n_cb + kb):
 *       dmin/dmax fp16 (n_blk), config u8 (n_blk), coeff u8 (n_blk),
 *       levels_hi u8 (n_blk*16), levels_lo u8 (n_blk*8)
 *       -- scripts/sx8_container_v43.py:30-35, scripts/kernel_sx8_v43.py:14-51
 *   v4.4 kb-major (bid = kb*N + n): hdr u8 (n_blk, hdr_bytes in {6,8}) =
 *       dmin|dmax|config|coeff(|pad), levels u8 (n_blk, 24) = qh[16]|ql[8]
 *       -- scripts/prepare_v44.py:35-79
 *   kb-major split arrays (the fused-WMMA form, scripts/integrate_fused.py:46-58):
 *       the split arrays above re-ordered to bid = kb*N + n.
 *   PCA side tables: basis f32 (n_cb, 64) = [b0 | b1], scales f32 (n_cb, 2).
 */
#ifndef SX8_HIP_H
#define SX8_HIP_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* 3: sx8_dec_gemv_rmsnorm_pair takes the up matrix's pointers; sx8_gemm_reload_tuning.
 * 4: deferred split-K sums: sx8_gemm_prefill_group_deferred, sx8_dec_gemm_silu_deferred and
 *    the consumers sx8_dec_add_rmsnorm_parts, sx8_dec_qk_rope_cache_rows_parts
 * 5: producer-written GEMM operands: sx8_gemm_prefill_packed(_workspace_bytes),
 *    sx8_dec_attn_prefill_packed, sx8_dec_gemm_gateup_silu(_workspace_bytes) */
#define SX8_ABI_VERSION 5

#define SX8_OK 0
#define SX8_ERR_INVALID 1      /* bad argument (null pointer, size, hdr_bytes, alignment) */
#define SX8_ERR_HIP 2          /* HIP runtime error (launch or allocation) */
#define SX8_ERR_UNSUPPORTED 3  /* shape outside what the kernels support */

/* ABI version of the loaded library (SX8_ABI_VERSION at build time). */
int32_t sx8_abi_version(void);

/* Message for the last error returned on the calling thread ("" if none). */
const char* sx8_last_error(void);

/* Canonical R64 dequant to fp16, split arrays in pkl order.
 * Replaces kernel_sx8_v43.decode_tensor_gpu_fast (scripts/kernel_sx8_v43.py:109-145)
 * and its numba kernel sx8_v43_kernel (:14-51).  out is (out_f, in_f) row-major fp16;
 * columns in_f .. n_cb*32-1 of the padded block grid are dropped.  Bit-exact. */
int32_t sx8_dequant_f16(const uint16_t* dmin, const uint16_t* dmax, const uint8_t* config,
                        const uint8_t* coeff, const uint8_t* levels_hi,
                        const uint8_t* levels_lo, const float* basis, const float* scales,
                        int64_t out_f, int64_t in_f, int64_t n_cb, uint16_t* out,
                        void* stream);

/* R64 dequant of selected rows from the v4.4 kb-major layout:
 *   out[t, :] = W16[ids[t], :]  for t < T (ids int64; ids outside [0, N) leave row t
 *   unwritten).  ids == NULL means ids[t] = t with T = N (whole-tensor dequant).
 * Replaces sx8_embed_v44 (cuda/sx8_embed_v44.cu:80-94, kernel :21-78), which computed
 * the rows in float32; this one is bit-exact to the canonical dequant.
 * out is (T, K) row-major fp16. */
int32_t sx8_embed_gather(const int64_t* ids, int64_t T, const uint8_t* hdr,
                         const uint8_t* levels, int32_t hdr_bytes, const float* basis,
                         const float* scales, int64_t K, int64_t N, int64_t n_cb,
                         uint16_t* out, void* stream);

/* Load-time layout transform: S-X8 v4.3 split arrays in pkl / .sx8v43 container order
 * (n-major, bid' = n*n_cb + kb: dmin/dmax fp16 as bytes, config, coeff, levels_hi
 * (16 B per block), levels_lo (8 B per block); no alignment required) -> the v4.4
 * kb-major device records (bid = kb*N + n): hdr (n_blk, hdr_bytes) = dmin | dmax | config
 * | coeff (| 2 zero bytes) and levels (n_blk, 24) = levels_hi | levels_lo.  Byte-identical
 * to the reference's to_v44 (scripts/prepare_v44.py:35-79), which it replaces on the
 * device side of a container load. */
int32_t sx8_v43_to_v44(const uint8_t* dmin, const uint8_t* dmax, const uint8_t* config,
                       const uint8_t* coeff, const uint8_t* levels_hi, const uint8_t* levels_lo,
                       int64_t out_f, int64_t n_cb, int32_t hdr_bytes, uint8_t* hdr,
                       uint8_t* levels, void* stream);

/* Same transform from GGUF block_sx8 records: `blocks` is (out_f * n_cb) interleaved 30-byte
 * records dmin | dmax | config | qh[16] | ql[8] | coeff in n-major order, the tensor data of
 * a GGUF SX8 tensor (llama-cpp-sx8.patch:131-144; converter blockify_vec,
 * scripts/convert_pkl_to_gguf_sx8.py:21-38).  No alignment required. */
int32_t sx8_blocks_to_v44(const uint8_t* blocks, int64_t out_f, int64_t n_cb, int32_t hdr_bytes,
                          uint8_t* hdr, uint8_t* levels, void* stream);

/* llama.cpp's no-PCA float32 dequant of block_sx8 records ("R32-ggml", dequantize_row_sx8,
 * llama-cpp-sx8.patch:746-767): out (out_f, in_f) float32 row-major, the coeff byte
 * ignored.  contract != 0 evaluates rlo, rhi and rlo + step*lv as fused multiply-adds (a
 * C build that contracts them); contract == 0 rounds every operation separately.  For
 * comparing this engine with the reference's llama.cpp fork on the same GGUF file. */
int32_t sx8_dequant_ggml_f32(const uint8_t* blocks, int64_t out_f, int64_t in_f, int64_t n_cb,
                             int32_t contract, float* out, void* stream);

/* V6 encode + level packing of a (out_f, in_f) fp16 weight (row pitch ld elements), the
 * deterministic half of the quantizer (scripts/quantize_qwen35_4b_sx8_v43_gpu.py:22-47
 * v6_encode_6bit_gpu, :148-167 pack_levels_6bit): per 32-weight block (columns past in_f
 * count as zero) dmin/dmax (fp16), config, levels_hi (16 B), levels_lo (8 B), in the
 * pkl / container n-major order; `levels` (optional, 32 B per block) receives the unpacked
 * 6-bit levels for the PCA step.  Binary32 arithmetic with every operation rounded, MSE
 * summed left to right, first strictly-lowest candidate wins. */
int32_t sx8_v6_encode(const uint16_t* W, int64_t out_f, int64_t in_f, int64_t ld, uint8_t* levels,
                      uint16_t* dmin, uint16_t* dmax, uint8_t* config, uint8_t* levels_hi,
                      uint8_t* levels_lo, void* stream);

/* PCA precompute Z[m, kb, j] = scales[kb, j] * sum_t X[m, kb*32+t] * basis[kb, 32j+t]
 * for m < M, in float32 with the reference's summation tree.
 * Replaces compute_z44 (cuda/sx8_decode1_v3.cu:185-195, kernel :44-65) for M = 1 and
 * compute_z44_batch (cuda/sx8_gemm_compact.cu:157-169, kernel :28-50) for M > 1.
 * X is (M, ldx) fp16 with ldx >= n_cb*32.  Z is (M, n_cb, 2) float32 (8-byte aligned);
 * basis 16-byte aligned.  M * n_cb below 2^31 (SX8_ERR_UNSUPPORTED otherwise). */
int32_t sx8_compute_z(const uint16_t* X, int64_t M, int64_t ldx, const float* basis,
                      const float* scales, int64_t n_cb, float* Z, void* stream);

/* M = 1 decode GEMV on the v4.4 layout: Y[n] = sum_k X[k] W[n, k], float32 result.
 * If Z_in != NULL it is used as the PCA precompute (n_cb, 2) (the two-launch form,
 * decode1_v44 at cuda/sx8_decode1_v3.cu:197-221); otherwise Z is computed from
 * basis/scales with the reference's summation tree and, when Z_out != NULL, also written
 * there (the combined form, decode1_v44_combined at :223-246).  X holds n_cb*32 fp16
 * values (16-byte aligned).  `workspace` (>= sx8_gemv_workspace_bytes(n_cb) bytes, 16-byte
 * aligned) receives the activation table of the two-launch forms (Z_out != NULL, or
 * n_cb > 640); the single-launch form builds it in LDS and takes workspace = NULL.  A call
 * that needs the workspace and gets NULL returns SX8_ERR_INVALID.
 * Tolerance against the float64 yardstick: max|dY| / max|Y| <= 1e-3. */
int32_t sx8_gemv(const uint16_t* X, const uint8_t* hdr, const uint8_t* levels,
                 int32_t hdr_bytes, const float* basis, const float* scales,
                 const float* Z_in, float* Z_out, int64_t N, int64_t n_cb, float* Y,
                 void* workspace, int64_t workspace_bytes, void* stream);

/* GEMVs of n_mats (1..4) v4.4 weights that share X (same K, same hdr_bytes), e.g. the
 * q/k/v or gate/up projections of a decoder layer, as one launch: Ys[i] (Ns[i],) float32 =
 * W_i . X.  Per matrix either Z_in[i] (Z_in non-NULL) or bases[i] + scales[i]; arrays are
 * host arrays of n_mats device pointers.  Each output is what sx8_gemv gives for that
 * matrix (same decode, same tolerance); one dispatch instead of n_mats, which is most of
 * an M = 1 GEMV's fixed cost.  n_cb > 640 runs one two-launch GEMV per matrix and then
 * needs `workspace` (sx8_gemv_workspace_bytes(n_cb) bytes); otherwise NULL.  No
 * counterpart in the reference, whose decode path runs one decode1_v44 per projection
 * (cuda/sx8_decode1_v3.cu:197-246). */
int32_t sx8_gemv_group(const uint16_t* X, int32_t n_mats, const uint8_t* const* hdrs,
                       const uint8_t* const* levels, int32_t hdr_bytes,
                       const float* const* bases, const float* const* scales,
                       const float* const* Z_in, const int64_t* Ns, int64_t n_cb,
                       float* const* Ys, void* workspace, int64_t workspace_bytes, void* stream);

/* Workspace bytes sx8_gemv needs for n_cb K blocks (112 per block). */
int64_t sx8_gemv_workspace_bytes(int64_t n_cb);

/* Workspace bytes of a prefill call over n_mats (1..4) matrices of Ns[i] output columns
 * that share an (M, K) X with n_cb = ceil(K / 32): the PCA operand of every matrix, the
 * packed copy of X and the split-K partials of the plan the call will run.  The same value
 * serves sx8_gemm_prefill, _split, _z, _core (n_mats = 1) and _group; sx8_dec_gemm_silu
 * (K = its inner size).  -1 for an invalid shape.  The plan depends only on (M, sum Ns,
 * the group's column tiles, n_cb) and on the tuning variables SX8_GEMM_TILE, SX8_GEMM_PLAN
 * and SX8_GEMM_W2 as the library last read them (see sx8_gemm_reload_tuning), so a size
 * returned here stays valid for later calls with the same sizes.  No counterpart in the
 * reference, whose wrappers allocate outputs and Z with torch inside each call
 * (cuda/sx8_gemm_compact.cu:157-194). */
int64_t sx8_gemm_prefill_workspace_bytes(int64_t M, int32_t n_mats, const int64_t* Ns, int64_t n_cb);

/* Prefill tuning variables (for tuning runs and tests; a default run sets none):
 * SX8_GEMM_TILE=256|512 forces the tile height, SX8_GEMM_PLAN=k<1|2>:<S> (128- or 256-row
 * tiles in S K ranges) or w<0|1>:<St> (512-row tiles; 1: whole rounds of 256 tiles first,
 * St K ranges for the rest) forces one plan when it is valid for the shape, SX8_GEMM_W2=0
 * runs 512-row plans on the one-wave-per-SIMD kernel.  The library reads them once, at the
 * first prefill call or query; this call reads them again.  Not to be called while prefill
 * calls or queries run on other threads.  No counterpart in the reference. */
int32_t sx8_gemm_reload_tuning(void);

/* The plan a prefill call with these sizes runs (for logs and tests): desc[0] tile rows
 * (128, 256 or 512), desc[1] work-groups, desc[2] K ranges, desc[3] K blocks per range,
 * desc[4] whole 512-row tiles before the split tail, desc[5] tiles of the split tail,
 * desc[6] workspace bytes, desc[7] 0.  No counterpart in the reference. */
int32_t sx8_gemm_prefill_plan(int64_t M, int32_t n_mats, const int64_t* Ns, int64_t n_cb,
                              int64_t* desc);

/* Prefill GEMM Y (M, N) float32 = X (M, ldx) fp16 . W^T on the v4.4 layout.
 * The PCA-free core weights rlo + step*lv are decoded with the reference's float32
 * range parameters (cuda/sx8_fused_wmma.cu:70-94), the multiply-add rounded once to fp16,
 * and fed to v_mfma_f32_32x32x16_f16 with float32 accumulation; the PCA term
 * sum_kb c0 Z0 + c1 Z1 is
 * added by extra MFMA k-steps over Z (split into fp16 hi + lo parts), which the call
 * computes first with the reference's summation tree.  The MFMA operands are therefore
 * not the canonical R64 fp16 weights (those come from sx8_dequant_f16); the product is
 * within the tolerance below.  `workspace` (256-byte aligned, >= sx8_gemm_prefill_
 * workspace_bytes(M, 1, &N, n_cb) bytes) holds Z, the packed X and any split-K partials;
 * calls that overlap in time need distinct workspaces.  Columns k >= K of X are never
 * read.  Tolerance against the float64 yardstick: max|dY| / max|Y| <= 1e-3.
 * Replaces gemm_compact (cuda/sx8_gemm_compact.cu:171-194, kernel :55-152) together
 * with its Z precompute compute_z44_batch (:157-169). */
int32_t sx8_gemm_prefill(const uint16_t* X, int64_t M, int64_t ldx, int64_t K,
                         const uint8_t* hdr, const uint8_t* levels, int32_t hdr_bytes,
                         const float* basis, const float* scales, int64_t N, int64_t n_cb,
                         float* Y, void* workspace, int64_t workspace_bytes, void* stream);

/* sx8_gemm_prefill without a workspace argument, for callers that cannot allocate (code
 * under HIP graph capture, tight serving loops, harnesses that forbid hipMalloc).  No
 * counterpart in the reference.  The call's scratch (Z, packed X, split-K partials) is a
 * 64 MiB device array inside the library (one per device, held until the process ends);
 * the call allocates, frees and synchronizes nothing.  Z plus the packed X must fit it,
 * about 72 * M * n_cb bytes (M <= 3000 at K = 9728, M <= 11000 at K = 2560); a larger call
 * returns SX8_ERR_UNSUPPORTED, and a split-K plan is used only if its partials fit the rest
 * (otherwise an unsplit plan, same result up to the fp32 summation order).  All calls on a
 * device share the array: calls that overlap in time on one device race (serialize them,
 * e.g. on one stream).  Same output as sx8_gemm_prefill whenever both run the same plan. */
int32_t sx8_gemm_prefill_static(const uint16_t* X, int64_t M, int64_t ldx, int64_t K,
                                const uint8_t* hdr, const uint8_t* levels, int32_t hdr_bytes,
                                const float* basis, const float* scales, int64_t N, int64_t n_cb,
                                float* Y, void* stream);

/* Same GEMM from kb-major split arrays (dmin/dmax fp16, config, coeff, hi (n_blk*16),
 * lo (n_blk*8), all in bid = kb*N + n order).  Same workspace as sx8_gemm_prefill.
 * Replaces fused_forward (cuda/sx8_fused_wmma.cu:134-154, kernel :11-132). */
int32_t sx8_gemm_prefill_split(const uint16_t* X, int64_t M, int64_t ldx, int64_t K,
                               const uint16_t* dmin, const uint16_t* dmax,
                               const uint8_t* config, const uint8_t* coeff,
                               const uint8_t* hi, const uint8_t* lo, const float* basis,
                               const float* scales, int64_t N, int64_t n_cb, float* Y,
                               void* workspace, int64_t workspace_bytes, void* stream);

/* Same GEMM with the PCA precompute supplied by the caller: Z (M, n_cb, 2) float32 as
 * written by sx8_compute_z.  Three launches: Z converted to the fp16 hi/lo operand and X
 * packed (both into `workspace`, sized as for sx8_gemm_prefill), the GEMM, and for a
 * split-K plan the fixed-order sum of the partials.
 * Replaces gemm_compact(X, hdr, levels, Z, n_cb, hdr_bytes) (cuda/sx8_gemm_compact.cu:
 * 171-194, kernel :55-152). */
int32_t sx8_gemm_prefill_z(const uint16_t* X, int64_t M, int64_t ldx, int64_t K,
                           const uint8_t* hdr, const uint8_t* levels, int32_t hdr_bytes,
                           const float* Z, int64_t N, int64_t n_cb, float* Y,
                           void* workspace, int64_t workspace_bytes, void* stream);

/* Prefill GEMMs of n_mats (1..4) v4.4 weights that share X (same K, same hdr_bytes), e.g.
 * the q/k/v or gate/up projections of a prompt: Ys[i] (M, Ns[i]) float32 = X . W_i^T + PCA,
 * each what sx8_gemm_prefill gives for that matrix up to the split-K summation order.
 * Host arrays of n_mats device pointers; workspace sized by
 * sx8_gemm_prefill_workspace_bytes(M, n_mats, Ns, n_cb).  One pass over X packs it for all
 * matrices and one launch covers the column tiles of the whole group.  No counterpart in
 * the reference, whose runtime calls gemm_sx8_compact once per projection
 * (scripts/sx8_gemm_compact.py:42-74). */
int32_t sx8_gemm_prefill_group(const uint16_t* X, int64_t M, int64_t ldx, int64_t K, int32_t n_mats,
                               const uint8_t* const* hdrs, const uint8_t* const* levels,
                               int32_t hdr_bytes, const float* const* bases,
                               const float* const* scales, const int64_t* Ns, int64_t n_cb,
                               float* const* Ys, void* workspace, int64_t workspace_bytes,
                               void* stream);

/* sx8_gemm_prefill_group with its split-K sum left to the caller.  When the plan splits K
 * into S ranges on 128- or 256-row tiles, Ys[i] receive the first range's products only and
 * the other S - 1 ranges' partial products stay in the workspace: *n_parts = S - 1, *parts =
 * the first partial slice (a device pointer into the workspace), *slice = floats per slice
 * (M * sum N_i); matrix i's (M, N_i) block of slice s starts at parts + s * slice +
 * M * (N_0 + .. + N_{i-1}).  Ys[i] + slice 0 + .. + slice S-2, added in that order, is what
 * sx8_gemm_prefill_group writes, bit for bit (sx8_dec_add_rmsnorm_parts and
 * sx8_dec_qk_rope_cache_rows_parts add them where they read Y).  Any other plan sums as
 * usual and reports *n_parts = 0.  The slices live until the workspace is used again.  No
 * counterpart in the reference (its prefill GEMM does not split K). */
int32_t sx8_gemm_prefill_group_deferred(const uint16_t* X, int64_t M, int64_t ldx, int64_t K,
                                        int32_t n_mats, const uint8_t* const* hdrs,
                                        const uint8_t* const* levels, int32_t hdr_bytes,
                                        const float* const* bases, const float* const* scales,
                                        const int64_t* Ns, int64_t n_cb, float* const* Ys,
                                        void* workspace, int64_t workspace_bytes, float** parts,
                                        int32_t* n_parts, int64_t* slice, void* stream);

/* sx8_gemm_prefill_group on operands a producer kernel already wrote, so the call runs no
 * pass over X (it launches the GEMM and, for a split plan, the partial sums only):
 *   Xp  -- the packed X of the M rows: for each 32-row group G (rows past M zero) and K
 *          block kb a 2 KB chunk at byte (G * n_cb + kb) * 2048, laid out [k-step st 0..1]
 *          [lane l = 32 hf + r, hf 0..1, r 0..31][8 fp16] holding X[32 G + r][32 kb + 16 hf
 *          + 8 st .. + 8]; ceil(M / 32) * n_cb * 2048 bytes, 16-byte aligned;
 *   Zhl[i] -- matrix i's PCA operand, (M, n_cb) entries of 8 bytes: Z0, Z1 of the row's K
 *          block (scale_j * sum_t x_t basis_j[t], the reference's tree order) each as fp16
 *          (hi, lo) with hi = fp16(z), lo = fp16(z - hi); M * n_cb * 8 bytes, 16-byte aligned.
 * sx8_dec_attn_prefill_packed writes both for the attention output.  The workspace holds
 * only the split-K partials (sx8_gemm_prefill_packed_workspace_bytes; NULL when that is 0).
 * parts / n_parts / slice: all NULL -- the call adds its split-K partials itself; all given
 * -- the partial slices are left to the caller as in sx8_gemm_prefill_group_deferred.  Same
 * outputs, bit for bit, as sx8_gemm_prefill_group on the X those operands came from.  No
 * counterpart in the reference (its prefill GEMM reads X as given). */
int32_t sx8_gemm_prefill_packed(const uint16_t* Xp, const uint32_t* const* Zhl, int64_t M, int64_t K,
                                int32_t n_mats, const uint8_t* const* hdrs, const uint8_t* const* levels,
                                int32_t hdr_bytes, const int64_t* Ns, int64_t n_cb, float* const* Ys,
                                void* workspace, int64_t workspace_bytes, float** parts, int32_t* n_parts,
                                int64_t* slice, void* stream);

/* Workspace bytes of sx8_gemm_prefill_packed (the plan's split-K partials; 0 when the plan
 * does not split K), or -1 for bad arguments. */
int64_t sx8_gemm_prefill_packed_workspace_bytes(int64_t M, int32_t n_mats, const int64_t* Ns, int64_t n_cb);

/* Output-side PCA: Y[m, n] += sum_kb c0(kb,n) Z[m,kb,0] + c1(kb,n) Z[m,kb,1], c0/c1 the
 * signed nibbles of the coeff byte in the v4.4 header (float32 FMAs, one thread per
 * column).  The PCA step of gemm_compact's epilogue (cuda/sx8_gemm_compact.cu:130-150)
 * as a separate pass, for callers that hold a core-only result. */
int32_t sx8_gemm_pca_z(const float* Z, int64_t M, const uint8_t* hdr, int32_t hdr_bytes,
                       int64_t N, int64_t n_cb, float* Y, void* stream);

/* Prefill GEMM of the PCA-free core weights only (rlo + step*lv); with sx8_gemm_pca_z it
 * gives the same product as sx8_gemm_prefill_z in two passes.  With X = the identity
 * (M = K = n_cb*32 rows of unit vectors) Y[k, n] is exactly the fp16 MFMA operand of weight
 * (n, k), which pins the operand decode bit for bit.  Workspace as for sx8_gemm_prefill. */
int32_t sx8_gemm_prefill_core(const uint16_t* X, int64_t M, int64_t ldx, int64_t K,
                              const uint8_t* hdr, const uint8_t* levels, int32_t hdr_bytes,
                              int64_t N, int64_t n_cb, float* Y, void* workspace,
                              int64_t workspace_bytes, void* stream);

#ifdef __cplusplus
}
#endif

#endif /* SX8_HIP_H */
