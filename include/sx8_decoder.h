/* sx8_decoder.h -- per-token ops of the end-to-end S-X8 decoder (libsx8_hip.so).
 *
 * These sit between the S-X8 GEMVs of sx8_hip.h in one decode step.  They replace the
 * Hugging Face Qwen module ops (RMSNorm, rotary embedding, SDPA over the KV cache, SiLU,
 * greedy argmax) that the reference's runtime runs around its S-X8 linears
 * (scripts/infer_sx8.py:109-173).  Every entry point reads the decode position from
 * device memory, so one step can be captured in a HIP graph and replayed.  Conventions as
 * in sx8_hip.h: device pointers, fp16 as uint16_t bits, int32_t status, stream as void*.
 */
#ifndef SX8_DECODER_H
#define SX8_DECODER_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* For each of M rows of H: resid = (init ? fp16 init : resid) + (delta ? delta : 0) in
 * float32 (the updated residual stream is written back), then out = fp16(resid *
 * rsqrt(mean(resid^2) + eps) * w).  delta and init may be NULL. */
int32_t sx8_dec_add_rmsnorm(float* resid, const float* delta, const uint16_t* init,
                            const uint16_t* w, uint16_t* out, int64_t M, int64_t H, float eps,
                            void* stream);

/* sx8_dec_add_rmsnorm where delta is a deferred split-K GEMM output (the *_deferred prefill
 * calls): each delta element is first summed with its n_parts (0..7) partial slices at
 * parts + s * slice, in slice order, the sum the GEMM would have written.  delta must be
 * given when n_parts > 0; parts 4-byte aligned, slice >= M * H. */
int32_t sx8_dec_add_rmsnorm_parts(float* resid, const float* delta, const uint16_t* init,
                                  const uint16_t* w, uint16_t* out, int64_t M, int64_t H, float eps,
                                  const float* parts, int32_t n_parts, int64_t slice, void* stream);

/* sx8_dec_add_rmsnorm_parts (the same h into resid, the same x, bit for bit) writing x not as
 * fp16 rows but as the prefill-GEMM operands of the n_mats (1..4) matrices that multiply
 * it (sx8_gemm_prefill_packed): Xp, the packed X (ceil(M / 32) * (H / 32) * 2048 bytes; rows
 * past M pack zeros), and Zhl[i], matrix i's PCA operand for its basis (H / 32, 2, 32) and
 * scales (M * (H / 32) * 8 bytes) -- what the GEMM's own pass over x writes, without that
 * launch.  H a multiple of 32, at most 4096; resid, delta, parts and Xp 16-byte aligned,
 * init and w 8-byte, bases 16-byte, scales and Zhl 8-byte.  No reference counterpart. */
int32_t sx8_dec_add_rmsnorm_packed(float* resid, const float* delta, const uint16_t* init, const uint16_t* w,
                                   int64_t M, int64_t H, float eps, const float* parts, int32_t n_parts,
                                   int64_t slice, int32_t n_mats, const float* const* bases,
                                   const float* const* scales, uint16_t* Xp, uint32_t* const* Zhl, void* stream);

/* One token at position *pos: per query/key head RMSNorm (q_norm/k_norm weights, over hd),
 * fp16 rounding, rotate-half RoPE with cos_t/sin_t rows (L, hd/2) float32; q into q_out
 * (nh*hd fp16), k and v into row *pos of k_cache / v_cache ((nk, L, hd) fp16 each).  A
 * position outside [0, L) writes nothing.  hd even and <= 256. */
int32_t sx8_dec_qk_rope_cache(const float* q_raw, const float* k_raw, const float* v_raw,
                              const uint16_t* q_norm, const uint16_t* k_norm, const float* cos_t,
                              const float* sin_t, const int64_t* pos, uint16_t* q_out,
                              uint16_t* k_cache, uint16_t* v_cache, int32_t nh, int32_t nk,
                              int32_t hd, int64_t L, float eps, void* stream);

/* The same for `rows` consecutive tokens at positions *pos .. *pos + rows - 1 (a prompt):
 * q_raw (rows, nh*hd), k_raw / v_raw (rows, nk*hd) float32, q_out (rows, nh*hd) fp16;
 * token y is what sx8_dec_qk_rope_cache computes at position *pos + y.  No reference
 * counterpart (the Hugging Face attention module's prompt pass, scripts/infer_sx8.py). */
int32_t sx8_dec_qk_rope_cache_rows(const float* q_raw, const float* k_raw, const float* v_raw,
                                   const uint16_t* q_norm, const uint16_t* k_norm,
                                   const float* cos_t, const float* sin_t, const int64_t* pos,
                                   int64_t rows, uint16_t* q_out, uint16_t* k_cache,
                                   uint16_t* v_cache, int32_t nh, int32_t nk, int32_t hd,
                                   int64_t L, float eps, void* stream);

/* sx8_dec_qk_rope_cache_rows on the deferred output of the q/k/v group GEMM
 * (sx8_gemm_prefill_group_deferred with matrices q, k, v and M = rows): every value read is
 * summed with its n_parts (0..7) partial slices first, in slice order (q's block of slice s
 * at parts + s * slice, k's at + rows*nh*hd, v's at + rows*(nh+nk)*hd).  parts 4-byte
 * aligned, slice >= rows * (nh + 2 nk) * hd. */
int32_t sx8_dec_qk_rope_cache_rows_parts(const float* q_raw, const float* k_raw, const float* v_raw,
                                         const uint16_t* q_norm, const uint16_t* k_norm,
                                         const float* cos_t, const float* sin_t, const int64_t* pos,
                                         int64_t rows, uint16_t* q_out, uint16_t* k_cache,
                                         uint16_t* v_cache, int32_t nh, int32_t nk, int32_t hd,
                                         int64_t L, float eps, const float* parts, int32_t n_parts,
                                         int64_t slice, void* stream);

/* Decode attention of one token: for each of nh query heads (kv head = h / (nh/nk)),
 * softmax(scale * q . K[0..*pos]) . V[0..*pos] over the caches written by
 * sx8_dec_qk_rope_cache; out (nh*hd) fp16.  hd 64 or 128, L <= 4096, q and caches
 * 16-byte aligned. */
int32_t sx8_dec_attn(const uint16_t* q, const uint16_t* k_cache, const uint16_t* v_cache,
                     const int64_t* pos, uint16_t* out, int32_t nh, int32_t nk, int32_t hd,
                     int64_t L, float scale, void* stream);

/* The same attention split over cache positions: two launches, n_kv x 16 work-groups each
 * taking one KV head's share of positions for all nh/nk query heads that share it (nh/nk
 * in {1, 2, 4, 8}), then a combine of the per-chunk partial softmax sums in fixed order.
 * `workspace` (16-byte aligned, >= sx8_dec_attn_workspace_bytes(nh, hd)) holds the
 * partials; it needs no clearing.  Each work-group streams its positions once with an
 * online softmax, so the cache length is limited only to 2^20.  Same result as
 * sx8_dec_attn up to float32 summation order. */
int32_t sx8_dec_attn_split(const uint16_t* q, const uint16_t* k_cache, const uint16_t* v_cache,
                           const int64_t* pos, uint16_t* out, int32_t nh, int32_t nk, int32_t hd,
                           int64_t L, float scale, void* workspace, int64_t workspace_bytes,
                           void* stream);

/* sx8_dec_qk_rope_cache followed by sx8_dec_attn_split in one pass over the cache: the
 * q/k RMSNorm + RoPE of the raw f32 projections are computed inside the attention
 * work-groups, and the work-group whose chunk holds *pos writes that position's k and v
 * into the caches and uses them from registers.  Same arguments as the two calls (cos_t,
 * sin_t: (L, hd / 2) tables), out (nh*hd) fp16; equal to the two-call form up to the
 * summation order of the RMSNorm sums.  Positions outside [0, L) write nothing.  No
 * reference counterpart (the Hugging Face attention module of scripts/infer_sx8.py). */
int32_t sx8_dec_attn_rope(const float* q_raw, const float* k_raw, const float* v_raw,
                          const uint16_t* q_norm, const uint16_t* k_norm, const float* cos_t,
                          const float* sin_t, const int64_t* pos, uint16_t* k_cache,
                          uint16_t* v_cache, uint16_t* out, int32_t nh, int32_t nk, int32_t hd,
                          int64_t L, float scale, float eps, void* workspace,
                          int64_t workspace_bytes, void* stream);

/* sx8_dec_silu_mul followed by sx8_gemm_prefill, without the intermediate: the prefill
 * GEMM's pass that packs X and computes Z reads g and u (M x K float32, row stride K)
 * and forms x = fp16(silu(g) * u) itself.  Y (M, N) float32 as sx8_gemm_prefill gives it
 * for that x; workspace as sx8_gemm_prefill_workspace_bytes(M, 1, &N, n_cb) with
 * n_cb = ceil(K / 32).  No reference counterpart: the MLP of scripts/infer_sx8.py's prompt
 * pass (Hugging Face SiLU * up, then SX8LinearV44.forward on the down projection). */
int32_t sx8_dec_gemm_silu(const float* g, const float* u, int64_t M, int64_t K, const uint8_t* hdr,
                          const uint8_t* levels, int32_t hdr_bytes, const float* basis,
                          const float* scales, int64_t N, int64_t n_cb, float* Y, void* workspace,
                          int64_t workspace_bytes, void* stream);

/* sx8_dec_gemm_silu with the split-K sum left to the caller, as
 * sx8_gemm_prefill_group_deferred (one matrix: slice s at parts + s * slice). */
int32_t sx8_dec_gemm_silu_deferred(const float* g, const float* u, int64_t M, int64_t K,
                                   const uint8_t* hdr, const uint8_t* levels, int32_t hdr_bytes,
                                   const float* basis, const float* scales, int64_t N, int64_t n_cb,
                                   float* Y, void* workspace, int64_t workspace_bytes, float** parts,
                                   int32_t* n_parts, int64_t* slice, void* stream);

/* The prompt pass's MLP up to the down projection's input: the gate and up prefill GEMMs
 * of X (M, K) fp16 -- or of its packed operands Xp_in, Zhl_in[gate, up] (the layouts of
 * sx8_gemm_prefill_packed, e.g. from sx8_dec_add_rmsnorm_packed; X NULL) -- (hdrs / levels /
 * bases / scales: [gate, up], N output columns each, n_cb K blocks) and x = fp16(silu(g) *
 * u), written straight as the down projection's
 * packed prefill-GEMM operands (sx8_gemm_prefill_packed): Xp (ceil(M / 32) * ceil(N / 32)
 * * 2048 bytes) and Zhl (M * ceil(N / 32) * 8 bytes) for the down projection's basis
 * (ceil(N / 32), 2, 32) and scales.  When the plan runs whole 512-row tiles, one GEMM
 * launch takes 64 gate and the same 64 up columns per tile and its epilogue writes the
 * operands (no float32 g and u in memory); otherwise the group GEMM writes g and u into the
 * workspace and a pack pass reads them back.  Both forms give the same bits, the bits of
 * sx8_gemm_prefill_group + sx8_dec_silu_mul + the down GEMM's own pass over x.  Workspace:
 * sx8_dec_gemm_gateup_silu_workspace_bytes.  No reference counterpart (the reference's MLP
 * runs gate, up, SiLU * up and down as separate torch ops, scripts/infer_sx8.py). */
int32_t sx8_dec_gemm_gateup_silu(const uint16_t* X, const uint16_t* Xp_in, const uint32_t* const* Zhl_in,
                                 int64_t M, int64_t K, const uint8_t* const* hdrs,
                                 const uint8_t* const* levels, int32_t hdr_bytes, const float* const* bases,
                                 const float* const* scales, int64_t N, int64_t n_cb, const float* down_basis,
                                 const float* down_scales, uint16_t* Xp, uint32_t* Zhl, void* workspace,
                                 int64_t workspace_bytes, void* stream);

/* Workspace bytes of sx8_dec_gemm_gateup_silu, or -1 for bad arguments. */
int64_t sx8_dec_gemm_gateup_silu_workspace_bytes(int64_t M, int64_t N, int64_t n_cb);

/* Causal attention of T prompt rows (prefill): q (T, nh, hd) fp16 (normalized and
 * rotated, as sx8_dec_qk_rope_cache_rows writes it), caches (nk, L, hd) fp16 holding
 * keys/values 0 .. start + T - 1; row i (position start + i) attends keys 0 .. start + i.
 * out (T, nh * hd) fp16; scale = 1 / sqrt(hd).  nh / nk in {1, 2, 4, 8} with 16 nh / nk
 * <= hd, hd 64 or 128, one KV head's cache (L * hd * 2 bytes) at most 0x7FF00000 bytes
 * (it is read through 32-bit buffer offsets).  fp16 products on MFMA with fp32 accumulation and an fp32 online
 * softmax (probabilities rounded to fp16 for the second product).  No reference
 * counterpart: the Hugging Face attention of the prompt pass in scripts/infer_sx8.py. */
int32_t sx8_dec_attn_prefill(const uint16_t* q, const uint16_t* k_cache, const uint16_t* v_cache,
                             uint16_t* out, int64_t T, int64_t start, int32_t nh, int32_t nk, int32_t hd,
                             int64_t L, float scale, void* stream);

/* sx8_dec_attn_prefill writing its output as the o projection's prefill-GEMM operands
 * (sx8_gemm_prefill_packed) instead of (T, nh * hd) fp16: Xp, the packed X of the T rows
 * (ceil(T / 32) * n_cb * 2048 bytes), and Zhl, the o projection's PCA operand (T * n_cb * 8
 * bytes), with n_cb = nh * hd / 32 and basis (n_cb, 2, 32) / scales (n_cb, 2) that
 * projection's.  Bit for bit what sx8_dec_attn_prefill followed by the prefill GEMM's own
 * pass over its output gives; the separate pass (one launch, X read and written) is gone.
 * basis, Xp and Zhl 16-byte aligned, scales 8-byte.  No reference counterpart. */
int32_t sx8_dec_attn_prefill_packed(const uint16_t* q, const uint16_t* k_cache, const uint16_t* v_cache,
                                    int64_t T, int64_t start, int32_t nh, int32_t nk, int32_t hd, int64_t L,
                                    float scale, const float* basis, const float* scales, uint16_t* Xp,
                                    uint32_t* Zhl, void* stream);

/* Workspace bytes of sx8_dec_attn_split. */
int64_t sx8_dec_attn_workspace_bytes(int32_t nh, int32_t hd);

/* out = fp16(silu(g) * u) over n float32 elements. */
int32_t sx8_dec_silu_mul(const float* g, const float* u, uint16_t* out, int64_t n, void* stream);

/* Decoder GEMVs with their input produced inside the GEMV (no separate launch for it).
 * No reference counterpart: in scripts/infer_sx8.py:109-173 the Hugging Face modules run
 * the RMSNorm / SiLU ops and SX8LinearV44.forward (scripts/integrate_fused_v44.py:43-77)
 * then runs the M = 1 GEMV (sx8_gemv_group above) on their output.
 *
 * sx8_dec_gemv_rmsnorm: x = fp16(h * rsqrt(mean(h^2) + eps) * norm_w) with h = (init ? fp16
 * init : resid) + (delta ? delta : 0) in float32 (K = n_cb * 32 values, as
 * sx8_dec_add_rmsnorm with M = 1, up to the summation order of mean(h^2)); then Ys[i] =
 * W_i . x for the n_mats matrices, as sx8_gemv_group.  When resid_out is not NULL it
 * receives h; it must not alias resid or delta.  State vectors 16-byte aligned.
 * sx8_dec_gemv_silu: the same with x = fp16(silu(g) * u) (as sx8_dec_silu_mul).
 * sx8_dec_gemv_silu_add / sx8_dec_gemv_add: x = fp16(silu(g) * u), or x given (fp16, 16-byte
 * aligned), and Ys[i] = adds[i] + W_i . x: the residual add of the decoder layer in the
 * GEMV's final store (each element read and written by one thread, so adds[i] may be
 * Ys[i]: the residual stream updated in place).  adds[i] is 4-byte aligned and either
 * equals Ys[i] or overlaps no output vector; any other overlap is refused.
 * All need n_cb <= 384 and take bases/scales (no caller Z). */
int32_t sx8_dec_gemv_rmsnorm(const float* resid, const uint16_t* init, const float* delta,
                             const uint16_t* norm_w, float eps, float* resid_out, int32_t n_mats,
                             const uint8_t* const* hdrs, const uint8_t* const* levels,
                             int32_t hdr_bytes, const float* const* bases,
                             const float* const* scales, const int64_t* Ns, int64_t n_cb,
                             float* const* Ys, void* stream);
int32_t sx8_dec_gemv_silu(const float* g, const float* u, int32_t n_mats,
                          const uint8_t* const* hdrs, const uint8_t* const* levels,
                          int32_t hdr_bytes, const float* const* bases, const float* const* scales,
                          const int64_t* Ns, int64_t n_cb, float* const* Ys, void* stream);
int32_t sx8_dec_gemv_silu_add(const float* g, const float* u, int32_t n_mats,
                              const uint8_t* const* hdrs, const uint8_t* const* levels,
                              int32_t hdr_bytes, const float* const* bases, const float* const* scales,
                              const int64_t* Ns, int64_t n_cb, const float* const* adds,
                              float* const* Ys, void* stream);
int32_t sx8_dec_gemv_add(const uint16_t* x, int32_t n_mats, const uint8_t* const* hdrs,
                         const uint8_t* const* levels, int32_t hdr_bytes, const float* const* bases,
                         const float* const* scales, const int64_t* Ns, int64_t n_cb,
                         const float* const* adds, float* const* Ys, void* stream);

/* The decoder MLP as two launches (no reference counterpart: the reference runs the gate,
 * up and down linears of the Hugging Face MLP separately, scripts/infer_sx8.py:109-173).
 * sx8_dec_gemv_rmsnorm_pair: x = fp16(resid * rsqrt(mean(resid^2) + eps) * norm_w) (as
 * sx8_dec_gemv_rmsnorm with the residual alone), g = W_gate x and u = W_up x in one
 * launch, m = fp16(silu(g) * u) (as sx8_dec_silu_mul) to m, and zp = the down projection's
 * PCA sums of m per K block in two partial slots, (N / 32, 2, 2) floats.  The up matrix's
 * headers, levels, bases and scales (up_*) must follow the gate matrix's in memory
 * (up_hdr = hdr + N * n_cb * hdr_bytes, up_levels = levels + N * n_cb * 24, up_bases =
 * bases + n_cb * 64, up_scales = scales + n_cb * 2: one allocation per field holding both),
 * otherwise SX8_ERR_INVALID; N a multiple of 32 in 32..12288 (the down projection's K, as
 * sx8_dec_gemv_zp_add accepts); down_bases its (N / 32, 64) bases.
 * sx8_dec_gemv_zp_add: Y = add + W_down m with the PCA term from zp (Z = (zp[kb][0][c] +
 * zp[kb][1][c]) * scales[kb][c]); add may be Y (the residual updated in place). */
int32_t sx8_dec_gemv_rmsnorm_pair(const float* resid, const uint16_t* norm_w, float eps,
                                  const uint8_t* hdr, const uint8_t* levels, int32_t hdr_bytes,
                                  const float* bases, const float* scales, const uint8_t* up_hdr,
                                  const uint8_t* up_levels, const float* up_bases,
                                  const float* up_scales, int64_t N, int64_t n_cb,
                                  const float* down_bases, uint16_t* m, float* zp, void* stream);
int32_t sx8_dec_gemv_zp_add(const uint16_t* m, const uint8_t* hdr, const uint8_t* levels,
                            int32_t hdr_bytes, const float* zp, const float* scales, int64_t N,
                            int64_t n_cb, const float* add, float* Y, void* stream);

/* The lm_head step of a decode: logits = W · fp16(resid · rsqrt(mean(resid^2) + eps) · norm_w)
 * (sx8_dec_gemv_rmsnorm on one matrix), then *tok = argmax(logits) (first index among
 * equal maxima, as sx8_dec_argmax_advance) and *pos += 1.  Each GEMV work-group also
 * writes the best of its own columns to parts (sx8_dec_argmax_parts_bytes(N, n_cb) bytes,
 * 8-byte aligned), so the argmax launch scans those instead of the N logits.  No
 * reference counterpart (the reference takes torch.argmax of the Hugging Face logits,
 * scripts/infer_sx8.py). */
int64_t sx8_dec_argmax_parts_bytes(int64_t N, int64_t n_cb);
int32_t sx8_dec_gemv_rmsnorm_argmax(const float* resid, const uint16_t* norm_w, float eps,
                                    const uint8_t* hdr, const uint8_t* levels, int32_t hdr_bytes,
                                    const float* bases, const float* scales, int64_t N, int64_t n_cb,
                                    float* logits, void* parts, int64_t parts_bytes, int64_t* tok,
                                    int64_t* pos, void* stream);

/* *tok = argmax(logits[0..n)) (first index among equal maxima), then *pos += 1. */
int32_t sx8_dec_argmax_advance(const float* logits, int64_t n, int64_t* tok, int64_t* pos,
                               void* stream);

#ifdef __cplusplus
}
#endif

#endif /* SX8_DECODER_H */
