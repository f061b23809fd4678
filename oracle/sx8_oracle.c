/*
 * sx8_oracle.c -- CPU restatement of the S-X8 v4.3 dequantization arithmetic.
 *
 * TEST INFRASTRUCTURE ONLY.  This file is the parity checker for the HIP kernels
 * under sx8-quantization_amd/csrc.  Only tests/, __graft_entry__.smoke() and the
 * cpu_baseline leg of bench.py may load it; the product path never does.
 *
 * Build: oracle/Makefile (gcc -O2 -ffp-contract=off -fopenmp).  Contraction MUST
 * stay off: every fused multiply-add below is written as an explicit fma().
 *
 * What is restated (all citations are to /root/reference):
 *   - the block field layout and 6-bit level extraction
 *       (docs/SX8_FLASH_V4_3_SPEC.md:13-25, scripts/kernel_sx8_v43.py:22-25);
 *   - R64, the canonical dequant of scripts/kernel_sx8_v43.py:14-51 under Numba's
 *     typing: dmin/dmax arrive as float32 (kernel_sx8_v43.py:123-124 casts the fp16
 *     arrays with astype(np.float32)); `hi_f - lo_f` is a binary32 subtraction; the
 *     0.25 / 0.015873 / 1e-10 / 1.0 literals are float64, so q, rlo, rhi, step and w
 *     are binary64; `weights` is a float32 buffer (store rounds to binary32, RNE);
 *     decode_tensor_gpu_fast (:141) then rounds to fp16 with torch .half() (RNE);
 *   - R32, the float32 variant used by the reference's .cu kernels
 *     (cuda/sx8_embed_v44.cu:46-75), kept only to count last-bit disagreements;
 *   - R32-ggml, llama.cpp's no-PCA float32 dequant of GGUF block_sx8 records
 *     (llama-cpp-sx8.patch:746-767), with and without fused multiply-adds;
 *   - the prefill GEMM's fp16 MFMA operand (the PCA-free core of the reference's float32
 *     decode, cuda/sx8_fused_wmma.cu:70-94, in the HIP kernel's evaluation order, the
 *     final multiply-add rounded once to fp16);
 *   - float64-accumulated GEMV/GEMM references used as the 1e-3 yardstick
 *     (scripts/sx8_decode1_v3.py:131-133, scripts/sx8_fused_wmma.py:128-132);
 *   - the CPU dequant + fp32-accumulated GEMV that bench.py reports as its CPU
 *     baseline (a restatement of decode_tensor_gpu_fast followed by X @ W.T).
 *
 * Block order everywhere in this file is the pkl/container order ("n-major"):
 * block bid covers row n = bid / n_cb, columns kb*32 .. kb*32+31 with kb = bid % n_cb
 * (kernel_sx8_v43.py:46, :137).
 */
#include <math.h>
#include <stdint.h>
#include <string.h>
#ifdef _OPENMP
#include <omp.h>
#endif

/* ---------------------------------------------------------------- fp16 <-> fp32 */

/* Exact binary16 -> binary32 widening (every fp16 value is representable). */
float sx8o_f16_to_f32(uint16_t h) {
    uint32_t sign = (uint32_t)(h & 0x8000u) << 16;
    uint32_t exp = (h >> 10) & 0x1Fu;
    uint32_t man = h & 0x3FFu;
    uint32_t bits;
    if (exp == 0) {
        if (man == 0) {
            bits = sign;
        } else {                       /* subnormal: renormalise */
            int e = -1;
            do { man <<= 1; e++; } while ((man & 0x400u) == 0);
            man &= 0x3FFu;
            bits = sign | ((uint32_t)(127 - 15 - e) << 23) | (man << 13);
        }
    } else if (exp == 0x1F) {
        bits = sign | 0x7F800000u | (man << 13);
    } else {
        bits = sign | ((exp + 127 - 15) << 23) | (man << 13);
    }
    float f;
    memcpy(&f, &bits, 4);
    return f;
}

/* binary32 -> binary16, round to nearest even, with fp16 subnormals and overflow
 * to infinity (IEEE 754 convertFormat).  NaN maps to a quiet NaN keeping the top
 * payload bits. */
uint16_t sx8o_f32_to_f16(float f) {
    uint32_t x;
    memcpy(&x, &f, 4);
    uint16_t sign = (uint16_t)((x >> 16) & 0x8000u);
    uint32_t exp = (x >> 23) & 0xFFu;
    uint32_t man = x & 0x7FFFFFu;
    if (exp == 0xFF) {
        if (man == 0) return sign | 0x7C00u;
        return (uint16_t)(sign | 0x7E00u | (man >> 13));
    }
    int e = (int)exp - 127;           /* unbiased exponent */
    if (e > 15) return sign | 0x7C00u;
    if (e >= -14) {                    /* normal fp16 range */
        uint32_t m = man;              /* 23 bits, keep 10 */
        uint32_t keep = m >> 13;
        uint32_t rest = m & 0x1FFFu;
        uint32_t he = (uint32_t)(e + 15);
        uint32_t r = (he << 10) | keep;
        if (rest > 0x1000u || (rest == 0x1000u && (keep & 1u))) r += 1; /* may carry into exp */
        return (uint16_t)(sign | r);   /* r == 0x7C00 is the correct overflow to inf */
    }
    /* subnormal or zero in fp16: value = man24 * 2^(e-23); target unit 2^-24 */
    if (exp == 0) return sign;         /* f32 subnormals are far below 2^-25 */
    uint32_t m24 = man | 0x800000u;    /* 24-bit significand */
    int shift = -e - 14 + 13;          /* bits to drop so the unit becomes 2^-24 */
    if (shift > 24) return sign;       /* below half of the smallest subnormal */
    uint32_t keep = m24 >> shift;
    uint32_t rest = m24 & ((1u << shift) - 1u);
    uint32_t half = 1u << (shift - 1);
    if (rest > half || (rest == half && (keep & 1u))) keep += 1;
    return (uint16_t)(sign | keep);    /* keep == 0x400 is the smallest normal */
}

/* ------------------------------------------------------------ level extraction */

/* 6-bit level of weight t (0..31) of one block: high nibble from qh, low quad from
 * ql (SPEC.md:20-21, kernel_sx8_v43.py:23-25). */
static inline int sx8o_level(const uint8_t* qh, const uint8_t* ql, int t) {
    int nib = (qh[t >> 1] >> ((t & 1) * 4)) & 0xF;
    int qua = (ql[t >> 2] >> ((3 - (t & 3)) * 2)) & 0x3;
    return (nib << 2) | qua;
}

int sx8o_level_of(const uint8_t* qh, const uint8_t* ql, int t) { return sx8o_level(qh, ql, t); }

/* ------------------------------------------------------------------------ R64 */

/* One weight under R64.  `fused` selects fma(step, lv, rlo) (NVVM contracts the
 * mul+add of kernel_sx8_v43.py:39 by default) or the separately rounded form.
 * The two PCA updates (kernel_sx8_v43.py:48-49) are written as fma: the product
 * (1.0*c)*scale*basis is exact in binary64 (4 + 24 + 24 significant bits), so fused
 * and unfused agree there by construction. Returns the binary32 store value. */
static inline float sx8o_r64_weight(float lo_f, float hi_f, int cfg, int coeff, int lv, int t,
                                    float s0, float s1, float b0, float b1, int fused) {
    double q = (double)(hi_f - lo_f) * 0.25;     /* binary32 subtract, binary64 scale */
    int strat = (cfg >> ((t >> 3) * 2)) & 3;
    double rlo, rhi;
    if (strat == 0)      { rlo = lo_f;     rhi = hi_f; }
    else if (strat == 1) { rlo = lo_f;     rhi = lo_f + q; }
    else if (strat == 2) { rlo = hi_f - q; rhi = hi_f; }
    else                 { rlo = lo_f + q; rhi = hi_f - q; }
    double step = (rhi - rlo) * 0.015873;
    if (step < 1e-10) step = 1e-10;              /* NaN compares false and passes */
    double w = fused ? fma(step, (double)lv, rlo) : rlo + step * (double)lv;
    int c0 = coeff & 0xF;        c0 = c0 < 8 ? c0 : c0 - 16;
    int c1 = (coeff >> 4) & 0xF; c1 = c1 < 8 ? c1 : c1 - 16;
    w = fma((1.0 * c0) * (double)s0, (double)b0, w);
    w = fma((1.0 * c1) * (double)s1, (double)b1, w);
    return (float)w;                             /* binary32 store, RNE */
}

/* Full-tensor R64 dequant in pkl block order.  dmin/dmax are fp16 bit patterns.
 * out16 (n_blocks*32 fp16 bit patterns) and/or out32 (binary32 store values) may be
 * NULL.  basis is (n_cb, 64) float32, scales (n_cb, 2) float32. */
void sx8o_dequant_r64(int64_t n_blocks, int32_t n_cb,
                      const uint16_t* dmin, const uint16_t* dmax,
                      const uint8_t* config, const uint8_t* coeff,
                      const uint8_t* hi, const uint8_t* lo,
                      const float* basis, const float* scales,
                      int32_t fused, uint16_t* out16, float* out32) {
#pragma omp parallel for schedule(static)
    for (int64_t bid = 0; bid < n_blocks; bid++) {
        float lo_f = sx8o_f16_to_f32(dmin[bid]);
        float hi_f = sx8o_f16_to_f32(dmax[bid]);
        int cfg = config[bid], cf = coeff[bid];
        int64_t cb = bid % n_cb;
        const float* bs = basis + cb * 64;
        float s0 = scales[cb * 2 + 0], s1 = scales[cb * 2 + 1];
        for (int t = 0; t < 32; t++) {
            int lv = sx8o_level(hi + bid * 16, lo + bid * 8, t);
            float w = sx8o_r64_weight(lo_f, hi_f, cfg, cf, lv, t, s0, s1, bs[t], bs[32 + t], fused);
            if (out32) out32[bid * 32 + t] = w;
            if (out16) out16[bid * 32 + t] = sx8o_f32_to_f16(w);
        }
    }
}

/* ------------------------------------------------------------------------ R32 */

/* The float32 decode of the reference's .cu kernels (sx8_embed_v44.cu:46-75):
 * branchless strategy, 0.015873f, 1e-10f clamp, per-weight PCA, __float2half.
 * Contraction is off here; the reference's nvcc build contracts with unknown
 * grouping, so this variant is only used to count last-bit disagreements. */
void sx8o_dequant_r32(int64_t n_blocks, int32_t n_cb,
                      const uint16_t* dmin, const uint16_t* dmax,
                      const uint8_t* config, const uint8_t* coeff,
                      const uint8_t* hi, const uint8_t* lo,
                      const float* basis, const float* scales, uint16_t* out16) {
#pragma omp parallel for schedule(static)
    for (int64_t bid = 0; bid < n_blocks; bid++) {
        float lo_f = sx8o_f16_to_f32(dmin[bid]);
        float hi_f = sx8o_f16_to_f32(dmax[bid]);
        int cfg = config[bid], cf = coeff[bid];
        int64_t cb = bid % n_cb;
        int c0 = cf & 0xF;        if (c0 >= 8) c0 -= 16;
        int c1 = (cf >> 4) & 0xF; if (c1 >= 8) c1 -= 16;
        float q = (hi_f - lo_f) * 0.25f;
        for (int t = 0; t < 32; t++) {
            int s = (cfg >> ((t >> 3) * 2)) & 3;
            float rlo = lo_f + q * (float)(3 * (s == 2) + (s == 3));
            float rhi = hi_f - q * (float)(3 * (s == 1) + (s == 3));
            float step = (rhi - rlo) * 0.015873f;
            if (step < 1e-10f) step = 1e-10f;
            int lv = sx8o_level(hi + bid * 16, lo + bid * 8, t);
            float w = rlo + step * (float)lv
                    + (float)c0 * scales[cb * 2] * basis[cb * 64 + t]
                    + (float)c1 * scales[cb * 2 + 1] * basis[cb * 64 + 32 + t];
            out16[bid * 32 + t] = sx8o_f32_to_f16(w);
        }
    }
}

/* ------------------------------------------------- prefill GEMM operand (core) */

/* binary64 -> binary16, round to nearest even, subnormals, overflow to infinity.  adj
 * breaks an exact tie the other way when a lower-order part of the value is known:
 * adj > 0 means the true value lies just above |x| in magnitude, adj < 0 just below. */
static uint16_t sx8o_f64_to_f16_adj(double x, double adj) {
    const uint16_t sign = signbit(x) ? 0x8000u : 0u;
    if (isnan(x)) return (uint16_t)(sign | 0x7E00u);
    const double ax = fabs(x);
    if (isinf(x)) return (uint16_t)(sign | 0x7C00u);
    if (ax == 0.0) return sign;
    int e2;
    (void)frexp(ax, &e2);                        /* ax = f 2^e2, f in [0.5, 1) */
    int ue = e2 - 1 - 10;                        /* exponent of the fp16 ulp at ax */
    if (ue < -24) ue = -24;                      /* subnormal range: ulp 2^-24 */
    const double q = ldexp(ax, -ue);             /* exact: a power-of-two scaling */
    double n = floor(q);
    const double frac = q - n;
    if (frac > 0.5 || (frac == 0.5 && (adj > 0 || (adj == 0 && fmod(n, 2.0) != 0)))) n += 1.0;
    /* n counts ulps of 2^ue; a normal result has n in [1024, 2048] (2048 carries) */
    uint32_t bits;
    if (ue == -24) {
        bits = (uint32_t)n;                      /* 1024 is the smallest normal, 0x0400 */
    } else {
        bits = ((uint32_t)(ue + 10 + 15) << 10) + ((uint32_t)n - 1024u);
    }
    if (bits >= 0x7C00u) bits = 0x7C00u;
    return (uint16_t)(sign | bits);
}

/* The fp16 operand the prefill GEMM feeds to its MFMAs for weight t of a block: the
 * PCA-free core rlo + step*lv of the reference's float32 decode (cuda/sx8_fused_wmma.cu:
 * 70-94, whose WMMA tiles hold that float32 weight plus the per-weight PCA, rounded with
 * __float2half), evaluated the way the HIP kernel does it (csrc/sx8_gemm.hip, sub_range /
 * dec_pair):
 *   d = hi - lo, q = d * 0.25f, m = d * 0.015873f           (binary32, each rounded)
 *   s = strategy of sub-block t/8; k1 = {0, 0, 3, 1}[s], e = {0, 2, 2, 1}[s]
 *   rlo  = fmaf(q, k1, lo)                                  (= lo + q*(3*(s==2)+(s==3)))
 *   step = d > 0 ? m * 2^-e : 1e-10f    (the range rhi - rlo is d * {1, 1/4, 1/4, 1/2})
 *   w16  = fp16(step * lv + rlo), the exact value rounded once (RNE) -- the kernel's
 *          v_fma_mix{lo,hi}_f16 evaluates the multiply-add at full precision and rounds
 *          straight to fp16, with no binary32 intermediate.
 * The PCA term is not part of the operand (the kernel adds it through Z).  The reference
 * floors step at 1e-10 after scaling; for hi > lo the unfloored step is at least
 * 2.4e-10 (the smallest fp16 range times 0.015873 / 4), so the floor binds exactly when
 * d <= 0 (NaN endpoints: d is NaN, step = 1e-10 and rlo NaN propagates).
 * out16: n_blocks * 32 fp16 bit patterns, pkl block order. */
void sx8o_core_f16(int64_t n_blocks, const uint16_t* dmin, const uint16_t* dmax,
                   const uint8_t* config, const uint8_t* hi, const uint8_t* lo, uint16_t* out16) {
#pragma omp parallel for schedule(static)
    for (int64_t bid = 0; bid < n_blocks; bid++) {
        const float lo_f = sx8o_f16_to_f32(dmin[bid]);
        const float hi_f = sx8o_f16_to_f32(dmax[bid]);
        const float d = hi_f - lo_f;
        const float q = d * 0.25f;
        const float m = d * 0.015873f;
        for (int t = 0; t < 32; t++) {
            const int s = (config[bid] >> ((t >> 3) * 2)) & 3;
            static const float k1t[4] = {0.f, 0.f, 3.f, 1.f};
            static const int et[4] = {0, 2, 2, 1};
            const float rlo = fmaf(q, k1t[s], lo_f);
            const float step = d > 0.f ? ldexpf(m, -et[s]) : 1e-10f;
            const double a = (double)step * (double)sx8o_level(hi + bid * 16, lo + bid * 8, t);  /* exact */
            const double b = (double)rlo;
            /* a + b = sum + err exactly (two-sum); a tie of the fp16 rounding of sum is
             * broken by err, so the result is the exact value rounded once */
            const double sum = a + b;
            const double bb = sum - a;
            const double err = (a - (sum - bb)) + (b - bb);
            out16[bid * 32 + t] = sx8o_f64_to_f16_adj(sum, signbit(sum) ? -err : err);
        }
    }
}

/* R32-ggml: llama.cpp's dequantize_row_sx8 (llama-cpp-sx8.patch:746-767) on interleaved
 * 30-byte block_sx8 records (patch:131-144): float32 arithmetic, no PCA (coeff ignored),
 * branch-free strategy offsets, 0.015873f and 1e-10f.  contract = 1 writes the three
 * a*b+c forms as fmaf (what a contracting C build computes), contract = 0 rounds every
 * operation.  out: n_blocks * 32 floats in block order. */
void sx8o_dequant_ggml(int64_t n_blocks, const uint8_t* blocks, int32_t contract, float* out) {
#pragma omp parallel for schedule(static)
    for (int64_t b = 0; b < n_blocks; b++) {
        const uint8_t* r = blocks + b * 30;
        const float lo_f = sx8o_f16_to_f32((uint16_t)(r[0] | (r[1] << 8)));
        const float hi_f = sx8o_f16_to_f32((uint16_t)(r[2] | (r[3] << 8)));
        const float q = (hi_f - lo_f) * 0.25f;
        for (int t = 0; t < 32; t++) {
            const int s = (r[4] >> ((t >> 3) * 2)) & 3;
            const float k1 = (float)(3 * (s == 2) + (s == 3));
            const float k2 = (float)(3 * (s == 1) + (s == 3));
            const float rlo = contract ? fmaf(q, k1, lo_f) : lo_f + q * k1;
            const float rhi = contract ? fmaf(-q, k2, hi_f) : hi_f - q * k2;
            float step = (rhi - rlo) * 0.015873f;
            if (step < 1e-10f) step = 1e-10f;
            const float lv = (float)sx8o_level(r + 5, r + 21, t);
            out[b * 32 + t] = contract ? fmaf(step, lv, rlo) : rlo + step * lv;
        }
    }
}

/* ------------------------------------------------------- float64 references */

/* Y[m, n] = sum_k X[m, k] * W[n, k] in binary64 (X, W are fp16 bit patterns;
 * W is (N, ldw) row-major and only its first K columns are used). */
void sx8o_gemm_f64(int32_t M, int32_t N, int32_t K, const uint16_t* X, int32_t ldx,
                   const uint16_t* W, int32_t ldw, double* Y) {
#pragma omp parallel for schedule(static)
    for (int32_t n = 0; n < N; n++) {
        for (int32_t m = 0; m < M; m++) {
            double acc = 0.0;
            for (int32_t k = 0; k < K; k++)
                acc += (double)sx8o_f16_to_f32(X[(int64_t)m * ldx + k]) *
                       (double)sx8o_f16_to_f32(W[(int64_t)n * ldw + k]);
            Y[(int64_t)m * N + n] = acc;
        }
    }
}

/* ------------------------------------------------------------ CPU baseline */

/* The CPU baseline of bench.py: R64 dequant of a whole tensor to fp16 (above)
 * followed by an fp32-accumulated GEMV y = W16 . x, one output row per OpenMP
 * iteration.  fp16 widening goes through a 64K-entry table built on first use.
 * Returns 0, or -1 when K exceeds the on-stack activation buffer. */
static float g_f16_lut[65536];
static int g_f16_lut_ready = 0;

static void sx8o_build_lut(void) {
    if (g_f16_lut_ready) return;
    for (uint32_t h = 0; h < 65536u; h++) g_f16_lut[h] = sx8o_f16_to_f32((uint16_t)h);
    g_f16_lut_ready = 1;
}

int32_t sx8o_gemv_f32(int32_t N, int32_t K, int32_t ldw, const uint16_t* W16,
                      const uint16_t* x16, float* y) {
    float xs[32768];
    if (K > 32768 || K > ldw) return -1;
    sx8o_build_lut();
    for (int32_t k = 0; k < K; k++) xs[k] = g_f16_lut[x16[k]];
#pragma omp parallel for schedule(static)
    for (int32_t n = 0; n < N; n++) {
        const uint16_t* w = W16 + (int64_t)n * ldw;
        float acc = 0.0f;
        for (int32_t k = 0; k < K; k++) acc += xs[k] * g_f16_lut[w[k]];
        y[n] = acc;
    }
    return 0;
}

int32_t sx8o_num_threads(void) {
#ifdef _OPENMP
    return omp_get_max_threads();
#else
    return 1;
#endif
}

void sx8o_set_num_threads(int32_t n) {
#ifdef _OPENMP
    if (n > 0) omp_set_num_threads(n);
#else
    (void)n;
#endif
}
