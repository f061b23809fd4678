"""CPU oracle for the S-X8 v4.3 hot path -- TEST INFRASTRUCTURE ONLY.

Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg may import
this module, and only as the checker.  The shipped package never imports it.

Contents (each restates a reference function; paths are relative to
/root/reference):

* ``lib()`` -- ctypes handle on oracle/build/libsx8_oracle.so, the C restatement of
  R64 (scripts/kernel_sx8_v43.py:14-51), R32 (cuda/sx8_embed_v44.cu:46-75), the
  float64 GEMM yardstick and the CPU baseline GEMV.
* ``pack_levels`` / ``unpack_levels`` -- scripts/quantize_qwen35_4b_sx8_v43_gpu.py:148-167
  and scripts/kernel_sx8_v43.py:23-25.
* ``v6_encode`` -- quantize_qwen35_4b_sx8_v43_gpu.py:22-47 (float32 numpy).
* ``pca_correct`` -- quantize_qwen35_4b_sx8_v43_gpu.py:75-142 (numpy SVD).
* ``quantize`` -- the tensor loop of quantize_qwen35_4b_sx8_v43_gpu.py:235-282 and the
  pkl serialisation of :383-395 (``qt`` and ``bases_info`` dicts).
* ``to_v44`` -- scripts/prepare_v44.py:35-79 (kb-major hdr/levels).
* ``dequant_r64`` -- C R64; ``dequant_r64_numpy`` -- an independent vectorised
  float64 restatement (unfused); ``dequant_r64_exact`` -- exact rational arithmetic
  for spot checks of the fused form.
* ``z44`` -- cuda/sx8_decode1_v3.cu:44-65 in float64.
* ``gemm_f64`` -- the float64 yardstick Y = X . W16^T.
* ``dequant_ggml`` -- C R32-ggml, llama.cpp's no-PCA float32 dequant of block_sx8
  records (llama-cpp-sx8.patch:746-767), with or without fused multiply-adds.
* ``core_f16`` -- C: the prefill GEMM's fp16 MFMA operand, the PCA-free core of the
  reference's float32 decode (cuda/sx8_fused_wmma.cu:70-94) in the kernel's evaluation
  order; ``core_exact_weight`` -- the same recipe in exact rational arithmetic with every
  binary32 operation correctly rounded (independent check).

Parity status of each function is recorded next to it.
"""
from __future__ import annotations

import ctypes
import os
import subprocess
from fractions import Fraction

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "build", "libsx8_oracle.so")

L63 = 63
C_STEP = 0.015873          # kernel_sx8_v43.py:37 (float64 literal, not 1/63)
STEP_FLOOR = 1e-10         # kernel_sx8_v43.py:38

_lib = None


def build() -> str:
    """Compile the C oracle with oracle/Makefile (idempotent)."""
    subprocess.run(["make", "-s", "-C", HERE], check=True)
    return LIB_PATH


def lib():
    """ctypes handle on the C oracle; builds it on first use if absent."""
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            build()
        L = ctypes.CDLL(LIB_PATH)
        p = ctypes.c_void_p
        i64, i32 = ctypes.c_int64, ctypes.c_int32
        L.sx8o_dequant_r64.argtypes = [i64, i32, p, p, p, p, p, p, p, p, i32, p, p]
        L.sx8o_dequant_r64.restype = None
        L.sx8o_dequant_r32.argtypes = [i64, i32, p, p, p, p, p, p, p, p, p]
        L.sx8o_dequant_ggml.restype = None
        L.sx8o_dequant_ggml.argtypes = [i64, p, i32, p]
        L.sx8o_dequant_r32.restype = None
        L.sx8o_core_f16.argtypes = [i64, p, p, p, p, p, p]
        L.sx8o_core_f16.restype = None
        L.sx8o_gemm_f64.argtypes = [i32, i32, i32, p, i32, p, i32, p]
        L.sx8o_gemm_f64.restype = None
        L.sx8o_gemv_f32.argtypes = [i32, i32, i32, p, p, p]
        L.sx8o_gemv_f32.restype = i32
        L.sx8o_f16_to_f32.argtypes = [ctypes.c_uint16]
        L.sx8o_f16_to_f32.restype = ctypes.c_float
        L.sx8o_f32_to_f16.argtypes = [ctypes.c_float]
        L.sx8o_f32_to_f16.restype = ctypes.c_uint16
        L.sx8o_num_threads.restype = i32
        L.sx8o_set_num_threads.argtypes = [i32]
        _lib = L
    return _lib


def _ptr(a: np.ndarray):
    assert a.flags["C_CONTIGUOUS"]
    return ctypes.c_void_p(a.ctypes.data)


# --------------------------------------------------------------------------- a1 levels

def pack_levels(lv: np.ndarray):
    """(n_blk, 32) levels 0..63 -> (levels_hi (n_blk*16,), levels_lo (n_blk*8,)).

    Restates pack_levels_6bit (quantize_qwen35_4b_sx8_v43_gpu.py:148-167): weight t's
    high nibble goes to qh[t>>1] bits (t&1)*4; its low quad to ql[t>>2] bits
    (3-(t&3))*2.  Pinned by the brute-force round trip with ``unpack_levels`` and by
    hand-built blocks in tests/test_oracle.py.
    """
    lv = np.asarray(lv, dtype=np.uint8).reshape(-1, 32)
    n = lv.shape[0]
    hi4 = (lv >> 2) & 0xF
    lo2 = lv & 0x3
    qh = (hi4[:, 0::2] | (hi4[:, 1::2] << 4)).astype(np.uint8)
    ql = ((lo2[:, 0::4] << 6) | (lo2[:, 1::4] << 4) | (lo2[:, 2::4] << 2) | lo2[:, 3::4]).astype(np.uint8)
    return qh.reshape(n * 16), ql.reshape(n * 8)


def unpack_levels(hi: np.ndarray, lo: np.ndarray) -> np.ndarray:
    """Inverse of pack_levels, following kernel_sx8_v43.py:23-25 weight by weight."""
    hi = np.asarray(hi, dtype=np.uint8).reshape(-1, 16)
    lo = np.asarray(lo, dtype=np.uint8).reshape(-1, 8)
    out = np.empty((hi.shape[0], 32), dtype=np.uint8)
    for t in range(32):
        nib = (hi[:, t >> 1] >> ((t & 1) * 4)) & 0xF
        qua = (lo[:, t >> 2] >> ((3 - (t & 3)) * 2)) & 0x3
        out[:, t] = (nib << 2) | qua
    return out


# ------------------------------------------------------------------------ a0 quantizer

def v6_encode(blocks: np.ndarray):
    """V6 encode of (n_blk, 32) float32 blocks (quantize…:22-47), float32 arithmetic.

    Candidate order [full, lower quarter, upper quarter, centre half]; strict `<`
    keeps the first candidate on MSE ties.  The per-sub-block MSE sums the eight
    squared errors left to right before dividing by 8 (the reference uses
    torch.mean, whose CUDA summation order is unspecified).
    Returns levels (n,32) u8, dmin f32, dmax f32, config u8, strategies (n,4).
    """
    b = np.asarray(blocks, dtype=np.float32)
    n = b.shape[0]
    sub = b.reshape(n, 4, 8)
    dmin = b.min(axis=1)
    dmax = b.max(axis=1)
    d = np.maximum(dmax - dmin, np.float32(1e-10))
    q = d / np.float32(4.0)
    slo = [dmin, dmin, dmax - q, dmin + q]
    shi = [dmax, dmin + q, dmax, dmax - q]
    best_mse = np.full((n, 4), np.inf, dtype=np.float32)
    best_lev = np.zeros((n, 4, 8), dtype=np.int32)
    best_str = np.zeros((n, 4), dtype=np.int32)
    for ri in range(4):
        lo = slo[ri][:, None, None]
        hi = shi[ri][:, None, None]
        step = np.maximum((hi - lo) / np.float32(L63), np.float32(1e-10))
        cand = np.clip(np.rint((sub - lo) / step), 0, L63).astype(np.int32)
        rec = lo + step * cand.astype(np.float32)
        sq = (sub - rec) ** 2
        acc = sq[..., 0]
        for j in range(1, 8):
            acc = acc + sq[..., j]
        mse = acc / np.float32(8.0)
        better = mse < best_mse
        best_mse = np.where(better, mse, best_mse)
        best_lev = np.where(better[..., None], cand, best_lev)
        best_str = np.where(better, ri, best_str)
    config = (best_str[:, 0] | (best_str[:, 1] << 2) | (best_str[:, 2] << 4) | (best_str[:, 3] << 6))
    return best_lev.astype(np.uint8).reshape(n, 32), dmin, dmax, config.astype(np.uint8), best_str


def pca_correct(levels, dmin, dmax, config, blocks, n_cb, n_bases=4, _plant=None):
    """PCA post-correction per column slice kb (quantize…:75-142), numpy float32.

    Pinned by known answers (tests/test_quantizer.py, test_pca_known_answers): residual
    slices built from orthonormal directions and mutually orthogonal coefficient rows of
    distinct energy, so the kept directions (Vh[:2], up to the sign the SVD returns), the
    lower-median / 3 scales and every coefficient byte (given that sign) are known in
    closed form.  The sign itself is not pinnable: it depends on the LAPACK build, and
    the [-8, 7] clamp makes a flip visible in the bytes.  ``_plant`` (tests only) swaps in
    a known mistake -- "median/4", "upper_median" or "vh1:3" -- to show the pin fails.
    Returns coeff (n_blk,1) u8, data (n_cb,64) f32, scales (n_cb,2) f32.
    """
    n_blk = blocks.shape[0]
    d = np.maximum(dmax - dmin, np.float32(1e-10)).astype(np.float32)
    Q = (d / np.float32(4.0)).astype(np.float32)
    L = np.float32(L63)
    lo_j = np.stack([dmin, dmin, dmax - Q, dmin + Q], axis=0)
    st_j = np.stack([d / L, Q / L, Q / L, np.maximum(d - 2 * Q, np.float32(1e-10)) / L], axis=0)
    lv_f = levels.astype(np.float32)
    coeff = np.zeros((n_blk, 1), dtype=np.uint8)
    data = np.zeros((n_cb, 64), dtype=np.float32)
    scales = np.zeros((n_cb, 2), dtype=np.float32)
    idx = np.arange(n_blk)
    for cb in range(n_cb):
        si = idx[idx % n_cb == cb]
        if si.shape[0] < 4:
            continue
        cfg = config[si].astype(np.int64)
        rec = np.zeros((si.shape[0], 32), dtype=np.float32)
        for sb in range(4):
            st = (cfg >> (sb * 2)) & 3
            lo_sb = lo_j[st, si]
            step_sb = st_j[st, si]
            rec[:, sb * 8:(sb + 1) * 8] = lo_sb[:, None] + step_sb[:, None] * lv_f[si][:, sb * 8:(sb + 1) * 8]
        err = (blocks[si] - rec).astype(np.float32)
        _, _, vh = np.linalg.svd(err, full_matrices=False)
        first = 1 if _plant == "vh1:3" else 0
        basis = vh[first:first + n_bases].astype(np.float32)
        craw = basis @ err.T
        # torch.median returns the lower median for even counts
        srt = np.sort(np.abs(craw), axis=1)
        med = srt[:, srt.shape[1] // 2 if _plant == "upper_median" else (srt.shape[1] - 1) // 2]
        div = np.float32(4.0 if _plant == "median/4" else 3.0)
        sc = np.maximum(med / div, np.float32(1e-10)).astype(np.float32)
        cq = np.clip(np.rint(craw / sc[:, None]), -8, 7).astype(np.int8)
        byte0 = (cq[0].view(np.uint8) & 0xF) | ((cq[1].view(np.uint8) & 0xF) << 4)
        coeff[si, 0] = byte0
        data[cb] = basis[:2].reshape(-1)
        scales[cb] = sc[:2]
    return coeff, data, scales


def quantize(W16: np.ndarray, name: str = "w"):
    """fp16 (N, K) weight -> (qt, bases_info) dicts in the pkl layout.

    Mirrors the per-tensor loop of quantize…:235-282 (zero-pad K to a multiple of
    32, V6 encode, PCA, pack) and the serialised dict keys of :383-395.
    """
    W = np.asarray(W16, dtype=np.float16)
    out_f, in_f = W.shape
    n_cb = (in_f + 31) // 32
    Wf = W.astype(np.float32)
    if n_cb * 32 != in_f:
        Wf = np.pad(Wf, ((0, 0), (0, n_cb * 32 - in_f)))
    blocks = np.ascontiguousarray(Wf.reshape(out_f * n_cb, 32))
    lv, dmin, dmax, config, _ = v6_encode(blocks)
    coeff, data, scales = pca_correct(lv, dmin, dmax, config, blocks, n_cb)
    hi, lo = pack_levels(lv)
    qt = {
        "shape": (out_f, in_f), "orig_shape": (out_f, in_f),
        "n_blocks": out_f * n_cb, "n_cb": n_cb,
        "dmin": dmin.astype(np.float16), "dmax": dmax.astype(np.float16),
        "config": config, "levels_hi": hi, "levels_lo": lo, "coeff": coeff,
    }
    bases_info = {"n_cb": n_cb, "data": data, "scales": scales}
    return qt, bases_info


# ------------------------------------------------------------------------- a3 layout

def to_v44(qt, bases_info, hdr_aligned=False):
    """kb-major v4.4 layout (prepare_v44.py:35-79), written from the field spec.

    hdr row = dmin fp16 LE | dmax fp16 LE | config | coeff (| 2 zero pad bytes);
    levels row = qh bytes 4sb..4sb+3 then ql bytes 2sb..2sb+1 per sub-block, which
    is byte-identical to qh[0:16] || ql[0:8].  Row order bid = kb*N + n.
    Pinned by byte-level invariants in tests/test_oracle.py.
    """
    out_f, in_f = qt["shape"]
    n_cb = qt["n_cb"]
    n_blk = qt["n_blocks"]
    hb = 8 if hdr_aligned else 6
    hi = np.asarray(qt["levels_hi"], dtype=np.uint8).reshape(n_blk, 16)
    lo = np.asarray(qt["levels_lo"], dtype=np.uint8).reshape(n_blk, 8)
    dmin = np.asarray(qt["dmin"]).astype(np.float16).reshape(n_blk).view(np.uint8).reshape(n_blk, 2)
    dmax = np.asarray(qt["dmax"]).astype(np.float16).reshape(n_blk).view(np.uint8).reshape(n_blk, 2)
    cfg = np.asarray(qt["config"], dtype=np.uint8).reshape(n_blk)
    cof = np.asarray(qt["coeff"], dtype=np.uint8).reshape(n_blk)
    lev = np.zeros((n_blk, 24), dtype=np.uint8)
    for sb in range(4):
        lev[:, 4 * sb:4 * sb + 4] = hi[:, 4 * sb:4 * sb + 4]
        lev[:, 16 + 2 * sb:16 + 2 * sb + 2] = lo[:, 2 * sb:2 * sb + 2]
    hdr = np.zeros((n_blk, hb), dtype=np.uint8)
    hdr[:, 0:2] = dmin
    hdr[:, 2:4] = dmax
    hdr[:, 4] = cfg
    hdr[:, 5] = cof
    perm = np.arange(n_blk).reshape(out_f, n_cb).T.reshape(-1)   # kb-major row -> pkl bid
    return {
        "levels": np.ascontiguousarray(lev[perm]),
        "hdr": np.ascontiguousarray(hdr[perm]),
        "n_cb": n_cb, "shape": (out_f, in_f),
        "bases": np.asarray(bases_info["data"], dtype=np.float32).reshape(-1, 64),
        "scales": np.asarray(bases_info["scales"], dtype=np.float32).reshape(-1, 2),
    }


# ------------------------------------------------------------------------- a2 dequant

def _fields(qt):
    n_blk = qt["n_blocks"]
    c = lambda a, dt: np.ascontiguousarray(np.asarray(a).reshape(-1).astype(dt, copy=False))
    return (n_blk,
            c(np.asarray(qt["dmin"]).astype(np.float16).view(np.uint16), np.uint16),
            c(np.asarray(qt["dmax"]).astype(np.float16).view(np.uint16), np.uint16),
            c(qt["config"], np.uint8), c(qt["coeff"], np.uint8),
            c(qt["levels_hi"], np.uint8), c(qt["levels_lo"], np.uint8))


def _bases(bases_info):
    data = np.ascontiguousarray(np.asarray(bases_info["data"], dtype=np.float32).reshape(-1))
    sc = np.ascontiguousarray(np.asarray(bases_info["scales"], dtype=np.float32).reshape(-1))
    return data, sc


def dequant_r64(qt, bases_info, fused=True, blocks_only=False):
    """R64 dequant via the C oracle.  Returns fp16 (out_f, in_f) (or the raw
    (n_blk, 32) block matrix when blocks_only)."""
    n_blk, dmin, dmax, cfg, cof, hi, lo = _fields(qt)
    data, sc = _bases(bases_info)
    out = np.empty(n_blk * 32, dtype=np.uint16)
    lib().sx8o_dequant_r64(n_blk, qt["n_cb"], _ptr(dmin), _ptr(dmax), _ptr(cfg), _ptr(cof),
                           _ptr(hi), _ptr(lo), _ptr(data), _ptr(sc), int(bool(fused)),
                           _ptr(out), None)
    w = out.view(np.float16)
    if blocks_only:
        return w.reshape(n_blk, 32)
    out_f, in_f = qt["shape"]
    return w.reshape(out_f, qt["n_cb"] * 32)[:, :in_f]


def dequant_r32(qt, bases_info):
    n_blk, dmin, dmax, cfg, cof, hi, lo = _fields(qt)
    data, sc = _bases(bases_info)
    out = np.empty(n_blk * 32, dtype=np.uint16)
    lib().sx8o_dequant_r32(n_blk, qt["n_cb"], _ptr(dmin), _ptr(dmax), _ptr(cfg), _ptr(cof),
                           _ptr(hi), _ptr(lo), _ptr(data), _ptr(sc), _ptr(out))
    out_f, in_f = qt["shape"]
    return out.view(np.float16).reshape(out_f, qt["n_cb"] * 32)[:, :in_f]


def dequant_ggml(blocks: np.ndarray, contract: bool = True) -> np.ndarray:
    """R32-ggml (llama-cpp-sx8.patch:746-767) of (n_blk, 30) u8 block_sx8 records ->
    (n_blk, 32) float32, no PCA."""
    b = np.ascontiguousarray(blocks, dtype=np.uint8).reshape(-1, 30)
    out = np.empty((b.shape[0], 32), dtype=np.float32)
    lib().sx8o_dequant_ggml(b.shape[0], _ptr(b), int(bool(contract)), _ptr(out))
    return out


def core_f16(qt):
    """fp16 (out_f, in_f) operand tile values of the prefill GEMM (no PCA), C oracle.

    Pinned by closed forms (degenerate block -> dmin, level 0 -> rlo per strategy, signed
    zero), by ``core_exact_weight`` on fuzzed and quantized blocks, and by its distance
    to R64 without PCA (at most one fp16 ulp, rarely nonzero): tests/test_oracle.py."""
    n_blk, dmin, dmax, cfg, _, hi, lo = _fields(qt)
    out = np.empty(n_blk * 32, dtype=np.uint16)
    lib().sx8o_core_f16(n_blk, _ptr(dmin), _ptr(dmax), _ptr(cfg), _ptr(hi), _ptr(lo), _ptr(out))
    out_f, in_f = qt["shape"]
    return out.view(np.float16).reshape(out_f, qt["n_cb"] * 32)[:, :in_f]


def _rn32(fr: Fraction) -> Fraction:
    """Correctly rounded binary32 (round to nearest, ties to even) of an exact rational,
    subnormals included (the three float32 neighbours of the float64 approximation
    bracket the exact value)."""
    if fr == 0:
        return Fraction(0)
    x = np.float32(float(fr))
    cands = [np.nextafter(x, np.float32(-np.inf)), x, np.nextafter(x, np.float32(np.inf))]

    def key(c):
        return abs(Fraction(float(c)) - fr), int(np.array(c, dtype=np.float32).view(np.uint32)) & 1
    return Fraction(float(min(cands, key=key)))


def _rn16(fr: Fraction) -> np.float16:
    """Correctly rounded binary16 (RNE) of an exact rational, subnormals included."""
    if fr == 0:
        return np.float16(0.0)
    x = np.float16(float(fr))
    cands = [np.nextafter(x, np.float16(-np.inf)), x, np.nextafter(x, np.float16(np.inf))]

    def key(c):
        return abs(Fraction(float(c)) - fr), int(np.array(c, dtype=np.float16).view(np.uint16)) & 1
    return min(cands, key=key)


def core_exact_weight(dmin16, dmax16, cfg, lv, t, c_step=None, f32_store=False):
    """One operand value of ``core_f16`` from exact rationals: every binary32 operation
    rounded once, and the final multiply-add step*lv + rlo rounded once to fp16 (what the
    kernel's v_fma_mix does).  ``f32_store`` rounds it to binary32 first (the reference's
    float w then __float2half); ``c_step`` overrides the 0.015873 constant.  Tests use
    both knobs to show that the checks discriminate.  Finite endpoints only."""
    lo = Fraction(float(np.float16(dmin16)))
    hi = Fraction(float(np.float16(dmax16)))
    c = Fraction(float(np.float32(C_STEP))) if c_step is None else Fraction(c_step)
    d = _rn32(hi - lo)
    q = _rn32(d / 4)
    m = _rn32(d * c)
    s = (cfg >> ((t >> 3) * 2)) & 3
    k1 = (0, 0, 3, 1)[s]
    e = (0, 2, 2, 1)[s]
    rlo = _rn32(q * k1 + lo)
    step = m / (2 ** e) if d > 0 else Fraction(float(np.float32(STEP_FLOOR)))
    w = step * lv + rlo
    return _rn16(_rn32(w) if f32_store else w)


def dequant_r64_numpy(qt, bases_info):
    """Independent vectorised restatement of R64, unfused, in numpy float64.

    Written from the Numba typing rules rather than from the C code: strategy
    ranges via masked assignment, the float32 subtraction done in numpy float32.
    Returns (n_blk, 32) float16.
    """
    n_blk, dmin, dmax, cfg, cof, hi, lo = _fields(qt)
    data, sc = _bases(bases_info)
    n_cb = qt["n_cb"]
    lo_f = dmin.view(np.float16).astype(np.float32)
    hi_f = dmax.view(np.float16).astype(np.float32)
    q = (hi_f - lo_f).astype(np.float64) * 0.25
    lo64 = lo_f.astype(np.float64)[:, None]
    hi64 = hi_f.astype(np.float64)[:, None]
    q2 = q[:, None]
    sb = np.arange(32) >> 3
    strat = (cfg.astype(np.int64)[:, None] >> (2 * sb)[None, :]) & 3
    rlo = np.where(strat == 2, hi64 - q2, np.where(strat == 3, lo64 + q2, lo64))
    rhi = np.where(strat == 1, lo64 + q2, np.where(strat == 3, hi64 - q2, hi64))
    rlo = np.broadcast_to(rlo, (n_blk, 32))
    rhi = np.broadcast_to(rhi, (n_blk, 32))
    with np.errstate(invalid="ignore", over="ignore"):
        step = (rhi - rlo) * C_STEP
        step = np.where(step < STEP_FLOOR, STEP_FLOOR, step)
        lv = unpack_levels(hi, lo).astype(np.float64)
        w = rlo + step * lv
        c0 = (cof & 0xF).astype(np.int64)
        c0 = np.where(c0 < 8, c0, c0 - 16).astype(np.float64)
        c1 = ((cof >> 4) & 0xF).astype(np.int64)
        c1 = np.where(c1 < 8, c1, c1 - 16).astype(np.float64)
        kb = np.arange(n_blk) % n_cb
        bs = data.reshape(n_cb, 64)[kb].astype(np.float64)
        s2 = sc.reshape(n_cb, 2)[kb].astype(np.float64)
        w = w + ((1.0 * c0) * s2[:, 0])[:, None] * bs[:, :32]
        w = w + ((1.0 * c1) * s2[:, 1])[:, None] * bs[:, 32:]
        return w.astype(np.float32).astype(np.float16)


def _f64_round(fr: Fraction) -> float:
    return float(fr)   # int/int true division in CPython is correctly rounded


def dequant_r64_exact_weight(dmin16, dmax16, cfg, coeff, lv, t, s0, s1, b0, b1):
    """One weight of fused R64 from exact rationals (slow; spot checks only)."""
    lo_f = np.float32(np.float16(dmin16))
    hi_f = np.float32(np.float16(dmax16))
    d32 = np.float32(hi_f - lo_f)
    q = float(d32) * 0.25
    s = (cfg >> ((t >> 3) * 2)) & 3
    lo64, hi64 = float(lo_f), float(hi_f)
    if s == 0:
        rlo, rhi = lo64, hi64
    elif s == 1:
        rlo, rhi = lo64, lo64 + q
    elif s == 2:
        rlo, rhi = hi64 - q, hi64
    else:
        rlo, rhi = lo64 + q, hi64 - q
    step = (rhi - rlo) * C_STEP
    if step < STEP_FLOOR:
        step = STEP_FLOOR
    w = _f64_round(Fraction(step) * lv + Fraction(rlo))
    c0 = coeff & 0xF
    c0 = c0 if c0 < 8 else c0 - 16
    c1 = (coeff >> 4) & 0xF
    c1 = c1 if c1 < 8 else c1 - 16
    w = _f64_round(Fraction(w) + Fraction((1.0 * c0) * float(np.float32(s0))) * Fraction(float(np.float32(b0))))
    w = _f64_round(Fraction(w) + Fraction((1.0 * c1) * float(np.float32(s1))) * Fraction(float(np.float32(b1))))
    return np.float16(np.float32(w))


# ------------------------------------------------------------------- a4 / references

def z44(X: np.ndarray, bases_info) -> np.ndarray:
    """Z[m, kb, j] = scales[kb, j] * sum_t X[m, kb*32+t] * bases[kb, 32j+t] (float64),
    the PCA precompute of cuda/sx8_decode1_v3.cu:44-65 and cuda/sx8_gemm_compact.cu:28-50."""
    X = np.asarray(X, dtype=np.float64)
    if X.ndim == 1:
        X = X[None, :]
    n_cb = int(bases_info["n_cb"])
    Kp = n_cb * 32
    Xp = np.zeros((X.shape[0], Kp))
    Xp[:, :X.shape[1]] = X
    B = np.asarray(bases_info["data"], dtype=np.float64).reshape(n_cb, 2, 32)
    S = np.asarray(bases_info["scales"], dtype=np.float64).reshape(n_cb, 2)
    return np.einsum("mct,cjt->mcj", Xp.reshape(-1, n_cb, 32), B) * S[None]


def z44_f32_tree(X16: np.ndarray, bases_info) -> np.ndarray:
    """Z in float32 with the reference's exact summation order: products x_t * b_t,
    then the warp xor-tree over offsets 16, 8, 4, 2, 1 (cuda/sx8_decode1_v3.cu:53-63:
    lane 0 ends with ((p0+p16)+(p8+p24)) + ...), then scale * sum.  Returns (M, n_cb, 2)."""
    X = np.asarray(X16, dtype=np.float16)
    if X.ndim == 1:
        X = X[None, :]
    n_cb = int(bases_info["n_cb"])
    Xp = np.zeros((X.shape[0], n_cb * 32), dtype=np.float32)
    Xp[:, :X.shape[1]] = X.astype(np.float32)
    B = np.asarray(bases_info["data"], dtype=np.float32).reshape(n_cb, 2, 32)
    S = np.asarray(bases_info["scales"], dtype=np.float32).reshape(n_cb, 2)
    p = Xp.reshape(-1, n_cb, 1, 32) * B[None]                      # float32 products
    off = 16
    while off >= 1:
        p = p[..., :off] + p[..., off:2 * off]
        off //= 2
    return (S[None] * p[..., 0]).astype(np.float32)


def gemm_f64(X16: np.ndarray, W16: np.ndarray) -> np.ndarray:
    """Y = X . W^T with float64 accumulation over fp16 inputs (C oracle)."""
    X = np.ascontiguousarray(np.asarray(X16, dtype=np.float16).reshape(-1, np.shape(X16)[-1]))
    W = np.ascontiguousarray(np.asarray(W16, dtype=np.float16))
    M, K = X.shape
    N = W.shape[0]
    Y = np.empty((M, N), dtype=np.float64)
    lib().sx8o_gemm_f64(M, N, K, _ptr(X.view(np.uint16)), K, _ptr(W.view(np.uint16)),
                        W.shape[1], _ptr(Y))
    return Y


def rel_err(Y, Y_ref) -> float:
    """max|Y - Y_ref| / max|Y_ref|, the reference's metric (sx8_fused_wmma.py:132)."""
    Y = np.asarray(Y, dtype=np.float64)
    Y_ref = np.asarray(Y_ref, dtype=np.float64)
    return float(np.max(np.abs(Y - Y_ref)) / (np.max(np.abs(Y_ref)) + 1e-30))
