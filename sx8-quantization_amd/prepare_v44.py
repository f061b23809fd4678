"""Load-time transform of S-X8 v4.3 tensors to the kb-major v4.4 device layout.

Interface of scripts/prepare_v44.py (reference): ``to_v44``, ``extract_levels_v43``,
``extract_levels_v44``, ``decode_v44_numpy`` and ``verify``, plus ``to_v44_device``,
which builds the same bytes with torch on the GPU so that large tensors (lm_head:
12.2 M blocks) are laid out without a host round trip per field.

v4.4 layout, 30 bytes per block exactly, row order bid = kb*N + n:
  hdr    (n_blk, 6|8) u8 = dmin fp16 LE | dmax fp16 LE | config | coeff (| 2 zero bytes)
  levels (n_blk, 24)  u8 = per sub-block sb: hi nibbles at 4sb..4sb+3, lo quads at
                           16+2sb..17+2sb -- byte-identical to qh[0:16] || ql[0:8].
"""
from __future__ import annotations

import numpy as np


def _nmajor_fields(qt):
    out_f, _ = qt["shape"]
    n_cb = qt["n_cb"]
    n_blk = qt["n_blocks"]
    if n_blk != out_f * n_cb:
        raise ValueError(f"n_blocks {n_blk} != out_f*n_cb {out_f * n_cb}")
    hi = np.asarray(qt["levels_hi"], dtype=np.uint8).reshape(out_f, n_cb, 16)
    lo = np.asarray(qt["levels_lo"], dtype=np.uint8).reshape(out_f, n_cb, 8)
    dmin = np.asarray(qt["dmin"]).astype(np.float16).reshape(out_f, n_cb)
    dmax = np.asarray(qt["dmax"]).astype(np.float16).reshape(out_f, n_cb)
    config = np.asarray(qt["config"]).astype(np.uint8).reshape(out_f, n_cb)
    coeff = np.asarray(qt["coeff"]).astype(np.uint8).reshape(out_f, n_cb)
    return out_f, n_cb, hi, lo, dmin, dmax, config, coeff


def to_v44(qt, bases_info, hdr_aligned=False):
    """numpy v4.3 (n-major pkl arrays) -> dict(levels, hdr, n_cb, shape, bases, scales)."""
    out_f, n_cb, hi, lo, dmin, dmax, config, coeff = _nmajor_fields(qt)
    hb = 8 if hdr_aligned else 6
    hdr = np.zeros((n_cb, out_f, hb), dtype=np.uint8)
    hdr[:, :, 0:2] = dmin.T.copy().view(np.uint8).reshape(n_cb, out_f, 2)
    hdr[:, :, 2:4] = dmax.T.copy().view(np.uint8).reshape(n_cb, out_f, 2)
    hdr[:, :, 4] = config.T
    hdr[:, :, 5] = coeff.T
    levels = np.concatenate([hi, lo], axis=2).transpose(1, 0, 2)
    return {
        "levels": np.ascontiguousarray(levels).reshape(-1, 24),
        "hdr": hdr.reshape(-1, hb),
        "n_cb": n_cb,
        "shape": tuple(qt["shape"]),
        "bases": np.asarray(bases_info["data"], dtype=np.float32).reshape(-1, 64),
        "scales": np.asarray(bases_info["scales"], dtype=np.float32).reshape(-1, 2),
    }


def to_v44_device(qt, bases_info, hdr_aligned=False, device="cuda"):
    """Same bytes as ``to_v44`` built with torch on `device`.
    Returns (hdr (n_blk, 6|8) u8, levels (n_blk, 24) u8, bases (n_cb,64) f32,
    scales (n_cb,2) f32) as device tensors."""
    import torch
    out_f, _ = qt["shape"]
    n_cb = qt["n_cb"]
    hb = 8 if hdr_aligned else 6

    def dev(a, dt):
        return torch.from_numpy(np.ascontiguousarray(np.asarray(a).reshape(-1)).view(dt)).to(device)

    hi = dev(qt["levels_hi"], np.uint8).view(out_f, n_cb, 16)
    lo = dev(qt["levels_lo"], np.uint8).view(out_f, n_cb, 8)
    dmin = dev(np.asarray(qt["dmin"]).astype(np.float16), np.uint8).view(out_f, n_cb, 2)
    dmax = dev(np.asarray(qt["dmax"]).astype(np.float16), np.uint8).view(out_f, n_cb, 2)
    cfg = dev(np.asarray(qt["config"]).astype(np.uint8), np.uint8).view(out_f, n_cb, 1)
    cof = dev(np.asarray(qt["coeff"]).astype(np.uint8), np.uint8).view(out_f, n_cb, 1)
    parts = [dmin, dmax, cfg, cof]
    if hb == 8:
        parts.append(torch.zeros(out_f, n_cb, 2, dtype=torch.uint8, device=device))
    hdr = torch.cat(parts, dim=2).transpose(0, 1).contiguous().view(-1, hb)
    levels = torch.cat([hi, lo], dim=2).transpose(0, 1).contiguous().view(-1, 24)
    bases = torch.from_numpy(np.ascontiguousarray(
        np.asarray(bases_info["data"], dtype=np.float32).reshape(-1, 64))).to(device)
    scales = torch.from_numpy(np.ascontiguousarray(
        np.asarray(bases_info["scales"], dtype=np.float32).reshape(-1, 2))).to(device)
    return hdr, levels, bases, scales


def extract_levels_v43(qt):
    """The 32 six-bit levels per block from the v4.3 arrays (pkl order)."""
    n_blk = qt["n_blocks"]
    hi = np.asarray(qt["levels_hi"], dtype=np.uint8).reshape(n_blk, 16)
    lo = np.asarray(qt["levels_lo"], dtype=np.uint8).reshape(n_blk, 8)
    t = np.arange(32)
    nib = (hi[:, t >> 1] >> ((t & 1) * 4)) & 0xF
    qua = (lo[:, t >> 2] >> ((3 - (t & 3)) * 2)) & 0x3
    return ((nib << 2) | qua).astype(np.uint8)


def extract_levels_v44(v44):
    """The 32 levels per block from the v4.4 level records (kb-major order)."""
    lev = np.asarray(v44["levels"], dtype=np.uint8)
    t = np.arange(32)
    sb, i = t >> 3, t & 7
    nib = (lev[:, 4 * sb + (i >> 1)] >> ((i & 1) * 4)) & 0xF
    qua = (lev[:, 16 + 2 * sb + (i >> 2)] >> ((3 - (i & 3)) * 2)) & 0x3
    return ((nib << 2) | qua).astype(np.uint8)


def decode_v44_numpy(v44, X, n):
    """float64 value of output column n with PCA applied through Z0/Z1 (the contract
    of the GEMV kernel, prepare_v44.py:109-158), branchless float64 strategy."""
    out_f, _ = v44["shape"]
    n_cb = v44["n_cb"]
    X = np.asarray(X, dtype=np.float64)
    Xp = np.zeros(n_cb * 32)
    Xp[:X.shape[0]] = X
    bases = np.asarray(v44["bases"], dtype=np.float64).reshape(n_cb, 2, 32)
    scales = np.asarray(v44["scales"], dtype=np.float64).reshape(n_cb, 2)
    Z = np.einsum("ct,cjt->cj", Xp.reshape(n_cb, 32), bases) * scales
    lv = extract_levels_v44({"levels": np.asarray(v44["levels"])[np.arange(n_cb) * out_f + n]})
    hdr = np.asarray(v44["hdr"])[np.arange(n_cb) * out_f + n]
    lo = hdr[:, 0:2].copy().view(np.float16).astype(np.float64).reshape(-1)
    hi = hdr[:, 2:4].copy().view(np.float16).astype(np.float64).reshape(-1)
    cfg = hdr[:, 4].astype(np.int64)
    co = hdr[:, 5].astype(np.int64)
    q = (hi - lo) * 0.25
    acc = 0.0
    for sb in range(4):
        s = (cfg >> (2 * sb)) & 3
        rlo = lo + q * (3 * (s == 2) + (s == 3))
        rhi = hi - q * (3 * (s == 1) + (s == 3))
        step = np.maximum((rhi - rlo) * 0.015873, 1e-10)
        w = rlo[:, None] + step[:, None] * lv[:, 8 * sb:8 * sb + 8]
        acc += float(np.sum(w * Xp.reshape(n_cb, 32)[:, 8 * sb:8 * sb + 8]))
    c0 = np.where((co & 0xF) < 8, co & 0xF, (co & 0xF) - 16)
    c1 = np.where((co >> 4) < 8, co >> 4, (co >> 4) - 16)
    return acc + float(np.sum(c0 * Z[:, 0] + c1 * Z[:, 1]))


def verify(qt, bases_info, name=""):
    """Layout checks of prepare_v44.verify (:161-203): 30 B per block, level bijection,
    header bytes equal to the v4.3 fields.  Returns True when all pass."""
    v44 = to_v44(qt, bases_info)
    n_blk = qt["n_blocks"]
    ok = v44["levels"].nbytes + v44["hdr"].nbytes == n_blk * 30
    out_f, _ = qt["shape"]
    n_cb = qt["n_cb"]
    lv43 = extract_levels_v43(qt).reshape(out_f, n_cb, 32).transpose(1, 0, 2).reshape(-1, 32)
    ok &= bool(np.array_equal(lv43, extract_levels_v44(v44)))
    dmin = np.asarray(qt["dmin"]).astype(np.float16).reshape(out_f, n_cb).T.reshape(-1)
    ok &= bool(np.array_equal(v44["hdr"][:, 0:2].copy().view(np.float16).reshape(-1).view(np.uint16),
                              dmin.view(np.uint16)))
    return ok
