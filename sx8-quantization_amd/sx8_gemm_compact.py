"""Prefill GEMM on the kb-major v4.4 layout (the M > 1 path of SX8LinearV44).

Interface of scripts/sx8_gemm_compact.py (reference): ``_ext()`` (an object with
``compute_z44_batch`` and ``gemm_compact``) and ``gemm_sx8_compact``.

``gemm_sx8_compact`` runs sx8_gemm_prefill: Z is computed inside the call, the core
weights rlo + step*lv (float32 range parameters, the multiply-add rounded once to fp16)
feed v_mfma_f32_32x32x16_f16, and the PCA term rides along as extra MFMA k-steps over Z.
``_ext().gemm_compact`` keeps the reference's caller-supplied-Z contract with the same
kernel (sx8_gemm_prefill_z).  The library allocates nothing: each call takes its
workspace (Z, packed X, split-K partials) from torch's caching allocator on the current
stream, the way the reference's wrappers allocate their outputs.
"""
from __future__ import annotations

import torch

import _sx8lib as _L


def _x2d(X, K=None):
    """Row-major fp16 (M, K) view usable by the kernels (contiguous rows)."""
    Xc = X.contiguous()
    if Xc.dtype != torch.float16:
        Xc = Xc.half()
    if Xc.dim() != 2:
        raise ValueError(f"X must be 2-D (M, K), got shape {tuple(X.shape)}")
    return Xc


class _Ext:
    """Drop-in for the reference's load_inline module (sx8_gemm_compact.py:24-39)."""

    @staticmethod
    def compute_z44_batch(X, basis, scales, n_cb):
        n_cb = int(n_cb)
        Xc = _x2d(X)
        M, K = Xc.shape
        if K < n_cb * 32:
            Xp = torch.zeros((M, n_cb * 32), dtype=torch.float16, device=Xc.device)
            Xp[:, :K] = Xc
            Xc = Xp
        Z = torch.empty((M, n_cb, 2), dtype=torch.float32, device=Xc.device)
        _L.call("sx8_compute_z", _L.ptr(Xc), M, Xc.shape[1], _L.ptr(basis.contiguous()),
                _L.ptr(scales.contiguous()), n_cb, _L.ptr(Z), _L.stream(Xc.device))
        return Z

    @staticmethod
    def gemm_compact(X, hdr, levels, Z, n_cb, hdr_bytes):
        n_cb = int(n_cb)
        Xc = _x2d(X)
        M, K = Xc.shape
        N = hdr.size(0) // n_cb
        Kc = min(K, n_cb * 32)
        Y = torch.empty((M, N), dtype=torch.float32, device=Xc.device)
        Zc = Z.contiguous().float()
        if Zc.numel() != M * n_cb * 2:
            raise ValueError(f"Z must hold (M, n_cb, 2) = ({M}, {n_cb}, 2) values")
        ws, nb = _L.gemm_workspace(M, (N,), n_cb, Xc.device)
        _L.call("sx8_gemm_prefill_z", _L.ptr(Xc), M, K, Kc, _L.ptr(hdr), _L.ptr(levels),
                int(hdr_bytes), _L.ptr(Zc), N, n_cb, _L.ptr(Y), _L.ptr(ws), nb, _L.stream(Xc.device))
        return Y


_cached = None


def _ext():
    global _cached
    if _cached is None:
        _L.lib()
        _cached = _Ext()
    return _cached


def gemm_sx8_compact(X, qt, bases_info, hdr_t=None, lvl_t=None, bas_t=None, sca_t=None,
                     hdr_bytes=6, in_f=None, n_cb=None):
    """Y = X @ W^T for X (M, K) fp16 CUDA -> Y (M, N) float32 CUDA (a fresh tensor).

    As upstream, a weight with fewer than 64 output rows is dequantized whole and
    multiplied with torch (F.linear in fp16, then .float()); K shorter than n_cb*32 is
    handled inside the kernel (the reference zero-padded X)."""
    if in_f is None:
        in_f = qt["shape"][1]
    if n_cb is None:
        n_cb = qt["n_cb"]
    out_f = qt["shape"][0]
    if out_f < 64:
        from kernel_sx8_v43 import decode_tensor_gpu_fast
        W = decode_tensor_gpu_fast(qt, bases_info).reshape(out_f, in_f)
        return torch.nn.functional.linear(X.contiguous(), W).float()
    if hdr_t is None:
        from sx8_decode1_v3 import make_tensors_v44
        hdr_t, lvl_t, bas_t, sca_t = make_tensors_v44(qt, bases_info,
                                                      hdr_aligned=(hdr_bytes == 8))
    Xc = _x2d(X)
    M, K = Xc.shape
    if K < in_f:
        raise ValueError(f"X has {K} columns, weight needs {in_f}")
    Y = torch.empty((M, out_f), dtype=torch.float32, device=Xc.device)
    ws, nb = _L.gemm_workspace(M, (out_f,), int(n_cb), Xc.device)
    _L.call("sx8_gemm_prefill", _L.ptr(Xc), M, K, int(in_f), _L.ptr(hdr_t), _L.ptr(lvl_t),
            int(hdr_bytes), _L.ptr(bas_t), _L.ptr(sca_t), out_f, int(n_cb), _L.ptr(Y), _L.ptr(ws), nb,
            _L.stream(Xc.device))
    return Y
