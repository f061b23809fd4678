"""Prefill GEMM from kb-major split arrays (the reference's fused WMMA contract).

Interface of scripts/sx8_fused_wmma.py (reference): ``_get_module()`` (an object with
``fused_forward``), ``make_tensors``, ``gemm_sx8_wmma_cached``, ``gemm_sx8_wmma`` and
``decode1_sx8_cached``; ``to_kbmajor`` restates scripts/kernel_sx8_fused.py:20-41,
which builds the kb-major dict these functions consume.

The kernel behind it is the same MFMA prefill as gemm_sx8_compact (sx8_gemm_prefill_
split): the PCA-free core weights rlo + step*lv with the reference's float32 range
parameters, each multiply-add rounded once to fp16, as v_mfma_f32_32x32x16_f16 operands;
PCA added through Z as extra k-steps.  Like the reference's WMMA tiles (cuda/sx8_fused_wmma.cu:70-97) these
operands are not the canonical R64 weights; the product meets the 1e-3 bar.
``make_tensors`` no longer builds the rlo/step fp16 tables of precompute_rlo_step.py: no
kernel here reads them.
"""
from __future__ import annotations

import numpy as np
import torch

import _sx8lib as _L


def to_kbmajor(qt, bases_info):
    """pkl (n-major) arrays -> kb-major dict {dmin, dmax, config, coeff, levels_hi,
    levels_lo} with bid' = kb*N + n (as integrate_fused.SX8Linear._kbm)."""
    N = qt["shape"][0]
    n_cb = qt["n_cb"]

    def reorder(a, per_block):
        a = np.asarray(a)
        if per_block == 1:
            return np.ascontiguousarray(a.reshape(N, n_cb).T.reshape(-1))
        return np.ascontiguousarray(a.reshape(N, n_cb, per_block).transpose(1, 0, 2).reshape(-1))

    kbm = {
        "dmin": reorder(np.asarray(qt["dmin"]).astype(np.float16), 1),
        "dmax": reorder(np.asarray(qt["dmax"]).astype(np.float16), 1),
        "config": reorder(np.asarray(qt["config"]).astype(np.uint8), 1),
        "coeff": reorder(np.asarray(qt["coeff"]).reshape(-1).astype(np.uint8), 1),
        "levels_hi": reorder(np.asarray(qt["levels_hi"]).astype(np.uint8), 16),
        "levels_lo": reorder(np.asarray(qt["levels_lo"]).astype(np.uint8), 8),
    }
    return kbm, bases_info


class _Module:
    @staticmethod
    def fused_forward(X, dmin, dmax, config, coeff, hi, lo, basis, scales, n_cb):
        n_cb = int(n_cb)
        Xc = X.contiguous().half()
        M, K = Xc.shape
        N = dmin.numel() // n_cb
        Y = torch.empty((M, N), dtype=torch.float32, device=Xc.device)
        ws, nb = _L.gemm_workspace(M, (N,), n_cb, Xc.device)
        _L.call("sx8_gemm_prefill_split", _L.ptr(Xc), M, K, min(K, n_cb * 32),
                _L.ptr(dmin), _L.ptr(dmax), _L.ptr(config), _L.ptr(coeff), _L.ptr(hi),
                _L.ptr(lo), _L.ptr(basis), _L.ptr(scales), N, n_cb, _L.ptr(Y), _L.ptr(ws), nb,
                _L.stream(Xc.device))
        return Y


_module = None


def _get_module():
    global _module
    if _module is None:
        _L.lib()
        _module = _Module()
    return _module


def make_tensors(qt_kbmajor, bases_info, device):
    """Device tensors of the kb-major metadata (created once and cached by callers)."""
    return {
        "dmin": _L.as_device(qt_kbmajor["dmin"], np.uint16, device),
        "dmax": _L.as_device(qt_kbmajor["dmax"], np.uint16, device),
        "config": _L.as_device(qt_kbmajor["config"], np.uint8, device),
        "coeff": _L.as_device(qt_kbmajor["coeff"], np.uint8, device),
        "hi": _L.as_device(qt_kbmajor["levels_hi"], np.uint8, device),
        "lo": _L.as_device(qt_kbmajor["levels_lo"], np.uint8, device),
        "basis": _L.as_device(bases_info["data"], np.float32, device),
        "scales": _L.as_device(bases_info["scales"], np.float32, device),
    }


def gemm_sx8_wmma_cached(X, tensors, n_cb):
    """Y = X @ W^T with cached device tensors.  X (M, K) fp16 -> Y (M, N) float32."""
    return _get_module().fused_forward(X.contiguous(), tensors["dmin"], tensors["dmax"],
                                       tensors["config"], tensors["coeff"], tensors["hi"],
                                       tensors["lo"], tensors["basis"], tensors["scales"],
                                       int(n_cb))


def gemm_sx8_wmma(X, qt_kbmajor, bases_info, n_cb):
    return gemm_sx8_wmma_cached(X, make_tensors(qt_kbmajor, bases_info, X.device), n_cb)


def decode1_sx8_cached(X, tensors, n_cb):
    """M = 1 product from the same tensors: X (K,) fp16 -> Y (N,) float32."""
    return gemm_sx8_wmma_cached(X.reshape(1, -1), tensors, n_cb).reshape(-1)
