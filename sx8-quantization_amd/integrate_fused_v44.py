"""nn.Module integration of the S-X8 kernels (the caller of the hot path).

Interface of scripts/integrate_fused_v44.py (reference): ``SX8LinearV44`` and
``clone_model_fused_v44``.  Dispatch follows integrate_fused_v44.py:43-77:
  * M == 1                -> decode1_v44 (HIP GEMV, kb-major v4.4 tensors);
  * M > 1                 -> gemm_sx8_compact (HIP MFMA prefill on the same tensors),
                             or gemm_sx8_wmma_cached on kb-major split arrays when
                             SX8_USE_WMMA=1;
  * output                -> y.half() (+ bias), reshaped to (*x.shape[:-1], out_f).
Embeddings are replaced by SX8EmbeddingV44.
"""
from __future__ import annotations

import os

import torch
import torch.nn as nn

from sx8_decode1_v3 import decode1_v44, best_split_k, make_tensors_v44
from sx8_embed_v44 import SX8EmbeddingV44
from sx8_fused_wmma import gemm_sx8_wmma_cached, make_tensors, to_kbmajor
from sx8_gemm_compact import gemm_sx8_compact

DEV = torch.device("cuda")


class SX8LinearV44(nn.Module):
    """nn.Linear whose weight is an S-X8 tensor (device tensors built lazily)."""

    def __init__(self, qt, bases_info, bias=None, out_f=None, in_f=None, hdr_bytes=6):
        super().__init__()
        self.qt = qt
        self.bases_info = bases_info
        self.bias = bias
        self.out_f = out_f if out_f is not None else qt["shape"][0]
        self.in_f = in_f if in_f is not None else qt["shape"][1]
        self.hdr_bytes = hdr_bytes
        self._t44 = None
        self._tensors = None

    def _load_t44(self):
        if self._t44 is None:
            self._t44 = make_tensors_v44(self.qt, self.bases_info,
                                         hdr_aligned=(self.hdr_bytes == 8))

    def forward(self, x):
        x = x.contiguous()
        orig_shape = x.shape
        if x.dim() != 2:
            x = x.reshape(-1, x.shape[-1])
        M = x.shape[0]
        if M == 1:
            self._load_t44()
            hdr_t, lvl_t, bas_t, sca_t = self._t44
            split_k = best_split_k(self.out_f, self.qt["n_cb"])
            y, _ = decode1_v44(x[0], self.qt, self.bases_info, hdr_t, lvl_t, bas_t, sca_t,
                               self.hdr_bytes, split_k)
            y = y.unsqueeze(0)
        elif os.environ.get("SX8_USE_WMMA") == "1":
            if self._tensors is None:
                kbm, _ = to_kbmajor(self.qt, self.bases_info)
                self._tensors = make_tensors(kbm, self.bases_info, x.device)
            y = gemm_sx8_wmma_cached(x, self._tensors, self.qt["n_cb"])
        else:
            self._load_t44()
            hdr_t, lvl_t, bas_t, sca_t = self._t44
            y = gemm_sx8_compact(x, self.qt, self.bases_info, hdr_t, lvl_t, bas_t, sca_t,
                                 self.hdr_bytes)
        y = y.half()
        if self.bias is not None:
            y = y + self.bias
        return y.reshape(*orig_shape[:-1], self.out_f)


def clone_model_fused_v44(model, wd, bd, hdr_bytes=6, t44=None):
    """Replace, in place, every nn.Linear / nn.Embedding whose parameter name is in
    ``wd`` by SX8LinearV44 / SX8EmbeddingV44.  Returns (model, n_replaced).
    ``t44`` (optional, not in the reference): {name: (hdr, levels, bases, scales)} device
    tensors already in the v4.4 layout, e.g. from sx8_container_v43.load_v44; the
    replaced modules use them instead of building their own."""
    n_replaced = 0
    for name, p in list(model.named_parameters()):
        if name not in wd or p.dim() < 2:
            continue
        qt, bi = wd[name], bd[name]
        parts = name.split(".")
        parent = model
        for part in parts[:-2]:
            parent = parent[int(part)] if part.isdigit() else getattr(parent, part)
        attr = parts[-2]
        mod = getattr(parent, attr)
        pre = t44.get(name) if t44 is not None else None
        if isinstance(mod, nn.Embedding):
            emb = SX8EmbeddingV44(qt, bi, hdr_bytes=6)
            if pre is not None and pre[0].shape[1] == 6:
                emb._t = pre
                emb._hdr, emb._lvl, emb._bas, emb._sca = pre
                emb.qt = emb.bases_info = None
            setattr(parent, attr, emb)
            n_replaced += 1
            continue
        if not isinstance(mod, nn.Linear):
            continue
        new = SX8LinearV44(qt, bi, mod.bias, mod.out_features, mod.in_features,
                           hdr_bytes=hdr_bytes)
        if pre is not None and pre[0].shape[1] == hdr_bytes:
            new._t44 = pre
        setattr(parent, attr, new)
        del mod.weight
        n_replaced += 1
    if torch.cuda.is_available():
        torch.cuda.empty_cache()
    return model, n_replaced
