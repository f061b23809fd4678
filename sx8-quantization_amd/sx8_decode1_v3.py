"""M = 1 decode GEMV on the kb-major v4.4 layout (the decode path of SX8LinearV44).

Interface of scripts/sx8_decode1_v3.py (reference): ``_ext()`` (an object with
``compute_z44``, ``decode1_v44`` and ``decode1_v44_combined``), ``make_tensors_v44``,
``best_split_k``, the ``_BUF``/``_buf`` output pools and ``decode1_v44``.
The CUDA extension is replaced by libsx8_hip.so (sx8_compute_z / sx8_gemv).  The GEMV is
one launch: every work-group builds the per-K-block activation table (x pairs, sums, Z)
in LDS while its first weight records stream in.  The combined form, which hands Z back
with the reference's summation tree, puts a small table kernel in front.
``decode1_v44_group`` (no counterpart upstream) runs the GEMVs of up to four weights that
share x -- q/k/v, gate/up -- as one launch.
"""
from __future__ import annotations

import ctypes

import torch

import _sx8lib as _L

DEV = torch.device("cuda")
# K blocks up to which sx8_gemv builds its activation table in LDS (single launch, no
# workspace); beyond it the table goes through the caller's workspace
_LDS_MAX_KB = 640


def _x_for_kernel(X, n_cb):
    """fp16 (K,) activation as the kernel needs it: contiguous, 16-byte aligned and
    zero-padded to n_cb*32 values (the reference read past K instead)."""
    Xc = X.reshape(-1).contiguous().half()
    Kp = n_cb * 32
    if Xc.numel() < Kp or Xc.data_ptr() % 16:
        Xp = torch.zeros(Kp, dtype=torch.float16, device=Xc.device)
        Xp[:min(Kp, Xc.numel())] = Xc[:Kp]
        Xc = Xp
    return Xc


def _workspace(n_cb, device):
    """Table workspace of sx8_gemv's two-launch forms (112 bytes per K block), fresh from
    torch's caching allocator on the current stream: stream-ordered and capture-safe."""
    n = (int(_L.lib().sx8_gemv_workspace_bytes(n_cb)) + 3) // 4
    return torch.empty(max(n, 4), dtype=torch.float32, device=device)


class _Ext:
    """Drop-in for the reference's load_inline module (sx8_decode1_v3.py:33-54)."""

    @staticmethod
    def compute_z44(X, basis, scales, n_cb, out=None):
        n_cb = int(n_cb)
        Xc = _x_for_kernel(X, n_cb)
        if out is None:
            out = torch.empty(n_cb, 2, dtype=torch.float32, device=Xc.device)
        _L.call("sx8_compute_z", _L.ptr(Xc), 1, n_cb * 32, _L.ptr(basis.contiguous()),
                _L.ptr(scales.contiguous()), n_cb, _L.ptr(out), _L.stream(Xc.device))
        return out

    @staticmethod
    def decode1_v44(X, hdr, levels, Z, n_cb, hdr_bytes, split_k=1, out=None):
        """GEMV with a precomputed Z; split_k is accepted and ignored (as upstream)."""
        n_cb = int(n_cb)
        N = hdr.size(0) // n_cb
        Xc = _x_for_kernel(X, n_cb)
        if out is None:
            out = torch.empty(N, dtype=torch.float32, device=Xc.device)
        ws = _workspace(n_cb, Xc.device)
        _L.call("sx8_gemv", _L.ptr(Xc), _L.ptr(hdr), _L.ptr(levels), int(hdr_bytes), None, None,
                _L.ptr(Z.contiguous()), None, N, n_cb, _L.ptr(out), _L.ptr(ws), ws.numel() * 4,
                _L.stream(Xc.device))
        return out

    @staticmethod
    def decode1_v44_combined(X, hdr, levels, basis, scales, n_cb, hdr_bytes, Z, out):
        n_cb = int(n_cb)
        N = hdr.size(0) // n_cb
        Xc = _x_for_kernel(X, n_cb)
        ws = _workspace(n_cb, Xc.device)
        _L.call("sx8_gemv", _L.ptr(Xc), _L.ptr(hdr), _L.ptr(levels), int(hdr_bytes),
                _L.ptr(basis.contiguous()), _L.ptr(scales.contiguous()), None, _L.ptr(Z), N,
                n_cb, _L.ptr(out), _L.ptr(ws), ws.numel() * 4, _L.stream(Xc.device))
        return out


_cached = None


def _ext():
    global _cached
    if _cached is None:
        _L.lib()          # fail loudly here if the HIP library is missing
        _cached = _Ext()
    return _cached


def make_tensors_v44(qt, bases_info, hdr_aligned=False):
    """v4.4 kb-major tensors on the current device: hdr (n_blk, 6|8) u8,
    levels (n_blk, 24) u8, bases (n_cb, 64) f32, scales (n_cb, 2) f32."""
    from prepare_v44 import to_v44_device
    return to_v44_device(qt, bases_info, hdr_aligned=hdr_aligned, device=DEV)


def best_split_k(N, n_cb):
    """The reference's split heuristic (sx8_decode1_v3.py:69-77).  Its result is
    accepted by decode1_v44 and ignored, as upstream; the HIP GEMV picks its own
    K split from the shape and the CU count."""
    n_blocks = (N + 63) // 64
    want = 540
    sk = max(1, (want + n_blocks - 1) // n_blocks)
    return min(sk, 16)


_BUF = {}


def _buf(key, shape):
    """Pooled float32 device buffer per key on the current device.  (The reference's
    check `b.device != DEV` compared cuda:0 with cuda and so reallocated on every call;
    here the pool is reused as its comment intended.)"""
    dev = torch.device("cuda", torch.cuda.current_device())
    b = _BUF.get((key, dev.index))
    if b is None or b.shape != tuple(shape):
        b = torch.empty(*shape, dtype=torch.float32, device=dev)
        _BUF[(key, dev.index)] = b
    return b


def decode1_v44(X, qt, bases_info, hdr_t=None, lvl_t=None, bas_t=None, sca_t=None,
                hdr_bytes=6, split_k=1):
    """Y = W . X for X (K,) fp16 -> (Y float32 (N,), (hdr_t, lvl_t, bas_t, sca_t)).
    Y is a pooled buffer keyed by N: the next call with the same N overwrites it."""
    if hdr_t is None:
        hdr_t, lvl_t, bas_t, sca_t = make_tensors_v44(qt, bases_info,
                                                      hdr_aligned=(hdr_bytes == 8))
    n_cb = qt["n_cb"]
    N = qt["shape"][0]
    _ext()
    Y = _buf(("Y", N), (N,))
    # The reference passes a pooled Z scratch to decode1_v44_combined; nothing reads it
    # afterwards, so the Z output is skipped here, which lets the HIP GEMV build its
    # activation table inside the single launch.
    Xc = _x_for_kernel(X, n_cb)
    ws = _workspace(n_cb, Xc.device) if n_cb > _LDS_MAX_KB else None
    _L.call("sx8_gemv", _L.ptr(Xc), _L.ptr(hdr_t), _L.ptr(lvl_t), int(hdr_bytes), _L.ptr(bas_t),
            _L.ptr(sca_t), None, None, N, n_cb, _L.ptr(Y), _L.ptr(ws), 0 if ws is None else ws.numel() * 4,
            _L.stream(Xc.device))
    return Y, (hdr_t, lvl_t, bas_t, sca_t)


def decode1_v44_group(X, tensors, Ns, n_cb, hdr_bytes=6, outs=None):
    """Y_i = W_i . X for up to four v4.4 weights with the same K, in one launch.
    tensors: [(hdr_t, lvl_t, bas_t, sca_t), ...]; Ns: output widths; outs: optional
    float32 (N_i,) outputs.  Returns the list of outputs.  Each Y_i equals what
    decode1_v44 gives for W_i (same panel decode; only the work split differs)."""
    n = len(tensors)
    Xc = _x_for_kernel(X, int(n_cb))
    if outs is None:
        outs = [torch.empty(int(N), dtype=torch.float32, device=Xc.device) for N in Ns]
    P = ctypes.c_void_p * n
    keep = [(t[2].contiguous(), t[3].contiguous()) for t in tensors]   # alive for the call
    hdrs = P(*[t[0].data_ptr() for t in tensors])
    lvls = P(*[t[1].data_ptr() for t in tensors])
    bas = P(*[k[0].data_ptr() for k in keep])
    sca = P(*[k[1].data_ptr() for k in keep])
    ys = P(*[y.data_ptr() for y in outs])
    ns = (ctypes.c_int64 * n)(*[int(N) for N in Ns])
    ws = _workspace(int(n_cb), Xc.device) if int(n_cb) > _LDS_MAX_KB else None
    _L.call("sx8_gemv_group", _L.ptr(Xc), n, hdrs, lvls, int(hdr_bytes), bas, sca, None, ns,
            int(n_cb), ys, _L.ptr(ws), 0 if ws is None else ws.numel() * 4, _L.stream(Xc.device))
    return outs
