"""End-to-end decoder stack on S-X8 weights: prefill, then greedy decode replayed from a
HIP graph (the caller role of scripts/infer_sx8.py:109-173 and the CUDA-graph decode
of results/fase4_v44_velocidad.json:70-80).

A Qwen3-style dense decoder (RMSNorm, q/k RMSNorm per head, RoPE, GQA attention with
a KV cache, SwiGLU MLP, tied S-X8 embedding / lm_head).  Every linear weight is an
SX8LinearV44 (M = 1 -> the HIP decode GEMV, M > 1 -> the HIP prefill GEMM), the token
embedding is an SX8EmbeddingV44 (HIP row gather); norms stay fp16.  The ops between
the S-X8 kernels (norms, RoPE, attention over the cache, SiLU) are plain torch ops.

Decode is graph-friendly: the step reads the current token and position from device
tensors, writes the KV cache at that position with index_copy_, masks the unused cache
tail, and writes the next token (argmax) and position back, so one captured step can be
replayed for every generated token.
"""
from __future__ import annotations

import ctypes
import math
import time

import torch
import torch.nn as nn

import _sx8lib as _L
from integrate_fused_v44 import SX8LinearV44
from prepare_v44 import to_v44_device
from quantize_sx8 import quantize_tensor
from sx8_embed_v44 import SX8EmbeddingV44

QWEN3_4B = dict(hidden=2560, n_layers=36, n_heads=32, n_kv=8, head_dim=128,
                inter=9728, vocab=151936, rope_theta=1.0e6, eps=1e-6)


def _rms(x, w, eps):
    xf = x.float()
    return (xf * torch.rsqrt(xf.pow(2).mean(-1, keepdim=True) + eps) * w.float()).half()


def sx8_linear(out_f, in_f, gen, device, std=0.02, degenerate_frac=0.0):
    """A random N(0, std) weight quantized to S-X8 on `device`, as an SX8LinearV44 with
    its v4.4 device tensors already built."""
    W = (torch.randn(out_f, in_f, generator=gen, device=device) * std).half()
    qt, bi = quantize_tensor(W, device=device, degenerate_frac=degenerate_frac,
                             seed=int(torch.randint(0, 1 << 30, (1,), generator=gen, device=device)))
    lin = SX8LinearV44(qt, bi, None, out_f, in_f, hdr_bytes=6)
    lin._t44 = to_v44_device(qt, bi, hdr_aligned=False, device=device)
    return lin


def clone_linear(lin):
    """Same values in new device memory (so every layer streams its own bytes)."""
    new = SX8LinearV44(lin.qt, lin.bases_info, None, lin.out_f, lin.in_f, hdr_bytes=6)
    new._t44 = tuple(t.clone() for t in lin._t44)
    return new


def pair_storage(a, b):
    """Move the device tensors of `a` and `b` into one allocation per field, b's right after
    a's (both keep views of it): sx8_dec_gemv_rmsnorm_pair reads a matrix pair through the
    first matrix's pointers and refuses a pair stored apart."""
    ta, tb = [], []
    for x, y in zip(a._t44, b._t44):
        buf = torch.cat([x.reshape(-1), y.reshape(-1)])
        ta.append(buf[:x.numel()].view(x.shape))
        tb.append(buf[x.numel():].view(y.shape))
    a._t44, b._t44 = tuple(ta), tuple(tb)


class Layer(nn.Module):
    def __init__(self, cfg, lins, device):
        super().__init__()
        H, hd = cfg["hidden"], cfg["head_dim"]
        self.q, self.k, self.v, self.o, self.gate, self.up, self.down = lins
        self.in_norm = torch.ones(H, dtype=torch.float16, device=device)
        self.post_norm = torch.ones(H, dtype=torch.float16, device=device)
        self.q_norm = torch.ones(hd, dtype=torch.float16, device=device)
        self.k_norm = torch.ones(hd, dtype=torch.float16, device=device)


class SX8Decoder(nn.Module):
    """Random-init decoder.  `n_distinct` layers get their own random weights; layer i
    reuses the values of layer i % n_distinct in its own device memory."""

    def __init__(self, cfg=QWEN3_4B, device=None, seed=0, n_distinct=None, max_len=1024,
                 log=None):
        super().__init__()
        self.cfg = cfg = dict(cfg)
        device = torch.device(device or "cuda")
        self.device = device
        gen = torch.Generator(device=device)
        gen.manual_seed(seed)
        H, nh, nk, hd, I = cfg["hidden"], cfg["n_heads"], cfg["n_kv"], cfg["head_dim"], cfg["inter"]
        L = cfg["n_layers"]
        n_distinct = L if n_distinct is None else max(1, min(n_distinct, L))
        t0 = time.time()
        base = []
        for i in range(n_distinct):
            base.append([sx8_linear(nh * hd, H, gen, device), sx8_linear(nk * hd, H, gen, device),
                         sx8_linear(nk * hd, H, gen, device), sx8_linear(H, nh * hd, gen, device),
                         sx8_linear(I, H, gen, device), sx8_linear(I, H, gen, device),
                         sx8_linear(H, I, gen, device)])
            if log:
                log(f"e2e: quantized layer {i} ({time.time() - t0:.1f}s)")
        layers = []
        for i in range(L):
            src = base[i % n_distinct]
            lins = src if i < n_distinct else [clone_linear(l) for l in src]
            layers.append(Layer(cfg, lins, device))
            pair_storage(layers[-1].gate, layers[-1].up)
        self.layers = layers
        self.head = sx8_linear(cfg["vocab"], H, gen, device)      # tied lm_head / embedding
        self.embed = SX8EmbeddingV44(self.head.qt, self.head.bases_info, hdr_bytes=6)
        self.embed._t = self.head._t44                              # share the device tensors
        self.embed._hdr, self.embed._lvl, self.embed._bas, self.embed._sca = self.head._t44
        self.final_norm = torch.ones(H, dtype=torch.float16, device=device)
        if log:
            log(f"e2e: quantized lm_head {cfg['vocab']}x{H} ({time.time() - t0:.1f}s)")
        # RoPE tables (neox halves) and the KV cache
        inv = 1.0 / (cfg["rope_theta"] ** (torch.arange(0, hd, 2, device=device).float() / hd))
        pos = torch.arange(max_len, device=device).float()
        ang = torch.outer(pos, inv)
        self.cos, self.sin = ang.cos(), ang.sin()                   # (max_len, hd / 2)
        self.max_len = max_len
        self.k_cache = [torch.zeros(nk, max_len, hd, dtype=torch.float16, device=device) for _ in range(L)]
        self.v_cache = [torch.zeros(nk, max_len, hd, dtype=torch.float16, device=device) for _ in range(L)]
        self.arange = torch.arange(max_len, device=device)

    # ---------------------------------------------------------------- helpers
    def _rope(self, x, cos, sin):
        """x (T, heads, hd) fp16; cos/sin (T, hd / 2) fp32."""
        h = x.shape[-1] // 2
        xf = x.float()
        x1, x2 = xf[..., :h], xf[..., h:]
        c, s = cos[:, None, :], sin[:, None, :]
        return torch.cat([x1 * c - x2 * s, x2 * c + x1 * s], dim=-1).half()

    def _mlp(self, ly, x):
        h = _rms(x, ly.post_norm, self.cfg["eps"])
        g = ly.gate(h)
        u = ly.up(h)
        return ly.down((torch.nn.functional.silu(g.float()) * u.float()).half())

    # ---------------------------------------------------------------- prefill
    @torch.no_grad()
    def prefill(self, ids):
        """ids (T,) int64 on the device -> next token (1,) int64; fills the KV cache."""
        cfg = self.cfg
        nh, nk, hd, eps = cfg["n_heads"], cfg["n_kv"], cfg["head_dim"], cfg["eps"]
        T = ids.shape[0]
        x = self.embed(ids)                                        # (T, H) fp16
        cos, sin = self.cos[:T], self.sin[:T]
        for li, ly in enumerate(self.layers):
            h = _rms(x, ly.in_norm, eps)
            q = _rms(ly.q(h).view(T, nh, hd), ly.q_norm, eps)
            k = _rms(ly.k(h).view(T, nk, hd), ly.k_norm, eps)
            v = ly.v(h).view(T, nk, hd)
            q, k = self._rope(q, cos, sin), self._rope(k, cos, sin)
            self.k_cache[li][:, :T, :] = k.permute(1, 0, 2)
            self.v_cache[li][:, :T, :] = v.permute(1, 0, 2)
            rep = nh // nk
            qf = q.permute(1, 0, 2).float().contiguous()                       # (nh, T, hd)
            kf = k.permute(1, 0, 2).float().repeat_interleave(rep, 0).contiguous()
            vf = v.permute(1, 0, 2).float().repeat_interleave(rep, 0).contiguous()
            a = torch.nn.functional.scaled_dot_product_attention(qf[None], kf[None], vf[None],
                                                                 is_causal=True)[0]
            x = x + ly.o(a.permute(1, 0, 2).reshape(T, nh * hd).half())
            x = x + self._mlp(ly, x)
        logits = self.head(_rms(x[-1:], self.final_norm, eps))
        return logits.float().argmax(-1)

    def _prefill_bufs(self, T):
        """Activation buffers of prefill_fused for T tokens (built once per T)."""
        pb = getattr(self, "_pb", None)
        if pb is not None and pb["T"] == T:
            return pb
        cfg, dev = self.cfg, self.device
        H, nh, nk, hd, I = cfg["hidden"], cfg["n_heads"], cfg["n_kv"], cfg["head_dim"], cfg["inter"]
        f32 = dict(dtype=torch.float32, device=dev)
        f16 = dict(dtype=torch.float16, device=dev)
        pb = {"T": T, "resid": torch.empty(T, H, **f32), "h": torch.empty(T, H, **f16),
              "q": torch.empty(T, nh * hd, **f32), "k": torch.empty(T, nk * hd, **f32),
              "v": torch.empty(T, nk * hd, **f32), "qh": torch.empty(T, nh, hd, **f16),
              # the attention output as the o projection's packed GEMM operands
              "xp": torch.empty((T + 31) // 32 * (nh * hd // 32) * 1024, dtype=torch.int16, device=dev),
              "zhl": torch.empty(T * (nh * hd // 32) * 4, dtype=torch.int16, device=dev),
              # the normalized rows as the q/k/v or gate/up GEMM's packed operands (one packed X,
              # up to four Zhl; each consumed by its GEMM before the next norm writes them)
              "xn": torch.empty((T + 31) // 32 * (H // 32) * 1024, dtype=torch.int16, device=dev),
              "zn": [torch.empty(T * (H // 32) * 4, dtype=torch.int16, device=dev) for _ in range(3)],
              # x = fp16(silu(g) u) as the down projection's packed GEMM operands
              "xpd": torch.empty((T + 31) // 32 * ((I + 31) // 32) * 1024, dtype=torch.int16, device=dev),
              "zhld": torch.empty(T * ((I + 31) // 32) * 4, dtype=torch.int16, device=dev),
              "o": torch.empty(T, H, **f32),
              "d": torch.empty(T, H, **f32),
              "pos0": torch.zeros(1, dtype=torch.int64, device=dev),
              "logits": torch.empty(cfg["vocab"], **f32), "tok": torch.zeros(1, dtype=torch.int64, device=dev),
              "scratch_pos": torch.zeros(1, dtype=torch.int64, device=dev)}
        pb["head_group"] = self._group_args((self.head,), (pb["logits"],))
        # one prefill workspace for every GEMM of the pass (the calls run in stream order),
        # sized for the largest of them
        ly0 = self.layers[0]
        need = max(int(_L.lib().sx8_gemm_prefill_workspace_bytes(T, len(Ns), (ctypes.c_int64 * len(Ns))(*Ns),
                                                                 n_cb))
                   for Ns, n_cb in (((ly0.q.out_f, ly0.k.out_f, ly0.v.out_f), ly0.q.qt["n_cb"]),
                                    ((ly0.o.out_f,), ly0.o.qt["n_cb"]),
                                    ((ly0.gate.out_f, ly0.up.out_f), ly0.gate.qt["n_cb"]),
                                    ((ly0.down.out_f,), ly0.down.qt["n_cb"])))
        need = max(need, int(_L.lib().sx8_dec_gemm_gateup_silu_workspace_bytes(T, I, ly0.gate.qt["n_cb"])))
        pb["ws"] = torch.empty(need, dtype=torch.uint8, device=dev)
        pb["groups"] = [(self._group_args((ly.q, ly.k, ly.v), (pb["q"], pb["k"], pb["v"])),
                         self._group_args((ly.gate, ly.up), ()),         # (no float32 outputs)
                         self._group_args((ly.o,), (pb["o"],)),
                         self._group_args((ly.down,), (pb["d"],))) for ly in self.layers]
        self._pb = pb
        return pb

    @staticmethod
    def _gemm_group(args, X, ws, st):
        """The prefill GEMMs of matrices sharing X (sx8_gemm_prefill_group), outputs (M, N_i)."""
        n, hdrs, lvls, bas, sca, ns, n_cb, ys = args
        M, K = X.shape
        _L.call("sx8_gemm_prefill_group", _L.ptr(X), M, K, K, n, hdrs, lvls, 6, bas, sca, ns, n_cb, ys,
                _L.ptr(ws), ws.numel(), st)

    @staticmethod
    def _gemm_group_deferred(args, X, ws, st):
        """_gemm_group with the split-K sum left to the consumer
        (sx8_gemm_prefill_group_deferred): returns (parts, n_parts, slice), n_parts = 0 when
        the outputs are complete."""
        n, hdrs, lvls, bas, sca, ns, n_cb, ys = args
        M, K = X.shape
        parts, n_parts, slc = ctypes.c_void_p(), ctypes.c_int32(), ctypes.c_int64()
        _L.call("sx8_gemm_prefill_group_deferred", _L.ptr(X), M, K, K, n, hdrs, lvls, 6, bas, sca, ns, n_cb, ys,
                _L.ptr(ws), ws.numel(), ctypes.addressof(parts), ctypes.addressof(n_parts), ctypes.addressof(slc),
                st)
        return parts.value, n_parts.value, slc.value

    @staticmethod
    def _gemm_packed(args, Xp, Zhls, M, K, ws, st, defer=True):
        """The prefill GEMMs of `args` on the packed X and the Zhl per matrix their producer
        wrote (sx8_gemm_prefill_packed); with defer the split-K sum is left to the consumer and
        (parts, n_parts, slice) is returned, else the outputs are complete."""
        n, hdrs, lvls, bas, sca, ns, n_cb, ys = args
        parts, n_parts, slc = ctypes.c_void_p(), ctypes.c_int32(), ctypes.c_int64()
        outs = (ctypes.addressof(parts), ctypes.addressof(n_parts), ctypes.addressof(slc)) if defer else (None,) * 3
        _L.call("sx8_gemm_prefill_packed", _L.ptr(Xp), (ctypes.c_void_p * n)(*[z.data_ptr() for z in Zhls[:n]]), M,
                K, n, hdrs, lvls, 6, ns, n_cb, ys, _L.ptr(ws), ws.numel(), *outs, st)
        return (parts.value, n_parts.value, slc.value) if defer else (None, 0, 0)

    @staticmethod
    def _norm_packed(pb, args, resid, delta, init, w, parts, eps, st):
        """add + RMSNorm of the T rows written as the packed GEMM operands of the matrices
        of `args` (sx8_dec_add_rmsnorm_packed into pb's xn / zn)."""
        n, hdrs, lvls, bas, sca, ns, n_cb, ys = args
        T, H = resid.shape
        P = _L.ptr
        _L.call("sx8_dec_add_rmsnorm_packed", P(resid), P(delta) if delta is not None else None,
                P(init) if init is not None else None, P(w), T, H, eps, parts[0], parts[1], parts[2], n, bas, sca,
                P(pb["xn"]), (ctypes.c_void_p * n)(*[z.data_ptr() for z in pb["zn"][:n]]), st)

    @staticmethod
    def _gemm(lin, X, Y, ws, st):
        """Y (M, N) f32 = X (M, K) fp16 . W^T through sx8_gemm_prefill."""
        hdr, lvl, bas, sca = lin._t44
        M, K = X.shape
        _L.call("sx8_gemm_prefill", _L.ptr(X), M, K, K, _L.ptr(hdr), _L.ptr(lvl), 6, _L.ptr(bas),
                _L.ptr(sca), lin.out_f, lin.qt["n_cb"], _L.ptr(Y), _L.ptr(ws), ws.numel(), st)

    @torch.no_grad()
    def prefill_fused(self, ids, all_logits=False):
        """prefill() with the library ops over the T prompt rows: add + RMSNorm written
        as the next GEMM's packed operands (sx8_dec_add_rmsnorm_packed, M = T), the prefill
        GEMMs on producer-written operands (sx8_gemm_prefill_packed), q/k
        norm + RoPE + KV-cache write (sx8_dec_qk_rope_cache_rows), causal attention over
        the cache rows writing the o projection's packed GEMM operands
        (sx8_dec_attn_prefill_packed, sx8_gemm_prefill_packed), the gate/up GEMM writing
        fp16(SiLU(g) * u) as the down projection's packed operands
        (sx8_dec_gemm_gateup_silu) and the final norm inside the lm_head GEMV.  The split-K sums
        of the q/k/v, o and down GEMMs (all but the last layer's) are added by the kernels
        that read those outputs (the *_deferred GEMM calls and the *_parts consumers), the
        same sums in the same order.  The residual stream is float32.  Returns the next token (1,); generation only needs the last
        row's logits, so that is all the lm_head computes.  all_logits=True instead runs
        the final norm over every row and the lm_head as a prefill GEMM (M = T), as a
        Hugging Face forward does (scripts/integrate_fused_v44.py:119-167 compares those
        logits), and returns the (T, vocab) float32 logits."""
        cfg = self.cfg
        H, nh, nk, hd, eps = cfg["hidden"], cfg["n_heads"], cfg["n_kv"], cfg["head_dim"], cfg["eps"]
        T = ids.shape[0]
        pb = self._prefill_bufs(T)
        st = _L.stream(self.device)
        P = _L.ptr
        emb = self.embed(ids)                                      # (T, H) fp16
        # split-K sums are left to the kernel that reads the GEMM output (the *_deferred
        # calls and the *_parts consumers; the same sums in the same order): q/k/v into the
        # RoPE pass, o into the second add + RMSNorm, down into the next layer's first
        pend = (None, 0, 0)                                        # down's, for the next layer
        last = len(self.layers) - 1
        for li, ly in enumerate(self.layers):
            # add + RMSNorm written as the q/k/v GEMM's packed operands (no pass over its rows)
            if li == 0:
                self._norm_packed(pb, pb["groups"][li][0], pb["resid"], None, emb, ly.in_norm, (None, 0, 0), eps, st)
            else:
                self._norm_packed(pb, pb["groups"][li][0], pb["resid"], pb["d"], None, ly.in_norm, pend, eps, st)
            qp = self._gemm_packed(pb["groups"][li][0], pb["xn"], pb["zn"], T, H, pb["ws"], st)     # q, k, v
            _L.call("sx8_dec_qk_rope_cache_rows_parts", P(pb["q"]), P(pb["k"]), P(pb["v"]), P(ly.q_norm),
                    P(ly.k_norm), P(self.cos), P(self.sin), P(pb["pos0"]), T, P(pb["qh"]),
                    P(self.k_cache[li]), P(self.v_cache[li]), nh, nk, hd, self.max_len, eps, qp[0], qp[1], qp[2],
                    st)
            # attention writes the o projection's packed X and Zhl itself (no pass over its output)
            _, _, obas, osca = ly.o._t44
            _L.call("sx8_dec_attn_prefill_packed", P(pb["qh"]), P(self.k_cache[li]), P(self.v_cache[li]), T, 0, nh,
                    nk, hd, self.max_len, 1.0 / math.sqrt(hd), P(obas), P(osca), P(pb["xp"]), P(pb["zhl"]), st)
            op = self._gemm_packed(pb["groups"][li][2], pb["xp"], [pb["zhl"]], T, nh * hd, pb["ws"], st)
            self._norm_packed(pb, pb["groups"][li][1], pb["resid"], pb["o"], None, ly.post_norm, op, eps, st)
            # gate/up GEMM ending in x = fp16(silu(g) u) as the down projection's packed operands
            _, hdrs, lvls, bas, sca, _, gcb, _ = pb["groups"][li][1]
            _, _, dbas, dsca = ly.down._t44
            _L.call("sx8_dec_gemm_gateup_silu", None, P(pb["xn"]), (ctypes.c_void_p * 2)(*[z.data_ptr() for z in pb["zn"][:2]]),
                    T, H, hdrs, lvls, 6, bas, sca, cfg["inter"], gcb, P(dbas), P(dsca), P(pb["xpd"]), P(pb["zhld"]),
                    P(pb["ws"]), pb["ws"].numel(), st)
            # down; the last layer's output feeds the final norm and the lm_head whole
            pend = self._gemm_packed(pb["groups"][li][3], pb["xpd"], [pb["zhld"]], T, cfg["inter"], pb["ws"], st,
                                     defer=li < last)
        if all_logits:
            # every row: residual + down output, final norm, lm_head GEMM over T rows
            _L.call("sx8_dec_add_rmsnorm", P(pb["resid"]), P(pb["d"]), None, P(self.final_norm), P(pb["h"]),
                    T, H, eps, st)
            logits = torch.empty(T, cfg["vocab"], dtype=torch.float32, device=self.device)
            ws, nb = _L.gemm_workspace(T, (cfg["vocab"],), self.head.qt["n_cb"], self.device)
            self._gemm(self.head, pb["h"], logits, ws, st)
            return logits
        # last row: residual + down output, final norm and lm_head in one launch
        self._gemv_rms(pb["head_group"], pb["resid"][T - 1], None, pb["d"][T - 1], self.final_norm, None,
                       eps, st)
        _L.call("sx8_dec_argmax_advance", P(pb["logits"]), cfg["vocab"], P(pb["tok"]), P(pb["scratch_pos"]), st)
        return pb["tok"].clone()

    # ---------------------------------------------------------------- decode
    @torch.no_grad()
    def decode_step(self, tok, pos):
        """One greedy step: tok (1,) int64, pos (1,) int64 device tensors (the position
        the token is written at).  Updates tok and pos in place; no host sync."""
        cfg = self.cfg
        nh, nk, hd, eps = cfg["n_heads"], cfg["n_kv"], cfg["head_dim"], cfg["eps"]
        rep = nh // nk
        x = self.embed(tok)                                        # (1, H)
        cos, sin = self.cos.index_select(0, pos), self.sin.index_select(0, pos)
        mask = torch.where(self.arange <= pos, 0.0, float("-inf"))            # (max_len,)
        scale = 1.0 / math.sqrt(hd)
        for li, ly in enumerate(self.layers):
            h = _rms(x, ly.in_norm, eps)
            q = _rms(ly.q(h).view(1, nh, hd), ly.q_norm, eps)
            k = _rms(ly.k(h).view(1, nk, hd), ly.k_norm, eps)
            v = ly.v(h).view(1, nk, hd)
            q, k = self._rope(q, cos, sin), self._rope(k, cos, sin)
            self.k_cache[li].index_copy_(1, pos, k.view(nk, 1, hd))
            self.v_cache[li].index_copy_(1, pos, v.view(nk, 1, hd))
            qt = q.view(nk, rep, hd).transpose(1, 2).contiguous()               # (nk, hd, rep)
            s = torch.matmul(self.k_cache[li], qt).transpose(1, 2).float() * scale + mask
            p = torch.softmax(s, dim=-1).half()                                 # (nk, rep, L)
            a = torch.matmul(p, self.v_cache[li])                                # (nk, rep, hd)
            x = x + ly.o(a.reshape(1, nh * hd))
            x = x + self._mlp(ly, x)
        logits = self.head(_rms(x, self.final_norm, eps))
        tok.copy_(logits.float().argmax(-1))
        pos.add_(1)
        return tok

    # ---------------------------------------------------------------- fused decode
    def _fused_setup(self):
        """Buffers and ctypes argument lists of the fused decode step (built once)."""
        if getattr(self, "_fz", None) is not None:
            return self._fz
        cfg, dev = self.cfg, self.device
        H, nh, nk, hd, I, V = (cfg["hidden"], cfg["n_heads"], cfg["n_kv"], cfg["head_dim"],
                               cfg["inter"], cfg["vocab"])
        f32 = dict(dtype=torch.float32, device=dev)
        f16 = dict(dtype=torch.float16, device=dev)
        z = {"ra": torch.zeros(H, **f32),
             "q": torch.zeros(nh * hd, **f32), "k": torch.zeros(nk * hd, **f32),
             "v": torch.zeros(nk * hd, **f32), "a": torch.zeros(nh * hd, **f16),
             "logits": torch.zeros(V, **f32)}
        # the MLP in two launches: m = silu(W_gate x) * W_up x and the down projection's
        # partial PCA sums zp from the gate/up pair, then the down GEMV from m and zp
        z["m"] = torch.zeros(I, **f16)
        z["zp"] = torch.zeros(I // 32, 2, 2, **f32)
        z["attn_ws"] = torch.zeros(int(_L.lib().sx8_dec_attn_workspace_bytes(nh, hd)) // 4 + 64, **f32)
        # grouped GEMV arguments (q/k/v and gate/up share their input): ctypes arrays of
        # device pointers, built once per layer; the o and down GEMVs add their output to
        # the residual stream ra in place
        z["groups"] = []
        for ly in self.layers:
            z["groups"].append((self._group_args((ly.q, ly.k, ly.v), (z["q"], z["k"], z["v"])),
                                self._group_args((ly.o,), (z["ra"],))))
        z["resid_adds"] = (ctypes.c_void_p * 1)(z["ra"].data_ptr())
        z["head_group"] = self._group_args((self.head,), (z["logits"],))
        # per-work-group argmax partials of the lm_head GEMV
        nb = int(_L.lib().sx8_dec_argmax_parts_bytes(V, self.head.qt["n_cb"]))
        z["head_parts"] = torch.zeros(max(nb, 8) // 4, dtype=torch.int32, device=dev)
        self._fz = z
        return z

    @staticmethod
    def _group_args(lins, ys):
        n = len(lins)
        P = ctypes.c_void_p * n
        return (n, P(*[l._t44[0].data_ptr() for l in lins]), P(*[l._t44[1].data_ptr() for l in lins]),
                P(*[l._t44[2].data_ptr() for l in lins]), P(*[l._t44[3].data_ptr() for l in lins]),
                (ctypes.c_int64 * n)(*[l.out_f for l in lins]), lins[0].qt["n_cb"],
                P(*[y.data_ptr() for y in ys]) if ys else None)

    @staticmethod
    def _gemv_rms(args, resid, init, delta, w, resid_out, eps, st):
        """GEMVs of `args` on RMSNorm((init or resid) + delta) * w, the sum to resid_out."""
        n, hdrs, lvls, bas, sca, ns, n_cb, ys = args
        P = _L.ptr
        _L.call("sx8_dec_gemv_rmsnorm", P(resid) if resid is not None else None,
                P(init) if init is not None else None, P(delta) if delta is not None else None,
                P(w), eps, P(resid_out) if resid_out is not None else None, n, hdrs, lvls, 6, bas,
                sca, ns, n_cb, ys, st)

    def _mlp_fused(self, ly, r, eps, st):
        """r += W_down (silu(W_gate x) * W_up x), x = RMSNorm(r) * post_norm, in two launches."""
        z, P = self._fz, _L.ptr
        gh, gl, gb, gs = ly.gate._t44
        uh, ul, ub, us = ly.up._t44
        dh, dl, db, ds = ly.down._t44
        _L.call("sx8_dec_gemv_rmsnorm_pair", P(r), P(ly.post_norm), eps, P(gh), P(gl), 6, P(gb), P(gs),
                P(uh), P(ul), P(ub), P(us), ly.gate.out_f, ly.gate.qt["n_cb"], P(db), P(z["m"]), P(z["zp"]), st)
        _L.call("sx8_dec_gemv_zp_add", P(z["m"]), P(dh), P(dl), 6, P(z["zp"]), P(ds), ly.down.out_f,
                ly.down.qt["n_cb"], P(r), P(r), st)

    @staticmethod
    def _gemv_add(args, x, adds, st):
        """Ys = adds + W x."""
        n, hdrs, lvls, bas, sca, ns, n_cb, ys = args
        _L.call("sx8_dec_gemv_add", _L.ptr(x), n, hdrs, lvls, 6, bas, sca, ns, n_cb, adds, ys, st)

    @torch.no_grad()
    def decode_step_fused(self, tok, pos):
        """decode_step with the per-token ops as single HIP launches (sx8_decoder.h) and the
        GEMVs called through the C ABI; the residual stream is float32.  Each RMSNorm runs
        inside the GEMV that consumes it (sx8_dec_gemv_rmsnorm: q/k/v, lm_head;
        sx8_dec_gemv_rmsnorm_pair: gate/up, whose epilogue also forms silu(g) * u and the
        down projection's PCA sums), and both residual adds inside the GEMVs that produce
        them (sx8_dec_gemv_add for o, sx8_dec_gemv_zp_add for down: the stream ra is
        updated in place); q/k norm + RoPE + KV-cache write inside attention
        (sx8_dec_attn_rope): per layer one launch each for q/k/v, attention (two: chunks,
        combine), o, gate/up and down."""
        cfg = self.cfg
        nh, nk, hd, eps = cfg["n_heads"], cfg["n_kv"], cfg["head_dim"], cfg["eps"]
        z = self._fused_setup()
        st = _L.stream(self.device)
        P = _L.ptr
        emb = self.embed(tok)                                       # (1, H) fp16
        L = self.max_len
        r, adds = z["ra"], z["resid_adds"]
        for li, ly in enumerate(self.layers):
            g_qkv, g_o = z["groups"][li]
            if li == 0:                                             # h = embedding row -> r
                self._gemv_rms(g_qkv, None, emb, None, ly.in_norm, r, eps, st)
            else:                                                   # h = r
                self._gemv_rms(g_qkv, r, None, None, ly.in_norm, None, eps, st)
            # q/k norm + RoPE + KV-cache write inside the attention pass
            _L.call("sx8_dec_attn_rope", P(z["q"]), P(z["k"]), P(z["v"]), P(ly.q_norm), P(ly.k_norm),
                    P(self.cos), P(self.sin), P(pos), P(self.k_cache[li]), P(self.v_cache[li]),
                    P(z["a"]), nh, nk, hd, L, 1.0 / math.sqrt(hd), eps, P(z["attn_ws"]),
                    z["attn_ws"].numel() * 4, st)
            self._gemv_add(g_o, z["a"], adds, st)                   # r += W_o a
            self._mlp_fused(ly, r, eps, st)                         # r += W_down silu(g) u
        # final norm + lm_head GEMV, whose work-groups leave argmax partials; argmax + pos += 1
        hh, hl, hb, hs = self.head._t44
        _L.call("sx8_dec_gemv_rmsnorm_argmax", P(r), P(self.final_norm), eps, P(hh), P(hl), 6, P(hb), P(hs),
                cfg["vocab"], self.head.qt["n_cb"], P(z["logits"]), P(z["head_parts"]),
                z["head_parts"].numel() * 4, P(tok), P(pos), st)
        return tok

    # ---------------------------------------------------------------- generation
    @torch.no_grad()
    def generate(self, ids, n_new, use_graph=True, fused=True, return_logits=False):
        """Prefill `ids`, then greedily decode `n_new` tokens.  Returns (tokens (n_new,)
        on the device, prefill seconds, decode seconds); with return_logits (fused path
        only) also the (n_new, vocab) float32 logits each token was picked from: row 0 the
        prefill's last row, row i the i-th decode step's (copied after each step, outside
        the timed figures' meaning: the copies add to the decode time)."""
        dev = self.device
        T = ids.shape[0]
        assert T + n_new <= self.max_len
        if return_logits and not fused:
            raise ValueError("return_logits needs the fused path")
        lg = torch.empty(n_new, self.cfg["vocab"], dtype=torch.float32, device=dev) if return_logits else None
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        first = self.prefill_fused(ids) if fused else self.prefill(ids)
        torch.cuda.synchronize()
        t_prefill = time.perf_counter() - t0
        if lg is not None:
            lg[0].copy_(self._pb["logits"])
        tok = first.clone()
        pos = torch.full((1,), T, dtype=torch.int64, device=dev)
        out = torch.empty(n_new, dtype=torch.int64, device=dev)
        out[0] = first[0]
        step = self.decode_step_fused if fused else self.decode_step
        if use_graph:
            # warm-up (pools, workspaces) on a side stream, then capture one step
            saved = (tok.clone(), pos.clone())
            s = torch.cuda.Stream()
            s.wait_stream(torch.cuda.current_stream())
            with torch.cuda.stream(s):
                step(tok, pos)
            torch.cuda.current_stream().wait_stream(s)
            tok.copy_(saved[0])
            pos.copy_(saved[1])
            g = torch.cuda.CUDAGraph()
            with torch.cuda.graph(g):
                step(tok, pos)
            tok.copy_(saved[0])
            pos.copy_(saved[1])
            torch.cuda.synchronize()
            t1 = time.perf_counter()
            for i in range(1, n_new):
                g.replay()
                out[i:i + 1].copy_(tok)
                if lg is not None:
                    lg[i].copy_(self._fz["logits"])
            torch.cuda.synchronize()
            t_decode = time.perf_counter() - t1
        else:
            torch.cuda.synchronize()
            t1 = time.perf_counter()
            for i in range(1, n_new):
                step(tok, pos)
                out[i:i + 1].copy_(tok)
                if lg is not None:
                    lg[i].copy_(self._fz["logits"])
            torch.cuda.synchronize()
            t_decode = time.perf_counter() - t1
        if lg is not None:
            return out, t_prefill, t_decode, lg
        return out, t_prefill, t_decode
