"""The per-token decoder ops of include/sx8_decoder.h on the GPU against float32 torch
references (the same math as the decode loop of scripts/infer_sx8.py:109-173)."""
import ctypes
import math

import numpy as np
import pytest

pytestmark = pytest.mark.gpu


def _attn_ref(q, kc, vc, pos, nh, nk, hd, scale):
    import torch
    n = pos + 1
    G = nh // nk
    out = torch.empty(nh, hd)
    for h in range(nh):
        K = kc[h // G, :n].float()
        V = vc[h // G, :n].float()
        s = (K @ q[h].float()) * scale
        out[h] = torch.softmax(s, 0) @ V
    return out


@pytest.mark.parametrize("nh,nk,hd,L,positions", [
    (32, 8, 128, 1024, [0, 1, 31, 32, 33, 700, 1023]),   # the decoder's shape (G = 4)
    (16, 16, 64, 300, [0, 5, 299]),                      # G = 1
    (8, 1, 64, 4096, [4095, 100]),                       # G = 8, longest cache of sx8_dec_attn
    (4, 2, 128, 6000, [5999, 4097, 64]),                 # G = 2, past sx8_dec_attn's limit
])
def test_decode_attention_split_and_single(hiplib, cuda, nh, nk, hd, L, positions):
    import torch
    import _sx8lib as _L
    g = torch.Generator().manual_seed(nh * 7 + hd)
    q = torch.randn(nh, hd, generator=g).half()
    kc = torch.randn(nk, L, hd, generator=g).half()
    vc = torch.randn(nk, L, hd, generator=g).half()
    qd, kd, vd = q.to(cuda), kc.to(cuda), vc.to(cuda)
    ws = torch.zeros(int(_L.lib().sx8_dec_attn_workspace_bytes(nh, hd)) // 4 + 16, device=cuda)
    scale = 1.0 / math.sqrt(hd)
    P = _L.ptr
    for pos in positions:
        print("attn", nh, nk, hd, L, pos, flush=True)
        pt = torch.tensor([pos], dtype=torch.int64, device=cuda)
        o1 = torch.empty(nh, hd, dtype=torch.float16, device=cuda)
        o2 = torch.empty_like(o1)
        if L <= 4096:
            _L.call("sx8_dec_attn", P(qd), P(kd), P(vd), P(pt), P(o1), nh, nk, hd, L, scale, _L.stream(cuda))
        _L.call("sx8_dec_attn_split", P(qd), P(kd), P(vd), P(pt), P(o2), nh, nk, hd, L, scale, P(ws),
                ws.numel() * 4, _L.stream(cuda))
        ref = _attn_ref(q, kc, vc, pos, nh, nk, hd, scale)
        for o in ((o1, o2) if L <= 4096 else (o2,)):
            err = (o.cpu().float() - ref).abs().max().item()
            assert err <= 2e-3 * max(1.0, ref.abs().max().item()), (pos, err)


@pytest.mark.parametrize("nh,nk,hd,L,T,start", [
    (32, 8, 128, 1024, 512, 0),     # the decoder's prompt pass (G = 4)
    (32, 8, 128, 1024, 77, 100),    # ragged tile, keys already in the cache before the prompt
    (4, 2, 64, 64, 12, 0),          # the tiny e2e decoder (G = 2)
    (16, 16, 64, 300, 33, 0),       # G = 1
    (8, 1, 128, 200, 70, 3),        # G = 8
    (8, 2, 64, 96, 64, 31),         # G = 4 at hd 64, start one short of a block
    (32, 8, 128, 64, 1, 0),         # one row
    (32, 8, 128, 128, 1, 77),       # one row after 77 cached positions
    (2, 1, 128, 160, 40, 5),        # G = 2 at hd 128
    (8, 8, 128, 256, 100, 0),       # G = 1 at hd 128
    (32, 8, 128, 1200, 1100, 50),   # G = 4 on a grid of 280 work-groups (four heads per group)
])
def test_prefill_attention(hiplib, cuda, nh, nk, hd, L, T, start):
    """sx8_dec_attn_prefill against float32 causal attention; cache rows past start + T
    hold NaN, which must never reach the output."""
    import torch
    import _sx8lib as _L
    g = torch.Generator().manual_seed(nh * 13 + T + start)
    q = torch.randn(T, nh, hd, generator=g).half()
    kc = torch.full((nk, L, hd), float("nan")).half()
    vc = torch.full((nk, L, hd), float("nan")).half()
    kc[:, :start + T] = torch.randn(nk, start + T, hd, generator=g).half()
    vc[:, :start + T] = torch.randn(nk, start + T, hd, generator=g).half()
    scale = 1.0 / math.sqrt(hd)
    out = torch.empty(T, nh * hd, dtype=torch.float16, device=cuda)
    qd, kd, vd = q.to(cuda), kc.to(cuda), vc.to(cuda)
    print("attn_prefill", nh, nk, hd, L, T, start, flush=True)
    _L.call("sx8_dec_attn_prefill", _L.ptr(qd), _L.ptr(kd), _L.ptr(vd), _L.ptr(out), T, start, nh, nk, hd, L,
            scale, _L.stream(cuda))
    G = nh // nk
    n = start + T
    mask = torch.arange(n)[None, :] > (start + torch.arange(T))[:, None]
    ref = torch.empty(T, nh, hd)
    for h in range(nh):
        s = (q[:, h].float() @ kc[h // G, :n].float().T) * scale
        s = s.masked_fill(mask, float("-inf"))
        ref[:, h] = torch.softmax(s, -1) @ vc[h // G, :n].float()
    got = out.cpu().float().view(T, nh, hd)
    assert torch.isfinite(got).all()
    err = (got - ref).abs().max().item()
    assert err <= 3e-3 * max(1.0, ref.abs().max().item()), err


def test_prefill_attention_rejects_bad_arguments(hiplib, cuda):
    import torch
    import _sx8lib as _L
    t = torch.zeros(4096, dtype=torch.float16, device=cuda)
    P = _L.ptr
    with pytest.raises(RuntimeError, match="bad shape"):      # start + T > L
        _L.call("sx8_dec_attn_prefill", P(t), P(t), P(t), P(t), 8, 1, 4, 2, 64, 8, 0.125, _L.stream(cuda))
    with pytest.raises(RuntimeError, match="bad shape"):      # 16 * G > hd
        _L.call("sx8_dec_attn_prefill", P(t), P(t), P(t), P(t), 8, 0, 8, 1, 64, 8, 0.125, _L.stream(cuda))


def test_attention_split_rejects_bad_arguments(hiplib, cuda):
    import torch
    import _sx8lib as _L
    t = torch.zeros(64, dtype=torch.float16, device=cuda)
    pt = torch.zeros(1, dtype=torch.int64, device=cuda)
    P = _L.ptr
    with pytest.raises(RuntimeError, match="workspace"):
        _L.call("sx8_dec_attn_split", P(t), P(t), P(t), P(pt), P(t), 4, 1, 64, 16, 1.0, P(t), 4, _L.stream(cuda))
    with pytest.raises(RuntimeError, match="bad shape"):
        _L.call("sx8_dec_attn_split", P(t), P(t), P(t), P(pt), P(t), 12, 4, 64, 16, 1.0, P(t), 1 << 20,
                _L.stream(cuda))                                  # nh / nk = 3


def test_add_rmsnorm_and_silu_mul(hiplib, cuda):
    import torch
    import _sx8lib as _L
    P = _L.ptr
    g = torch.Generator().manual_seed(3)
    H = 2560
    resid = torch.randn(1, H, generator=g)
    delta = torch.randn(1, H, generator=g)
    w = (torch.rand(H, generator=g) + 0.5).half()
    rd, dd, wd = resid.to(cuda), delta.to(cuda), w.to(cuda)
    out = torch.empty(1, H, dtype=torch.float16, device=cuda)
    _L.call("sx8_dec_add_rmsnorm", P(rd), P(dd), None, P(wd), P(out), 1, H, 1e-6, _L.stream(cuda))
    x = resid + delta
    ref = x * torch.rsqrt((x * x).mean(-1, keepdim=True) + 1e-6) * w.float()
    assert torch.allclose(rd.cpu(), x, atol=0, rtol=0)
    assert (out.cpu().float() - ref).abs().max().item() <= 2e-3 * ref.abs().max().item()
    a = torch.randn(9728, generator=g)
    b = torch.randn(9728, generator=g)
    ad, bd = a.to(cuda), b.to(cuda)      # held: a temporary's memory could be reused at once
    o = torch.empty(9728, dtype=torch.float16, device=cuda)
    _L.call("sx8_dec_silu_mul", P(ad), P(bd), P(o), 9728, _L.stream(cuda))
    refm = torch.nn.functional.silu(a) * b
    assert (o.cpu().float() - refm).abs().max().item() <= 2e-3 * refm.abs().max().item()


@pytest.mark.parametrize("M,H,use_init,use_delta,shift", [
    (3, 2560, True, True, 0),     # four-wide loads, residual from the fp16 embedding rows
    (2, 4096, False, True, 0),    # four-wide, the longest such row
    (2, 2562, True, False, 0),    # H % 4 != 0: one value per load
    (2, 2560, False, True, 1),    # a residual one float past 16-byte alignment
    (2, 2560, True, False, 0),    # four-wide, the fp16 rows alone
    (3, 1024, False, False, 0),   # four-wide, the residual alone
    (2, 5000, True, True, 0),     # longer than the unrolled forms hold
    (1, 7, False, False, 0),      # a row shorter than a wave
])
def test_add_rmsnorm_forms(hiplib, cuda, M, H, use_init, use_delta, shift):
    """sx8_dec_add_rmsnorm in each of its load forms against float32 torch: resid written
    back exactly (init, when given, replacing resid before delta is added) and the fp16
    normed rows within half-precision rounding."""
    import torch
    import _sx8lib as _L
    P = _L.ptr
    g = torch.Generator().manual_seed(M * H + shift)
    resid = torch.randn(M, H, generator=g)
    delta = torch.randn(M, H, generator=g)
    init = torch.randn(M, H, generator=g).half()
    w = (torch.rand(H, generator=g) + 0.5).half()
    rbuf = torch.zeros(M * H + shift, device=cuda)
    rbuf[shift:] = resid.flatten().to(cuda)
    rd = rbuf[shift:]
    dd, idd, wd = delta.to(cuda), init.to(cuda), w.to(cuda)
    out = torch.empty(M, H, dtype=torch.float16, device=cuda)
    print("add_rmsnorm", M, H, use_init, use_delta, shift, flush=True)
    _L.call("sx8_dec_add_rmsnorm", P(rd), P(dd) if use_delta else None, P(idd) if use_init else None, P(wd),
            P(out), M, H, 1e-6, _L.stream(cuda))
    x = init.float() if use_init else resid.clone()
    if use_delta:
        x = x + delta
    ref = x * torch.rsqrt((x * x).mean(-1, keepdim=True) + 1e-6) * w.float()
    assert torch.equal(rd.cpu().view(M, H), x)
    assert bool(((out.cpu().float() - ref).abs() <= 2.0 ** -9 * ref.abs() + 1e-4).all())


def _group(lins_t, Ns, n_cb, ys):
    import ctypes
    n = len(lins_t)
    P = ctypes.c_void_p * n
    return (n, P(*[t[0].data_ptr() for t in lins_t]), P(*[t[1].data_ptr() for t in lins_t]),
            P(*[t[2].data_ptr() for t in lins_t]), P(*[t[3].data_ptr() for t in lins_t]),
            (ctypes.c_int64 * n)(*Ns), n_cb, P(*[y.data_ptr() for y in ys]))


def _mats(cuda, Ns, K, seed, hb=6):
    import torch
    from quantize_sx8 import quantize_tensor
    from sx8_decode1_v3 import make_tensors_v44
    out = []
    for i, N in enumerate(Ns):
        g = torch.Generator().manual_seed(seed + i)
        W = (torch.randn(N, K, generator=g) * 0.02).half()
        qt, bi = quantize_tensor(W, device=cuda, degenerate_frac=0.01, seed=seed + 100 + i)
        t = make_tensors_v44(qt, bi, hdr_aligned=hb == 8)
        assert t[0].shape[-1] == hb
        out.append(t)
    return out


@pytest.mark.parametrize("hb", [6, 8])
def test_fused_gemv_rmsnorm(hiplib, cuda, hb):
    """sx8_dec_gemv_rmsnorm against sx8_dec_add_rmsnorm + sx8_gemv_group (q/k/v-like group)."""
    import torch
    import _sx8lib as _L
    P = _L.ptr
    st = _L.stream(cuda)
    K, Ns, eps = 2560, [1024, 512, 300], 1e-6
    ts = _mats(cuda, Ns, K, 40, hb)
    g = torch.Generator().manual_seed(7)
    resid = torch.randn(K, generator=g).to(cuda)
    delta = torch.randn(K, generator=g).to(cuda)
    w = (torch.rand(K, generator=g) + 0.5).half().to(cuda)
    init = torch.randn(K, generator=g).half().to(cuda)
    for use_init in (False, True):
        # reference: the two-launch path
        r_ref = (torch.zeros(1, K) if use_init else resid.cpu().clone().view(1, K)).to(cuda)
        h16 = torch.empty(1, K, dtype=torch.float16, device=cuda)
        _L.call("sx8_dec_add_rmsnorm", P(r_ref), None if use_init else P(delta),
                P(init) if use_init else None, P(w), P(h16), 1, K, eps, st)
        y_ref = [torch.empty(N, device=cuda) for N in Ns]
        n, hd, lv, bs, sc, ns, n_cb, ys = _group(ts, Ns, K // 32, y_ref)
        _L.call("sx8_gemv_group", P(h16), n, hd, lv, hb, bs, sc, None, ns, n_cb, ys, None, 0, st)
        # fused
        r_out = torch.full((K,), float("nan"), device=cuda)
        y = [torch.empty(N, device=cuda) for N in Ns]
        n, hd, lv, bs, sc, ns, n_cb, ys = _group(ts, Ns, K // 32, y)
        _L.call("sx8_dec_gemv_rmsnorm", None if use_init else P(resid), P(init) if use_init else None,
                None if use_init else P(delta), P(w), eps, P(r_out), n, hd, lv, hb, bs, sc, ns, n_cb, ys, st)
        torch.cuda.synchronize()
        assert torch.equal(r_out.cpu(), r_ref.cpu().view(K))        # h = resid + delta, exact
        for a, b in zip(y, y_ref):
            rel = (a - b).abs().max().item() / b.abs().max().item()
            assert rel <= 1e-5, rel
    # the residual alone (no delta, no init, no resid_out): the group takes h and the norm
    # weight from its preloaded argument slots; the same x, so the same outputs as the
    # two-launch path with delta = 0
    r_ref = resid.cpu().clone().view(1, K).to(cuda)
    h16 = torch.empty(1, K, dtype=torch.float16, device=cuda)
    _L.call("sx8_dec_add_rmsnorm", P(r_ref), None, None, P(w), P(h16), 1, K, eps, st)
    y_ref = [torch.empty(N, device=cuda) for N in Ns]
    n, hd, lv, bs, sc, ns, n_cb, ys = _group(ts, Ns, K // 32, y_ref)
    _L.call("sx8_gemv_group", P(h16), n, hd, lv, hb, bs, sc, None, ns, n_cb, ys, None, 0, st)
    y = [torch.empty(N, device=cuda) for N in Ns]
    n, hd, lv, bs, sc, ns, n_cb, ys = _group(ts, Ns, K // 32, y)
    _L.call("sx8_dec_gemv_rmsnorm", P(resid), None, None, P(w), eps, None, n, hd, lv, hb, bs, sc, ns, n_cb, ys, st)
    torch.cuda.synchronize()
    for a, b in zip(y, y_ref):
        rel = (a - b).abs().max().item() / b.abs().max().item()
        assert rel <= 1e-5, rel
    # resid_out may not alias an input still being read by other work-groups
    with pytest.raises(RuntimeError, match="alias"):
        _L.call("sx8_dec_gemv_rmsnorm", P(resid), None, P(delta), P(w), eps, P(resid), n, hd, lv, hb, bs,
                sc, ns, n_cb, ys, st)


def test_fused_gemv_silu(hiplib, cuda):
    """sx8_dec_gemv_silu equals sx8_dec_silu_mul + sx8_gemv_group bit for bit (down-like,
    K = 9728: three table passes)."""
    import torch
    import _sx8lib as _L
    P = _L.ptr
    st = _L.stream(cuda)
    K, Ns = 9728, [2560]
    ts = _mats(cuda, Ns, K, 60)
    g = torch.Generator().manual_seed(8)
    a = torch.randn(K, generator=g).to(cuda)
    b = torch.randn(K, generator=g).to(cuda)
    m = torch.empty(K, dtype=torch.float16, device=cuda)
    _L.call("sx8_dec_silu_mul", P(a), P(b), P(m), K, st)
    y_ref = [torch.empty(N, device=cuda) for N in Ns]
    n, hd, lv, bs, sc, ns, n_cb, ys = _group(ts, Ns, K // 32, y_ref)
    _L.call("sx8_gemv_group", P(m), n, hd, lv, 6, bs, sc, None, ns, n_cb, ys, None, 0, st)
    y = [torch.empty(N, device=cuda) for N in Ns]
    n, hd, lv, bs, sc, ns, n_cb, ys = _group(ts, Ns, K // 32, y)
    _L.call("sx8_dec_gemv_silu", P(a), P(b), n, hd, lv, 6, bs, sc, ns, n_cb, ys, st)
    torch.cuda.synchronize()
    assert torch.equal(y[0].cpu(), y_ref[0].cpu())
    # more K blocks than the up-front table passes hold: refused
    with pytest.raises(RuntimeError, match="n_cb"):
        _L.call("sx8_dec_gemv_silu", P(a), P(b), n, hd, lv, 6, bs, sc, ns, 385, ys, st)


@pytest.mark.parametrize("hb", [6, 8])
def test_fused_gemv_residual_add(hiplib, cuda, hb):
    """sx8_dec_gemv_add and sx8_dec_gemv_silu_add: Ys[i] = adds[i] + W_i x bit for bit against
    sx8_gemv_group (resp. sx8_dec_silu_mul + sx8_gemv_group) plus a float32 add, both with a
    separate residual and with the residual updated in place (adds[i] = Ys[i]), with 6- and
    8-byte headers; a residual that partly overlaps an output is refused."""
    import torch
    import _sx8lib as _L
    P = _L.ptr
    st = _L.stream(cuda)
    g = torch.Generator().manual_seed(12)
    # o-like group of one matrix and a q/k/v-like group of three, plain x
    for K, Ns in ((4096, [2560]), (2560, [4096, 1024, 1024])):
        ts = _mats(cuda, Ns, K, 70 + len(Ns), hb)
        x = torch.randn(K, generator=g).half().to(cuda)
        res = [torch.randn(N, generator=g).to(cuda) for N in Ns]
        y_ref = [torch.empty(N, device=cuda) for N in Ns]
        n, hd, lv, bs, sc, ns, n_cb, ys = _group(ts, Ns, K // 32, y_ref)
        _L.call("sx8_gemv_group", P(x), n, hd, lv, hb, bs, sc, None, ns, n_cb, ys, None, 0, st)
        exp = [yr + r for yr, r in zip(y_ref, res)]
        y = [torch.empty(N, device=cuda) for N in Ns]
        n, hd, lv, bs, sc, ns, n_cb, ys = _group(ts, Ns, K // 32, y)
        adds = (ctypes.c_void_p * n)(*[r.data_ptr() for r in res])
        _L.call("sx8_dec_gemv_add", P(x), n, hd, lv, hb, bs, sc, ns, n_cb, adds, ys, st)
        inplace = [r.clone() for r in res]
        n, hd, lv, bs, sc, ns, n_cb, ys = _group(ts, Ns, K // 32, inplace)
        adds2 = (ctypes.c_void_p * n)(*[r.data_ptr() for r in inplace])
        _L.call("sx8_dec_gemv_add", P(x), n, hd, lv, hb, bs, sc, ns, n_cb, adds2, ys, st)
        torch.cuda.synchronize()
        for i in range(n):
            assert torch.equal(y[i].cpu(), exp[i].cpu()), (K, i)
            assert torch.equal(inplace[i].cpu(), exp[i].cpu()), (K, i)
    # down-like: x = silu(g) * u, residual updated in place; g and u adjacent (u = g + K:
    # both from one preloaded argument), then apart
    K, Ns = 9728, [2560]
    ts = _mats(cuda, Ns, K, 61, hb)
    ab = torch.randn(2, K, generator=g).to(cuda)
    a, b = ab[0], ab[1]
    m = torch.empty(K, dtype=torch.float16, device=cuda)
    _L.call("sx8_dec_silu_mul", P(a), P(b), P(m), K, st)
    y_ref = [torch.empty(N, device=cuda) for N in Ns]
    n, hd, lv, bs, sc, ns, n_cb, ys = _group(ts, Ns, K // 32, y_ref)
    _L.call("sx8_gemv_group", P(m), n, hd, lv, hb, bs, sc, None, ns, n_cb, ys, None, 0, st)
    res = torch.randn(Ns[0], generator=g).to(cuda)
    exp = y_ref[0] + res
    res0 = res.clone()
    n, hd, lv, bs, sc, ns, n_cb, ys = _group(ts, Ns, K // 32, [res])
    adds = (ctypes.c_void_p * 1)(res.data_ptr())
    _L.call("sx8_dec_gemv_silu_add", P(a), P(b), n, hd, lv, hb, bs, sc, ns, n_cb, adds, ys, st)
    b2 = b.clone()                                          # u no longer at g + K
    res2 = res0.clone()
    n, hd, lv, bs, sc, ns, n_cb, ys2 = _group(ts, Ns, K // 32, [res2])
    adds2 = (ctypes.c_void_p * 1)(res2.data_ptr())
    _L.call("sx8_dec_gemv_silu_add", P(a), P(b2), n, hd, lv, hb, bs, sc, ns, n_cb, adds2, ys2, st)
    # u = g + K (one preloaded argument for both) with a separate residual: Ys = adds + W x
    res3 = res0.clone()
    out3 = torch.full((Ns[0],), float("nan"), device=cuda)
    n, hd, lv, bs, sc, ns, n_cb, ys3 = _group(ts, Ns, K // 32, [out3])
    adds3 = (ctypes.c_void_p * 1)(res3.data_ptr())
    _L.call("sx8_dec_gemv_silu_add", P(a), P(b), n, hd, lv, hb, bs, sc, ns, n_cb, adds3, ys3, st)
    torch.cuda.synchronize()
    assert torch.equal(res.cpu(), exp.cpu())
    assert torch.equal(res2.cpu(), exp.cpu())
    assert torch.equal(out3.cpu(), exp.cpu())
    assert torch.equal(res3.cpu(), res0.cpu())              # the separate residual is only read
    # a residual that overlaps its output without being it: refused before any launch
    big = torch.zeros(Ns[0] + 8, device=cuda)
    n, hd, lv, bs, sc, ns, n_cb, ysb = _group(ts, Ns, K // 32, [big[8:]])
    with pytest.raises(RuntimeError, match="overlaps"):
        _L.call("sx8_dec_gemv_silu_add", P(a), P(b), n, hd, lv, hb, bs, sc, ns, n_cb,
                (ctypes.c_void_p * 1)(big.data_ptr()), ysb, st)
    with pytest.raises(RuntimeError, match="residual"):
        bad = (ctypes.c_void_p * 1)(None)
        _L.call("sx8_dec_gemv_silu_add", P(a), P(b), n, hd, lv, hb, bs, sc, ns, n_cb, bad, ys, st)


@pytest.mark.parametrize("M,K,N,hb", [(512, 9728, 2560, 6), (512, 9728, 2560, 8), (77, 9728, 300, 6),
                                      (40, 1000, 130, 8)])
def test_gemm_silu_matches_two_calls(hiplib, cuda, M, K, N, hb):
    """sx8_dec_gemm_silu equals sx8_dec_silu_mul + sx8_gemm_prefill bit for bit (the pack
    pass forms the same fp16 x); K = 1000 takes the unaligned, ragged-tail loads."""
    import torch
    import _sx8lib as _L
    P = _L.ptr
    st = _L.stream(cuda)
    (hdr, lvl, bas, sca), = _mats(cuda, [N], K, 70 + M, hb)
    n_cb = (K + 31) // 32
    g = torch.Generator().manual_seed(M + K)
    a = (torch.randn(M, K, generator=g) * 3).to(cuda)
    b = torch.randn(M, K, generator=g).to(cuda)
    m = torch.empty(M, K, dtype=torch.float16, device=cuda)
    _L.call("sx8_dec_silu_mul", P(a), P(b), P(m), M * K, st)
    y_ref = torch.empty(M, N, device=cuda)
    ws, nb = _L.gemm_workspace(M, (N,), n_cb, cuda)
    _L.call("sx8_gemm_prefill", P(m), M, K, K, P(hdr), P(lvl), hb, P(bas), P(sca), N, n_cb, P(y_ref), P(ws), nb,
            st)
    y = torch.empty(M, N, device=cuda)
    print("gemm_silu", M, K, N, hb, flush=True)
    _L.call("sx8_dec_gemm_silu", P(a), P(b), M, K, P(hdr), P(lvl), hb, P(bas), P(sca), N, n_cb, P(y), P(ws), nb,
            st)
    torch.cuda.synchronize()
    assert torch.equal(y.cpu(), y_ref.cpu())


@pytest.mark.parametrize("n,offset", [(151936, 0), (151937, 1), (5, 0), (4099, 3)])
def test_argmax_advance(hiplib, cuda, n, offset):
    import torch
    import _sx8lib as _L
    g = torch.Generator().manual_seed(n)
    buf = torch.randn(n + offset, generator=g)
    x = buf[offset:]
    if n > 10:
        x[n // 3] = 7.5                  # tie: the first index wins
        x[n - 2] = 7.5
        x[n // 2] = float("nan")         # skipped
    xd = buf.to(cuda)[offset:]           # offset 1/3: not 16-byte aligned -> scalar path
    tok = torch.zeros(1, dtype=torch.int64, device=cuda)
    pos = torch.full((1,), 41, dtype=torch.int64, device=cuda)
    _L.call("sx8_dec_argmax_advance", _L.ptr(xd), n, _L.ptr(tok), _L.ptr(pos), _L.stream(cuda))
    torch.cuda.synchronize()
    assert tok.item() == int(np.nanargmax(x.numpy()))
    assert pos.item() == 42


@pytest.mark.parametrize("nh,nk,hd,L,positions", [
    (32, 8, 128, 1024, [0, 31, 32, 700, 1023]),
    (16, 16, 64, 300, [0, 5, 299]),
    (8, 4, 64, 64, [0, 63]),
    (32, 8, 128, 1500, [0, 700, 1499]),
    (16, 2, 128, 400, [0, 399]),                   # G = 8
    (8, 2, 128, 3000, [0, 2047, 2999]),            # a longer cache (94 positions per chunk)
])
def test_attn_rope_matches_two_calls(hiplib, cuda, nh, nk, hd, L, positions):
    """sx8_dec_attn_rope against sx8_dec_qk_rope_cache + sx8_dec_attn_split: the new k/v rows
    written into the caches, every other row untouched, and the attention output (the two
    forms differ only in the summation order of the q/k RMSNorm sums)."""
    import torch
    import _sx8lib as _L
    P = _L.ptr
    st = _L.stream(cuda)
    g = torch.Generator().manual_seed(nh * 7 + L)
    half = hd // 2
    inv = 1.0 / (1e6 ** (torch.arange(half, dtype=torch.float32) / half))
    ang = torch.arange(L, dtype=torch.float32)[:, None] * inv[None]
    cos, sin = ang.cos().to(cuda), ang.sin().to(cuda)
    qn = (torch.rand(hd, generator=g) + 0.5).half().to(cuda)
    kn = (torch.rand(hd, generator=g) + 0.5).half().to(cuda)
    ws_n = int(_L.lib().sx8_dec_attn_workspace_bytes(nh, hd)) // 4 + 64
    base_k = (torch.randn(nk, L, hd, generator=g) * 0.5).half()
    base_v = torch.randn(nk, L, hd, generator=g).half()
    for p in positions:
        q = torch.randn(nh * hd, generator=g).to(cuda)
        k = torch.randn(nk * hd, generator=g).to(cuda)
        v = torch.randn(nk * hd, generator=g).to(cuda)
        pos = torch.full((1,), p, dtype=torch.int64, device=cuda)
        # two calls
        kc1, vc1 = base_k.clone().to(cuda), base_v.clone().to(cuda)
        qh = torch.empty(nh * hd, dtype=torch.float16, device=cuda)
        out1 = torch.empty(nh * hd, dtype=torch.float16, device=cuda)
        ws1 = torch.zeros(ws_n, device=cuda)
        _L.call("sx8_dec_qk_rope_cache", P(q), P(k), P(v), P(qn), P(kn), P(cos), P(sin), P(pos), P(qh),
                P(kc1), P(vc1), nh, nk, hd, L, 1e-6, st)
        _L.call("sx8_dec_attn_split", P(qh), P(kc1), P(vc1), P(pos), P(out1), nh, nk, hd, L,
                1.0 / math.sqrt(hd), P(ws1), ws_n * 4, st)
        # fused
        kc2, vc2 = base_k.clone().to(cuda), base_v.clone().to(cuda)
        out2 = torch.empty(nh * hd, dtype=torch.float16, device=cuda)
        ws2 = torch.zeros(ws_n, device=cuda)
        _L.call("sx8_dec_attn_rope", P(q), P(k), P(v), P(qn), P(kn), P(cos), P(sin), P(pos), P(kc2), P(vc2),
                P(out2), nh, nk, hd, L, 1.0 / math.sqrt(hd), 1e-6, P(ws2), ws_n * 4, st)
        torch.cuda.synchronize()
        kc1, vc1, kc2, vc2 = kc1.cpu(), vc1.cpu(), kc2.cpu(), vc2.cpu()
        keep = torch.ones(L, dtype=torch.bool)
        keep[p] = False
        assert torch.equal(kc2[:, keep], base_k[:, keep]) and torch.equal(vc2[:, keep], base_v[:, keep])
        assert torch.equal(vc2[:, p], vc1[:, p])
        dk = (kc2[:, p].float() - kc1[:, p].float()).abs().max().item()
        assert dk <= 2e-3 * kc1[:, p].float().abs().max().item(), dk
        o1, o2 = out1.cpu().float(), out2.cpu().float()
        assert (o1 - o2).abs().max().item() <= 5e-3 * o1.abs().max().item()


def _qk_rope_ref(x, w, cos_row, sin_row, eps):
    """One head's RMSNorm (fp16-rounded, as the model's fp16 activations are) and rotate-half
    RoPE in float32; x (hd,) float32, w (hd,) fp16, cos_row / sin_row (hd/2,)."""
    import torch
    half = x.numel() // 2
    n = (x * torch.rsqrt((x * x).mean() + eps) * w.float()).half().float()
    n1, n2 = n[:half], n[half:]
    return torch.cat([n1 * cos_row - n2 * sin_row, n2 * cos_row + n1 * sin_row])


@pytest.mark.parametrize("nh,nk,hd,L,rows,pos0", [
    (32, 8, 128, 64, 9, 3),      # the decoder's heads, a ragged last block of rows
    (4, 2, 256, 40, 7, 36),      # hd 256 (two waves per head); rows 4..6 fall past the cache
    (6, 2, 96, 32, 5, 0),        # hd 96; 10 heads in blocks of 4
    (3, 1, 160, 16, 4, 0),       # hd 160: a value head's upper elements at d + 128
    (8, 8, 64, 20, 1, 19),       # one row at the last cache position
    (2, 1, 200, 8, 3, -1),       # the first row before the cache writes nothing
])
def test_qk_rope_cache_rows(hiplib, cuda, nh, nk, hd, L, rows, pos0):
    """sx8_dec_qk_rope_cache_rows against a float32 per-head reference (q, the cache rows it
    writes, every other cache row and every out-of-cache q row untouched), and bit for bit
    against one sx8_dec_qk_rope_cache call per row."""
    import torch
    import _sx8lib as _L
    P = _L.ptr
    st = _L.stream(cuda)
    eps = 1e-6
    g = torch.Generator().manual_seed(hd * 31 + rows)
    half = hd // 2
    inv = 1.0 / (1e6 ** (torch.arange(half, dtype=torch.float32) / half))
    ang = torch.arange(L, dtype=torch.float32)[:, None] * inv[None]
    cos, sin = ang.cos(), ang.sin()
    qn = (torch.rand(hd, generator=g) + 0.5).half()
    kn = (torch.rand(hd, generator=g) + 0.5).half()
    q = torch.randn(rows, nh * hd, generator=g)
    k = torch.randn(rows, nk * hd, generator=g) * 3.0
    v = torch.randn(rows, nk * hd, generator=g)
    base_k = torch.randn(nk, L, hd, generator=g).half()
    base_v = torch.randn(nk, L, hd, generator=g).half()
    sentinel = torch.full((rows, nh * hd), 7.0).half()
    d = {n: t.to(cuda) for n, t in dict(q=q, k=k, v=v, qn=qn, kn=kn, cos=cos, sin=sin).items()}
    print("qk_rope_rows", nh, nk, hd, L, rows, pos0, flush=True)
    # the rows form
    qo, kc, vc = sentinel.to(cuda), base_k.to(cuda), base_v.to(cuda)
    pos = torch.tensor([pos0], dtype=torch.int64, device=cuda)
    _L.call("sx8_dec_qk_rope_cache_rows", P(d["q"]), P(d["k"]), P(d["v"]), P(d["qn"]), P(d["kn"]),
            P(d["cos"]), P(d["sin"]), P(pos), rows, P(qo), P(kc), P(vc), nh, nk, hd, L, eps, st)
    # one single-token call per row
    qo1, kc1, vc1 = sentinel.to(cuda), base_k.to(cuda), base_v.to(cuda)
    for y in range(rows):
        py = torch.tensor([pos0 + y], dtype=torch.int64, device=cuda)
        _L.call("sx8_dec_qk_rope_cache", P(d["q"][y]), P(d["k"][y]), P(d["v"][y]), P(d["qn"]), P(d["kn"]),
                P(d["cos"]), P(d["sin"]), P(py), P(qo1[y]), P(kc1), P(vc1), nh, nk, hd, L, eps, st)
    torch.cuda.synchronize()
    qo, kc, vc = qo.cpu(), kc.cpu(), vc.cpu()
    assert torch.equal(qo, qo1.cpu()) and torch.equal(kc, kc1.cpu()) and torch.equal(vc, vc1.cpu())
    ref_k, ref_v = base_k.clone(), base_v.clone()
    ref_q = sentinel.clone().float()
    for y in range(rows):
        p = pos0 + y
        if not 0 <= p < L:
            continue
        for h in range(nh):
            ref_q[y, h * hd:(h + 1) * hd] = _qk_rope_ref(q[y, h * hd:(h + 1) * hd], qn, cos[p], sin[p], eps)
        for h in range(nk):
            ref_k[h, p] = _qk_rope_ref(k[y, h * hd:(h + 1) * hd], kn, cos[p], sin[p], eps).half()
            ref_v[h, p] = v[y, h * hd:(h + 1) * hd].half()
    assert torch.equal(vc, ref_v)
    # fp16 outputs: the output's own rounding, plus one fp16 step of a normed value below 8
    # (the reference's norm sum, in another order, can round a normed element the other way)
    def close(a, r):
        return bool(((a.float() - r).abs() <= 2.0 ** -10 * r.abs() + 2.0 ** -7).all())
    assert close(qo, ref_q), (qo.float() - ref_q).abs().max().item()
    assert close(kc, ref_k.float()), (kc.float() - ref_k.float()).abs().max().item()


@pytest.mark.gpu
@pytest.mark.parametrize("nh,nk,L,rows,pos0,n_parts", [
    (32, 8, 2048, 512, 0, 1),      # the prompt pass's call: 512 rows, the q/k/v GEMM's one pending slice
    (32, 8, 600, 77, 530, 1),      # rows past the cache's end write nothing
    (16, 2, 400, 33, -2, 2),       # rows before the cache write nothing
    (12, 4, 100, 5, 0, 3),         # 20 heads: work-groups' units straddle q, k and v heads and rows
    (8, 8, 40, 1, 39, 0),          # one row at the last position
])
def test_qk_rope_cache_rows_vector_kernel(hiplib, cuda, nh, nk, L, rows, pos0, n_parts):
    """Head dim 128 with aligned rows runs the 16-byte kernel (k_qk_rope128); a q buffer 4 bytes
    off 16-byte alignment runs the general one (k_qk_rope_cache).  Both write the same q rows
    and K/V cache rows bit for bit, with and without pending partial slices."""
    import torch
    import _sx8lib as _L
    P = _L.ptr
    st = _L.stream(cuda)
    hd = 128
    g = torch.Generator().manual_seed(nh * 5 + rows)
    half = hd // 2
    inv = 1.0 / (1e6 ** (torch.arange(half, dtype=torch.float32) / half))
    ang = torch.arange(L, dtype=torch.float32)[:, None] * inv[None]
    cos, sin = ang.cos().to(cuda), ang.sin().to(cuda)
    qn = (torch.rand(hd, generator=g) + 0.5).half().to(cuda)
    kn = (torch.rand(hd, generator=g) + 0.5).half().to(cuda)
    q = torch.randn(rows, nh * hd, generator=g).to(cuda)
    k = (torch.randn(rows, nk * hd, generator=g) * 3).to(cuda)
    v = torch.randn(rows, nk * hd, generator=g).to(cuda)
    slice_ = rows * (nh + 2 * nk) * hd + 32
    parts = torch.randn(max(n_parts, 1) * slice_, generator=g).to(cuda)
    pos = torch.tensor([pos0], dtype=torch.int64, device=cuda)
    base_k = torch.randn(nk, L, hd, generator=g).half().to(cuda)
    base_v = torch.randn(nk, L, hd, generator=g).half().to(cuda)
    qbuf = torch.empty(rows * nh * hd + 1, device=cuda)
    qbuf[1:] = q.reshape(-1)
    print("qk_rope vector kernel", nh, nk, L, rows, pos0, n_parts, flush=True)
    outs = []
    for qsrc in (q, qbuf[1:]):
        qo = torch.full((rows, nh * hd), 7.0, device=cuda).half()
        kc, vc = base_k.clone(), base_v.clone()
        _L.call("sx8_dec_qk_rope_cache_rows_parts", P(qsrc), P(k), P(v), P(qn), P(kn), P(cos), P(sin), P(pos), rows,
                P(qo), P(kc), P(vc), nh, nk, hd, L, 1e-6, P(parts) if n_parts else None, n_parts,
                slice_ if n_parts else 0, st)
        outs.append((qo, kc, vc))
    torch.cuda.synchronize()
    for a, b in zip(*outs):
        assert torch.equal(a.cpu().view(torch.int16), b.cpu().view(torch.int16))
    # rows outside the cache leave q (sentinel) and the caches untouched
    for y in range(rows):
        if not 0 <= pos0 + y < L:
            assert bool((outs[0][0][y] == 7.0).all())


@pytest.mark.parametrize("H,I,hb", [(2560, 9728, 6), (2560, 9728, 8), (1024, 8224, 6), (512, 1056, 8)])
def test_gemv_pair_and_zp_down(hiplib, cuda, H, I, hb):
    """sx8_dec_gemv_rmsnorm_pair + sx8_dec_gemv_zp_add against the three-launch MLP
    (sx8_dec_gemv_rmsnorm over gate and up as a group, sx8_dec_silu_mul, sx8_dec_gemv_add):
    m within one fp16 step (g and u are summed in another order), the partial sums' Z
    against sx8_compute_z on the same m, and the down GEMV from the partial sums against
    sx8_dec_gemv_add on the same m.  I = 8224 leaves the last panel partly empty; I = 1056
    runs at the 32-pair minimum panel width.  A pair stored apart, or an N the down GEMV
    would refuse, is refused."""
    import torch
    import _sx8lib as _L
    P = _L.ptr
    st = _L.stream(cuda)
    eps = 1e-6
    gu = _mats(cuda, [I, I], H, 80 + H, hb)
    (dh, dl, db, ds), = _mats(cuda, [H], I, 90 + H, hb)
    # the up matrix's arrays right behind the gate matrix's
    cat = [torch.cat([gu[0][f].reshape(-1), gu[1][f].reshape(-1)]) for f in range(4)]
    up = [c[gu[0][f].numel():] for f, c in enumerate(cat)]
    g = torch.Generator().manual_seed(H)
    resid = torch.randn(H, generator=g).to(cuda)
    w = (torch.rand(H, generator=g) + 0.5).half().to(cuda)
    y_gu = torch.empty(2, I, device=cuda)
    n, hd, lv, bs, sc, ns, n_cb, ys = _group(gu, [I, I], H // 32, [y_gu[0], y_gu[1]])
    _L.call("sx8_dec_gemv_rmsnorm", P(resid), None, None, P(w), eps, None, n, hd, lv, hb, bs, sc, ns, n_cb,
            ys, st)
    m_ref = torch.empty(I, dtype=torch.float16, device=cuda)
    _L.call("sx8_dec_silu_mul", P(y_gu[0]), P(y_gu[1]), P(m_ref), I, st)
    m = torch.full((I,), float("nan"), dtype=torch.float16, device=cuda)
    zp = torch.full((I // 32, 2, 2), float("nan"), device=cuda)
    _L.call("sx8_dec_gemv_rmsnorm_pair", P(resid), P(w), eps, P(cat[0]), P(cat[1]), hb, P(cat[2]), P(cat[3]),
            *[P(u) for u in up], I, H // 32, P(db), P(m), P(zp), st)
    torch.cuda.synchronize()
    mf, mr = m.cpu().float(), m_ref.cpu().float()
    assert torch.isfinite(mf).all()
    step = torch.where(mr.abs() < 2.0 ** -14, torch.full_like(mr, 2.0 ** -24),
                       2.0 ** (torch.floor(torch.log2(mr.abs().clamp_min(2.0 ** -14))) - 10))
    assert ((mf - mr).abs() <= step).all()
    assert (mf == mr).float().mean().item() > 0.99
    # Z from the partial sums against sx8_compute_z on the pair's own m
    z_ref = torch.empty(I // 32, 2, device=cuda)
    _L.call("sx8_compute_z", P(m), 1, I, P(db), P(ds), I // 32, P(z_ref), st)
    torch.cuda.synchronize()
    zpc = zp.cpu()
    assert torch.isfinite(zpc).all()
    z = (zpc[:, 0, :] + zpc[:, 1, :]) * ds.cpu().view(I // 32, 2)
    zr = z_ref.cpu()
    assert (z - zr).abs().max().item() <= 1e-5 * zr.abs().max().item()
    # the down GEMV: partial sums vs its own Z, separate output and in place
    res = torch.randn(H, generator=g).to(cuda)
    y_ref = res.clone()
    n, hd, lv, bs, sc, ns, n_cb, ys = _group([(dh, dl, db, ds)], [H], I // 32, [y_ref])
    adds = (ctypes.c_void_p * 1)(y_ref.data_ptr())
    _L.call("sx8_dec_gemv_add", P(m), n, hd, lv, hb, bs, sc, ns, n_cb, adds, ys, st)
    y = torch.full((H,), float("nan"), device=cuda)
    _L.call("sx8_dec_gemv_zp_add", P(m), P(dh), P(dl), hb, P(zp), P(ds), H, I // 32, P(res), P(y), st)
    y_in = res.clone()
    _L.call("sx8_dec_gemv_zp_add", P(m), P(dh), P(dl), hb, P(zp), P(ds), H, I // 32, P(y_in), P(y_in), st)
    torch.cuda.synchronize()
    scale = (y_ref - res).abs().max().item()
    for out in (y, y_in):
        assert (out - y_ref).abs().max().item() <= 1e-5 * scale
    def pair(ptrs, Ncols):
        _L.call("sx8_dec_gemv_rmsnorm_pair", P(resid), P(w), eps, P(ptrs[0]), P(ptrs[1]), hb, P(ptrs[2]),
                P(ptrs[3]), *[P(u) for u in ptrs[4:]], Ncols, H // 32, P(db), P(m), P(zp), st)

    with pytest.raises(RuntimeError, match="multiple of 32"):
        pair(cat + up, I - 16)
    # the up matrix in its own allocations (as to_v44_device makes them): refused on the host
    for f in range(4):
        apart = list(cat) + list(up)
        apart[4 + f] = gu[1][f]
        with pytest.raises(RuntimeError, match="follow the gate"):
            pair(apart, I)
    # N past what sx8_dec_gemv_zp_add accepts (n_cb <= 384, N <= 12288)
    with pytest.raises(RuntimeError, match="multiple of 32"):
        pair(cat + up, 12288 + 32)


@pytest.mark.parametrize("K,N,hb", [
    (2560, 20000, 6),      # fewer panels than co-resident work-groups: one panel each
    (256, 100000, 6),      # 128-column panels, one K round per panel (R < ring)
    (2560, 151936, 8),     # the vocab-sized lm_head (128-column panels), 8-byte headers
])
def test_head_argmax_partials(hiplib, cuda, K, N, hb):
    """sx8_dec_gemv_rmsnorm_argmax: logits bit for bit those of sx8_dec_gemv_rmsnorm, and the
    token that sx8_dec_argmax_advance picks from them -- with four equal maxima (rows 5, 6
    and 70 in the first panel, 70 in the second wave of a 128-column panel, and 17000 in
    another panel; identical weights give identical logits) the first index wins -- and
    the position advanced."""
    import torch
    import _sx8lib as _L
    from quantize_sx8 import quantize_tensor
    from sx8_decode1_v3 import make_tensors_v44
    P = _L.ptr
    st = _L.stream(cuda)
    eps = 1e-6
    print("head argmax", K, N, hb, flush=True)
    g = torch.Generator().manual_seed(31)
    resids = [torch.randn(K, generator=g) for _ in range(2)]
    W = torch.randn(N, K, generator=g) * 0.02
    top = torch.sign(resids[0]) * 0.05           # the largest logit for the first residual
    W[5], W[6], W[70], W[17000] = top, top, top, top
    qt, bi = quantize_tensor(W.half(), device=cuda, degenerate_frac=0.0, seed=32)   # equal rows stay equal
    hdr, lvl, bas, sca = make_tensors_v44(qt, bi, hdr_aligned=hb == 8)
    assert hdr.shape[-1] == hb
    w = (torch.rand(K, generator=g) + 0.5).half().to(cuda)
    nb = int(_L.lib().sx8_dec_argmax_parts_bytes(N, K // 32))
    assert nb > 0
    parts = torch.empty(nb // 4, dtype=torch.int32, device=cuda)
    for k, r in enumerate(resids):
        rd = r.to(cuda)
        ref = torch.empty(N, device=cuda)
        n, hd, lv, bs, sc, ns, n_cb, ys = _group([(hdr, lvl, bas, sca)], [N], K // 32, [ref])
        _L.call("sx8_dec_gemv_rmsnorm", P(rd), None, None, P(w), eps, None, n, hd, lv, hb, bs, sc, ns, n_cb, ys, st)
        tok_ref = torch.zeros(1, dtype=torch.int64, device=cuda)
        pos_ref = torch.full((1,), 40, dtype=torch.int64, device=cuda)
        _L.call("sx8_dec_argmax_advance", P(ref), N, P(tok_ref), P(pos_ref), st)
        logits = torch.full((N,), float("nan"), device=cuda)
        tok = torch.full((1,), -1, dtype=torch.int64, device=cuda)
        pos = torch.full((1,), 40, dtype=torch.int64, device=cuda)
        _L.call("sx8_dec_gemv_rmsnorm_argmax", P(rd), P(w), eps, P(hdr), P(lvl), hb, P(bas), P(sca), N, K // 32,
                P(logits), P(parts), nb, P(tok), P(pos), st)
        torch.cuda.synchronize()
        assert torch.equal(logits.cpu(), ref.cpu()), k
        assert tok.item() == tok_ref.item() and pos.item() == 41, (k, tok.item(), tok_ref.item())
        if k == 0:
            assert tok.item() == 5 and ref[5].item() == ref[70].item() == ref[17000].item() == ref.max().item()
    with pytest.raises(RuntimeError, match="parts"):
        _L.call("sx8_dec_gemv_rmsnorm_argmax", P(rd), P(w), eps, P(hdr), P(lvl), hb, P(bas), P(sca), N, K // 32,
                P(logits), P(parts), nb - 8, P(tok), P(pos), st)


@pytest.mark.parametrize("N,top", [
    (16384, 48),     # 64-column panels (256 of them): 48 is 16's partner across 32 lanes
    (70000, 100),    # 128-column panels: 100 is in the panel's second wave
])
def test_head_argmax_partials_nan_logit(hiplib, cuda, N, top):
    """A NaN logit in a panel never hides the panel's other columns from the argmax: column
    16's first header decodes a NaN range (dmin = fp16 NaN), column `top` -- in the same
    panel, across the 32-lane step of the butterfly of 64-column panels, or in the second
    wave of a 128-column panel -- holds the largest logit.  sx8_dec_gemv_rmsnorm_argmax must
    pick `top`, as sx8_dec_argmax_advance does on the same logits."""
    import torch
    import _sx8lib as _L
    from quantize_sx8 import quantize_tensor
    from sx8_decode1_v3 import make_tensors_v44
    P = _L.ptr
    st = _L.stream(cuda)
    K, eps = 2560, 1e-6
    g = torch.Generator().manual_seed(41)
    resid = torch.randn(K, generator=g)
    W = torch.randn(N, K, generator=g) * 0.02
    W[top] = torch.sign(resid) * 0.05
    qt, bi = quantize_tensor(W.half(), device=cuda, degenerate_frac=0.0, seed=42)
    hdr, lvl, bas, sca = make_tensors_v44(qt, bi)
    hdr.view(-1, 6)[16, 0:2] = torch.tensor([0x00, 0x7E], dtype=torch.uint8, device=cuda)  # kb 0, n 16
    w = (torch.rand(K, generator=g) + 0.5).half().to(cuda)
    rd = resid.to(cuda)
    ref = torch.empty(N, device=cuda)
    n, hd, lv, bs, sc, ns, n_cb, ys = _group([(hdr, lvl, bas, sca)], [N], K // 32, [ref])
    _L.call("sx8_dec_gemv_rmsnorm", P(rd), None, None, P(w), eps, None, n, hd, lv, 6, bs, sc, ns, n_cb, ys, st)
    tok_ref = torch.zeros(1, dtype=torch.int64, device=cuda)
    pos_ref = torch.zeros(1, dtype=torch.int64, device=cuda)
    _L.call("sx8_dec_argmax_advance", P(ref), N, P(tok_ref), P(pos_ref), st)
    nb = int(_L.lib().sx8_dec_argmax_parts_bytes(N, K // 32))
    parts = torch.empty(nb // 4, dtype=torch.int32, device=cuda)
    logits = torch.empty(N, device=cuda)
    tok = torch.full((1,), -1, dtype=torch.int64, device=cuda)
    pos = torch.zeros(1, dtype=torch.int64, device=cuda)
    _L.call("sx8_dec_gemv_rmsnorm_argmax", P(rd), P(w), eps, P(hdr), P(lvl), 6, P(bas), P(sca), N, K // 32,
            P(logits), P(parts), nb, P(tok), P(pos), st)
    torch.cuda.synchronize()
    lr = ref.cpu()
    assert torch.isnan(lr[16]) and torch.isnan(lr).sum().item() == 1
    assert torch.equal(logits.cpu().view(torch.int32), lr.view(torch.int32))
    assert tok_ref.item() == top
    assert tok.item() == top and pos.item() == 1


def _deferred(name, *args):
    """Call a *_deferred entry point; returns (parts, n_parts, slice)."""
    import ctypes
    import _sx8lib as _L
    parts, n_parts, slc = ctypes.c_void_p(), ctypes.c_int32(), ctypes.c_int64()
    _L.call(name, *args[:-1], ctypes.addressof(parts), ctypes.addressof(n_parts), ctypes.addressof(slc), args[-1])
    return parts.value, n_parts.value, slc.value


@pytest.mark.parametrize("M,K,Ns,hb,want_np", [
    (512, 4096, [2560], 6, 3),          # o at M = 512: 4 K ranges
    (512, 4096, [2560], 8, 3),
    (300, 2600, [1001], 6, None),       # ragged N (H % 4 != 0: the scalar add path)
    (512, 2560, [9728, 9728], 6, 0),    # gate/up at M = 512: unsplit 512-row tiles
    (2048, 2560, [9728], 6, 0),         # gate at M = 2048: split tiles, summed as usual
])
def test_gemm_deferred_sums_into_add_rmsnorm(hiplib, cuda, M, K, Ns, hb, want_np):
    """sx8_gemm_prefill_group_deferred + sx8_dec_add_rmsnorm_parts give the residual and the
    normalized rows of sx8_gemm_prefill_group + sx8_dec_add_rmsnorm bit for bit (the
    partial slices are added in the order the split-K sum adds them); plans without K
    slices report no parts and write the full sums."""
    import torch
    import _sx8lib as _L
    P = _L.ptr
    st = _L.stream(cuda)
    ts = _mats(cuda, Ns, K, 300 + M, hb)
    n_cb = (K + 31) // 32
    g = torch.Generator().manual_seed(M + K)
    X = torch.randn(M, K, generator=g).half().to(cuda)
    H = Ns[0]
    resid0 = torch.randn(M, H, generator=g).to(cuda)
    w = (torch.rand(H, generator=g) + 0.5).half().to(cuda)
    ws, nb = _L.gemm_workspace(M, Ns, n_cb, cuda)
    print("deferred gemm", M, K, Ns, hb, flush=True)
    ya = [torch.empty(M, N, device=cuda) for N in Ns]
    ga = _group(ts, Ns, n_cb, ya)
    _L.call("sx8_gemm_prefill_group", P(X), M, K, K, ga[0], ga[1], ga[2], hb, ga[3], ga[4], ga[5], ga[6], ga[7],
            P(ws), nb, st)
    ra, ha = resid0.clone(), torch.empty(M, H, dtype=torch.float16, device=cuda)
    _L.call("sx8_dec_add_rmsnorm", P(ra), P(ya[0]), None, P(w), P(ha), M, H, 1e-6, st)
    yb = [torch.empty(M, N, device=cuda) for N in Ns]
    grp = _group(ts, Ns, n_cb, yb)
    parts, n_parts, slc = _deferred("sx8_gemm_prefill_group_deferred", P(X), M, K, K, grp[0], grp[1], grp[2], hb,
                                    grp[3], grp[4], grp[5], grp[6], grp[7], P(ws), nb, st)
    rb, hb16 = resid0.clone(), torch.empty(M, H, dtype=torch.float16, device=cuda)
    _L.call("sx8_dec_add_rmsnorm_parts", P(rb), P(yb[0]), None, P(w), P(hb16), M, H, 1e-6, parts, n_parts, slc, st)
    torch.cuda.synchronize()
    plan = _L.gemm_plan(M, Ns, n_cb)
    print("   plan", plan, "n_parts", n_parts, flush=True)
    if want_np is not None:
        assert n_parts == want_np
    assert n_parts == (plan["k_ranges"] - 1 if plan["tile"] != 512 else 0)
    if n_parts:
        assert slc == M * sum(Ns)
    else:
        for a, b in zip(ya, yb):
            assert torch.equal(a.cpu(), b.cpu())
    assert torch.equal(rb.cpu(), ra.cpu())
    assert torch.equal(hb16.cpu().view(torch.int16), ha.cpu().view(torch.int16))


@pytest.mark.parametrize("T", [512, 13])
def test_qkv_deferred_sums_into_rope(hiplib, cuda, T):
    """The q/k/v group deferred + sx8_dec_qk_rope_cache_rows_parts write the q rows and the
    K/V cache rows of the group call + sx8_dec_qk_rope_cache_rows bit for bit (32/8 heads of
    128, K = 2560: two K ranges at T = 512)."""
    import torch
    import _sx8lib as _L
    P = _L.ptr
    st = _L.stream(cuda)
    nh, nk, hd, L, K, eps = 32, 8, 128, 600, 2560, 1e-6
    Ns = [nh * hd, nk * hd, nk * hd]
    ts = _mats(cuda, Ns, K, 500 + T)
    n_cb = K // 32
    g = torch.Generator().manual_seed(T)
    X = torch.randn(T, K, generator=g).half().to(cuda)
    qn = (torch.rand(hd, generator=g) + 0.5).half().to(cuda)
    kn = (torch.rand(hd, generator=g) + 0.5).half().to(cuda)
    ang = torch.rand(L, hd // 2, generator=g) * 6.0
    cos, sin = ang.cos().to(cuda), ang.sin().to(cuda)
    pos0 = torch.full((1,), 7, dtype=torch.int64, device=cuda)
    ws, nb = _L.gemm_workspace(T, Ns, n_cb, cuda)
    out = []
    print("deferred qkv", T, flush=True)
    for deferred in (False, True):
        ys = [torch.empty(T, N, device=cuda) for N in Ns]
        grp = _group(ts, Ns, n_cb, ys)
        qh = torch.zeros(T, nh, hd, dtype=torch.float16, device=cuda)
        kc = torch.zeros(nk, L, hd, dtype=torch.float16, device=cuda)
        vc = torch.zeros(nk, L, hd, dtype=torch.float16, device=cuda)
        common = (P(ys[0]), P(ys[1]), P(ys[2]), P(qn), P(kn), P(cos), P(sin), P(pos0), T, P(qh), P(kc), P(vc),
                  nh, nk, hd, L, eps)
        if deferred:
            parts, n_parts, slc = _deferred("sx8_gemm_prefill_group_deferred", P(X), T, K, K, grp[0], grp[1],
                                            grp[2], 6, grp[3], grp[4], grp[5], grp[6], grp[7], P(ws), nb, st)
            _L.call("sx8_dec_qk_rope_cache_rows_parts", *common, parts, n_parts, slc, st)
            print("   n_parts", n_parts, flush=True)
            if T == 512:
                assert n_parts == 1
        else:
            _L.call("sx8_gemm_prefill_group", P(X), T, K, K, grp[0], grp[1], grp[2], 6, grp[3], grp[4], grp[5],
                    grp[6], grp[7], P(ws), nb, st)
            _L.call("sx8_dec_qk_rope_cache_rows", *common, st)
        torch.cuda.synchronize()
        out.append((qh.cpu(), kc.cpu(), vc.cpu()))
    for a, b in zip(*out):
        assert torch.equal(a.view(torch.int16), b.view(torch.int16))


def test_gemm_silu_deferred_sums_into_add_rmsnorm(hiplib, cuda):
    """sx8_dec_gemm_silu_deferred (down at M = 512: 6 K ranges) + sx8_dec_add_rmsnorm_parts
    equal sx8_dec_gemm_silu + sx8_dec_add_rmsnorm bit for bit."""
    import torch
    import _sx8lib as _L
    P = _L.ptr
    st = _L.stream(cuda)
    M, K, N = 512, 9728, 2560
    (hdr, lvl, bas, sca), = _mats(cuda, [N], K, 77)
    n_cb = K // 32
    g = torch.Generator().manual_seed(5)
    a = (torch.randn(M, K, generator=g) * 3).to(cuda)
    b = torch.randn(M, K, generator=g).to(cuda)
    resid0 = torch.randn(M, N, generator=g).to(cuda)
    w = (torch.rand(N, generator=g) + 0.5).half().to(cuda)
    ws, nb = _L.gemm_workspace(M, (N,), n_cb, cuda)
    args = (P(a), P(b), M, K, P(hdr), P(lvl), 6, P(bas), P(sca), N, n_cb)
    y = torch.empty(M, N, device=cuda)
    _L.call("sx8_dec_gemm_silu", *args, P(y), P(ws), nb, st)
    ra, ha = resid0.clone(), torch.empty(M, N, dtype=torch.float16, device=cuda)
    _L.call("sx8_dec_add_rmsnorm", P(ra), P(y), None, P(w), P(ha), M, N, 1e-6, st)
    y2 = torch.empty(M, N, device=cuda)
    parts, n_parts, slc = _deferred("sx8_dec_gemm_silu_deferred", *args, P(y2), P(ws), nb, st)
    rb, hb16 = resid0.clone(), torch.empty(M, N, dtype=torch.float16, device=cuda)
    _L.call("sx8_dec_add_rmsnorm_parts", P(rb), P(y2), None, P(w), P(hb16), M, N, 1e-6, parts, n_parts, slc, st)
    torch.cuda.synchronize()
    print("deferred silu n_parts", n_parts, flush=True)
    assert n_parts == 5 and slc == M * N
    assert torch.equal(rb.cpu(), ra.cpu())
    assert torch.equal(hb16.cpu().view(torch.int16), ha.cpu().view(torch.int16))


def _packed_operands_ref(x16, Zf, n_cb):
    """The packed X and Zhl (include/sx8_hip.h, sx8_gemm_prefill_packed) of an fp16 (T, 32 n_cb)
    matrix given as uint16 and its float32 Z (T, n_cb, 2), built in numpy: X[32 G + r][32 kb +
    16 hf + 8 st + i] at chunk (G, kb), k-step st, lane 32 hf + r, value i (rows past T
    zero); Z as (fp16(z), fp16(z - fp16(z)))."""
    T = x16.shape[0]
    Gs = (T + 31) // 32
    X = np.zeros((Gs * 32, n_cb * 32), np.uint16)
    X[:T] = x16
    Xp = X.reshape(Gs, 32, n_cb, 2, 2, 8).transpose(0, 2, 4, 3, 1, 5)   # G, kb, st, hf, r, i
    hi = Zf.astype(np.float16)
    lo = (Zf - hi.astype(np.float32)).astype(np.float16)
    return np.ascontiguousarray(Xp).ravel(), np.stack([hi, lo], -1).view(np.uint16).ravel()


@pytest.mark.parametrize("nh,nk,hd,L,T,start,N,hb", [
    (32, 8, 128, 1024, 512, 0, 2560, 6),   # the decoder's prompt pass: o at T = 512 (4 K ranges)
    (32, 8, 128, 1200, 1100, 50, 640, 8),  # G = 4 with four heads per work-group, ragged tile
    (8, 1, 128, 200, 70, 3, 300, 6),       # G = 8 (one wave set)
    (16, 16, 64, 300, 33, 0, 96, 8),       # G = 1 at hd 64
    (2, 1, 128, 160, 40, 5, 1001, 6),      # G = 2 at hd 128
    (32, 8, 128, 64, 1, 0, 256, 6),        # one row
])
def test_attention_packed_operands(hiplib, cuda, nh, nk, hd, L, T, start, N, hb):
    """sx8_dec_attn_prefill_packed writes, bit for bit, the packed X and Zhl that the prefill
    GEMM's own pass makes from sx8_dec_attn_prefill's output (packed rows padded with zeros,
    Z in the reference's tree order: sx8_compute_z), every byte of both buffers; and
    sx8_gemm_prefill_packed on them gives sx8_gemm_prefill_group's output bit for bit, with
    the split-K sum inside the call and left to the caller."""
    import torch
    import _sx8lib as _L
    P = _L.ptr
    st = _L.stream(cuda)
    K = nh * hd
    n_cb = K // 32
    g = torch.Generator().manual_seed(nh * 17 + T + start)
    q = torch.randn(T, nh, hd, generator=g).half().to(cuda)
    kc = torch.full((nk, L, hd), float("nan")).half()
    vc = torch.full((nk, L, hd), float("nan")).half()
    kc[:, :start + T] = torch.randn(nk, start + T, hd, generator=g).half()
    vc[:, :start + T] = torch.randn(nk, start + T, hd, generator=g).half()
    kd, vd = kc.to(cuda), vc.to(cuda)
    ts = _mats(cuda, [N], K, 900 + T, hb)
    hdr, lvl, bas, sca = ts[0]
    scale = 1.0 / math.sqrt(hd)
    print("attn packed", nh, nk, hd, L, T, start, N, hb, flush=True)
    out = torch.empty(T, K, dtype=torch.float16, device=cuda)
    _L.call("sx8_dec_attn_prefill", P(q), P(kd), P(vd), P(out), T, start, nh, nk, hd, L, scale, st)
    Gs = (T + 31) // 32
    Xp = torch.full((Gs * n_cb * 1024,), 0x7E7E, dtype=torch.int16, device=cuda)   # sentinel bytes
    Zhl = torch.full((T * n_cb * 4,), 0x7E7E, dtype=torch.int16, device=cuda)
    _L.call("sx8_dec_attn_prefill_packed", P(q), P(kd), P(vd), T, start, nh, nk, hd, L, scale, P(bas), P(sca),
            P(Xp), P(Zhl), st)
    Zf = torch.empty(T, n_cb, 2, device=cuda)
    _L.call("sx8_compute_z", P(out), T, K, P(bas), P(sca), n_cb, P(Zf), st)
    torch.cuda.synchronize()
    xp_ref, zhl_ref = _packed_operands_ref(out.cpu().view(torch.int16).numpy().view(np.uint16),
                                           Zf.cpu().numpy(), n_cb)
    assert np.array_equal(Xp.cpu().numpy().view(np.uint16), xp_ref)
    assert np.array_equal(Zhl.cpu().numpy().view(np.uint16), zhl_ref)
    # the GEMM on the producer's operands
    ws, nb = _L.gemm_workspace(T, [N], n_cb, cuda)
    ya = torch.empty(T, N, device=cuda)
    ga = _group(ts, [N], n_cb, [ya])
    _L.call("sx8_gemm_prefill_group", P(out), T, K, K, ga[0], ga[1], ga[2], hb, ga[3], ga[4], ga[5], ga[6], ga[7],
            P(ws), nb, st)
    nbp = int(_L.lib().sx8_gemm_prefill_packed_workspace_bytes(T, 1, (ctypes.c_int64 * 1)(N), n_cb))
    assert 0 <= nbp <= nb
    wsp = torch.empty(max(nbp, 256), dtype=torch.uint8, device=cuda)
    zp = (ctypes.c_void_p * 1)(Zhl.data_ptr())
    yb = torch.empty(T, N, device=cuda)
    gb = _group(ts, [N], n_cb, [yb])
    _L.call("sx8_gemm_prefill_packed", P(Xp), zp, T, K, 1, gb[1], gb[2], hb, gb[5], n_cb, gb[7],
            P(wsp) if nbp else None, nbp, None, None, None, st)
    yc = torch.empty(T, N, device=cuda)
    gc = _group(ts, [N], n_cb, [yc])
    parts, n_parts, slc = _deferred("sx8_gemm_prefill_packed", P(Xp), zp, T, K, 1, gc[1], gc[2], hb, gc[5], n_cb,
                                    gc[7], P(wsp) if nbp else None, nbp, st)
    yd = yc.clone()
    if n_parts:                        # the slices sit in the workspace; added in slice order
        assert slc == T * N
        off = (parts - wsp.data_ptr()) // 4
        f = wsp.view(torch.float32)
        for s in range(n_parts):
            yd += f[off + s * slc:off + s * slc + T * N].view(T, N)
    torch.cuda.synchronize()
    print("   plan", _L.gemm_plan(T, [N], n_cb), "n_parts", n_parts, flush=True)
    assert torch.equal(ya.cpu(), yb.cpu())
    assert torch.equal(ya.cpu(), yd.cpu())


@pytest.mark.parametrize("M,K,N,hb", [
    (512, 2560, 9728, 6),     # the prompt pass's gate/up at T = 512: whole 512-row tiles (fused)
    (512, 2560, 9728, 8),
    (700, 640, 1536, 6),      # ragged rows
    (2048, 2560, 9728, 6),    # split tail tiles: the group GEMM + pack pass form
    (96, 512, 1000, 6),       # small M, N not a multiple of 32
    (512, 2560, 9760, 6),     # whole tiles with a half-empty last paired tile (N = 152.5 x 64)
])
def test_gateup_silu_packed_operands(hiplib, cuda, monkeypatch, M, K, N, hb):
    """sx8_dec_gemm_gateup_silu writes, bit for bit, the down projection's packed X and Zhl of
    x = sx8_dec_silu_mul(gate X, up X) (sx8_gemm_prefill_group for g and u, sx8_compute_z for
    Z), in both of its forms: the paired-tile GEMM with the SiLU epilogue and the group GEMM +
    pack pass (SX8_GEMM_W2=0 takes the second); the down GEMM on them equals
    sx8_gemm_prefill on x."""
    import torch
    import _sx8lib as _L
    P = _L.ptr
    st = _L.stream(cuda)
    n_cb = (K + 31) // 32
    n_cb_d = (N + 31) // 32
    ts = _mats(cuda, [N, N], K, 40 + M, hb)
    dn = _mats(cuda, [256], N, 70 + M, hb)[0]                   # a down-like matrix: K = N
    g = torch.Generator().manual_seed(M + N)
    X = torch.randn(M, K, generator=g).half().to(cuda)
    # reference: g, u by the group GEMM, x by the SiLU launch, Z by sx8_compute_z
    ws, nb = _L.gemm_workspace(M, [N, N], n_cb, cuda)
    gu = [torch.empty(M, N, device=cuda) for _ in range(2)]
    ga = _group(ts, [N, N], n_cb, gu)
    _L.call("sx8_gemm_prefill_group", P(X), M, K, K, ga[0], ga[1], ga[2], hb, ga[3], ga[4], ga[5], ga[6], ga[7],
            P(ws), nb, st)
    x = torch.zeros(M, n_cb_d * 32, dtype=torch.float16, device=cuda)
    xs = torch.empty(M, N, dtype=torch.float16, device=cuda)
    _L.call("sx8_dec_silu_mul", P(gu[0]), P(gu[1]), P(xs), M * N, st)
    x[:, :N] = xs
    Zf = torch.empty(M, n_cb_d, 2, device=cuda)
    _L.call("sx8_compute_z", P(x), M, n_cb_d * 32, P(dn[2]), P(dn[3]), n_cb_d, P(Zf), st)
    torch.cuda.synchronize()
    xp_ref, zhl_ref = _packed_operands_ref(x.cpu().view(torch.int16).numpy().view(np.uint16), Zf.cpu().numpy(),
                                           n_cb_d)
    Gs = (M + 31) // 32
    print("gateup silu plan (group tiling)", _L.gemm_plan(M, [N, N], n_cb), flush=True)
    for w2 in ("1", "0"):
        monkeypatch.setenv("SX8_GEMM_W2", w2)
        _L.lib().sx8_gemm_reload_tuning()
        print("gateup silu", M, K, N, hb, "w2", w2, flush=True)
        need = int(_L.lib().sx8_dec_gemm_gateup_silu_workspace_bytes(M, N, n_cb))
        wsg = torch.empty(need, dtype=torch.uint8, device=cuda)
        Xp = torch.full((Gs * n_cb_d * 1024,), 0x7E7E, dtype=torch.int16, device=cuda)
        Zhl = torch.full((M * n_cb_d * 4,), 0x7E7E, dtype=torch.int16, device=cuda)
        _L.call("sx8_dec_gemm_gateup_silu", P(X), None, None, M, K, ga[1], ga[2], hb, ga[3], ga[4], N, n_cb, P(dn[2]),
                P(dn[3]), P(Xp), P(Zhl), P(wsg), need, st)
        torch.cuda.synchronize()
        assert np.array_equal(Xp.cpu().numpy().view(np.uint16), xp_ref)
        assert np.array_equal(Zhl.cpu().numpy().view(np.uint16), zhl_ref)
    monkeypatch.delenv("SX8_GEMM_W2")
    _L.lib().sx8_gemm_reload_tuning()
    # the down GEMM on the packed operands against sx8_gemm_prefill on x
    yd = torch.empty(M, 256, device=cuda)
    wsd, nbd = _L.gemm_workspace(M, [256], n_cb_d, cuda)
    _L.call("sx8_gemm_prefill", P(x), M, n_cb_d * 32, n_cb_d * 32, P(dn[0]), P(dn[1]), hb, P(dn[2]), P(dn[3]), 256,
            n_cb_d, P(yd), P(wsd), nbd, st)
    yp = torch.empty(M, 256, device=cuda)
    gd = _group([dn], [256], n_cb_d, [yp])
    _L.call("sx8_gemm_prefill_packed", P(Xp), (ctypes.c_void_p * 1)(Zhl.data_ptr()), M, N, 1, gd[1], gd[2], hb, gd[5],
            n_cb_d, gd[7], P(wsd), nbd, None, None, None, st)
    torch.cuda.synchronize()
    assert torch.equal(yd.cpu(), yp.cpu())


@pytest.mark.parametrize("M,H,n_mats,np_,form", [
    (512, 2560, 3, 5, "delta"),     # q/k/v's producer: the previous down projection's 5 slices
    (512, 2560, 2, 3, "delta"),     # gate/up's producer: o's 3 slices
    (77, 640, 1, 0, "init"),        # layer 0 (fp16 init, no delta), ragged rows
    (33, 4096, 4, 1, "delta"),      # the widest row, four matrices
    (64, 2560, 2, 2, "both"),       # fp16 init plus delta and its slices
    (40, 1024, 3, 0, "none"),       # the residual alone
])
def test_add_rmsnorm_packed_operands(hiplib, cuda, M, H, n_mats, np_, form):
    """sx8_dec_add_rmsnorm_packed writes the residual of sx8_dec_add_rmsnorm_parts and the
    packed X / Zhl of its fp16 rows (every byte, rows past M packed as zeros) bit for bit;
    sx8_gemm_prefill_packed on them equals sx8_gemm_prefill_group on the rows, and
    sx8_dec_gemm_gateup_silu takes them in place of X."""
    import torch
    import _sx8lib as _L
    P = _L.ptr
    st = _L.stream(cuda)
    n_cb = H // 32
    Ns = [256 + 64 * i for i in range(n_mats)]
    ts = _mats(cuda, Ns, H, 500 + M, 6)
    g = torch.Generator().manual_seed(M * 3 + H)
    resid0 = torch.randn(M, H, generator=g).to(cuda)
    delta = torch.randn(M, H, generator=g).to(cuda)
    init = torch.randn(M, H, generator=g).half().to(cuda)
    parts = torch.randn(max(np_, 1), M * H + 8, generator=g).to(cuda)
    slc = M * H + 8                                             # a slice longer than the rows
    w = (torch.rand(H, generator=g) + 0.5).half().to(cuda)
    d_arg = P(delta) if form in ("delta", "both") else None
    i_arg = P(init) if form in ("init", "both") else None
    pp = P(parts) if np_ else None
    print("rmsnorm packed", M, H, n_mats, np_, form, flush=True)
    ra, xa = resid0.clone(), torch.empty(M, H, dtype=torch.float16, device=cuda)
    _L.call("sx8_dec_add_rmsnorm_parts", P(ra), d_arg, i_arg, P(w), P(xa), M, H, 1e-6, pp, np_, slc, st)
    rb = resid0.clone()
    Gs = (M + 31) // 32
    Xp = torch.full((Gs * n_cb * 1024,), 0x7E7E, dtype=torch.int16, device=cuda)
    Zs = [torch.full((M * n_cb * 4,), 0x7E7E, dtype=torch.int16, device=cuda) for _ in range(n_mats)]
    V = ctypes.c_void_p * n_mats
    _L.call("sx8_dec_add_rmsnorm_packed", P(rb), d_arg, i_arg, P(w), M, H, 1e-6, pp, np_, slc, n_mats,
            V(*[t[2].data_ptr() for t in ts]), V(*[t[3].data_ptr() for t in ts]), P(Xp),
            V(*[z.data_ptr() for z in Zs]), st)
    torch.cuda.synchronize()
    assert torch.equal(ra.cpu(), rb.cpu())
    x16 = xa.cpu().view(torch.int16).numpy().view(np.uint16)
    for i, t in enumerate(ts):
        Zf = torch.empty(M, n_cb, 2, device=cuda)
        _L.call("sx8_compute_z", P(xa), M, H, P(t[2]), P(t[3]), n_cb, P(Zf), st)
        torch.cuda.synchronize()
        xp_ref, zhl_ref = _packed_operands_ref(x16, Zf.cpu().numpy(), n_cb)
        if i == 0:
            assert np.array_equal(Xp.cpu().numpy().view(np.uint16), xp_ref)
        assert np.array_equal(Zs[i].cpu().numpy().view(np.uint16), zhl_ref), i
    # the GEMM on the operands
    ws, nb = _L.gemm_workspace(M, Ns, n_cb, cuda)
    ya = [torch.empty(M, N, device=cuda) for N in Ns]
    ga = _group(ts, Ns, n_cb, ya)
    _L.call("sx8_gemm_prefill_group", P(xa), M, H, H, ga[0], ga[1], ga[2], 6, ga[3], ga[4], ga[5], ga[6], ga[7],
            P(ws), nb, st)
    yb = [torch.empty(M, N, device=cuda) for N in Ns]
    gb = _group(ts, Ns, n_cb, yb)
    _L.call("sx8_gemm_prefill_packed", P(Xp), V(*[z.data_ptr() for z in Zs]), M, H, n_mats, gb[1], gb[2], 6, gb[5],
            n_cb, gb[7], P(ws), nb, None, None, None, st)
    torch.cuda.synchronize()
    for a, b in zip(ya, yb):
        assert torch.equal(a.cpu(), b.cpu())
    if n_mats == 2:
        # gate/up on the packed operands = gate/up on the rows
        N = Ns[0]
        t2 = _mats(cuda, [N, N], H, 600 + M, 6)
        dn = _mats(cuda, [64], N, 700 + M, 6)[0]
        Zg = [torch.empty(M * n_cb * 4, dtype=torch.int16, device=cuda) for _ in range(2)]
        rc = resid0.clone()
        _L.call("sx8_dec_add_rmsnorm_packed", P(rc), d_arg, i_arg, P(w), M, H, 1e-6, pp, np_, slc, 2,
                (ctypes.c_void_p * 2)(*[t[2].data_ptr() for t in t2]), (ctypes.c_void_p * 2)(*[t[3].data_ptr() for t in t2]),
                P(Xp), (ctypes.c_void_p * 2)(*[z.data_ptr() for z in Zg]), st)
        n_cb_d = (N + 31) // 32
        need = int(_L.lib().sx8_dec_gemm_gateup_silu_workspace_bytes(M, N, n_cb))
        wsg = torch.empty(need, dtype=torch.uint8, device=cuda)
        outs = []
        for packed in (False, True):
            XpD = torch.empty(Gs * n_cb_d * 1024, dtype=torch.int16, device=cuda)
            ZD = torch.empty(M * n_cb_d * 4, dtype=torch.int16, device=cuda)
            g2 = _group(t2, [N, N], n_cb, [])
            if packed:
                _L.call("sx8_dec_gemm_gateup_silu", None, P(Xp), (ctypes.c_void_p * 2)(*[z.data_ptr() for z in Zg]), M, H,
                        g2[1], g2[2], 6, g2[3], g2[4], N, n_cb, P(dn[2]), P(dn[3]), P(XpD), P(ZD), P(wsg), need, st)
            else:
                _L.call("sx8_dec_gemm_gateup_silu", P(xa), None, None, M, H, g2[1], g2[2], 6, g2[3], g2[4], N, n_cb,
                        P(dn[2]), P(dn[3]), P(XpD), P(ZD), P(wsg), need, st)
            torch.cuda.synchronize()
            outs.append((XpD.cpu(), ZD.cpu()))
        assert torch.equal(outs[0][0], outs[1][0]) and torch.equal(outs[0][1], outs[1][1])
