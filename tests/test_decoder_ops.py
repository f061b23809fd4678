"""The per-token decoder ops of include/sx8_decoder.h on the GPU against float32 torch
references (the same math as the decode loop of scripts/infer_sx8.py:109-173)."""
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
