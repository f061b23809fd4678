"""Seeded random shapes through the decode GEMV and the prefill GEMM (GPU).

Twelve (N, K, M) drawn from a fixed generator -- N in [64, 3000), K in [32, 2048) (most
not a multiple of 32, so the last K block is ragged), M in [1, 300) -- with 6- and 8-byte
headers alternating.  Weights are seeded N(0, 0.02) fp16 quantized with 1% degenerate
blocks; W16 is the C oracle's canonical R64 dequant.  Bars as in the other parity tests:
the GEMV within 1e-3 of the oracle's float64 product, the GEMM (through whatever plan the
library picks for the shape) within 1e-3 of X . W16^T in float64.
"""
import numpy as np
import pytest

pytestmark = pytest.mark.gpu


def _cases():
    rng = np.random.default_rng(2027)
    out = []
    for i in range(12):
        N = int(rng.integers(64, 3000))
        K = int(rng.integers(32, 2048))
        M = int(rng.integers(1, 300))
        out.append((i, N, K, M, 6 if i % 2 == 0 else 8))
    return out


@pytest.mark.parametrize("i,N,K,M,hb", _cases())
def test_random_shape_gemv_and_gemm(hiplib, oracle, cuda, i, N, K, M, hb):
    import torch
    from quantize_sx8 import quantize_tensor
    from sx8_decode1_v3 import decode1_v44, make_tensors_v44
    from sx8_gemm_compact import gemm_sx8_compact
    print("fuzz", i, "N", N, "K", K, "M", M, "hdr", hb, flush=True)
    g = torch.Generator(device="cpu").manual_seed(9000 + i)
    W = (torch.randn(N, K, generator=g) * 0.02).half()
    qt, bi = quantize_tensor(W, device=cuda, degenerate_frac=0.01, seed=9100 + i)
    W16 = oracle.dequant_r64(qt, bi)                         # (N, K) fp16, the oracle's bits
    t = make_tensors_v44(qt, bi, hdr_aligned=(hb == 8))
    assert t[0].shape[-1] == hb
    # decode GEMV
    x = torch.randn(K, generator=g).half()
    y, _ = decode1_v44(x.to(cuda), qt, bi, *t, hdr_bytes=hb)
    y_ref = oracle.gemm_f64(x.numpy()[None], W16)[0]
    rel = oracle.rel_err(y.cpu().numpy().astype(np.float64), y_ref)
    print("   gemv rel", rel, flush=True)
    assert rel <= 1e-3
    # prefill GEMM, the planner's plan for this shape
    X = torch.randn(M, K, generator=g).half().to(cuda)
    Y = gemm_sx8_compact(X, qt, bi, *t, hdr_bytes=hb)
    Wd = torch.from_numpy(np.ascontiguousarray(W16)).to(cuda)
    Y_ref = X.double() @ Wd.double().T
    rel = ((Y.double() - Y_ref).abs().max() / Y_ref.abs().max()).item()
    print("   gemm rel", rel, flush=True)
    assert rel <= 1e-3
