"""sx8_gemm_prefill_static, the prefill entry point that allocates nothing (its scratch is
a device array inside the library), against sx8_gemm_prefill with a caller workspace,
through the C ABI: bit-identical when both run the same plan, on two calls in a row with
the second one smaller (the array keeps the first call's contents); a plan whose split-K
partials would not fit falls back to an unsplit one (same product up to the fp32
summation order); oversize calls are refused on the host."""
import ctypes

import numpy as np
import pytest

pytestmark = pytest.mark.gpu

SCRATCH = 64 << 20


def _say(*a):
    print(*a, flush=True)


def _case(N, K, M, seed, cuda):
    import torch
    from prepare_v44 import to_v44_device
    from quantize_sx8 import quantize_tensor
    g = torch.Generator(device="cpu").manual_seed(seed)
    W = (torch.randn(N, K, generator=g) * 0.02).half()
    qt, bi = quantize_tensor(W, device=cuda, degenerate_frac=0.01, seed=seed + 1)
    t = to_v44_device(qt, bi, hdr_aligned=False, device=cuda)
    X = torch.randn(M, K, generator=g).half().to(cuda)
    return qt, bi, t, X


def _with_workspace(L, X, t, N, n_cb, cuda):
    import torch
    M, K = X.shape
    Y = torch.empty(M, N, device=cuda)
    ws, nb = L.gemm_workspace(M, (N,), n_cb, cuda)
    L.call("sx8_gemm_prefill", L.ptr(X), M, K, K, L.ptr(t[0]), L.ptr(t[1]), 6, L.ptr(t[2]), L.ptr(t[3]), N,
           n_cb, L.ptr(Y), L.ptr(ws), nb, L.stream(cuda))
    return Y


def _static(L, X, t, N, n_cb, cuda):
    import torch
    M, K = X.shape
    Y = torch.full((M, N), float("nan"), device=cuda)
    L.call("sx8_gemm_prefill_static", L.ptr(X), M, K, K, L.ptr(t[0]), L.ptr(t[1]), 6, L.ptr(t[2]),
           L.ptr(t[3]), N, n_cb, L.ptr(Y), L.stream(cuda))
    return Y


def _ref_rel(Y, X, qt, bi, cuda):
    from kernel_sx8_v43 import decode_tensor_gpu_fast
    W16 = decode_tensor_gpu_fast(qt, bi).to(cuda)
    ref = X.double() @ W16.double().T
    return ((Y.double() - ref).abs().max() / ref.abs().max()).item()


def test_static_matches_workspace_path_twice(hiplib, cuda):
    """Two calls in a row, the second smaller: each output equals sx8_gemm_prefill's."""
    import torch
    import _sx8lib as L
    for N, K, M, seed in [(4096, 2560, 512, 11), (1024, 2560, 130, 12)]:
        qt, bi, t, X = _case(N, K, M, seed, cuda)
        plan = L.gemm_plan(M, (N,), qt["n_cb"])
        _say("static", N, K, M, plan)
        assert plan["workspace"] <= SCRATCH                 # same plan on both paths
        Yw = _with_workspace(L, X, t, N, qt["n_cb"], cuda)
        Ys = _static(L, X, t, N, qt["n_cb"], cuda)
        torch.cuda.synchronize()
        assert torch.equal(Ys, Yw)
        rel = _ref_rel(Ys, X, qt, bi, cuda)
        _say("   rel", rel)
        assert rel <= 1e-3


def test_static_caps_split_partials(hiplib, cuda):
    """down_proj at M = 2048: the workspace path's split-K plan needs more partial bytes than
    the array has left after Z and the packed X, so the static call runs an unsplit plan."""
    import torch
    import _sx8lib as L
    N, K, M = 2560, 9728, 2048
    qt, bi, t, X = _case(N, K, M, 13, cuda)
    plan = L.gemm_plan(M, (N,), qt["n_cb"])
    _say("static capped", plan)
    assert plan["workspace"] > SCRATCH and plan["k_ranges"] > 1
    Yw = _with_workspace(L, X, t, N, qt["n_cb"], cuda)
    Ys = _static(L, X, t, N, qt["n_cb"], cuda)
    torch.cuda.synchronize()
    rel_w = ((Ys - Yw).abs().max() / Yw.abs().max()).item()
    rel = _ref_rel(Ys, X, qt, bi, cuda)
    _say("   vs workspace path", rel_w, "vs float64", rel)
    assert rel_w <= 1e-5 and rel <= 1e-3


def test_static_refuses_oversize(hiplib):
    """Z plus the packed X beyond the array: refused on the host, before any launch."""
    import _sx8lib as L
    lib = L.lib()
    p = ctypes.c_void_p(4096)
    rc = lib.sx8_gemm_prefill_static(p, 4096, 9728, 9728, p, p, 6, p, p, 2560, 304, p, None)
    assert rc == 3
    assert "static scratch" in lib.sx8_last_error().decode()
