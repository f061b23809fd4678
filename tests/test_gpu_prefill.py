"""GPU parity of the prefill GEMM at the configuration its throughput is quoted on
(the seven Qwen3-4B-class layer shapes at M = 128, 512 and
2048, each through the plan the library picks), the grouped calls a prompt pass makes,
the MFMA operand decode bit for bit, and HIP-graph capture of the wrapper.

Yardstick (the reference's own fused-GEMM check, scripts/sx8_fused_wmma.py:107-132, with
float64 in place of its float32 matmul): max|Y - Y_ref| / max|Y_ref| <= 1e-3 with
Y_ref = X . W16^T accumulated in float64, W16 the canonical R64 dequant.  W16 comes from
the device dequant, checked bit for bit against the C oracle first; the float64 product
runs on the GPU and a few of its rows are checked against the oracle's float64 GEMM.
"""
import ctypes

import numpy as np
import pytest

pytestmark = pytest.mark.gpu

LAYER = [("q_proj", 4096, 2560), ("k_proj", 1024, 2560), ("v_proj", 1024, 2560),
         ("o_proj", 2560, 4096), ("gate_proj", 9728, 2560), ("up_proj", 9728, 2560),
         ("down_proj", 2560, 9728)]
SEED = {name: 1000 + i for i, (name, _, _) in enumerate(LAYER)}
SHAPE = {name: (N, K) for name, N, K in LAYER}
TOL = 1e-3


def _say(*a):
    print(*a, flush=True)


_W = {}


def _weight(name, cuda, oracle):
    """(qt, bi, v4.4 tensors, W16 on the device) for a layer shape: seeded N(0, 0.02)
    fp16, quantized on the GPU with 1% degenerate blocks (as bench.py builds the layer);
    the device R64 dequant checked against the C oracle bit for bit."""
    if name not in _W:
        import torch
        from kernel_sx8_v43 import decode_tensor_gpu_fast
        from prepare_v44 import to_v44_device
        from quantize_sx8 import quantize_tensor
        N, K = SHAPE[name]
        g = torch.Generator(device="cpu").manual_seed(SEED[name])
        W = (torch.randn(N, K, generator=g) * 0.02).half()
        qt, bi = quantize_tensor(W, device=cuda, degenerate_frac=0.01, seed=SEED[name] + 1)
        t = to_v44_device(qt, bi, hdr_aligned=False, device=cuda)
        W16 = decode_tensor_gpu_fast(qt, bi).to(cuda)
        exp = oracle.dequant_r64(qt, bi).view(np.uint16)
        assert np.array_equal(W16.cpu().numpy().view(np.uint16), exp), name
        _W[name] = (qt, bi, t, W16)
    return _W[name]


def _x(M, K, seed, cuda):
    import torch
    g = torch.Generator(device="cpu").manual_seed(seed)
    return torch.randn(M, K, generator=g).half().to(cuda)


def _ref64(X, W16):
    return X.double() @ W16.double().T


def _rel(Y, Yref):
    return ((Y.double() - Yref).abs().max() / Yref.abs().max()).item()


@pytest.mark.parametrize("M", [128, 512, 2048])
@pytest.mark.parametrize("name", [n for n, _, _ in LAYER])
def test_prefill_layer_shapes(hiplib, oracle, cuda, name, M):
    """gemm_sx8_compact (the plan the library picks) on every layer shape at every M of the
    prefill sweep, against the float64 yardstick."""
    import _sx8lib as L
    from sx8_gemm_compact import gemm_sx8_compact
    qt, bi, t, W16 = _weight(name, cuda, oracle)
    N, K = SHAPE[name]
    plan = L.gemm_plan(M, (N,), qt["n_cb"])
    _say("prefill", name, N, K, "M", M, "plan", plan)
    X = _x(M, K, 11 + M, cuda)
    Y = gemm_sx8_compact(X, qt, bi, *t)
    Yref = _ref64(X, W16)
    if M == 128:
        # the device float64 product against the C oracle's on a few rows
        rows = [0, 77, 127]
        Yc = oracle.gemm_f64(X[rows].cpu().numpy(), W16.cpu().numpy())
        assert np.max(np.abs(Yc - Yref[rows].cpu().numpy())) <= 1e-12 * np.max(np.abs(Yc))
    rel = _rel(Y, Yref)
    _say("   rel", rel)
    assert rel <= TOL


@pytest.mark.parametrize("group", [("q_proj", "k_proj", "v_proj"), ("gate_proj", "up_proj")])
def test_prefill_group_m2048(hiplib, oracle, cuda, group):
    """sx8_gemm_prefill_group as the prompt pass calls it, at M = 2048: every output within
    the bar of the float64 yardstick."""
    import torch
    import _sx8lib as L
    M = 2048
    mats = [_weight(n, cuda, oracle) for n in group]
    Ns = [SHAPE[n][0] for n in group]
    K = SHAPE[group[0]][1]
    n_cb = mats[0][0]["n_cb"]
    _say("prefill group", group, "M", M, "plan", L.gemm_plan(M, Ns, n_cb))
    X = _x(M, K, 5, cuda)
    ys = [torch.empty(M, N, device=cuda) for N in Ns]
    n = len(group)
    Pa = ctypes.c_void_p * n
    ws, nb = L.gemm_workspace(M, Ns, n_cb, cuda)
    L.call("sx8_gemm_prefill_group", L.ptr(X), M, K, K, n, Pa(*[m[2][0].data_ptr() for m in mats]),
           Pa(*[m[2][1].data_ptr() for m in mats]), 6, Pa(*[m[2][2].data_ptr() for m in mats]),
           Pa(*[m[2][3].data_ptr() for m in mats]), (ctypes.c_int64 * n)(*Ns), n_cb,
           Pa(*[y.data_ptr() for y in ys]), L.ptr(ws), nb, L.stream(cuda))
    for name, m, y in zip(group, mats, ys):
        rel = _rel(y, _ref64(X, m[3]))
        _say("   ", name, "rel", rel)
        assert rel <= TOL


def _operand_case(kind, cuda, oracle):
    import torch
    from quantize_sx8 import quantize_tensor
    if kind == "quantized":
        g = torch.Generator(device="cpu").manual_seed(31)
        W = (torch.randn(2560, 2560, generator=g) * 0.02).half()
        return quantize_tensor(W, device=cuda, degenerate_frac=0.01, seed=32)[0]
    if kind == "ragged":
        g = torch.Generator(device="cpu").manual_seed(33)
        W = (torch.randn(300, 80, generator=g) * 0.02).half()
        return quantize_tensor(W, device=cuda, degenerate_frac=0.05, seed=34)[0]
    import os
    import sys
    sys.path.insert(0, os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden"))
    from make_golden import fuzz_blocks
    return fuzz_blocks(np.random.default_rng(35), 256, 8)[0]


@pytest.mark.parametrize("kind", ["quantized", "fuzz", "ragged"])
def test_prefill_mfma_operand_bit_exact(hiplib, oracle, cuda, kind):
    """The fp16 operand the GEMM decodes for every weight, read back through the core-only
    GEMM with X = the identity (Y[k, n] = 1 * w(n, k) + zeros: exact in the float32
    accumulators), against the oracle's core_f16 bit for bit (-0 reads back as +0): the
    reference's float32 range parameters (cuda/sx8_fused_wmma.cu:70-94), step*lv + rlo
    rounded once to fp16.  Fuzz blocks: every strategy and level, degenerate, reversed and
    subnormal ranges."""
    import torch
    import _sx8lib as L
    from prepare_v44 import to_v44_device
    qt = _operand_case(kind, cuda, oracle)
    N, K = qt["shape"]
    n_cb = qt["n_cb"]
    zero = {"n_cb": n_cb, "data": np.zeros((n_cb, 64), np.float32), "scales": np.zeros((n_cb, 2), np.float32)}
    hdr, lvl, _, _ = to_v44_device(qt, zero, hdr_aligned=False, device=cuda)
    X = torch.eye(K, dtype=torch.float16, device=cuda)
    Y = torch.empty(K, N, dtype=torch.float32, device=cuda)
    ws, nb = L.gemm_workspace(K, (N,), n_cb, cuda)
    _say("operand", kind, N, K, L.gemm_plan(K, (N,), n_cb))
    L.call("sx8_gemm_prefill_core", L.ptr(X), K, K, K, L.ptr(hdr), L.ptr(lvl), 6, N, n_cb, L.ptr(Y),
           L.ptr(ws), nb, L.stream(cuda))
    got = Y.T.contiguous().cpu().numpy()
    exp = oracle.core_f16(qt).astype(np.float32)
    exp[exp == 0] = 0.0                                  # -0 -> +0
    diff = np.nonzero(got.view(np.uint32) != exp.view(np.uint32))
    _say("   mismatches", diff[0].size)
    assert diff[0].size == 0, (got[diff][:8], exp[diff][:8])
    # the operand is the reference's float32 decode without PCA, not R64: within 1 ulp
    r64 = oracle.dequant_r64(qt, zero).astype(np.float32)
    assert np.max(np.abs(got - r64)) <= np.max(np.abs(r64)) * 2.0 ** -10


def test_prefill_wrapper_graph_capture(hiplib, oracle, cuda):
    """gemm_sx8_compact captured in a HIP graph (its workspace and output come from torch's
    allocator inside the capture; the library allocates and synchronizes nothing) replays
    bit-identically to the eager call, with eager work on the same buffers in between."""
    import torch
    from sx8_gemm_compact import gemm_sx8_compact
    qt, bi, t, W16 = _weight("k_proj", cuda, oracle)
    X = _x(512, 2560, 7, cuda)
    eager = gemm_sx8_compact(X, qt, bi, *t)
    torch.cuda.synchronize()
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        gemm_sx8_compact(X, qt, bi, *t)                   # warm the graph pool's sizes
    torch.cuda.current_stream().wait_stream(s)
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        Yg = gemm_sx8_compact(X, qt, bi, *t)
    for i in range(4):
        Yg.fill_(float("nan"))
        other = gemm_sx8_compact(_x(512, 2560, 100 + i, cuda), qt, bi, *t)   # eager in between
        graph.replay()
        torch.cuda.synchronize()
        assert torch.equal(Yg, eager), i
        assert not torch.equal(other, eager)


# ------------------------------------------------------------ 8-byte headers
# The reference's compact GEMM is instantiated for 6- and 8-byte headers
# (cuda/sx8_gemm_compact.cu:55, HDR template; scripts/sx8_decode1_v3.py:57-66 builds the
# 8-byte form with hdr_aligned=True: two pad bytes after coeff).  The header width changes
# only the record stride, so every 8-byte call must give the 6-byte call's output bit for
# bit, besides meeting the float64 yardstick.

_T8 = {}


def _t8(name, cuda, oracle):
    """The v4.4 tensors of a layer shape with 8-byte headers."""
    if name not in _T8:
        from prepare_v44 import to_v44_device
        qt, bi, t6, _ = _weight(name, cuda, oracle)
        t8 = to_v44_device(qt, bi, hdr_aligned=True, device=cuda)
        h6 = t6[0].reshape(-1, 6)
        h8 = t8[0].reshape(-1, 8)
        assert h8.shape[0] == h6.shape[0]
        assert np.array_equal(h8[:, :6].cpu().numpy(), h6.cpu().numpy())
        assert int(h8[:, 6:].abs().sum()) == 0
        assert np.array_equal(t8[1].cpu().numpy(), t6[1].cpu().numpy())
        _T8[name] = t8
    return _T8[name]


@pytest.mark.parametrize("name,M", [("gate_proj", 2048), ("down_proj", 2048), ("o_proj", 512),
                                    ("k_proj", 128)])
def test_prefill_hdr8_layer_shapes(hiplib, oracle, cuda, name, M):
    """gemm_sx8_compact(..., hdr_bytes=8) through the plan the library picks: within 1e-3
    of the float64 yardstick and bit-identical to the 6-byte-header call."""
    from sx8_gemm_compact import gemm_sx8_compact
    import _sx8lib as L
    qt, bi, t6, W16 = _weight(name, cuda, oracle)
    t8 = _t8(name, cuda, oracle)
    N, K = SHAPE[name]
    _say("prefill hdr8", name, N, K, "M", M, "plan", L.gemm_plan(M, (N,), qt["n_cb"]))
    X = _x(M, K, 21 + M, cuda)
    Y8 = gemm_sx8_compact(X, qt, bi, *t8, hdr_bytes=8)
    rel = _rel(Y8, _ref64(X, W16))
    _say("   rel", rel)
    assert rel <= TOL
    Y6 = gemm_sx8_compact(X, qt, bi, *t6, hdr_bytes=6)
    assert Y8.equal(Y6)


def test_prefill_hdr8_ragged(hiplib, oracle, cuda):
    """8-byte headers on a ragged shape: N not a multiple of the column tile, K not a
    multiple of 32 (last K block partly past the end), M not a multiple of 32."""
    import torch
    from kernel_sx8_v43 import decode_tensor_gpu_fast
    from prepare_v44 import to_v44_device
    from quantize_sx8 import quantize_tensor
    from sx8_gemm_compact import gemm_sx8_compact
    N, K, M = 1000, 2600, 300
    g = torch.Generator(device="cpu").manual_seed(77)
    W = (torch.randn(N, K, generator=g) * 0.02).half()
    qt, bi = quantize_tensor(W, device=cuda, degenerate_frac=0.02, seed=78)
    W16 = decode_tensor_gpu_fast(qt, bi).to(cuda)
    assert np.array_equal(W16.cpu().numpy().view(np.uint16), oracle.dequant_r64(qt, bi).view(np.uint16))
    X = _x(M, K, 79, cuda)
    t8 = to_v44_device(qt, bi, hdr_aligned=True, device=cuda)
    t6 = to_v44_device(qt, bi, hdr_aligned=False, device=cuda)
    Y8 = gemm_sx8_compact(X, qt, bi, *t8, hdr_bytes=8)
    rel = _rel(Y8, _ref64(X, W16))
    _say("prefill hdr8 ragged", N, K, M, "rel", rel)
    assert rel <= TOL
    assert Y8.equal(gemm_sx8_compact(X, qt, bi, *t6, hdr_bytes=6))


@pytest.mark.parametrize("group", [("q_proj", "k_proj", "v_proj"), ("gate_proj", "up_proj")])
def test_prefill_hdr8_group_m2048(hiplib, oracle, cuda, group):
    """sx8_gemm_prefill_group with 8-byte headers at M = 2048: every output within the bar
    of the float64 yardstick and bit-identical to the 6-byte-header group call."""
    import torch
    import _sx8lib as L
    M = 2048
    mats = [_weight(n, cuda, oracle) for n in group]
    t8s = [_t8(n, cuda, oracle) for n in group]
    Ns = [SHAPE[n][0] for n in group]
    K = SHAPE[group[0]][1]
    n_cb = mats[0][0]["n_cb"]
    _say("prefill hdr8 group", group, "M", M, "plan", L.gemm_plan(M, Ns, n_cb))
    X = _x(M, K, 25, cuda)
    n = len(group)
    Pa = ctypes.c_void_p * n

    def run(ts, hb):
        ys = [torch.empty(M, N, device=cuda) for N in Ns]
        ws, nb = L.gemm_workspace(M, Ns, n_cb, cuda)
        L.call("sx8_gemm_prefill_group", L.ptr(X), M, K, K, n, Pa(*[t[0].data_ptr() for t in ts]),
               Pa(*[t[1].data_ptr() for t in ts]), hb, Pa(*[t[2].data_ptr() for t in ts]),
               Pa(*[t[3].data_ptr() for t in ts]), (ctypes.c_int64 * n)(*Ns), n_cb,
               Pa(*[y.data_ptr() for y in ys]), L.ptr(ws), nb, L.stream(cuda))
        return ys

    y8 = run(t8s, 8)
    y6 = run([m[2] for m in mats], 6)
    for name, m, a, b in zip(group, mats, y8, y6):
        rel = _rel(a, _ref64(X, m[3]))
        _say("   ", name, "rel", rel)
        assert rel <= TOL
        assert a.equal(b), name


def test_prefill_hdr8_z_core_and_pca_z(hiplib, oracle, cuda):
    """The 8-byte-header forms of the caller-supplied-Z contract (gemm_compact ->
    sx8_gemm_prefill_z) and of the two-pass form (sx8_gemm_prefill_core + sx8_gemm_pca_z):
    each equal to its 6-byte-header call bit for bit and within the float64 yardstick."""
    import torch
    import _sx8lib as L
    from sx8_gemm_compact import _ext
    name, M = "q_proj", 512
    qt, bi, t6, W16 = _weight(name, cuda, oracle)
    t8 = _t8(name, cuda, oracle)
    N, K = SHAPE[name]
    n_cb = qt["n_cb"]
    X = _x(M, K, 27, cuda)
    Yref = _ref64(X, W16)
    ext = _ext()
    Z = ext.compute_z44_batch(X, t6[2], t6[3], n_cb)
    Yz8 = ext.gemm_compact(X, t8[0], t8[1], Z, n_cb, 8)
    Yz6 = ext.gemm_compact(X, t6[0], t6[1], Z, n_cb, 6)
    assert _rel(Yz8, Yref) <= TOL
    assert Yz8.equal(Yz6)

    def two_pass(t, hb):
        Yc = torch.empty(M, N, device=cuda)
        ws, nb = L.gemm_workspace(M, (N,), n_cb, cuda)
        L.call("sx8_gemm_prefill_core", L.ptr(X), M, K, K, L.ptr(t[0]), L.ptr(t[1]), hb, N, n_cb,
               L.ptr(Yc), L.ptr(ws), nb, L.stream(cuda))
        core = Yc.clone()
        L.call("sx8_gemm_pca_z", L.ptr(Z), M, L.ptr(t[0]), hb, N, n_cb, L.ptr(Yc), L.stream(cuda))
        return core, Yc

    c8, y8 = two_pass(t8, 8)
    c6, y6 = two_pass(t6, 6)
    assert c8.equal(c6) and y8.equal(y6)
    rel = _rel(y8, Yref)
    _say("prefill hdr8 two-pass rel", rel)
    assert rel <= TOL
    # the PCA pass added something: the core alone misses the PCA term
    assert not c8.equal(y8)


def test_prefill_hdr8_mfma_operand_bit_exact(hiplib, oracle, cuda):
    """The fp16 MFMA operand decoded from 8-byte headers, read back through the core-only
    GEMM with X = the identity, against the oracle's core_f16 bit for bit (fuzz blocks:
    every strategy and level, degenerate, reversed and subnormal ranges)."""
    import torch
    import _sx8lib as L
    from prepare_v44 import to_v44_device
    qt = _operand_case("fuzz", cuda, oracle)
    N, K = qt["shape"]
    n_cb = qt["n_cb"]
    zero = {"n_cb": n_cb, "data": np.zeros((n_cb, 64), np.float32), "scales": np.zeros((n_cb, 2), np.float32)}
    hdr, lvl, _, _ = to_v44_device(qt, zero, hdr_aligned=True, device=cuda)
    X = torch.eye(K, dtype=torch.float16, device=cuda)
    Y = torch.empty(K, N, dtype=torch.float32, device=cuda)
    ws, nb = L.gemm_workspace(K, (N,), n_cb, cuda)
    L.call("sx8_gemm_prefill_core", L.ptr(X), K, K, K, L.ptr(hdr), L.ptr(lvl), 8, N, n_cb, L.ptr(Y),
           L.ptr(ws), nb, L.stream(cuda))
    got = Y.T.contiguous().cpu().numpy()
    exp = oracle.core_f16(qt).astype(np.float32)
    exp[exp == 0] = 0.0
    assert np.array_equal(got.view(np.uint32), exp.view(np.uint32))
