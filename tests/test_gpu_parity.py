"""GPU parity of the HIP hot path against the CPU oracle (run with -m gpu).

Bars:
  * dequantized fp16 weights (full-tensor dequant and embedding rows) are bit-exact to
    the canonical R64 dequant, including the degenerate-block step = 1e-10 floor (the
    prefill GEMM's MFMA operands follow the reference's float32 decode instead and are
    pinned against their own oracle recipe in test_gpu_prefill.py);
  * GEMV / GEMM outputs are within max|dY| / max|Y_ref| <= 1e-3 of the float64-
    accumulated X . W16^T (the reference's metric, sx8_fused_wmma.py:132).
"""
import os

import numpy as np
import pytest

pytestmark = pytest.mark.gpu
HERE = os.path.dirname(os.path.abspath(__file__))

SHAPES_4B = {  # name: (N, K)  -- BASELINE.json configs[1]
    "q_proj": (4096, 2560), "k_proj": (1024, 2560), "o_proj": (2560, 4096),
    "gate_proj": (9728, 2560), "down_proj": (2560, 9728),
}


def _say(*a):
    print(*a, flush=True)


def _golden_qt(prefix):
    g = np.load(os.path.join(HERE, "golden", "sx8_golden.npz"))
    out_f, in_f, n_cb = (int(v) for v in g[prefix + "shape"])
    qt = {"shape": (out_f, in_f), "orig_shape": (out_f, in_f), "n_blocks": out_f * n_cb,
          "n_cb": n_cb}
    for k in ("dmin", "dmax", "config", "levels_hi", "levels_lo", "coeff"):
        qt[k] = g[prefix + k]
    bi = {"n_cb": n_cb, "data": g[prefix + "basis"], "scales": g[prefix + "scales"]}
    return qt, bi, g[prefix + "w16"].reshape(out_f, in_f)


_QCACHE = {}


def _quantized(N, K, seed, cuda, degenerate=0.01):
    """Seeded N(0, 0.02) fp16 weight, quantized with 1% degenerate blocks."""
    key = (N, K, seed, degenerate)
    if key not in _QCACHE:
        import torch
        from quantize_sx8 import quantize_tensor
        g = torch.Generator(device="cpu").manual_seed(seed)
        W = (torch.randn(N, K, generator=g) * 0.02).half()
        _QCACHE[key] = quantize_tensor(W, device=cuda, degenerate_frac=degenerate, seed=seed + 1)
    return _QCACHE[key]


def _x(M, K, seed):
    import torch
    g = torch.Generator(device="cpu").manual_seed(seed)
    return torch.randn(M, K, generator=g).half()


# ------------------------------------------------------------------------ dequant

@pytest.mark.parametrize("prefix", ["fuzz_", "q_"])
def test_dequant_matches_golden(hiplib, cuda, prefix):
    import torch
    from kernel_sx8_v43 import decode_tensor_gpu_fast
    qt, bi, w16 = _golden_qt(prefix)
    _say("dequant golden", prefix, qt["shape"])
    W = decode_tensor_gpu_fast(qt, bi)
    torch.cuda.synchronize()
    assert np.array_equal(W.cpu().numpy().view(np.uint16), w16)
    out = torch.empty(qt["shape"], dtype=torch.float16, device=cuda)
    assert decode_tensor_gpu_fast(qt, bi, out=out) is out
    assert np.array_equal(out.cpu().numpy().view(np.uint16), w16)
    with pytest.raises(ValueError):
        decode_tensor_gpu_fast(qt, bi, out=torch.empty(3, 3, dtype=torch.float16, device=cuda))


@pytest.mark.parametrize("N,K", [(2560, 2560), (1024, 2560), (300, 80), (64, 4096)])
def test_dequant_quantized_bit_exact(hiplib, oracle, cuda, N, K):
    from kernel_sx8_v43 import decode_tensor_gpu_fast
    qt, bi = _quantized(N, K, 0 if (N, K) == (2560, 2560) else N + K, cuda)
    _say("dequant quantized", N, K)
    got = decode_tensor_gpu_fast(qt, bi).cpu().numpy().view(np.uint16)
    exp = oracle.dequant_r64(qt, bi).view(np.uint16)
    assert np.array_equal(got, exp)
    # the 1% degenerate blocks decode to their constant value
    dm = np.asarray(qt["dmin"]).view(np.uint16)
    dx = np.asarray(qt["dmax"]).view(np.uint16)
    deg = np.nonzero(dm == dx)[0]
    assert deg.size > 0
    n_cb = qt["n_cb"]
    for bid in deg[:50]:
        n, kb = divmod(int(bid), n_cb)
        cols = got[n, kb * 32:min(K, kb * 32 + 32)]
        v = dm[bid] if dm[bid] != 0x8000 else 0
        assert np.all(cols == v)


# ---------------------------------------------------------------------- embedding

@pytest.mark.parametrize("hdr_bytes", [6, 8])
def test_embed_gather_bit_exact(hiplib, oracle, cuda, hdr_bytes):
    import torch
    from sx8_decode1_v3 import make_tensors_v44
    from sx8_embed_v44 import SX8EmbeddingV44, ext
    N, K = 3000, 2560
    qt, bi = _quantized(N, K, 77, cuda)
    _say("embed", hdr_bytes)
    W = oracle.dequant_r64(qt, bi).view(np.uint16)
    g = torch.Generator(device="cpu").manual_seed(5)
    ids = torch.randint(0, N, (512,), generator=g)
    ids[7], ids[100], ids[511] = -1, N, N + 12          # out of range: rows untouched
    hdr, lvl, bas, sca = make_tensors_v44(qt, bi, hdr_aligned=(hdr_bytes == 8))
    out = torch.full((512, K), 7.0, dtype=torch.float16, device=cuda)
    ext().sx8_embed_v44(ids.to(cuda), hdr, lvl, bas, sca, K, N, qt["n_cb"], out)
    got = out.cpu().numpy().view(np.uint16)
    idn = ids.numpy()
    ok = (idn >= 0) & (idn < N)
    assert np.array_equal(got[ok], W[idn[ok]])
    assert np.all(got[~ok] == np.float16(7.0).view(np.uint16))
    emb = SX8EmbeddingV44(qt, bi, hdr_bytes=hdr_bytes)
    ids2 = torch.randint(0, N, (4, 33), generator=g).to(cuda)
    e = emb(ids2)
    assert e.shape == (4, 33, K)
    assert np.array_equal(e.cpu().numpy().view(np.uint16).reshape(-1, K), W[ids2.cpu().numpy().reshape(-1)])


def test_embed_ragged_k(hiplib, oracle, cuda):
    import torch
    from sx8_embed_v44 import SX8EmbeddingV44
    qt, bi = _quantized(257, 80, 9, cuda)              # K = 80: last block half used
    W = oracle.dequant_r64(qt, bi).view(np.uint16)
    ids = torch.tensor([0, 256, 3, 3, 128], device=cuda)
    e = SX8EmbeddingV44(qt, bi)(ids)
    assert np.array_equal(e.cpu().numpy().view(np.uint16), W[ids.cpu().numpy()])


# --------------------------------------------------------------------------- GEMV

GEMV_CASES = [("cpu_config", 2560, 2560, 0)] + [
    (k, n, kk, 1000 + i) for i, (k, (n, kk)) in enumerate(SHAPES_4B.items())] + [
    ("odd_N", 1000, 2560, 7), ("tiny", 65, 96, 8), ("ragged_K", 200, 80, 9),
    # n_cb = 512: table inputs beyond the three up-front passes; 64-column panels
    # with 10 rounds: the record-buffer ring
    ("long_K", 300, 16384, 10), ("wide_N", 20000, 2560, 11),
    # past 65536 columns: 128-column panels (four slices per column), the last one partial
    ("wide_panels", 70001, 256, 12)]


@pytest.mark.parametrize("hdr_bytes", [6, 8])
@pytest.mark.parametrize("name,N,K,seed", GEMV_CASES)
def test_gemv_within_1e3(hiplib, oracle, cuda, name, N, K, seed, hdr_bytes):
    import torch
    from sx8_decode1_v3 import _ext, decode1_v44, make_tensors_v44
    qt, bi = _quantized(N, K, seed, cuda)
    _say("gemv", name, N, K, hdr_bytes)
    x = _x(1, K, seed + 2)[0]
    W = oracle.dequant_r64(qt, bi)
    y_ref = oracle.gemm_f64(x.numpy()[None], W)[0]
    t = make_tensors_v44(qt, bi, hdr_aligned=(hdr_bytes == 8))
    Y, _ = decode1_v44(x.to(cuda), qt, bi, *t, hdr_bytes=hdr_bytes)
    y = Y.cpu().numpy().astype(np.float64)
    rel = oracle.rel_err(y, y_ref)
    _say("   rel", rel)
    assert rel <= 1e-3
    # the two-launch form (Z precomputed by compute_z44) agrees: its Z is the reference
    # tree, the single-launch form sums the 32 products left to right
    ext = _ext()
    Z = ext.compute_z44(x.to(cuda), t[2], t[3], qt["n_cb"])
    Y2 = ext.decode1_v44(x.to(cuda), t[0], t[1], Z, qt["n_cb"], hdr_bytes, 1)
    assert oracle.rel_err(Y2.cpu().numpy(), y_ref) <= 1e-3
    assert oracle.rel_err(Y2.cpu().numpy(), y) <= 1e-5
    # Z equals the reference's float32 warp tree bit for bit, from both entry points
    zref = oracle.z44_f32_tree(x.numpy(), bi)[0]
    assert np.array_equal(Z.cpu().numpy(), zref)
    Zc = torch.empty(qt["n_cb"], 2, dtype=torch.float32, device=cuda)
    Y3 = torch.empty(N, dtype=torch.float32, device=cuda)
    ext.decode1_v44_combined(x.to(cuda), t[0], t[1], t[2], t[3], qt["n_cb"], hdr_bytes, Zc, Y3)
    assert np.array_equal(Zc.cpu().numpy(), zref)
    assert oracle.rel_err(Y3.cpu().numpy(), y_ref) <= 1e-3


def test_gemv_deterministic_and_pool(hiplib, cuda):
    import torch
    from sx8_decode1_v3 import decode1_v44, make_tensors_v44
    qt, bi = _quantized(1024, 2560, 1001, cuda)      # 4-column panels, one round
    t = make_tensors_v44(qt, bi)
    x = _x(1, 2560, 3)[0].to(cuda)
    first = decode1_v44(x, qt, bi, *t)[0].clone()
    for _ in range(20):
        y, _ = decode1_v44(x, qt, bi, *t)
        assert torch.equal(y, first)
    # pooled output: same N -> same buffer, overwritten by the next call
    y2, _ = decode1_v44(x * 2, qt, bi, *t)
    assert y2.data_ptr() == y.data_ptr()


GROUP_CASES = [  # name, [N_i], K
    ("qkv", [4096, 1024, 1024], 2560), ("gate_up", [9728, 9728], 2560),
    ("ragged", [1000, 65, 300, 7], 96), ("long_K", [64, 100], 20512),
    # 70001 columns in all: a group on 128-column panels, each matrix ending in a partial one
    ("wide_group", [40000, 30001], 256)]


@pytest.mark.parametrize("name,Ns,K", GROUP_CASES)
def test_gemv_group_matches_single(hiplib, oracle, cuda, name, Ns, K):
    """One launch over weights that share x: each output within 1e-3 of the float64
    yardstick and within 1e-5 of the single-matrix GEMV (only the panel split, hence the
    fp32 summation order, differs).  long_K (n_cb = 641) takes the per-matrix path."""
    import torch
    from sx8_decode1_v3 import decode1_v44, decode1_v44_group, make_tensors_v44
    _say("gemv_group", name, Ns, K)
    x = _x(1, K, 77)[0]
    qts = [_quantized(N, K, 500 + i, cuda) for i, N in enumerate(Ns)]
    tens = [make_tensors_v44(qt, bi) for qt, bi in qts]
    n_cb = qts[0][0]["n_cb"]
    ys = decode1_v44_group(x.to(cuda), tens, Ns, n_cb)
    torch.cuda.synchronize()
    for i, ((qt, bi), t) in enumerate(zip(qts, tens)):
        y_ref = oracle.gemm_f64(x.numpy()[None], oracle.dequant_r64(qt, bi))[0]
        y = ys[i].cpu().numpy().astype(np.float64)
        rel = oracle.rel_err(y, y_ref)
        single = decode1_v44(x.to(cuda), qt, bi, *t)[0].cpu().numpy()
        _say("   ", i, "rel", rel, "vs single", oracle.rel_err(y, single))
        assert rel <= 1e-3
        assert oracle.rel_err(y, single) <= 1e-5


@pytest.mark.parametrize("hdr_bytes", [6, 8])
def test_container_load_v44_matches_to_v44(hiplib, oracle, cuda, tmp_path, hdr_bytes):
    """.sx8v43 -> device v4.4 layout through sx8_v43_to_v44: byte-identical to the numpy
    to_v44 (prepare_v44.py:35-79) for every tensor, and the loaded tensors drive the GEMV
    to the same output as tensors built in memory."""
    import torch
    import sx8_container_v43 as C
    from prepare_v44 import to_v44
    from sx8_decode1_v3 import decode1_v44, make_tensors_v44
    wd, bd = {}, {}
    for i, (N, K) in enumerate([(300, 2560), (64, 96), (1000, 80), (4096, 2560)]):
        wd[f"t{i}.weight"], bd[f"t{i}.weight"] = _quantized(N, K, 600 + i, cuda)
    path = tmp_path / "m.sx8v43"
    C.write_sx43((wd, bd, {"test": 1}), path, verbose=False)
    _say("container", hdr_bytes, path.stat().st_size)
    t44 = C.load_v44(path, device=cuda, hdr_bytes=hdr_bytes)
    torch.cuda.synchronize()
    for name, (qt, bi) in ((n, (wd[n], bd[n])) for n in sorted(wd)):
        ref = to_v44(qt, bi, hdr_aligned=(hdr_bytes == 8))
        hdr, lvl, bas, sca = t44[name]
        assert np.array_equal(hdr.cpu().numpy(), ref["hdr"]), name
        assert np.array_equal(lvl.cpu().numpy(), ref["levels"]), name
        assert np.array_equal(bas.cpu().numpy(), ref["bases"]), name
        assert np.array_equal(sca.cpu().numpy(), ref["scales"]), name
    qt, bi = wd["t3.weight"], bd["t3.weight"]
    x = _x(1, 2560, 41)[0].to(cuda)
    y_file = decode1_v44(x, qt, bi, *t44["t3.weight"], hdr_bytes=hdr_bytes)[0].clone()
    y_mem = decode1_v44(x, qt, bi, *make_tensors_v44(qt, bi, hdr_aligned=(hdr_bytes == 8)),
                        hdr_bytes=hdr_bytes)[0]
    assert torch.equal(y_file, y_mem)


@pytest.mark.parametrize("hdr_bytes", [6, 8])
def test_gguf_load_and_r32_ggml(hiplib, oracle, cuda, tmp_path, hdr_bytes):
    """GGUF SX8 tensors (convert_pkl_to_gguf_sx8.py's layout): sx8_blocks_to_v44 gives
    to_v44's bytes; the fork's no-PCA float32 dequant (R32-ggml) is bit-exact to the
    oracle with and without contraction, NaN blocks included; the GEMV on the GGUF tensors
    (zero PCA bases) is within 1e-3 of the float64 product with those weights."""
    import torch
    import sx8_gguf as G
    from prepare_v44 import to_v44
    from sx8_decode1_v3 import decode1_v44
    wd = {f"t{i}": _quantized(N, K, 700 + i, cuda)[0] for i, (N, K) in enumerate([(300, 2560), (1000, 96)])}
    path = tmp_path / "m.gguf"
    G.convert(wd, path)
    t44 = G.load_v44(path, device=cuda, hdr_bytes=hdr_bytes)
    torch.cuda.synchronize()
    for name, qt in wd.items():
        zero = {"n_cb": qt["n_cb"], "data": np.zeros((qt["n_cb"], 64), np.float32),
                "scales": np.zeros((qt["n_cb"], 2), np.float32)}
        ref = to_v44(qt, zero, hdr_aligned=(hdr_bytes == 8))
        assert np.array_equal(t44[name][0].cpu().numpy(), ref["hdr"]), name
        assert np.array_equal(t44[name][1].cpu().numpy(), ref["levels"]), name
        assert not t44[name][2].any() and not t44[name][3].any()
    # R32-ggml, bit for bit (golden fuzz blocks: degenerate, reversed, NaN/inf endpoints)
    g = np.load(os.path.join(HERE, "golden", "sx8_golden.npz"))
    fq = {"n_blocks": 384}
    for k in ("dmin", "dmax", "config", "levels_hi", "levels_lo", "coeff"):
        fq[k] = g["fuzz_" + k]
    cases = [(G.blockify(fq), 64, 6, 192)] + [
        (G.blockify(qt), qt["shape"][0], qt["n_cb"], qt["shape"][1]) for qt in wd.values()]
    for blocks, out_f, n_cb, in_f in cases:
        dev_blocks = torch.from_numpy(blocks.reshape(-1).copy()).to(cuda)
        for contract in (True, False):
            got = G.dequant_ggml(dev_blocks, out_f, n_cb, in_f, contract=contract).cpu().numpy()
            exp = oracle.dequant_ggml(blocks, contract).reshape(out_f, n_cb * 32)[:, :in_f]
            _say("r32-ggml", out_f, n_cb, in_f, contract)
            assert np.array_equal(got, exp, equal_nan=True)
            fin = np.isfinite(exp)
            assert np.array_equal(got[fin].view(np.uint32), exp[fin].view(np.uint32))
    # GEMV through the GGUF-loaded tensors
    qt = wd["t0"]
    x = _x(1, 2560, 51)[0]
    W = oracle.dequant_ggml(G.blockify(qt), True).reshape(300, 2560).astype(np.float64)
    y_ref = W @ x.numpy().astype(np.float64)
    y = decode1_v44(x.to(cuda), qt, None, *t44["t0"], hdr_bytes=hdr_bytes)[0].cpu().numpy()
    assert oracle.rel_err(y, y_ref) <= 1e-3


# -------------------------------------------------------------------------- GEMM

PREFILL_CASES = [
    ("q_proj", 4096, 2560, 128, "auto"), ("k_proj", 1024, 2560, 512, "auto"),
    ("down", 2560, 9728, 130, "auto"), ("odd", 1000, 2560, 7, "auto"), ("tiny", 64, 96, 1, "auto"),
    ("ragged_K", 300, 80, 33, "auto"),
    # the 512-row tile kernel (k_gemm_w2; k_gemm_w1 with SX8_GEMM_W2=0), forced: ragged M and N, split K, long K, the
    # 256-row kernel on the same shape for comparison
    ("w1_ragged", 1000, 2560, 700, "512"), ("w1_ragged_256", 1000, 2560, 700, "256"),
    ("w1_q", 4096, 2560, 1024, "512"), ("w1_long_k", 640, 9728, 600, "512"),
    ("w1_ragged_k", 384, 2080, 513, "512"),
    # 272 tiles of 512 x 128: one full round of 256, the other 16 split over K (partial tiles
    # added by the tile reducer)
    ("w1_tail", 17408, 640, 600, "512"),
    # the one-wave-per-SIMD 512-row kernel (k_gemm_w1, SX8_GEMM_W2=0) on the same kinds of case
    ("w1only_ragged", 1000, 2560, 700, "512w1"), ("w1only_long_k", 640, 9728, 600, "512w1"),
    ("w1only_tail", 17408, 640, 600, "512w1"),
]


@pytest.mark.parametrize("name,N,K,M,tile", PREFILL_CASES)
def test_prefill_gemm(hiplib, oracle, cuda, gemm_tuning, name, N, K, M, tile):
    import torch
    if tile == "512w1":
        gemm_tuning(TILE="512", W2="0")
    elif tile != "auto":
        gemm_tuning(TILE=tile)
    from sx8_decode1_v3 import make_tensors_v44
    from sx8_gemm_compact import _ext, gemm_sx8_compact
    from sx8_fused_wmma import gemm_sx8_wmma_cached, make_tensors, to_kbmajor
    qt, bi = _quantized(N, K, N * 3 + K, cuda)
    _say("prefill", name, N, K, M)
    X = _x(M, K, 11)
    W = oracle.dequant_r64(qt, bi)
    Y_ref = oracle.gemm_f64(X.numpy(), W)
    t = make_tensors_v44(qt, bi)
    Y = gemm_sx8_compact(X.to(cuda), qt, bi, *t)
    rel = oracle.rel_err(Y.cpu().numpy(), Y_ref)
    _say("   rel", rel)
    assert rel <= 1e-3
    # against fp32 accumulation over the exact fp16 W (the kernel rounds the PCA-free
    # core weights to fp16 and adds PCA through Z, so the two differ by fp16 rounding)
    Y32 = X.float() @ torch.from_numpy(W.astype(np.float32)).T
    _say("   rel vs fp32(W_R64)", oracle.rel_err(Y.cpu().numpy(), Y32.numpy()))
    assert oracle.rel_err(Y.cpu().numpy(), Y32.numpy()) <= 1e-3
    # the split-array (fused-WMMA) contract runs the same kernel: identical output
    kbm, _ = to_kbmajor(qt, bi)
    Yw = gemm_sx8_wmma_cached(X.to(cuda), make_tensors(kbm, bi, cuda), qt["n_cb"])
    assert torch.equal(Yw.cpu(), Y.cpu())
    # caller-supplied Z contract: same kernel, same Z values -> identical output
    ext = _ext()
    Xp = torch.zeros(M, qt["n_cb"] * 32, dtype=torch.float16)
    Xp[:, :K] = X
    Z = ext.compute_z44_batch(Xp.to(cuda), t[2], t[3], qt["n_cb"])
    Yz = ext.gemm_compact(Xp.to(cuda), t[0], t[1], Z, qt["n_cb"], 6)
    assert torch.equal(Yz.cpu(), Y.cpu())
    # two-pass form: core-only GEMM, then the output-side PCA pass over Z
    import _sx8lib as L
    Yc = torch.empty_like(Yz)
    Xd = Xp.to(cuda)
    ws, nb = L.gemm_workspace(M, (N,), qt["n_cb"], cuda)
    L.call("sx8_gemm_prefill_core", L.ptr(Xd), M, Xd.shape[1], Xd.shape[1], L.ptr(t[0]),
           L.ptr(t[1]), 6, N, qt["n_cb"], L.ptr(Yc), L.ptr(ws), nb, L.stream(cuda))
    L.call("sx8_gemm_pca_z", L.ptr(Z), M, L.ptr(t[0]), 6, N, qt["n_cb"], L.ptr(Yc), L.stream(cuda))
    assert oracle.rel_err(Yc.cpu().numpy(), Y_ref) <= 1e-3


def test_prefill_deterministic(hiplib, cuda):
    import torch
    from sx8_decode1_v3 import make_tensors_v44
    from sx8_gemm_compact import gemm_sx8_compact
    qt, bi = _quantized(1024, 2560, 1001, cuda)
    t = make_tensors_v44(qt, bi)
    X = _x(256, 2560, 4).to(cuda)
    a = gemm_sx8_compact(X, qt, bi, *t)
    for _ in range(5):
        assert torch.equal(gemm_sx8_compact(X, qt, bi, *t), a)


def test_prefill_small_n_fallback(hiplib, oracle, cuda):
    from sx8_gemm_compact import gemm_sx8_compact
    qt, bi = _quantized(32, 2560, 5, cuda)              # N < 64 -> dequant + F.linear
    X = _x(16, 2560, 6)
    Y = gemm_sx8_compact(X.to(cuda), qt, bi)
    Y_ref = oracle.gemm_f64(X.numpy(), oracle.dequant_r64(qt, bi))
    assert oracle.rel_err(Y.cpu().numpy(), Y_ref) <= 1e-3


# ------------------------------------------------------------------------ modules

def test_linear_module_dispatch(hiplib, oracle, cuda, monkeypatch):
    import torch
    from integrate_fused_v44 import SX8LinearV44
    qt, bi = _quantized(512, 2560, 21, cuda)
    bias = torch.randn(512, dtype=torch.float16, device=cuda)
    lin = SX8LinearV44(qt, bi, bias=bias)
    W = oracle.dequant_r64(qt, bi)
    for shape in [(1, 2560), (1, 1, 2560), (2, 9, 2560)]:
        x = _x(int(np.prod(shape[:-1])), 2560, 8).reshape(shape)
        y = lin(x.to(cuda))
        assert y.shape == (*shape[:-1], 512) and y.dtype == torch.float16
        ref = oracle.gemm_f64(x.reshape(-1, 2560).numpy(), W) + bias.float().cpu().numpy()
        assert oracle.rel_err(y.float().cpu().numpy().reshape(-1, 512), ref) <= 2e-3
    monkeypatch.setenv("SX8_USE_WMMA", "1")
    x = _x(5, 2560, 9)
    y = lin(x.to(cuda))
    ref = oracle.gemm_f64(x.numpy(), W) + bias.float().cpu().numpy()
    assert oracle.rel_err(y.float().cpu().numpy(), ref) <= 2e-3


def test_clone_model_replaces_linears(hiplib, cuda):
    import torch
    import torch.nn as nn
    from integrate_fused_v44 import SX8EmbeddingV44, SX8LinearV44, clone_model_fused_v44
    from quantize_sx8 import quantize_tensor

    class Tiny(nn.Module):
        def __init__(self):
            super().__init__()
            self.embed = nn.Embedding(100, 64)
            self.layers = nn.ModuleList([nn.Linear(64, 128), nn.Linear(128, 64)])

        def forward(self, ids):
            h = self.embed(ids)
            for l in self.layers:
                h = l(h)
            return h

    torch.manual_seed(0)
    m = Tiny().half().to(cuda)
    wd, bd = {}, {}
    for name, p in m.named_parameters():
        if p.dim() == 2:
            wd[name], bd[name] = quantize_tensor(p.detach().cpu(), device="cpu")
    ids = torch.tensor([[1, 5, 99]], device=cuda)
    with torch.no_grad():
        ref = m(ids).float()
    m2, n = clone_model_fused_v44(m, wd, bd)
    assert n == 3
    assert isinstance(m2.embed, SX8EmbeddingV44) and isinstance(m2.layers[0], SX8LinearV44)
    with torch.no_grad():
        out = m2(ids).float()
    assert (out - ref).abs().max().item() / ref.abs().max().item() < 5e-2


@pytest.mark.parametrize("name,Ns,K,M,tile", [
    ("qkv_m512", [4096, 1024, 1024], 2560, 512, "auto"),
    ("gate_up_m700_w1", [1000, 1300], 2560, 700, "512"),
    ("ragged_four", [300, 64, 129, 700], 80, 33, "auto"),
])
def test_prefill_gemm_group(hiplib, oracle, cuda, gemm_tuning, name, Ns, K, M, tile):
    """sx8_gemm_prefill_group against the oracle (1e-3) and against one sx8_gemm_prefill per
    matrix (the same kernel arithmetic; only the split-K summation order can differ)."""
    import ctypes
    import torch
    import _sx8lib as L
    from sx8_decode1_v3 import make_tensors_v44
    if tile == "512w1":
        gemm_tuning(TILE="512", W2="0")
    elif tile != "auto":
        gemm_tuning(TILE=tile)
    _say("prefill group", name, Ns, K, M)
    mats = [_quantized(N, K, 500 + i, cuda) for i, N in enumerate(Ns)]
    ts = [make_tensors_v44(qt, bi) for qt, bi in mats]
    n_cb = mats[0][0]["n_cb"]
    X = _x(M, K, 13)
    Xd = X.to(cuda)
    n = len(Ns)
    Pa = ctypes.c_void_p * n
    ys = [torch.empty(M, N, device=cuda) for N in Ns]
    ws, nb = L.gemm_workspace(M, Ns, n_cb, cuda)
    L.call("sx8_gemm_prefill_group", L.ptr(Xd), M, K, K, n, Pa(*[t[0].data_ptr() for t in ts]),
           Pa(*[t[1].data_ptr() for t in ts]), 6, Pa(*[t[2].data_ptr() for t in ts]),
           Pa(*[t[3].data_ptr() for t in ts]), (ctypes.c_int64 * n)(*Ns), n_cb,
           Pa(*[y.data_ptr() for y in ys]), L.ptr(ws), nb, L.stream(cuda))
    for i, (qt, bi) in enumerate(mats):
        y1 = torch.empty(M, Ns[i], device=cuda)
        t = ts[i]
        ws1, nb1 = L.gemm_workspace(M, (Ns[i],), n_cb, cuda)
        L.call("sx8_gemm_prefill", L.ptr(Xd), M, K, K, L.ptr(t[0]), L.ptr(t[1]), 6, L.ptr(t[2]), L.ptr(t[3]),
               Ns[i], n_cb, L.ptr(y1), L.ptr(ws1), nb1, L.stream(cuda))
        ref = oracle.gemm_f64(X.numpy(), oracle.dequant_r64(qt, bi))
        got = ys[i].cpu().numpy()
        assert oracle.rel_err(got, ref) <= 1e-3, i
        assert oracle.rel_err(got, y1.cpu().numpy()) <= 1e-5, i


def test_vocab_sized_tensor_full(hiplib, oracle, cuda):
    """BASELINE config 4 at its full size: one 151936 x 2560 S-X8 matrix (seeded N(0, 0.02),
    1% degenerate blocks).  lm_head GEMV (M = 1) within 1e-3 of the float64 oracle; prefill
    GEMM at M = 512 within 1e-3 of a float32 matmul of the bit-exact R64 weights; 512
    uniform ids gathered bit-exact against the oracle's rows."""
    import torch
    from kernel_sx8_v43 import decode_tensor_gpu_fast
    from sx8_decode1_v3 import decode1_v44, make_tensors_v44
    from sx8_embed_v44 import ext
    from sx8_gemm_compact import gemm_sx8_compact
    N, K = 151936, 2560
    qt, bi = _quantized(N, K, 4, cuda)
    _say("vocab", N, K)
    W = oracle.dequant_r64(qt, bi)                               # (N, K) fp16, the oracle's bits
    t = make_tensors_v44(qt, bi)
    x = _x(1, K, 21)
    y, _ = decode1_v44(x[0].to(cuda), qt, bi, *t)
    rel = oracle.rel_err(y.cpu().numpy(), oracle.gemm_f64(x.numpy(), W)[0])
    _say("   gemv rel", rel)
    assert rel <= 1e-3
    # the device dequant is the oracle's bits, so the GEMM reference can be an fp32 matmul
    Wd = decode_tensor_gpu_fast(qt, bi).to(cuda)
    assert np.array_equal(Wd.cpu().numpy().view(np.uint16), W.view(np.uint16))
    X = _x(512, K, 22).to(cuda)
    Y = gemm_sx8_compact(X, qt, bi, *t)
    Y32 = X.float() @ Wd.float().T
    rel = (Y - Y32).abs().max().item() / Y32.abs().max().item()
    _say("   gemm rel", rel)
    assert rel <= 1e-3
    del Y, Y32, Wd
    g = torch.Generator(device="cpu").manual_seed(23)
    ids = torch.randint(0, N, (512,), generator=g)
    out = torch.empty(512, K, dtype=torch.float16, device=cuda)
    ext().sx8_embed_v44(ids.to(cuda), t[0], t[1], t[2], t[3], K, N, qt["n_cb"], out)
    assert np.array_equal(out.cpu().numpy().view(np.uint16), W.view(np.uint16)[ids.numpy()])
