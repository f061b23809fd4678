"""The product quantizer's deterministic half against the oracle (CPU); its PCA half
(scripts/quantize_qwen35_4b_sx8_v43_gpu.py:75-142) by known answers -- residual slices
whose principal directions, lower-median / 3 scales and coefficient bytes follow in
closed form, up to the singular-vector sign the decomposition returns (that sign depends
on the LAPACK / rocSOLVER build) -- and by invariants on quantized Gaussian weights."""
import numpy as np
import pytest
import torch


def _blocks(seed, n=4096):
    """fp16-valued blocks: Gaussian rows, exact-tie rows, constant (degenerate) rows,
    two-value rows and tiny-range rows."""
    rng = np.random.default_rng(seed)
    b = (rng.standard_normal((n, 32)) * 0.02).astype(np.float16)
    b[0:64] = b[0:64, :1]                                   # degenerate
    b[64:128] = np.where(rng.random((64, 32)) < 0.5, np.float16(-0.01), np.float16(0.02))
    b[128:192] = (np.float16(1.0) + rng.integers(0, 3, (64, 32)) * np.float16(2 ** -10)).astype(np.float16)
    b[192:256] = (rng.integers(-64, 64, (64, 32)) * np.float16(2 ** -12)).astype(np.float16)
    return b


def _kat_block():
    """One block whose four sub-blocks each lie exactly on one candidate's grid
    (dmin = 0, dmax = 63/64, q = 63/256): sub-block 0 on the full range (step 1/64), 1 on
    the lower quarter (step 1/256), 2 on the upper quarter [189/256, 252/256] (step 1/256),
    3 on the centre half [63/256, 189/256] (step 2/256), off the coarser grids."""
    lv = np.zeros(32, np.int64)
    lv[0:8] = [0, 63, 5, 17, 30, 41, 2, 60]           # full range: values lv/64
    lv[8:16] = [1, 3, 5, 7, 9, 13, 61, 62]            # j/256, j % 4 != 0
    lv[16:24] = [1, 2, 5, 6, 10, 33, 50, 62]          # (189 + j)/256
    lv[24:32] = [0, 1, 7, 12, 20, 33, 40, 63]         # (63 + 2j)/256, odd numerators
    x = np.empty(32)
    x[0:8] = lv[0:8] / 64
    x[8:16] = lv[8:16] / 256
    x[16:24] = (189 + lv[16:24]) / 256
    x[24:32] = (63 + 2 * lv[24:32]) / 256
    return x.astype(np.float16), lv, 0 | 1 << 2 | 2 << 4 | 3 << 6


def test_v6_known_answers(oracle):
    """Candidate order and ranges, the /63 step, rint and the strict-< tie rule, pinned by
    blocks with exact answers (both the oracle and the product's torch encoder)."""
    from quantize_sx8 import v6_encode_6bit
    x, lv, cfg = _kat_block()
    deg = np.full(32, np.float16(0.3))                   # degenerate: config 0, levels 0
    tie = x.copy()
    tie[8:16] = np.float16(0.0)                          # candidates 0 and 1 both exact: 0 wins
    b = np.stack([x, deg, tie]).astype(np.float32)
    for got in (oracle.v6_encode(b), tuple(t.numpy() for t in v6_encode_6bit(torch.from_numpy(b)))):
        glv, gmin, gmax, gcfg = got[0], got[1], got[2], got[3]
        assert np.array_equal(glv[0], lv) and int(gcfg[0]) == cfg
        assert gmin[0] == 0.0 and gmax[0] == np.float32(63 / 64)
        assert int(gcfg[1]) == 0 and not glv[1].any() and gmin[1] == gmax[1] == np.float32(np.float16(0.3))
        assert int(gcfg[2]) == cfg & ~0b1100 and not glv[2][8:16].any()


def test_torch_v6_encode_matches_oracle(oracle):
    from quantize_sx8 import v6_encode_6bit, pack_levels_6bit
    b = _blocks(3)
    lv, dmin, dmax, cfg = v6_encode_6bit(torch.from_numpy(b.astype(np.float32)))
    olv, odmin, odmax, ocfg, _ = oracle.v6_encode(b.astype(np.float32))
    assert np.array_equal(lv.numpy(), olv)
    assert np.array_equal(dmin.numpy(), odmin) and np.array_equal(dmax.numpy(), odmax)
    assert np.array_equal(cfg.numpy().astype(np.uint8), ocfg)
    hi, lo = pack_levels_6bit(lv.numpy())
    ohi, olo = oracle.pack_levels(olv)
    assert np.array_equal(hi, ohi) and np.array_equal(lo, olo)


# ------------------------------------------------------------- PCA known answers

def _hadamard(n):
    H = np.array([[1.0]])
    while H.shape[0] < n:
        H = np.block([[H, H], [H, -H]])
    return H


_PCA_K = np.array([1, -2, 3, -3, 4, -6, 9, 12])       # magnitudes k_w, w = 0..7
_PCA_A = np.array([8.0, 4.0, 2.0, 1.0])               # component weights: distinct energies
_PCA_TAU = 1.0 / 64
_PCA_ROWS = {0: (1, 2, 3, 5), 1: (6, 9, 12, 17)}      # Walsh rows used as directions per kb


def _pca_case():
    """Two K blocks (n_cb = 2) of 32 rows each.  Row r = 8u + w of block kb holds the
    residual sum_i c_i[r] V_i with V_i = Walsh row _PCA_ROWS[kb][i] / sqrt(32) (orthonormal)
    and c_i[r] = a_i H4[i, u] k_w tau.  The c_i are mutually orthogonal (H4 rows), so
    V_0..V_3 are the right singular vectors in order of a_i.  |c_i| takes the values
    a_i tau |k_w| four times each: sorted, positions 8-15 hold 3 and 16-19 hold 4, so the
    lower median (position 15 of 32) is 3 a_i tau and the scale a_i tau; c_i / scale =
    H4[i, u] k_w exactly, clamped to [-8, 7].  dmin = dmax = 0, levels 0, config 0 make the
    V6 reconstruction zero, so the residual equals the block values."""
    H32, H4 = _hadamard(32) / np.sqrt(32.0), _hadamard(4)
    n_rows, n_cb = 32, 2
    blocks = np.zeros((n_rows, n_cb, 32))
    for kb in range(n_cb):
        V = H32[list(_PCA_ROWS[kb])]
        for r in range(n_rows):
            u, w = divmod(r, 8)
            c = _PCA_A * H4[:, u] * _PCA_K[w] * _PCA_TAU
            blocks[r, kb] = c @ V
    n_blk = n_rows * n_cb
    return (np.zeros((n_blk, 32), np.uint8), np.zeros(n_blk, np.float32), np.zeros(n_blk, np.float32),
            np.zeros(n_blk, np.uint8), blocks.reshape(n_blk, 32).astype(np.float32), n_cb, H32, H4)


def _check_pca_known_answers(coeff, data, scales):
    _, _, _, _, _, n_cb, H32, H4 = _pca_case()
    coeff = np.asarray(coeff).reshape(32, n_cb)
    data = np.asarray(data, np.float64).reshape(n_cb, 2, 32)
    scales = np.asarray(scales, np.float64).reshape(n_cb, 2)
    for kb in range(n_cb):
        V = H32[list(_PCA_ROWS[kb])]
        cq = []
        for i in range(2):
            # the kept direction is +-V_i; its sign decides the coefficient signs
            sgn = np.sign(data[kb, i] @ V[i])
            assert np.allclose(data[kb, i], sgn * V[i], atol=1e-5), (kb, i)
            assert abs(scales[kb, i] - _PCA_A[i] * _PCA_TAU) <= 1e-5 * _PCA_A[i] * _PCA_TAU, (kb, i)
            cq.append(np.array([np.clip(sgn * H4[i, r // 8] * _PCA_K[r % 8], -8, 7) for r in range(32)]))
        exp = (cq[0].astype(np.int64) & 0xF) | ((cq[1].astype(np.int64) & 0xF) << 4)
        assert np.array_equal(coeff[:, kb].astype(np.int64), exp), kb


def test_pca_known_answers_oracle(oracle):
    lv, dmin, dmax, cfg, blocks, n_cb, _, _ = _pca_case()
    _check_pca_known_answers(*oracle.pca_correct(lv, dmin, dmax, cfg, blocks, n_cb))


@pytest.mark.parametrize("plant", ["median/4", "upper_median", "vh1:3"])
def test_pca_known_answers_catch_planted_mistakes(oracle, plant):
    lv, dmin, dmax, cfg, blocks, n_cb, _, _ = _pca_case()
    with pytest.raises(AssertionError):
        _check_pca_known_answers(*oracle.pca_correct(lv, dmin, dmax, cfg, blocks, n_cb, _plant=plant))


def _product_pca(method, device):
    from quantize_sx8 import pca_correct
    lv, dmin, dmax, cfg, blocks, n_cb, _, _ = _pca_case()
    t = lambda a: torch.from_numpy(a).to(device)
    return pca_correct(t(lv), t(dmin), t(dmax), t(cfg), t(blocks), n_cb, pca_method=method)


@pytest.mark.parametrize("method", ["svd", "gram"])
def test_pca_known_answers_product_cpu(method):
    _check_pca_known_answers(*_product_pca(method, "cpu"))


@pytest.mark.gpu
@pytest.mark.parametrize("method", ["svd", "gram"])
def test_pca_known_answers_product_gpu(hiplib, cuda, method):
    _check_pca_known_answers(*_product_pca(method, cuda))


def test_cpu_quantizer_pca_invariants():
    from quantize_sx8 import quantize_tensor
    g = torch.Generator().manual_seed(5)
    W = (torch.randn(256, 96, generator=g) * 0.02).half()
    qt, bi = quantize_tensor(W, device="cpu")
    _check_pca(qt, bi, W.float().numpy())


def _check_pca(qt, bi, W):
    """Orthonormal bases, |c| <= 8, and the PCA-corrected reconstruction (float64) is no
    worse than the V6 one without the correction."""
    data = np.asarray(bi["data"], np.float64).reshape(-1, 2, 32)
    for kb in range(data.shape[0]):
        G = data[kb] @ data[kb].T
        if np.any(G):
            assert np.allclose(G, np.eye(2), atol=1e-5)
    cf = np.asarray(qt["coeff"]).reshape(-1)
    for c in (cf & 0xF, cf >> 4):
        s = np.where(c >= 8, c.astype(int) - 16, c.astype(int))
        assert s.min() >= -8 and s.max() <= 7
    import oracle as O
    full = O.dequant_r64(qt, bi).astype(np.float64)
    nopca = O.dequant_r64(qt, {"n_cb": bi["n_cb"], "data": np.zeros_like(bi["data"]),
                               "scales": np.zeros_like(bi["scales"])}).astype(np.float64)
    ref = np.asarray(W, np.float64)[:, :full.shape[1]]
    assert np.mean((full - ref) ** 2) <= np.mean((nopca - ref) ** 2)


@pytest.mark.gpu
def test_hip_v6_encode_matches_oracle(hiplib, oracle, cuda):
    from quantize_sx8 import v6_encode_hip
    b = _blocks(7, 8192)
    lv, dmin, dmax, cfg, hi, lo = v6_encode_hip(torch.from_numpy(b).to(cuda))
    olv, odmin, odmax, ocfg, _ = oracle.v6_encode(b.astype(np.float32))
    assert np.array_equal(lv.cpu().numpy(), olv)
    assert np.array_equal(dmin.cpu().numpy().astype(np.float32), odmin)
    assert np.array_equal(dmax.cpu().numpy().astype(np.float32), odmax)
    assert np.array_equal(cfg.cpu().numpy().astype(np.uint8), ocfg)
    ohi, olo = oracle.pack_levels(olv)
    assert np.array_equal(hi.cpu().numpy(), ohi) and np.array_equal(lo.cpu().numpy(), olo)


@pytest.mark.gpu
@pytest.mark.parametrize("N,K", [(1024, 2560), (300, 80)])
def test_gpu_quantizer(hiplib, oracle, cuda, N, K):
    """GPU quantize_tensor: V6 fields identical to the CPU quantizer's (same bits), PCA by
    invariants (its bases come from a different decomposition, so they may differ)."""
    from quantize_sx8 import quantize_tensor
    g = torch.Generator().manual_seed(N + K)
    W = (torch.randn(N, K, generator=g) * 0.02).half()
    qg, bg = quantize_tensor(W, device=cuda, degenerate_frac=0.01, seed=1)
    qc, _ = quantize_tensor(W, device="cpu", degenerate_frac=0.01, seed=1)
    for k in ("dmin", "dmax", "config", "levels_hi", "levels_lo"):
        assert np.array_equal(np.asarray(qg[k]).view(np.uint8), np.asarray(qc[k]).view(np.uint8)), k
    Wd = W.float().numpy().copy()
    n_cb = qg["n_cb"]
    Wp = np.zeros((N, n_cb * 32), np.float32)
    Wp[:, :K] = Wd
    blk = Wp.reshape(-1, 32)
    gq = torch.Generator(device="cpu").manual_seed(1)
    idx = torch.randperm(blk.shape[0], generator=gq)[:int(round(0.01 * blk.shape[0]))].numpy()
    blk[idx] = blk[idx, :1]
    _check_pca(qg, bg, Wp[:, :K])
