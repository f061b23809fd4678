"""CPU-side checks of the C ABI: the library loads, exports every symbol that
include/*.h declare, and rejects bad arguments on the host (before any HIP
call) with an error code and a message.  No kernel is launched here."""
import ctypes
import glob
import os
import re

import pytest

REPO = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADERS = sorted(glob.glob(os.path.join(REPO, "include", "*.h")))


def _declared():
    text = "".join(open(h).read() for h in HEADERS)
    return sorted(set(re.findall(r"^\s*(?:int32_t|int64_t|const char\*)\s+(sx8_\w+)\s*\(", text, re.M)))


def test_header_declares_the_abi():
    names = _declared()
    assert "sx8_gemv" in names and "sx8_gemm_prefill" in names and "sx8_embed_gather" in names
    assert len(names) >= 10


def test_library_exports_every_declared_symbol(hiplib):
    import _sx8lib
    for name in _declared():
        assert hasattr(hiplib, name), name
    assert sorted(n for n, _, _ in _sx8lib.SIGNATURES) == _declared()
    assert hiplib.sx8_abi_version() == _sx8lib.ABI_VERSION


NULL = ctypes.c_void_p(None)


def _err(lib):
    return lib.sx8_last_error().decode()


def test_invalid_arguments_rejected_on_host(hiplib):
    L = hiplib
    p = ctypes.c_void_p(4096)   # never dereferenced: validation fails first
    # null pointers
    assert L.sx8_gemv(NULL, p, p, 6, p, p, NULL, NULL, 64, 2, p, NULL, 0, NULL) == 1
    assert "null" in _err(L)
    # hdr_bytes outside {6, 8}
    assert L.sx8_gemv(p, p, p, 7, p, p, NULL, NULL, 64, 2, p, NULL, 0, NULL) == 1
    assert "hdr_bytes" in _err(L)
    # misaligned Y, and a workspace that is too small
    assert L.sx8_gemv(p, p, p, 6, p, p, NULL, NULL, 64, 2, ctypes.c_void_p(4098), NULL, 0, NULL) == 1
    assert "misaligned" in _err(L)
    assert L.sx8_gemv(p, p, p, 6, p, p, NULL, NULL, 64, 2, p, p, 100, NULL) == 1
    assert "workspace" in _err(L)
    assert L.sx8_gemv_workspace_bytes(80) == 80 * 112
    # inconsistent K / n_cb
    assert L.sx8_dequant_f16(p, p, p, p, p, p, p, p, 4, 100, 2, p, NULL) == 1
    assert "bad shape" in _err(L)
    assert L.sx8_gemm_prefill(p, 4, 64, 64, p, p, 6, p, p, 0, 2, p, p, 1 << 20, NULL) == 1
    assert L.sx8_gemm_prefill(p, 4, 32, 64, p, p, 6, p, p, 64, 2, p, p, 1 << 20, NULL) == 1   # ldx < K
    assert L.sx8_embed_gather(p, 4, p, p, 5, p, p, 64, 10, 2, p, NULL) == 1
    assert L.sx8_compute_z(p, 1, 16, p, p, 1, p, NULL) == 1                      # ldx < 32
    assert L.sx8_compute_z(p, 1 << 26, 2048, p, p, 64, p, NULL) == 3             # M n_cb >= 2^31
    assert "2^31" in _err(L)
    assert L.sx8_gemm_pca_z(NULL, 1, p, 6, 64, 2, p, NULL) == 1
    assert L.sx8_gemm_prefill_z(p, 4, 64, 64, p, p, 6, NULL, 64, 2, p, p, 1 << 20, NULL) == 1   # Z missing
    assert L.sx8_gemm_prefill_z(p, 4, 64, 64, p, p, 6, p, 64, 3, p, p, 1 << 20, NULL) == 1      # n_cb != K/32


def test_gemv_group_rejects_bad_arguments(hiplib):
    L = hiplib
    p = ctypes.c_void_p(4096)
    P2 = ctypes.c_void_p * 2
    ptrs = P2(4096, 8192)
    ns = (ctypes.c_int64 * 2)(64, 32)
    # n_mats out of range, hdr_bytes, null bases without Z, misaligned X
    assert L.sx8_gemv_group(p, 0, ptrs, ptrs, 6, ptrs, ptrs, NULL, ns, 2, ptrs, NULL, 0, NULL) == 1
    assert "n_mats" in _err(L)
    assert L.sx8_gemv_group(p, 5, ptrs, ptrs, 6, ptrs, ptrs, NULL, ns, 2, ptrs, NULL, 0, NULL) == 1
    assert L.sx8_gemv_group(p, 2, ptrs, ptrs, 7, ptrs, ptrs, NULL, ns, 2, ptrs, NULL, 0, NULL) == 1
    assert "hdr_bytes" in _err(L)
    assert L.sx8_gemv_group(p, 2, ptrs, ptrs, 6, NULL, NULL, NULL, ns, 2, ptrs, NULL, 0, NULL) == 1
    assert "bases" in _err(L)
    assert L.sx8_gemv_group(ctypes.c_void_p(4098), 2, ptrs, ptrs, 6, ptrs, ptrs, NULL, ns, 2,
                            ptrs, NULL, 0, NULL) == 1
    bad_n = (ctypes.c_int64 * 2)(64, 0)
    assert L.sx8_gemv_group(p, 2, ptrs, ptrs, 6, ptrs, ptrs, NULL, bad_n, 2, ptrs, NULL, 0, NULL) == 1
    assert "bad N" in _err(L)
    # K beyond the LDS table (n_cb > 640) without the workspace it then needs
    assert L.sx8_gemv_group(p, 2, ptrs, ptrs, 6, ptrs, ptrs, NULL, ns, 641, ptrs, NULL, 0, NULL) == 1
    assert "workspace" in _err(L)


def test_workspace_contract(hiplib):
    """The library allocates nothing: prefill calls need a caller workspace of the size the
    query gives (256-byte aligned), and the GEMV's two-launch forms need theirs; a missing
    or short workspace is refused on the host."""
    L = hiplib
    p = ctypes.c_void_p(4096)
    N = (ctypes.c_int64 * 1)(4096)
    nb = L.sx8_gemm_prefill_workspace_bytes(2048, 1, N, 80)
    # Zhl (M * n_cb * 8) + packed X (M * n_cb * 64) at least
    assert nb >= 2048 * 80 * 72
    assert L.sx8_gemm_prefill_workspace_bytes(0, 1, N, 80) == -1
    assert L.sx8_gemm_prefill_workspace_bytes(16, 5, N, 80) == -1
    desc = (ctypes.c_int64 * 8)()
    assert L.sx8_gemm_prefill_plan(2048, 1, N, 80, desc) == 0
    assert desc[0] in (128, 256, 512) and desc[1] > 0 and desc[6] == nb
    # K = 2560 -> n_cb = 80; no workspace, a short one, a misaligned one
    assert L.sx8_gemm_prefill(p, 2048, 2560, 2560, p, p, 6, p, p, 4096, 80, p, NULL, 0, NULL) == 1
    assert "workspace" in _err(L)
    assert L.sx8_gemm_prefill(p, 2048, 2560, 2560, p, p, 6, p, p, 4096, 80, p, p, nb - 1, NULL) == 1
    assert "workspace" in _err(L)
    assert L.sx8_gemm_prefill(p, 2048, 2560, 2560, p, p, 6, p, p, 4096, 80, p, ctypes.c_void_p(4096 + 16),
                              nb, NULL) == 1
    assert "workspace" in _err(L)
    # GEMV: the Z-returning form needs the table workspace
    assert L.sx8_gemv(p, p, p, 6, p, p, NULL, p, 64, 2, p, NULL, 0, NULL) == 1
    assert "workspace" in _err(L)


def test_product_modules_import():
    """Every Python module of the package imports without a GPU (no work at import)."""
    import importlib
    for m in ("_sx8lib", "kernel_sx8_v43", "prepare_v44", "quantize_sx8", "sx8_decode1_v3",
              "sx8_embed_v44", "sx8_fused_wmma", "sx8_gemm_compact", "integrate_fused_v44",
              "e2e_decoder"):
        importlib.import_module(m)


def test_wrapper_raises_runtime_error(hiplib):
    import _sx8lib
    with pytest.raises(RuntimeError, match="hdr_bytes"):
        _sx8lib.call("sx8_gemv", ctypes.c_void_p(4096), ctypes.c_void_p(4096),
                     ctypes.c_void_p(4096), 9, ctypes.c_void_p(4096), ctypes.c_void_p(4096),
                     NULL, NULL, 64, 2, ctypes.c_void_p(4096), NULL, 0, NULL)


def test_missing_library_fails_loudly(monkeypatch, tmp_path):
    import _sx8lib
    monkeypatch.setattr(_sx8lib, "_lib", None)
    monkeypatch.setenv("SX8_HIP_LIB", str(tmp_path / "nope.so"))
    with pytest.raises(RuntimeError, match="not found"):
        _sx8lib.lib()


def test_decoder_pair_and_residual_refusals_on_host(hiplib):
    """sx8_dec_gemv_rmsnorm_pair reads the up matrix at the gate's pointers plus the gate's
    size: up arrays stored anywhere else are refused before any launch, as is an N the
    down GEMV (sx8_dec_gemv_zp_add) would refuse; the *_add GEMVs refuse a residual that
    overlaps an output without being it."""
    L = hiplib
    N, n_cb, hb = 9728, 80, 6
    n_blk = N * n_cb
    hdr, lvl, bas, sca = 1 << 28, 2 << 28, 3 << 28, 4 << 28
    up = [hdr + n_blk * hb, lvl + n_blk * 24, bas + n_cb * 64 * 4, sca + n_cb * 2 * 4]
    p = ctypes.c_void_p(4096)
    V = ctypes.c_void_p

    def pair(ups, Ncols=N, nc=n_cb):
        return L.sx8_dec_gemv_rmsnorm_pair(p, p, ctypes.c_float(1e-6), V(hdr), V(lvl), hb, V(bas), V(sca),
                                           *[V(u) for u in ups], Ncols, nc, p, p, p, NULL)

    for f in range(4):
        bad = list(up)
        bad[f] += 256
        assert pair(bad) == 1, f
        assert "follow the gate" in _err(L)
    assert pair(up, 12288 + 32) == 3 and "multiple of 32" in _err(L)
    assert pair(up, 16384) == 3
    # residual add: adds[0] 8 floats into Ys[0], and adds[1] == Ys[0] (another matrix's output)
    P2 = ctypes.c_void_p * 2
    ns = (ctypes.c_int64 * 2)(1024, 1024)
    ptrs = P2(1 << 20, 2 << 20)
    ys = P2(5 << 20, 6 << 20)
    for adds in (P2((5 << 20) + 32, 7 << 20), P2(7 << 20, 5 << 20)):
        assert L.sx8_dec_gemv_add(p, 2, ptrs, ptrs, 6, ptrs, ptrs, ns, 80, adds, ys, NULL) == 1
        assert "overlaps" in _err(L)


def test_deferred_sum_refusals_on_host(hiplib):
    """The deferred-sum entry points refuse bad arguments before any launch: missing
    out-parameters, a partial count outside 0..7, partial sums without delta or parts, a
    slice shorter than the rows it must cover, misaligned parts."""
    L = hiplib
    V = ctypes.c_void_p
    p = V(1 << 24)
    M, H = 512, 2560
    # out-parameters of the deferred GEMMs
    P1 = ctypes.c_void_p * 1
    ns = (ctypes.c_int64 * 1)(2560)
    ptrs = P1(1 << 20)
    assert L.sx8_gemm_prefill_group_deferred(p, M, 4096, 4096, 1, ptrs, ptrs, 6, ptrs, ptrs, ns, 128, ptrs,
                                             p, 1 << 30, NULL, NULL, NULL, NULL) == 1
    assert "out-parameter" in _err(L)
    assert L.sx8_dec_gemm_silu_deferred(p, p, M, 9728, p, p, 6, p, p, 2560, 304, p, p, 1 << 30,
                                        NULL, NULL, NULL, NULL) == 1
    assert "out-parameter" in _err(L)

    def add(delta, parts, n, slc):
        return L.sx8_dec_add_rmsnorm_parts(p, delta, NULL, p, p, M, H, ctypes.c_float(1e-6), parts, n, slc, NULL)

    assert add(p, p, 8, M * H) == 1 and "n_parts" in _err(L)
    assert add(p, p, -1, M * H) == 1 and "n_parts" in _err(L)
    assert add(NULL, p, 1, M * H) == 1 and "need delta" in _err(L)
    assert add(p, NULL, 1, M * H) == 1 and "parts" in _err(L)
    assert add(p, p, 1, M * H - 1) == 1 and "slice" in _err(L)
    assert add(p, V((1 << 24) + 2), 1, M * H) == 1 and "aligned" in _err(L)

    def rope(parts, n, slc):
        return L.sx8_dec_qk_rope_cache_rows_parts(p, p, p, p, p, p, p, p, M, p, p, p, 32, 8, 128, 1024,
                                                  ctypes.c_float(1e-6), parts, n, slc, NULL)

    need = M * (32 + 2 * 8) * 128
    assert rope(p, 8, need) == 1 and "n_parts" in _err(L)
    assert rope(NULL, 1, need) == 1
    assert rope(p, 2, need - 1) == 1 and "slice" in _err(L)


def test_packed_operand_refusals_on_host(hiplib):
    """sx8_gemm_prefill_packed and sx8_dec_attn_prefill_packed refuse bad arguments before any
    launch; the packed workspace holds the split-K partials only (none for an unsplit plan)."""
    L = hiplib
    V = ctypes.c_void_p
    p = V(1 << 24)
    M, K = 512, 4096
    P1 = ctypes.c_void_p * 1
    ns = (ctypes.c_int64 * 1)(2560)
    ptrs = P1(1 << 20)
    n_out = ctypes.c_int32()

    def gemm(xp, ws, nbytes, parts, n_parts, slc, Ns=ns, n_mats=1, hb=6):
        return L.sx8_gemm_prefill_packed(xp, ptrs, M, K, n_mats, ptrs, ptrs, hb, Ns, 128, ptrs, ws, nbytes,
                                         parts, n_parts, slc, NULL)

    assert gemm(p, p, 1 << 30, p, NULL, NULL) == 1 and "all three" in _err(L)
    assert gemm(p, p, 1 << 30, NULL, ctypes.addressof(n_out), NULL) == 1 and "all three" in _err(L)
    assert gemm(V((1 << 24) + 8), p, 1 << 30, NULL, NULL, NULL) == 1 and "aligned" in _err(L)
    assert gemm(NULL, p, 1 << 30, NULL, NULL, NULL) == 1 and "null" in _err(L)
    assert gemm(p, p, 1 << 30, NULL, NULL, NULL, n_mats=5) == 1 and "n_mats" in _err(L)
    assert gemm(p, p, 1 << 30, NULL, NULL, NULL, hb=7) == 1 and "hdr_bytes" in _err(L)
    # o at M = 512 splits K into 4 ranges: 3 partial slices of M x N floats
    need = L.sx8_gemm_prefill_packed_workspace_bytes(M, 1, ns, 128)
    assert need == 3 * M * 2560 * 4
    assert gemm(p, NULL, 0, NULL, NULL, NULL) == 1 and "workspace" in _err(L)
    assert gemm(p, p, need - 256, NULL, NULL, NULL) == 1 and "workspace" in _err(L)
    gu = (ctypes.c_int64 * 2)(9728, 9728)     # gate/up at M = 512: unsplit 512-row tiles
    assert L.sx8_gemm_prefill_packed_workspace_bytes(M, 2, gu, 80) == 0
    assert L.sx8_gemm_prefill_packed_workspace_bytes(0, 1, ns, 128) == -1
    assert L.sx8_gemm_prefill_packed_workspace_bytes(M, 1, ns, 128) <= L.sx8_gemm_prefill_workspace_bytes(
        M, 1, ns, 128)

    def attn(basis, xp, T=512, start=0, nh=32, nk=8, hd=128, Lc=1024):
        return L.sx8_dec_attn_prefill_packed(p, p, p, T, start, nh, nk, hd, Lc, ctypes.c_float(0.088), basis, p,
                                             xp, p, NULL)

    assert attn(NULL, p) == 1 and "null" in _err(L)
    assert attn(p, V((1 << 24) + 4)) == 1 and "aligned" in _err(L)
    assert attn(p, p, T=1000, start=100) == 1 and "bad shape" in _err(L)
    assert attn(p, p, nh=24, nk=8) == 1 and "bad shape" in _err(L)
    # one KV head's cache is read through 32-bit buffer offsets: at most 0x7FF00000 bytes
    assert attn(p, p, Lc=(0x7FF00000 // 256) + 1) == 1 and "2 GiB" in _err(L)
    assert L.sx8_dec_attn_prefill(p, p, p, p, 512, 0, 32, 8, 128, 1 << 23, ctypes.c_float(0.088), NULL) == 1
    assert "2 GiB" in _err(L)


def test_producer_operand_refusals_on_host(hiplib):
    """sx8_dec_gemm_gateup_silu and sx8_dec_add_rmsnorm_packed refuse bad arguments before any
    launch: both or neither of X and the packed input, n_mats outside 1..4, H not a multiple
    of 32 or past 4096, misaligned operands, a short workspace."""
    L = hiplib
    V = ctypes.c_void_p
    p = V(1 << 24)
    P2 = ctypes.c_void_p * 2
    two = P2(1 << 20, 1 << 21)
    M, K, N = 512, 2560, 9728
    need = L.sx8_dec_gemm_gateup_silu_workspace_bytes(M, N, K // 32)
    assert need > 0 and L.sx8_dec_gemm_gateup_silu_workspace_bytes(0, N, 80) == -1

    def gu(x, xp, zin, ws=p, nbytes=1 << 30, xpo=p):
        return L.sx8_dec_gemm_gateup_silu(x, xp, zin, M, K, two, two, 6, two, two, N, K // 32, p, p, xpo, p, ws,
                                          nbytes, NULL)

    assert gu(p, p, two) == 1 and "not both" in _err(L)            # X and the packed input
    assert gu(NULL, NULL, NULL) == 1 and "not both" in _err(L)     # neither
    assert gu(NULL, p, NULL) == 1 and "Zhl_in" in _err(L)
    assert gu(p, NULL, NULL, xpo=V((1 << 24) + 4)) == 1 and "misaligned" in _err(L)
    assert gu(p, NULL, NULL, nbytes=need - 256) == 1 and "workspace" in _err(L)

    def norm(n_mats=3, H=2560, xp=p, parts=NULL, n_parts=0, slc=0, delta=p):
        return L.sx8_dec_add_rmsnorm_packed(p, delta, NULL, p, M, H, ctypes.c_float(1e-6), parts, n_parts, slc,
                                            n_mats, (ctypes.c_void_p * 4)(*[1 << 20] * 4),
                                            (ctypes.c_void_p * 4)(*[1 << 20] * 4), xp,
                                            (ctypes.c_void_p * 4)(*[1 << 20] * 4), NULL)

    assert norm(n_mats=0) == 1 and "n_mats" in _err(L)
    assert norm(n_mats=5) == 1 and "n_mats" in _err(L)
    assert norm(H=2570) == 1 and "bad shape" in _err(L)
    assert norm(H=8192) == 1 and "bad shape" in _err(L)
    assert norm(xp=V((1 << 24) + 8)) == 1 and "aligned" in _err(L)
    assert norm(parts=p, n_parts=2, slc=M * 2560, delta=NULL) == 1 and "need delta" in _err(L)
    assert norm(parts=p, n_parts=2, slc=M * 2560 - 1) == 1 and "slice" in _err(L)
