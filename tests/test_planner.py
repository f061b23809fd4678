"""The prefill planner on the host (sx8_gemm_prefill_plan / _workspace_bytes; no kernel runs):
every plan covers each output tile and K block exactly once with K ranges of whole 4-block
groups, its grid and workspace follow from that cover, a forced plan is honoured, and the
layer shapes get the plans that the prefill profile was measured with."""
import itertools

import pytest

BN = 128              # output columns per tile
W_ROWS = 512          # rows of a 512-row (k_gemm_w2) tile


def _plan(M, Ns, n_cb):
    import _sx8lib as L
    return L.gemm_plan(M, Ns, n_cb)


def _ws_bytes(M, Ns, n_cb):
    import ctypes
    import _sx8lib as L
    n = len(Ns)
    return int(L.lib().sx8_gemm_prefill_workspace_bytes(M, n, (ctypes.c_int64 * n)(*Ns), n_cb))


def _ceil(a, b):
    return -(-a // b)


def _round256(v):
    return _ceil(v, 256) * 256


def _check(M, Ns, n_cb, forced=False):
    p = _plan(M, Ns, n_cb)
    NB = sum(_ceil(N, BN) for N in Ns)
    Ntot = sum(Ns)
    tile, G, S, kbs = p["tile"], p["groups"], p["k_ranges"], p["kb_per_range"]
    ctx = (M, Ns, n_cb, p)
    # K ranges: whole 4-block groups, every range non-empty, together exactly the n_cb blocks
    assert kbs % 4 == 0 and kbs > 0, ctx
    assert 1 <= S <= 8 and (S - 1) * kbs < n_cb <= S * kbs, ctx
    assert G < 2 ** 31, ctx
    if tile == W_ROWS:
        assert M > 256, ctx
        T = _ceil(M, W_ROWS) * NB
        Tf, n_split = p["whole_tiles"], p["split_tiles"]
        # whole tiles fill whole rounds of the 256 CUs; the rest run split (or all whole)
        assert Tf % 256 == 0 and 0 <= Tf <= T, ctx
        assert n_split == (T - Tf if S > 1 else 0), ctx
        assert G == (T if S == 1 else Tf + n_split * S), ctx
        part = n_split * (S - 1) * W_ROWS * BN * 4
    else:
        # 128-row tiles up to 128 rows; past that 256-row tiles, or 128-row ones when the
        # 256-row plan would leave more than half the CUs idle (or a plan is forced)
        assert tile in (128, 256) and (forced or M > 128 or tile == 128), ctx
        assert p["whole_tiles"] == 0 and p["split_tiles"] == 0, ctx
        assert G == _ceil(M, tile) * NB * S, ctx
        part = (S - 1) * M * Ntot * 4
    z = _round256(M * n_cb * 8) * len(Ns)
    xp = _round256(_ceil(M, 32) * n_cb * 2048)
    assert p["workspace"] == z + xp + part == _ws_bytes(M, Ns, n_cb), ctx
    return p


LAYER = [(4096,), (1024,), (2560,), (9728,), (4096, 1024, 1024), (9728, 9728)]
ODD = [(1,), (100,), (129, 300), (128, 128, 128, 128)]


@pytest.mark.parametrize("n_cb", [80, 128, 304])
def test_plan_invariants_layer_shapes(hiplib, n_cb):
    Ms = [1, 31, 32, 33, 128, 129, 256, 257, 511, 512, 513, 1000, 2048, 3000, 4096, 8192]
    for M, Ns in itertools.product(Ms, LAYER):
        _check(M, Ns, n_cb)


@pytest.mark.parametrize("n_cb", [1, 3, 4, 5, 7, 9, 33])
def test_plan_invariants_ragged(hiplib, n_cb):
    for M, Ns in itertools.product([1, 2, 127, 257, 600, 2049], ODD + LAYER[:2]):
        _check(M, Ns, n_cb)


@pytest.mark.parametrize("force,tile,S", [("k1:3", 128, 3), ("k2:5", 256, 5), ("w0:2", 512, 2),
                                          ("w1:4", 512, 4)])
def test_forced_plan(hiplib, gemm_tuning, force, tile, S):
    """SX8_GEMM_PLAN selects one plan (the tuning knob the parity tests use to reach every
    kernel form); w1 runs whole rounds of tiles first."""
    gemm_tuning(PLAN=force)
    p = _check(2048, (9728, 9728), 80, forced=True)
    assert (p["tile"], p["k_ranges"]) == (tile, S), p
    T = 4 * 152
    assert p["whole_tiles"] == (T // 256 * 256 if force.startswith("w1") else 0), p


def test_forced_plan_out_of_range_falls_back(hiplib, gemm_tuning):
    base = _plan(512, (2560,), 80)
    for bad in ("k2:9", "k3:2", "w2:1", "x1:1", "w0:0", "k1"):
        gemm_tuning(PLAN=bad)
        assert _plan(512, (2560,), 80) == base, bad


@pytest.mark.parametrize("M,Ns,n_cb,want", [
    # (tile, groups, k_ranges, whole_tiles, split_tiles) as the prefill profile lists them
    (2048, (4096,), 80, (256, 256, 1, 0, 0)),                  # q: unsplit 256-row tiles
    (2048, (1024,), 80, (256, 256, 4, 0, 0)),                  # k, v: 64 tiles x 4
    (2048, (2560,), 128, (512, 240, 3, 0, 80)),                # o: 80 tiles x 3
    (2048, (9728,), 80, (512, 448, 4, 256, 48)),               # gate, up: 256 whole + 48 x 4
    (2048, (2560,), 304, (512, 240, 3, 0, 80)),                # down: 80 tiles x 3
    (2048, (4096, 1024, 1024), 80, (512, 192, 1, 0, 0)),       # q/k/v group
    (2048, (9728, 9728), 80, (512, 704, 2, 512, 96)),          # gate/up group
    (512, (4096, 1024, 1024), 80, (256, 192, 2, 0, 0)),        # q/k/v group at M = 512
    (512, (2560,), 128, (256, 160, 4, 0, 0)),                  # o at M = 512
    (512, (9728, 9728), 80, (512, 152, 1, 0, 0)),              # gate/up group at M = 512
    (512, (2560,), 304, (256, 240, 6, 0, 0)),                  # down at M = 512
    (512, (1024,), 80, (128, 160, 5, 0, 0)),                   # k, v at M = 512: 128-row tiles
    (512, (4096,), 80, (256, 256, 4, 0, 0)),                   # q at M = 512
])
def test_layer_plans(hiplib, M, Ns, n_cb, want):
    """The planner's choices for the layer's calls (a change here moves the measured
    prefill figures and needs a new measurement)."""
    p = _check(M, Ns, n_cb)
    got = (p["tile"], p["groups"], p["k_ranges"], p["whole_tiles"], p["split_tiles"])
    assert got == want, (M, Ns, n_cb, p)
