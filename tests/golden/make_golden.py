"""Writes tests/golden/sx8_golden.npz: frozen S-X8 inputs with their canonical (R64) fp16
dequant.  Run from the repo root: python tests/golden/make_golden.py

The reference ships no fixtures or golden vectors for this path (its tests need an
unshipped 4.38 GB model file, a CUDA GPU and numba), so these are produced by the
CPU oracle in oracle/ after it has been pinned by the known-answer and brute-force
tests in tests/test_oracle.py (the hand-built known-answer blocks live in that file).
Each set stores the n-major block arrays, the PCA tables and `<set>_w16`, the
(out_f, in_f) fp16 dequant as uint16 bit patterns.  Sets:
  fuzz_*  random blocks: every strategy, all 64 levels, random coeff bytes, fp16
          endpoints drawn from normal, subnormal, equal (degenerate) and reversed
          (dmin > dmax) ranges;
  q_*     a seeded N(0, 0.02) 96 x 80 fp16 weight quantized by the oracle's
          restatement of the reference quantizer (K = 80 is not a multiple of 32).
"""
import os
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
REPO = os.path.dirname(os.path.dirname(HERE))
sys.path.insert(0, os.path.join(REPO, "oracle"))
import oracle as O  # noqa: E402


def fuzz_blocks(rng, out_f, n_cb):
    n = out_f * n_cb
    kind = rng.integers(0, 5, n)
    a = (rng.standard_normal(n) * 0.05).astype(np.float16)
    b = (a.astype(np.float32) + np.abs(rng.standard_normal(n) * 0.05)).astype(np.float16)
    sub = (rng.integers(1, 1024, n) * 2.0 ** -24).astype(np.float16)          # subnormals
    sub2 = (sub.astype(np.float32) + rng.integers(0, 2048, n) * 2.0 ** -24).astype(np.float16)
    dmin = np.where(kind == 0, a, np.where(kind == 1, sub, np.where(kind == 2, a, np.where(kind == 3, b, a))))
    dmax = np.where(kind == 0, b, np.where(kind == 1, sub2, np.where(kind == 2, a, np.where(kind == 3, a, b * 40))))
    # kind 2: degenerate (dmin == dmax); kind 3: reversed range; kind 4: wide range
    qt = {
        "shape": (out_f, n_cb * 32), "orig_shape": (out_f, n_cb * 32),
        "n_blocks": n, "n_cb": n_cb,
        "dmin": dmin.astype(np.float16), "dmax": dmax.astype(np.float16),
        "config": rng.integers(0, 256, n).astype(np.uint8),
        "levels_hi": rng.integers(0, 256, n * 16).astype(np.uint8),
        "levels_lo": rng.integers(0, 256, n * 8).astype(np.uint8),
        "coeff": rng.integers(0, 256, (n, 1)).astype(np.uint8),
    }
    basis = rng.standard_normal((n_cb, 64)).astype(np.float32)
    basis /= np.linalg.norm(basis.reshape(n_cb, 2, 32), axis=2).repeat(32, axis=1)
    bi = {"n_cb": n_cb, "data": basis.astype(np.float32),
          "scales": (np.abs(rng.standard_normal((n_cb, 2))) * 2e-3 + 1e-6).astype(np.float32)}
    return qt, bi


def main():
    O.build()
    rng = np.random.default_rng(20261201)
    out = {}
    qt, bi = fuzz_blocks(rng, 64, 6)
    for k in ("dmin", "dmax", "config", "levels_hi", "levels_lo", "coeff"):
        out["fuzz_" + k] = np.asarray(qt[k])
    out["fuzz_shape"] = np.array([64, 6 * 32, 6])
    out["fuzz_basis"] = bi["data"]
    out["fuzz_scales"] = bi["scales"]
    out["fuzz_w16"] = O.dequant_r64(qt, bi).view(np.uint16)

    g = np.random.default_rng(7)
    W = (g.standard_normal((96, 80)) * 0.02).astype(np.float16)
    qt, bi = O.quantize(W)
    for k in ("dmin", "dmax", "config", "levels_hi", "levels_lo", "coeff"):
        out["q_" + k] = np.asarray(qt[k])
    out["q_shape"] = np.array([96, 80, qt["n_cb"]])
    out["q_basis"] = bi["data"]
    out["q_scales"] = bi["scales"]
    out["q_w16"] = O.dequant_r64(qt, bi).view(np.uint16)
    out["q_weight"] = W.view(np.uint16)
    np.savez_compressed(os.path.join(HERE, "sx8_golden.npz"), **out)
    print("wrote", os.path.join(HERE, "sx8_golden.npz"))


if __name__ == "__main__":
    main()
