"""Runs the product's R64 device decode (sx8_r64_subblock from csrc/sx8_device.h),
compiled for the host, against the oracle: the same function the dequant and embedding
kernels call must be bit-exact on the CPU before it reaches a GPU.  (The prefill GEMM's
operand decode is a different recipe, pinned on the GPU by
tests/test_gpu_prefill.py::test_prefill_mfma_operand_bit_exact.)"""
import ctypes
import os
import subprocess

import numpy as np
import pytest

HERE = os.path.dirname(os.path.abspath(__file__))
REPO = os.path.dirname(HERE)
SRC = os.path.join(HERE, "emul", "sx8_emul.hip")
OUT = os.path.join(HERE, "emul", "build", "libsx8_emul.so")
HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")


@pytest.fixture(scope="module")
def emul():
    if not os.path.exists(HIPCC):
        pytest.skip("hipcc not available")
    os.makedirs(os.path.dirname(OUT), exist_ok=True)
    subprocess.run([HIPCC, "--cuda-host-only", "-O2", "-std=c++17", "-fPIC", "-shared",
                    "-ffp-contract=off", "-I", os.path.join(REPO, "sx8-quantization_amd", "csrc"),
                    "-I", os.path.join(REPO, "include"), "-o", OUT, SRC],
                   check=True, capture_output=True)
    L = ctypes.CDLL(OUT)
    p = ctypes.c_void_p
    L.sx8e_dequant_split.argtypes = [ctypes.c_int64, ctypes.c_int64] + [p] * 8 + [ctypes.c_int32, p]
    return L


def _run(emul, oracle, qt, bi, pca=True):
    n_blk, dmin, dmax, cfg, cof, hi, lo = oracle._fields(qt)
    data, sc = oracle._bases(bi)
    out = np.empty(n_blk * 32, dtype=np.uint16)
    P = oracle._ptr
    emul.sx8e_dequant_split(n_blk, qt["n_cb"], P(dmin), P(dmax), P(cfg), P(cof), P(hi), P(lo),
                            P(data), P(sc), int(pca), P(out))
    return out.reshape(n_blk, 32)


@pytest.mark.parametrize("prefix", ["fuzz_", "q_"])
def test_device_decode_matches_golden(emul, oracle, prefix):
    from test_oracle import _golden, _qt_from_golden
    g = _golden()
    qt, bi = _qt_from_golden(g, prefix)
    got = _run(emul, oracle, qt, bi)
    exp = oracle.dequant_r64(qt, bi, blocks_only=True).view(np.uint16)
    assert np.array_equal(got, exp)


def test_device_decode_fuzz(emul, oracle):
    import sys
    sys.path.insert(0, os.path.join(HERE, "golden"))
    from make_golden import fuzz_blocks
    qt, bi = fuzz_blocks(np.random.default_rng(99), 300, 8)
    got = _run(emul, oracle, qt, bi)
    exp = oracle.dequant_r64(qt, bi, blocks_only=True).view(np.uint16)
    assert np.array_equal(got, exp)


def test_device_decode_core_without_pca(emul, oracle):
    from test_oracle import _golden, _qt_from_golden
    g = _golden()
    qt, bi = _qt_from_golden(g, "fuzz_")
    got = _run(emul, oracle, qt, bi, pca=False)
    bi0 = {"n_cb": bi["n_cb"], "data": np.zeros_like(bi["data"]), "scales": np.zeros_like(bi["scales"])}
    exp = oracle.dequant_r64(qt, bi0, blocks_only=True).view(np.uint16)
    assert np.array_equal(got, exp)
