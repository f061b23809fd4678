"""GGUF interop on the CPU: block_sx8 records, the GGUF v3 writer/reader, and the oracle's
R32-ggml (llama.cpp's no-PCA float32 dequant).

* block_sx8 bytes are built here with struct from the field table of
  llama-cpp-sx8.patch:131-144 (dmin, dmax, config, qh[16], ql[8], coeff; 30 bytes);
* GGUF bytes are built here with struct from the public GGUF v3 layout (magic "GGUF",
  version, tensor and key-value counts, typed values, tensor infos with ne0 first, data
  aligned to general.alignment = 32);
* R32-ggml (patch:746-767) is recomputed with exact rational arithmetic and
  correctly rounded binary32 operations, separately for the fused (a C build that
  contracts a*b+c) and the unfused evaluation, and compared bit for bit."""
import os
import struct
from fractions import Fraction

import numpy as np
import pytest

import sx8_gguf as G

HERE = os.path.dirname(os.path.abspath(__file__))


def _golden_qt(prefix):
    g = np.load(os.path.join(HERE, "golden", "sx8_golden.npz"))
    out_f, in_f, n_cb = (int(v) for v in g[prefix + "shape"])
    qt = {"shape": (out_f, in_f), "orig_shape": None, "n_blocks": out_f * n_cb, "n_cb": n_cb}
    for k in ("dmin", "dmax", "config", "levels_hi", "levels_lo", "coeff"):
        qt[k] = g[prefix + k]
    return qt


def _struct_blocks(qt):
    n = qt["n_blocks"]
    hi = np.asarray(qt["levels_hi"]).reshape(n, 16)
    lo = np.asarray(qt["levels_lo"]).reshape(n, 8)
    cf = np.asarray(qt["coeff"]).reshape(n)
    return b"".join(struct.pack("<eeB16s8sB", float(qt["dmin"][i]), float(qt["dmax"][i]),
                                int(qt["config"][i]), hi[i].tobytes(), lo[i].tobytes(), int(cf[i]))
                    for i in range(n))


@pytest.mark.parametrize("prefix", ["fuzz_", "q_"])
def test_blockify_is_the_block_sx8_layout(prefix):
    qt = _golden_qt(prefix)
    fin = np.isfinite(qt["dmin"].astype(np.float32)) & np.isfinite(qt["dmax"].astype(np.float32))
    b = G.blockify(qt)
    assert b.shape == (qt["n_blocks"], 30)
    want = np.frombuffer(_struct_blocks(qt), dtype=np.uint8).reshape(-1, 30)
    # struct's 'e' re-encodes NaN payloads; compare those blocks' other bytes only
    assert np.array_equal(b[fin], want[fin])
    assert np.array_equal(b[:, 4:], want[:, 4:])
    back = G.unblockify(b, qt["shape"][0], qt["n_cb"], qt["shape"][1])
    for k in ("config", "levels_hi", "levels_lo"):
        assert np.array_equal(back[k], np.asarray(qt[k]).reshape(-1))
    assert np.array_equal(back["coeff"], np.asarray(qt["coeff"]).reshape(-1))
    assert np.array_equal(back["dmin"].view(np.uint16), qt["dmin"].view(np.uint16))
    assert np.array_equal(back["dmax"].view(np.uint16), qt["dmax"].view(np.uint16))


def _gguf_str(s):
    return struct.pack("<Q", len(s)) + s.encode()


def test_writer_matches_the_gguf_layout(tmp_path):
    blocks = bytes(range(60)) * 2                              # 4 records: 2 rows x 2 blocks
    norm = np.arange(3, dtype=np.float16)
    p = tmp_path / "t.gguf"
    G.write_gguf(p, [("w", [64, 2], G.GGML_TYPE_SX8, blocks), ("n", [3], G.GGML_TYPE_F16, norm.tobytes())],
                 {"general.architecture": "toy", "toy.block_count": 2, "toy.eps": 0.5,
                  "toy.sections": G.Typed(G.T_ARR, [1, 2], elem=G.T_I32)})
    hdr = b"GGUF" + struct.pack("<IQQ", 3, 2, 4)
    kv = (_gguf_str("general.architecture") + struct.pack("<I", 8) + _gguf_str("toy") +
          _gguf_str("toy.block_count") + struct.pack("<II", 4, 2) +
          _gguf_str("toy.eps") + struct.pack("<If", 6, 0.5) +
          _gguf_str("toy.sections") + struct.pack("<IIQii", 9, 5, 2, 1, 2))
    infos = (_gguf_str("w") + struct.pack("<IQQIQ", 2, 64, 2, 41, 0) +
             _gguf_str("n") + struct.pack("<IQIQ", 1, 3, 1, 128))   # 120 B of blocks -> next at 128
    head = hdr + kv + infos
    head += b"\0" * ((-len(head)) % 32)
    data = blocks + b"\0" * 8 + norm.tobytes() + b"\0" * 26
    assert p.read_bytes() == head + data
    kvr, t = G.read_gguf(p)
    assert kvr == {"general.architecture": "toy", "toy.block_count": 2, "toy.eps": 0.5, "toy.sections": [1, 2]}
    assert t["w"]["dims"] == [64, 2] and t["w"]["type"] == 41 and bytes(t["w"]["data"]) == blocks
    assert np.array_equal(t["n"]["data"].view(np.float16), norm)


def test_reader_rejects_bad_files(tmp_path):
    (tmp_path / "a").write_bytes(b"GGUX" + bytes(40))
    with pytest.raises(ValueError, match="magic"):
        G.read_gguf(tmp_path / "a")
    (tmp_path / "b").write_bytes(b"GGUF" + struct.pack("<IQQ", 3, 1, 0) + _gguf_str("w") +
                                 struct.pack("<IQQIQ", 2, 64, 4, 41, 0))
    with pytest.raises(ValueError, match="past the end"):
        G.read_gguf(tmp_path / "b")


def test_convert_and_sx8_tensors_round_trip(tmp_path):
    qt = _golden_qt("q_")
    p = tmp_path / "m.gguf"
    small = {"model.norm.weight": {"shape": (80,), "dtype": "fp16", "data": np.ones(80, np.float16)}}
    G.convert({"layers.0.w": qt}, p, arch="qwen35", kv={"qwen35.block_count": 1}, small=small)
    kv, t = G.read_gguf(p)
    assert kv["general.architecture"] == "qwen35" and kv["qwen35.block_count"] == 1
    st = G.sx8_tensors(p)
    blocks, out_f, n_cb = st["layers.0.w"]
    assert (out_f, n_cb) == (qt["shape"][0], qt["n_cb"])
    assert np.array_equal(blocks, G.blockify(qt))
    assert np.array_equal(t["model.norm.weight"]["data"].view(np.float16), small["model.norm.weight"]["data"])


# ------------------------------------------------------------ R32-ggml, exact check
_F32_STEP = Fraction(float(np.float32(0.015873)))
_F32_FLOOR = Fraction(float(np.float32(1e-10)))


def _r32(fr: Fraction) -> Fraction:
    """Correctly rounded binary32 (RNE) of an exact rational."""
    if fr == 0:
        return Fraction(0)
    x = np.float32(float(fr))
    cands = [np.nextafter(x, np.float32(-np.inf)), x, np.nextafter(x, np.float32(np.inf))]

    def key(c):
        return abs(Fraction(float(c)) - fr), int(np.array(c, dtype=np.float32).view(np.uint32)) & 1
    return Fraction(float(min(cands, key=key)))


def _ggml_exact(rec: bytes, contract: bool):
    lo = Fraction(float(np.frombuffer(rec[0:2], np.float16)[0]))
    hi = Fraction(float(np.frombuffer(rec[2:4], np.float16)[0]))
    q = _r32(_r32(hi - lo) / 4)
    out = []
    for t in range(32):
        s = (rec[4] >> ((t >> 3) * 2)) & 3
        k1, k2 = 3 * (s == 2) + (s == 3), 3 * (s == 1) + (s == 3)
        rlo = _r32(q * k1 + lo) if contract else _r32(lo + _r32(q * k1))
        rhi = _r32(hi - q * k2) if contract else _r32(hi - _r32(q * k2))
        step = _r32(_r32(rhi - rlo) * _F32_STEP)
        if step < _F32_FLOOR:
            step = _F32_FLOOR
        nib = (rec[5 + (t >> 1)] >> ((t & 1) * 4)) & 0xF
        qua = (rec[21 + (t >> 2)] >> ((3 - (t & 3)) * 2)) & 3
        lv = (nib << 2) | qua
        out.append(float(_r32(step * lv + rlo) if contract else _r32(rlo + _r32(step * lv))))
    return np.array(out, dtype=np.float32)


@pytest.mark.parametrize("contract", [True, False])
def test_oracle_r32_ggml_is_exact(oracle, contract):
    qt = _golden_qt("fuzz_")
    b = G.blockify(qt)
    fin = np.isfinite(qt["dmin"].astype(np.float32)) & np.isfinite(qt["dmax"].astype(np.float32))
    got = oracle.dequant_ggml(b, contract)
    idx = np.nonzero(fin)[0][:160]
    for i in idx:
        assert np.array_equal(got[i].view(np.uint32), _ggml_exact(b[i].tobytes(), contract).view(np.uint32)), i
    # NaN endpoints propagate
    bad = np.nonzero(~fin & (np.isnan(qt["dmin"].astype(np.float32)) | np.isnan(qt["dmax"].astype(np.float32))))[0]
    for i in bad:
        assert np.all(np.isnan(got[i]))


def test_oracle_r32_ggml_closed_forms(oracle):
    # degenerate block (dmin == dmax = v): step floors at 1e-10f, w = v + 1e-10 * lv
    # rounds back to v for |v| >= 2^-7 (63e-10 is below half an ulp there)
    rec = bytearray(30)
    v = np.float16(0.75)
    rec[0:2] = rec[2:4] = v.tobytes()
    rec[4] = 0b11100100                       # strategies 0, 1, 2, 3
    rec[5:21] = bytes([0xFF] * 16)
    rec[21:29] = bytes([0xFF] * 8)            # every level 63
    for contract in (True, False):
        assert np.all(oracle.dequant_ggml(np.frombuffer(bytes(rec), np.uint8), contract) == np.float32(0.75))
    # level 0 gives rlo exactly: strategy 0 -> dmin, 2 -> dmin + 3q (exact here), 3 -> dmin + q
    rec = bytearray(30)
    rec[0:2] = np.float16(-1.0).tobytes()
    rec[2:4] = np.float16(1.0).tobytes()
    rec[4] = 0b11100100
    w = oracle.dequant_ggml(np.frombuffer(bytes(rec), np.uint8), True)[0]
    assert w[0] == -1.0 and w[8] == -1.0 and w[16] == 0.5 and w[24] == -0.5
