"""The .sx8v43 container (v1.0 records, v1.1 SXT1 section) on the CPU.

Expected bytes are built here field by field from the reference's format document
(formats/SX8_FLASH_V4_3_CONTAINER.md, sections 1, 2 and 6), independently of the writer
under test; round trips, the v1.0/v1.1 compatibility rules and the safe metadata parse
follow the same document and scripts/sx8_container_v43.py:89-209."""
import io
import struct

import numpy as np
import pytest

import sx8_container_v43 as C


def _tensor(rng, out_f, n_cb, orig_shape=None):
    nb = out_f * n_cb
    qt = {"shape": (out_f, n_cb * 32), "orig_shape": orig_shape, "n_blocks": nb, "n_cb": n_cb,
          "dmin": rng.standard_normal(nb).astype(np.float16),
          "dmax": rng.standard_normal(nb).astype(np.float16),
          "config": rng.integers(0, 256, nb, dtype=np.uint8),
          "levels_hi": rng.integers(0, 256, nb * 16, dtype=np.uint8),
          "levels_lo": rng.integers(0, 256, nb * 8, dtype=np.uint8),
          "coeff": rng.integers(0, 256, nb, dtype=np.uint8)}
    bi = {"n_cb": n_cb, "data": rng.standard_normal((n_cb, 64)).astype(np.float32),
          "scales": rng.standard_normal((n_cb, 2)).astype(np.float32)}
    return qt, bi


def _model(seed=0):
    rng = np.random.default_rng(seed)
    wd, bd = {}, {}
    for name, (o, c, os_) in {"b.weight": (3, 2, None), "a.conv": (4, 1, (4, 2, 16))}.items():
        wd[name], bd[name] = _tensor(rng, o, c, os_)
    meta = {"method": "sx8_v43", "bpw": 7.5, "layers": 2}
    return wd, bd, meta


def _spec_bytes(wd, bd, meta, config=None, small=None):
    """The container as the format document lays it out, written field by field."""
    out = io.BytesIO()
    out.write(b"SX43FILE")
    out.write(bytes([1]))
    mb = repr(sorted(meta.items())).encode()
    out.write(struct.pack("<I", len(mb)) + mb)
    out.write(struct.pack("<I", len(wd)))
    for name in sorted(wd):
        qt, bi = wd[name], bd[name]
        out.write(struct.pack("<I", len(name)) + name.encode())
        out.write(struct.pack("<II", *qt["shape"]))
        os_ = qt["orig_shape"] or qt["shape"]
        out.write(struct.pack("<B", len(os_)) + struct.pack("<%dI" % len(os_), *os_))
        out.write(struct.pack("<II", qt["n_blocks"], qt["n_cb"]))
        for k in ("dmin", "dmax", "config", "levels_hi", "levels_lo", "coeff"):
            out.write(qt[k].tobytes())
        out.write(struct.pack("<I", bi["n_cb"]))
        out.write(bi["data"].astype("<f4").tobytes() + bi["scales"].astype("<f4").tobytes())
    if config is not None:
        import json
        cb = json.dumps(config).encode()
        out.write(b"SXT1" + struct.pack("<I", len(cb)) + cb + struct.pack("<I", len(small)))
        for name in sorted(small):
            st = small[name]
            out.write(struct.pack("<I", len(name)) + name.encode())
            out.write(struct.pack("<B", len(st["shape"])) + struct.pack("<%dI" % len(st["shape"]), *st["shape"]))
            out.write(bytes([0 if st["dtype"] == "fp16" else 1]) + st["data"].tobytes())
    return out.getvalue()


def _small():
    return {"norm.weight": {"shape": (5,), "dtype": "fp16", "data": np.arange(5, dtype=np.float16)},
            "A_log": {"shape": (2, 3), "dtype": "fp32",
                      "data": np.linspace(-1, 1, 6, dtype=np.float32).reshape(2, 3)}}


def test_writer_matches_the_format_document(tmp_path):
    wd, bd, meta = _model()
    p = tmp_path / "m.sx8v43"
    C.write_sx43({"weights": wd, "bases": bd, "meta": meta}, p, verbose=False)
    assert p.read_bytes() == _spec_bytes(wd, bd, meta)
    cfg = {"hidden_size": 8, "model_type": "toy"}
    p11 = tmp_path / "m11.sx8v43"
    C.write_sx43((wd, bd, meta), p11, verbose=False, config=cfg, small=_small())
    assert p11.read_bytes() == _spec_bytes(wd, bd, meta, cfg, _small())
    # the v1.1 file starts with the v1.0 file byte for byte (its records are unchanged)
    assert p11.read_bytes().startswith(p.read_bytes())


def test_round_trip_and_v10_v11_compatibility(tmp_path):
    wd, bd, meta = _model(1)
    p = tmp_path / "m.sx8v43"
    C.write_sx43((wd, bd, meta), p, verbose=False, config={"k": [1, 2]}, small=_small())
    rw, rb, rmeta = C.read_all(p)               # v1.0 reader: ignores the SXT1 section
    assert rmeta == meta and sorted(rw) == sorted(wd)
    for name in wd:
        for k in ("dmin", "dmax", "config", "levels_hi", "levels_lo", "coeff"):
            assert np.array_equal(rw[name][k].view(np.uint8), np.asarray(wd[name][k]).view(np.uint8))
        assert rw[name]["shape"] == wd[name]["shape"]
        assert rw[name]["orig_shape"] == wd[name]["orig_shape"]
        assert np.array_equal(rb[name]["data"], bd[name]["data"])
        assert np.array_equal(rb[name]["scales"], bd[name]["scales"])
    assert rw["a.conv"]["orig_shape"] == (4, 2, 16) and rw["b.weight"]["orig_shape"] is None
    w2, b2, m2, cfg, small = C.read_all_v11(p)
    assert cfg == {"k": [1, 2]} and sorted(small) == sorted(_small())
    for name, st in _small().items():
        assert small[name]["dtype"] == st["dtype"] and small[name]["shape"] == st["shape"]
        assert np.array_equal(small[name]["data"], st["data"])
    assert C.verify_sx43((wd, bd, meta), p, verbose=False)
    # a v1.0 file has no section: read_all_v11 gives (None, None) for it
    p10 = tmp_path / "m10.sx8v43"
    C.write_sx43((wd, bd, meta), p10, verbose=False)
    assert C.read_all_v11(p10)[3:] == (None, None)


def test_read_small_section_positions(tmp_path):
    f = io.BytesIO()
    f.write(b"prefix")
    C.write_small_section(f, {"a": 1}, _small())
    f.seek(6)
    cfg, small = C.read_small_section(f)
    assert cfg == {"a": 1} and f.tell() == len(f.getvalue())
    f.seek(0)
    assert C.read_small_section(f) == (None, None) and f.tell() == 0


def test_metadata_is_parsed_without_eval(tmp_path):
    wd, bd, _ = _model(2)
    p = tmp_path / "m.sx8v43"
    C.write_sx43((wd, bd, {}), p, verbose=False)
    raw = bytearray(p.read_bytes())
    evil = b"[('x', __import__('os').getcwd())]"
    ml = struct.unpack_from("<I", raw, 9)[0]
    raw[9:13 + ml] = struct.pack("<I", len(evil)) + evil
    bad = tmp_path / "evil.sx8v43"
    bad.write_bytes(bytes(raw))
    with pytest.raises(ValueError, match="metadata"):
        C.read_all(bad)


def test_rejects_bad_magic_and_truncation(tmp_path):
    wd, bd, meta = _model(3)
    p = tmp_path / "m.sx8v43"
    C.write_sx43((wd, bd, meta), p, verbose=False)
    data = p.read_bytes()
    (tmp_path / "bad").write_bytes(b"XXXXXXXX" + data[8:])
    with pytest.raises(ValueError, match="magic"):
        C.read_all(tmp_path / "bad")
    (tmp_path / "cut").write_bytes(data[:-7])
    with pytest.raises(ValueError, match="truncated"):
        C.read_all(tmp_path / "cut")


def test_verify_detects_a_changed_byte(tmp_path):
    wd, bd, meta = _model(4)
    p = tmp_path / "m.sx8v43"
    C.write_sx43((wd, bd, meta), p, verbose=False)
    wd["b.weight"]["levels_lo"] = wd["b.weight"]["levels_lo"].copy()
    wd["b.weight"]["levels_lo"][3] ^= 1
    assert not C.verify_sx43((wd, bd, meta), p, verbose=False)


def test_iter_records_payload_is_the_block_bytes(tmp_path):
    wd, bd, meta = _model(5)
    p = tmp_path / "m.sx8v43"
    C.write_sx43((wd, bd, meta), p, verbose=False)
    seen = []
    for name, info, payload in C.iter_records(p):
        qt = wd[name]
        want = b"".join(np.asarray(qt[k]).tobytes() for k in
                        ("dmin", "dmax", "config", "levels_hi", "levels_lo", "coeff"))
        assert bytes(payload) == want and info["n_blocks"] == qt["n_blocks"]
        assert np.array_equal(info["bases"], bd[name]["data"])
        seen.append(name)
        del payload, info
    assert seen == sorted(wd)
