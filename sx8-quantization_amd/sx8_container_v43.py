"""The .sx8v43 container: S-X8 v4.3 tensor records (v1.0) and the trailing SXT1
small-tensor section (v1.1), and its load straight into the v4.4 device layout.

Interface of scripts/sx8_container_v43.py (reference): ``MAGIC``, ``VERSION``,
``BYTES_PER_BLOCK``, ``write_sx43``, ``verify_sx43``, ``read_all``, ``SMALL_MAGIC``,
``write_small_section``, ``read_small_section``, ``read_all_v11``.  Format: the reference's
formats/SX8_FLASH_V4_3_CONTAINER.md (all fields little-endian):

    "SX43FILE" | version u8 (1) | meta_len u32 | meta (repr of sorted meta items)
    | n_tensors u32 | tensor records ... | [v1.1: "SXT1" | cfg_len u32 | cfg JSON
    | n_small u32 | small records ...]
    tensor record: name_len u32 | name | out_f u32 | in_f u32 | n_os u8 | orig_shape
                   n_os x u32 | n_blocks u32 | n_cb u32 | dmin f16[nb] | dmax f16[nb]
                   | config u8[nb] | levels_hi u8[16 nb] | levels_lo u8[8 nb]
                   | coeff u8[nb] | bi_n_cb u32 | bases f32[bi_n_cb * 64]
                   | scales f32[bi_n_cb * 2]
    small record:  name_len u32 | name | ndim u8 | shape ndim x u32 | dtype u8 (0 fp16,
                   1 fp32) | data

Additions: ``load_v44`` maps the file and, per tensor, copies the contiguous 30-byte-per-
block payload to the GPU once and lays it out there (``sx8_v43_to_v44``) -- the load path
the reference runs as a numba full-tensor decode (eval_common.py:77-151) or a numpy
to_v44 at first forward (prepare_v44.py:35-79).  ``iter_records`` walks the records of
a mapped file without copying them.

Differences: the metadata blob is parsed with ``ast.literal_eval`` (the reference calls
``eval`` on it, so a crafted file could run code); ``write_sx43`` / ``verify_sx43`` take
the in-memory ``{'weights', 'bases', 'meta'}`` dict (or a (weights, bases, meta) tuple)
rather than unpickling a path.  Record order, field order and bytes are the reference's.
"""
from __future__ import annotations

import ast
import json
import mmap
import os
import struct

import numpy as np

MAGIC = b"SX43FILE"
VERSION = 1
BYTES_PER_BLOCK = 30
SMALL_MAGIC = b"SXT1"
_SMALL_DTYPES = {0: ("fp16", np.float16), 1: ("fp32", np.float32)}


def _unpack_source(src):
    if isinstance(src, dict):
        return src["weights"], src["bases"], src.get("meta", {})
    if isinstance(src, (tuple, list)) and len(src) == 3:
        return src
    raise TypeError("expected {'weights', 'bases', 'meta'} or (weights, bases, meta); "
                    "pickle files are not loaded here")


def _meta_bytes(meta):
    return repr(sorted(meta.items())).encode()


def _write_record(f, name, qt, bi):
    nb, ncb = int(qt["n_blocks"]), int(qt["n_cb"])
    sh = tuple(int(v) for v in qt["shape"])
    os_ = qt.get("orig_shape")
    os_ = tuple(int(v) for v in (os_ if os_ is not None else sh))
    nm = name.encode()
    f.write(struct.pack("<I", len(nm)))
    f.write(nm)
    f.write(struct.pack("<II", sh[0], sh[1]))
    f.write(struct.pack("<B", len(os_)))
    f.write(struct.pack("<%dI" % len(os_), *os_))
    f.write(struct.pack("<II", nb, ncb))
    for key, dt, per in (("dmin", np.float16, 1), ("dmax", np.float16, 1), ("config", np.uint8, 1),
                         ("levels_hi", np.uint8, 16), ("levels_lo", np.uint8, 8),
                         ("coeff", np.uint8, 1)):
        a = np.ascontiguousarray(np.asarray(qt[key]).astype(dt, copy=False)).reshape(-1)
        if a.size != nb * per:
            raise ValueError(f"{name}: {key} has {a.size} entries, expected {nb * per}")
        f.write(a.tobytes())
    data = np.ascontiguousarray(np.asarray(bi["data"], dtype=np.float32)).reshape(-1)
    scales = np.ascontiguousarray(np.asarray(bi["scales"], dtype=np.float32)).reshape(-1)
    bn = int(bi["n_cb"])
    if data.size != bn * 64 or scales.size != bn * 2:
        raise ValueError(f"{name}: bases/scales do not match n_cb {bn}")
    f.write(struct.pack("<I", bn))
    f.write(data.tobytes())
    f.write(scales.tobytes())
    return nb


def write_sx43(src, out_path, verbose=True, config=None, small=None):
    """Write the container from (weights, bases, meta); tensors in sorted name order.
    With ``config`` and ``small`` the v1.1 SXT1 section is appended.  Returns out_path."""
    wd, bd, meta = _unpack_source(src)
    n_tot = 0
    with open(out_path, "wb") as f:
        f.write(MAGIC)
        f.write(struct.pack("<B", VERSION))
        mb = _meta_bytes(meta)
        f.write(struct.pack("<I", len(mb)))
        f.write(mb)
        f.write(struct.pack("<I", len(wd)))
        for name in sorted(wd):
            n_tot += _write_record(f, name, wd[name], bd[name])
        if config is not None or small is not None:
            write_small_section(f, config if config is not None else {}, small or {})
    if verbose:
        sz = os.path.getsize(out_path)
        print(f"wrote {out_path}: {len(wd)} tensors, {n_tot} blocks, {sz / 1e9:.3f} GB "
              f"({n_tot * BYTES_PER_BLOCK / 1e9:.3f} GB of 30-byte blocks)")
    return out_path


class _Cursor:
    """Sequential little-endian reader over a bytes-like buffer (an mmap or bytes)."""

    def __init__(self, buf, pos=0):
        self.buf = buf
        self.pos = pos

    def take(self, n):
        if self.pos + n > len(self.buf):
            raise ValueError("truncated .sx8v43 file")
        v = memoryview(self.buf)[self.pos:self.pos + n]
        self.pos += n
        return v

    def unpack(self, fmt):
        n = struct.calcsize(fmt)
        return struct.unpack(fmt, self.take(n))

    def array(self, dtype, count):
        dt = np.dtype(dtype)
        if self.pos + dt.itemsize * count > len(self.buf):
            raise ValueError("truncated .sx8v43 file")
        a = np.frombuffer(self.buf, dtype=dt, count=count, offset=self.pos)
        self.pos += dt.itemsize * count
        return a


def _parse_meta(raw):
    try:
        items = ast.literal_eval(bytes(raw).decode())
        return dict(items)
    except (ValueError, SyntaxError, TypeError) as e:
        raise ValueError(f"container metadata is not a literal list of items: {e}") from None


def _read_header(cur):
    if bytes(cur.take(8)) != MAGIC:
        raise ValueError("not an .sx8v43 file (bad magic)")
    (ver,) = cur.unpack("<B")
    if ver != VERSION:
        raise ValueError(f"unsupported .sx8v43 version {ver}")
    (ml,) = cur.unpack("<I")
    meta = _parse_meta(cur.take(ml))
    (nt,) = cur.unpack("<I")
    return meta, nt


def _read_record(cur):
    """One tensor record -> (name, shape, orig_shape, nb, ncb, payload_offset, bi_n_cb,
    bases, scales); the six block arrays are the 30*nb bytes at payload_offset."""
    (nl,) = cur.unpack("<I")
    name = bytes(cur.take(nl)).decode()
    sh = cur.unpack("<II")
    (n_os,) = cur.unpack("<B")
    os_ = cur.unpack("<%dI" % n_os)
    nb, ncb = cur.unpack("<II")
    off = cur.pos
    cur.take(nb * BYTES_PER_BLOCK)
    (bn,) = cur.unpack("<I")
    data = cur.array(np.float32, bn * 64).reshape(bn, 64)
    scales = cur.array(np.float32, bn * 2).reshape(bn, 2)
    return name, tuple(sh), tuple(os_), nb, ncb, off, bn, data, scales


def _fields(buf, off, nb):
    """The six block arrays of a record as views of `buf` (container field order)."""
    o = off
    dmin = np.frombuffer(buf, np.float16, nb, o); o += 2 * nb
    dmax = np.frombuffer(buf, np.float16, nb, o); o += 2 * nb
    config = np.frombuffer(buf, np.uint8, nb, o); o += nb
    hi = np.frombuffer(buf, np.uint8, 16 * nb, o); o += 16 * nb
    lo = np.frombuffer(buf, np.uint8, 8 * nb, o); o += 8 * nb
    coeff = np.frombuffer(buf, np.uint8, nb, o)
    return dmin, dmax, config, hi, lo, coeff


def _records(buf):
    cur = _Cursor(buf)
    meta, nt = _read_header(cur)
    wd, bd = {}, {}
    for _ in range(nt):
        name, sh, os_, nb, ncb, off, bn, data, scales = _read_record(cur)
        dmin, dmax, config, hi, lo, coeff = _fields(buf, off, nb)
        wd[name] = {"shape": sh, "orig_shape": os_ if os_ != sh else None, "n_blocks": nb,
                    "n_cb": ncb, "dmin": dmin, "dmax": dmax, "config": config,
                    "levels_hi": hi, "levels_lo": lo, "coeff": coeff}
        bd[name] = {"n_cb": bn, "data": data, "scales": scales}
    return wd, bd, meta, cur


def _file_bytes(path):
    with open(path, "rb") as f:
        return f.read()


def read_all(sx43_path):
    """(weights, bases, meta) from a v1.0 or v1.1 file; a v1.1 SXT1 section is ignored.
    Arrays are read-only numpy views of the file's bytes (like np.frombuffer upstream)."""
    wd, bd, meta, _ = _records(_file_bytes(sx43_path))
    return wd, bd, meta


def write_small_section(f, config, small_tensors):
    """Append the v1.1 section to an open binary file.  small_tensors:
    {name: {'shape': tuple, 'dtype': 'fp16'|'fp32', 'data': ndarray}}."""
    cb = json.dumps(config).encode()
    f.write(SMALL_MAGIC)
    f.write(struct.pack("<I", len(cb)))
    f.write(cb)
    f.write(struct.pack("<I", len(small_tensors)))
    for name in sorted(small_tensors):
        st = small_tensors[name]
        shape = tuple(int(v) for v in st["shape"])
        dt = 0 if st["dtype"] == "fp16" else 1
        data = np.ascontiguousarray(np.asarray(st["data"], dtype=_SMALL_DTYPES[dt][1]))
        if data.size != int(np.prod(shape)):
            raise ValueError(f"small tensor {name}: {data.size} values for shape {shape}")
        nb = name.encode()
        f.write(struct.pack("<I", len(nb)))
        f.write(nb)
        f.write(struct.pack("<B", len(shape)))
        f.write(struct.pack("<%dI" % len(shape), *shape))
        f.write(struct.pack("<B", dt))
        f.write(data.tobytes())


def _read_small(cur):
    if cur.pos + 4 > len(cur.buf) or bytes(memoryview(cur.buf)[cur.pos:cur.pos + 4]) != SMALL_MAGIC:
        return None, None
    cur.take(4)
    (cl,) = cur.unpack("<I")
    config = json.loads(bytes(cur.take(cl)))
    (n,) = cur.unpack("<I")
    small = {}
    for _ in range(n):
        (nl,) = cur.unpack("<I")
        name = bytes(cur.take(nl)).decode()
        (nd,) = cur.unpack("<B")
        shape = cur.unpack("<%dI" % nd)
        (dt,) = cur.unpack("<B")
        if dt not in _SMALL_DTYPES:
            raise ValueError(f"small tensor {name}: unknown dtype code {dt}")
        tag, npdt = _SMALL_DTYPES[dt]
        data = cur.array(npdt, int(np.prod(shape))).reshape(shape)
        small[name] = {"shape": tuple(shape), "dtype": tag, "data": data}
    return config, small


def read_small_section(f):
    """Read the SXT1 section at the current position of an open binary file ->
    (config, small), or (None, None) with the position unchanged when there is none."""
    pos = f.tell()
    rest = f.read()
    cur = _Cursor(rest)
    config, small = _read_small(cur)
    if config is None:
        f.seek(pos)
        return None, None
    f.seek(pos + cur.pos)
    return config, small


def read_all_v11(sx43_path):
    """(weights, bases, meta, config, small); config and small are None for a v1.0 file."""
    wd, bd, meta, cur = _records(_file_bytes(sx43_path))
    config, small = _read_small(cur)
    return wd, bd, meta, config, small


def verify_sx43(src, sx43_path, verbose=True):
    """Every array read back from the file equals the source's, byte for byte."""
    wd, bd, _ = _unpack_source(src)
    rw, rb, _ = read_all(sx43_path)
    ok_all = set(rw) == set(wd)
    for name in sorted(wd):
        if name not in rw:
            continue
        qt, bi, q2, b2 = wd[name], bd[name], rw[name], rb[name]
        ok = all(np.array_equal(np.asarray(qt[k]).reshape(-1).view(np.uint8)
                                if np.asarray(qt[k]).dtype == np.float16 else np.asarray(qt[k]).reshape(-1),
                                np.asarray(q2[k]).reshape(-1).view(np.uint8)
                                if q2[k].dtype == np.float16 else q2[k].reshape(-1))
                 for k in ("dmin", "dmax", "config", "levels_hi", "levels_lo", "coeff"))
        ok = ok and np.array_equal(np.asarray(bi["data"], np.float32).reshape(-1).view(np.uint32),
                                   b2["data"].reshape(-1).view(np.uint32))
        ok = ok and np.array_equal(np.asarray(bi["scales"], np.float32).reshape(-1).view(np.uint32),
                                   b2["scales"].reshape(-1).view(np.uint32))
        ok_all &= ok
        if verbose and not ok:
            print(f"  mismatch: {name}")
    if verbose:
        print(f"verify {sx43_path}: {'identical' if ok_all else 'DIFFERENT'} ({len(wd)} tensors)")
    return ok_all


def iter_records(sx43_path):
    """Walk the tensor records of a mapped file: yields (name, info, payload) where
    payload is a memoryview of the record's 30 * n_blocks block bytes and info holds
    shape, orig_shape, n_blocks, n_cb, bases and scales (read-only views)."""
    with open(sx43_path, "rb") as f:
        mm = mmap.mmap(f.fileno(), 0, access=mmap.ACCESS_READ)
    try:
        cur = _Cursor(mm)
        _, nt = _read_header(cur)
        for _ in range(nt):
            name, sh, os_, nb, ncb, off, bn, data, scales = _read_record(cur)
            info = {"shape": sh, "orig_shape": os_ if os_ != sh else None, "n_blocks": nb,
                    "n_cb": ncb, "bases": data, "scales": scales}
            yield name, info, memoryview(mm)[off:off + nb * BYTES_PER_BLOCK]
            del data, scales, info
    finally:
        del cur
        try:
            mm.close()
        except BufferError:
            pass      # a caller still holds a view; the map closes when it is released


def load_v44(sx43_path, device="cuda", hdr_bytes=6, names=None):
    """Load tensors of a container straight into the v4.4 device layout.

    Per tensor the 30 * n_blocks block bytes are copied to the device once and laid out
    there by ``sx8_v43_to_v44``.  Returns {name: (hdr (n_blk, hdr_bytes) u8, levels
    (n_blk, 24) u8, bases (n_cb, 64) f32, scales (n_cb, 2) f32)} for every tensor (or
    those in ``names``), ready for SX8LinearV44 / SX8EmbeddingV44 / the C ABI."""
    import ctypes
    import warnings

    import torch

    import _sx8lib as _L
    if hdr_bytes not in (6, 8):
        raise ValueError(f"hdr_bytes must be 6 or 8, got {hdr_bytes}")
    dev = torch.device(device)
    out = {}
    for name, info, payload in iter_records(sx43_path):
        if names is not None and name not in names:
            continue
        nb, ncb = info["n_blocks"], info["n_cb"]
        out_f = info["shape"][0]
        if nb != out_f * ncb:
            raise ValueError(f"{name}: n_blocks {nb} != out_f * n_cb {out_f * ncb}")
        with warnings.catch_warnings():      # read-only source: copied to the device at once
            warnings.simplefilter("ignore", UserWarning)
            raw = torch.from_numpy(np.frombuffer(payload, dtype=np.uint8)).to(dev)
        del payload
        hdr = torch.empty(nb, hdr_bytes, dtype=torch.uint8, device=dev)
        lvl = torch.empty(nb, 24, dtype=torch.uint8, device=dev)
        base = raw.data_ptr()
        P = ctypes.c_void_p
        _L.call("sx8_v43_to_v44", P(base), P(base + 2 * nb), P(base + 4 * nb), P(base + 29 * nb),
                P(base + 5 * nb), P(base + 21 * nb), out_f, ncb, hdr_bytes, _L.ptr(hdr), _L.ptr(lvl),
                _L.stream(dev))
        bas = torch.from_numpy(np.array(info["bases"], dtype=np.float32)).to(dev)
        sca = torch.from_numpy(np.array(info["scales"], dtype=np.float32)).to(dev)
        out[name] = (hdr, lvl, bas, sca)
        del raw
    return out
