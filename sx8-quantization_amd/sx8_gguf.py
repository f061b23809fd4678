"""GGUF interop for S-X8 tensors (the format of the reference's llama.cpp fork).

Role of scripts/convert_pkl_to_gguf_sx8.py (reference) and of the fork's GGML_TYPE_SX8
(llama-cpp-sx8.patch:131-144, type traits :851-858): an S-X8 tensor is stored in GGUF as
n-major 30-byte ``block_sx8`` records -- dmin f16 | dmax f16 | config | qh[16] | ql[8] |
coeff -- the same 30 bytes as the pkl / .sx8v43 block, interleaved.  GGUF has no place for
the PCA bases and scales, so the fork's engine ignores ``coeff`` (no PCA).

Here:
* ``blockify`` / ``unblockify`` -- the byte permutation between the split arrays and
  the records (the reference's ``blockify_vec``, convert_pkl_to_gguf_sx8.py:21-38);
* ``write_gguf`` / ``read_gguf`` -- a self-contained GGUF v3 writer / reader (the public
  GGUF layout: header, typed key-value pairs, tensor infos, aligned data), enough for
  S-X8 tensors (type 41, 32 weights per 30-byte block) plus fp16 / fp32 small tensors;
  the reference relies on the fork's gguf-py package instead;
* ``convert`` -- the converter's job: S-X8 tensors (and optional small tensors) of a
  model to one GGUF file;
* ``load_v44`` -- GGUF SX8 tensors straight into the v4.4 device layout
  (``sx8_blocks_to_v44``), with zero PCA bases, so this engine's GEMV / GEMM / gather run
  the fork's no-PCA weights;
* ``dequant_ggml`` -- the fork's float32 no-PCA dequant ("R32-ggml",
  ``dequantize_row_sx8``, patch:746-767) on the GPU, bit-exact, for comparing the two
  engines on the same file.
"""
from __future__ import annotations

import mmap
import struct

import numpy as np

GGUF_MAGIC = b"GGUF"
GGUF_VERSION = 3
GGML_TYPE_F32 = 0
GGML_TYPE_F16 = 1
GGML_TYPE_SX8 = 41            # GGMLQuantizationType.SX8 in the fork (patch:851-858)
QK_SX8 = 32
SX8_BLOCK_BYTES = 30
DEFAULT_ALIGNMENT = 32

# GGUF metadata value types
T_U8, T_I8, T_U16, T_I16, T_U32, T_I32, T_F32, T_BOOL, T_STR, T_ARR, T_U64, T_I64, T_F64 = range(13)
_SCALAR = {T_U8: "<B", T_I8: "<b", T_U16: "<H", T_I16: "<h", T_U32: "<I", T_I32: "<i",
           T_F32: "<f", T_BOOL: "<?", T_U64: "<Q", T_I64: "<q", T_F64: "<d"}


# ------------------------------------------------------------------ block records
def blockify(qt) -> np.ndarray:
    """(n_blocks, 30) u8 block_sx8 records, n-major, from the split arrays of ``qt``."""
    n = int(qt["n_blocks"])
    out = np.empty((n, SX8_BLOCK_BYTES), dtype=np.uint8)
    out[:, 0:2] = np.asarray(qt["dmin"]).astype(np.float16).reshape(n).view(np.uint8).reshape(n, 2)
    out[:, 2:4] = np.asarray(qt["dmax"]).astype(np.float16).reshape(n).view(np.uint8).reshape(n, 2)
    out[:, 4] = np.asarray(qt["config"], dtype=np.uint8).reshape(n)
    out[:, 5:21] = np.asarray(qt["levels_hi"], dtype=np.uint8).reshape(n, 16)
    out[:, 21:29] = np.asarray(qt["levels_lo"], dtype=np.uint8).reshape(n, 8)
    out[:, 29] = np.asarray(qt["coeff"], dtype=np.uint8).reshape(n)
    return out


def unblockify(blocks, out_f: int, n_cb: int, in_f: int | None = None) -> dict:
    """The split arrays (a ``qt`` dict, as the pkl holds them) of block_sx8 records."""
    b = np.ascontiguousarray(np.asarray(blocks, dtype=np.uint8)).reshape(-1, SX8_BLOCK_BYTES)
    n = out_f * n_cb
    if b.shape[0] != n:
        raise ValueError(f"{b.shape[0]} records for {out_f} x {n_cb} blocks")
    return {"shape": (out_f, in_f if in_f is not None else n_cb * QK_SX8), "orig_shape": None,
            "n_blocks": n, "n_cb": n_cb,
            "dmin": np.ascontiguousarray(b[:, 0:2]).view(np.float16).reshape(n),
            "dmax": np.ascontiguousarray(b[:, 2:4]).view(np.float16).reshape(n),
            "config": np.ascontiguousarray(b[:, 4]), "levels_hi": np.ascontiguousarray(b[:, 5:21]).reshape(-1),
            "levels_lo": np.ascontiguousarray(b[:, 21:29]).reshape(-1), "coeff": np.ascontiguousarray(b[:, 29])}


# ------------------------------------------------------------------ GGUF v3 writer
def _str(s: str) -> bytes:
    b = s.encode()
    return struct.pack("<Q", len(b)) + b


class Typed:
    """A metadata value with an explicit GGUF type (for arrays: `elem` is the element
    type), e.g. Typed(T_U64, 7) or Typed(T_ARR, [11, 11, 10, 0], elem=T_I32)."""

    def __init__(self, vtype, value, elem=None):
        self.vtype, self.value, self.elem = vtype, value, elem


def _infer_type(v):
    if isinstance(v, Typed):
        return v.vtype
    if isinstance(v, bool):
        return T_BOOL
    if isinstance(v, int):
        return T_U32 if 0 <= v < 2 ** 32 else T_I64
    if isinstance(v, float):
        return T_F32
    if isinstance(v, str):
        return T_STR
    if isinstance(v, (list, tuple)):
        return T_ARR
    raise TypeError(f"no GGUF type for {type(v).__name__}")


def _value(vtype, v) -> bytes:
    elem = None
    if isinstance(v, Typed):
        vtype, elem, v = v.vtype, v.elem, v.value
    if vtype == T_STR:
        return _str(v)
    if vtype == T_ARR:
        items = list(v)
        et = elem if elem is not None else (_infer_type(items[0]) if items else T_I32)
        return struct.pack("<IQ", et, len(items)) + b"".join(_value(et, x) for x in items)
    return struct.pack(_SCALAR[vtype], v)


def _kv(key, v) -> bytes:
    vtype = _infer_type(v)
    return _str(key) + struct.pack("<I", vtype) + _value(vtype, v)


def _nbytes(dims, gtype) -> int:
    ne = int(np.prod(dims))
    if gtype == GGML_TYPE_SX8:
        if dims[0] % QK_SX8:
            raise ValueError("SX8 rows must hold whole 32-weight blocks")
        return ne // QK_SX8 * SX8_BLOCK_BYTES
    if gtype == GGML_TYPE_F16:
        return ne * 2
    if gtype == GGML_TYPE_F32:
        return ne * 4
    raise ValueError(f"unsupported ggml type {gtype}")


def write_gguf(path, tensors, kv=None, alignment=DEFAULT_ALIGNMENT):
    """Write a GGUF v3 file.  tensors: [(name, dims (ne0 first), ggml_type, data bytes)];
    kv: {key: value} (type inferred: bool, int -> u32 / i64, float -> f32, str, list) or
    {key: Typed(...)}.  general.alignment is written when not the default."""
    kv = dict(kv or {})
    if alignment != DEFAULT_ALIGNMENT:
        kv["general.alignment"] = Typed(T_U32, int(alignment))
    infos, offset, datas = [], 0, []
    for name, dims, gtype, data in tensors:
        data = bytes(data) if not isinstance(data, (bytes, bytearray)) else data
        if len(data) != _nbytes(dims, gtype):
            raise ValueError(f"{name}: {len(data)} bytes, dims {dims} type {gtype} need {_nbytes(dims, gtype)}")
        infos.append(_str(name) + struct.pack("<I", len(dims)) +
                     b"".join(struct.pack("<Q", int(d)) for d in dims) + struct.pack("<IQ", gtype, offset))
        datas.append(data)
        offset += len(data)
        offset += (-offset) % alignment
    with open(path, "wb") as f:
        f.write(GGUF_MAGIC + struct.pack("<IQQ", GGUF_VERSION, len(tensors), len(kv)))
        for k in kv:
            f.write(_kv(k, kv[k]))
        for info in infos:
            f.write(info)
        f.write(b"\0" * ((-f.tell()) % alignment))
        for data in datas:
            f.write(data)
            f.write(b"\0" * ((-len(data)) % alignment))
    return path


# ------------------------------------------------------------------ GGUF v3 reader
class _R:
    def __init__(self, buf):
        self.buf, self.pos = buf, 0

    def get(self, fmt):
        n = struct.calcsize(fmt)
        if self.pos + n > len(self.buf):
            raise ValueError("truncated GGUF file")
        v = struct.unpack_from(fmt, self.buf, self.pos)
        self.pos += n
        return v[0] if len(v) == 1 else v

    def string(self):
        n = self.get("<Q")
        if self.pos + n > len(self.buf):
            raise ValueError("truncated GGUF file")
        s = bytes(self.buf[self.pos:self.pos + n]).decode()
        self.pos += n
        return s

    def value(self, vtype):
        if vtype == T_STR:
            return self.string()
        if vtype == T_ARR:
            et, n = self.get("<I"), self.get("<Q")
            return [self.value(et) for _ in range(n)]
        if vtype not in _SCALAR:
            raise ValueError(f"unknown GGUF value type {vtype}")
        return self.get(_SCALAR[vtype])


def read_gguf(path):
    """(kv, tensors) of a GGUF v2/v3 file; tensors: {name: {'dims', 'type', 'nbytes',
    'data' (read-only numpy u8 view of the mapped file)}} in file order."""
    with open(path, "rb") as f:
        mm = mmap.mmap(f.fileno(), 0, access=mmap.ACCESS_READ)
    r = _R(mm)
    if bytes(mm[:4]) != GGUF_MAGIC:
        raise ValueError("not a GGUF file (bad magic)")
    r.pos = 4
    version = r.get("<I")
    if version not in (2, 3):
        raise ValueError(f"unsupported GGUF version {version}")
    n_t, n_kv = r.get("<Q"), r.get("<Q")
    kv = {}
    for _ in range(n_kv):
        k = r.string()
        kv[k] = r.value(r.get("<I"))
    align = int(kv.get("general.alignment", DEFAULT_ALIGNMENT))
    infos = []
    for _ in range(n_t):
        name = r.string()
        nd = r.get("<I")
        dims = [r.get("<Q") for _ in range(nd)]
        gtype, off = r.get("<I"), r.get("<Q")
        infos.append((name, dims, gtype, off))
    base = r.pos + (-r.pos) % align
    tensors = {}
    for name, dims, gtype, off in infos:
        nb = _nbytes(dims, gtype)
        if base + off + nb > len(mm):
            raise ValueError(f"tensor {name} runs past the end of the file")
        tensors[name] = {"dims": dims, "type": gtype, "nbytes": nb,
                         "data": np.frombuffer(mm, dtype=np.uint8, count=nb, offset=base + off)}
    return kv, tensors


# ------------------------------------------------------------------ model level
def convert(wd, out_path, arch="qwen35", kv=None, small=None):
    """The converter's job (convert_pkl_to_gguf_sx8.py:41-89) on in-memory tensors: every
    2-D S-X8 tensor of ``wd`` as a GGUF SX8 tensor (dims [n_cb*32, out_f]), plus optional
    small tensors {name: {'shape', 'dtype': 'fp16'|'fp32', 'data'}}; ``kv`` adds metadata
    after general.architecture."""
    meta = {"general.architecture": arch}
    meta.update(kv or {})
    tens = []
    for name in wd:
        qt = wd[name]
        if len(qt["shape"]) != 2:
            continue
        out_f, n_cb = int(qt["shape"][0]), int(qt["n_cb"])
        tens.append((name, [n_cb * QK_SX8, out_f], GGML_TYPE_SX8, blockify(qt).tobytes()))
    for name in sorted(small or {}):
        st = small[name]
        dt = GGML_TYPE_F16 if st["dtype"] == "fp16" else GGML_TYPE_F32
        arr = np.ascontiguousarray(np.asarray(st["data"], dtype=np.float16 if dt == GGML_TYPE_F16 else np.float32))
        tens.append((name, list(reversed([int(v) for v in st["shape"]])), dt, arr.tobytes()))
    return write_gguf(out_path, tens, meta)


def sx8_tensors(path):
    """{name: (blocks (n_blk, 30) u8 view, out_f, n_cb)} for the SX8 tensors of a GGUF."""
    _, tensors = read_gguf(path)
    out = {}
    for name, t in tensors.items():
        if t["type"] != GGML_TYPE_SX8:
            continue
        ne0, rows = t["dims"][0], int(np.prod(t["dims"][1:]))
        out[name] = (t["data"].reshape(-1, SX8_BLOCK_BYTES), rows, ne0 // QK_SX8)
    return out


def load_v44(path, device="cuda", hdr_bytes=6, names=None):
    """GGUF SX8 tensors -> {name: (hdr, levels, bases, scales)} on `device` in the v4.4
    layout.  GGUF carries no PCA bases: bases and scales are zero, so this engine computes
    the same no-PCA weights as the fork's engine (coeff is kept but contributes 0)."""
    import ctypes
    import warnings

    import torch

    import _sx8lib as _L
    dev = torch.device(device)
    out = {}
    for name, (blocks, out_f, n_cb) in sx8_tensors(path).items():
        if names is not None and name not in names:
            continue
        with warnings.catch_warnings():
            warnings.simplefilter("ignore", UserWarning)
            raw = torch.from_numpy(blocks.reshape(-1)).to(dev)
        nb = out_f * n_cb
        hdr = torch.empty(nb, hdr_bytes, dtype=torch.uint8, device=dev)
        lvl = torch.empty(nb, 24, dtype=torch.uint8, device=dev)
        _L.call("sx8_blocks_to_v44", ctypes.c_void_p(raw.data_ptr()), out_f, n_cb, int(hdr_bytes),
                _L.ptr(hdr), _L.ptr(lvl), _L.stream(dev))
        out[name] = (hdr, lvl, torch.zeros(n_cb, 64, dtype=torch.float32, device=dev),
                     torch.zeros(n_cb, 2, dtype=torch.float32, device=dev))
        del raw
    return out


def dequant_ggml(blocks, out_f, n_cb, in_f=None, contract=True, out=None):
    """The fork's no-PCA float32 dequant of block_sx8 records on the GPU: blocks is a
    device u8 tensor of out_f * n_cb * 30 bytes (n-major) -> (out_f, in_f) float32."""
    import torch

    import _sx8lib as _L
    in_f = n_cb * QK_SX8 if in_f is None else in_f
    if out is None:
        out = torch.empty(out_f, in_f, dtype=torch.float32, device=blocks.device)
    _L.call("sx8_dequant_ggml_f32", _L.ptr(blocks.contiguous()), out_f, in_f, n_cb, int(bool(contract)),
            _L.ptr(out), _L.stream(blocks.device))
    return out
