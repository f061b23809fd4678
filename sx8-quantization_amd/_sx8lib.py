"""ctypes binding of libsx8_hip.so, the gfx950 HIP library behind every wrapper here.

The library is built in-tree (``build()`` drives hipcc) and loaded from this
directory, or from the path in the SX8_HIP_LIB environment variable.  There is no
fallback: if the library cannot be loaded, every GPU entry point raises
RuntimeError.  The C signatures are declared in include/sx8_hip.h.
"""
from __future__ import annotations

import ctypes
import os
import subprocess
import threading

PKG_DIR = os.path.dirname(os.path.abspath(__file__))
REPO_DIR = os.path.dirname(PKG_DIR)
CSRC_DIR = os.path.join(PKG_DIR, "csrc")
INCLUDE_DIR = os.path.join(REPO_DIR, "include")
LIB_NAME = "libsx8_hip.so"
LIB_PATH = os.path.join(PKG_DIR, LIB_NAME)
SOURCES = ["sx8_abi.hip", "sx8_dequant.hip", "sx8_layout.hip", "sx8_quant.hip", "sx8_gemv.hip",
           "sx8_gemm.hip", "sx8_decoder.hip"]
HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")

# hipcc flags: gfx950 only, no packed-fp32 instruction selection (those forms have
# given silent wrong results on the target pool), IEEE denormals, no fast-math.
HIP_FLAGS = [
    "--offload-arch=gfx950", "-mcode-object-version=5", "-O3", "-std=c++17", "-fPIC", "-shared",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-fno-fast-math", "-fno-gpu-flush-denormals-to-zero",
    "-Wall", "-Wno-unused-function",
]

# Per-source extra flags: the GEMV kernels take their leading arguments (matrix pointers,
# N, n_cb) preloaded into SGPRs at wave launch (8 arguments = 14 SGPRs); so do the decoder
# kernels (as many of their first eight arguments as fit: the decode attention gets its
# cache pointers and the position pointer without a kernel-argument load).
_PRELOAD8 = ["-mllvm", "-amdgpu-kernarg-preload-count=8"]
SOURCE_FLAGS = {"sx8_gemv.hip": _PRELOAD8, "sx8_decoder.hip": _PRELOAD8}

# (name, restype, argtypes) for every exported symbol of include/sx8_hip.h
_P = ctypes.c_void_p
_I32, _I64 = ctypes.c_int32, ctypes.c_int64
SIGNATURES = [
    ("sx8_abi_version", _I32, []),
    ("sx8_last_error", ctypes.c_char_p, []),
    ("sx8_dequant_f16", _I32, [_P, _P, _P, _P, _P, _P, _P, _P, _I64, _I64, _I64, _P, _P]),
    ("sx8_v43_to_v44", _I32, [_P, _P, _P, _P, _P, _P, _I64, _I64, _I32, _P, _P, _P]),
    ("sx8_blocks_to_v44", _I32, [_P, _I64, _I64, _I32, _P, _P, _P]),
    ("sx8_dequant_ggml_f32", _I32, [_P, _I64, _I64, _I64, _I32, _P, _P]),
    ("sx8_v6_encode", _I32, [_P, _I64, _I64, _I64, _P, _P, _P, _P, _P, _P, _P]),
    ("sx8_embed_gather", _I32, [_P, _I64, _P, _P, _I32, _P, _P, _I64, _I64, _I64, _P, _P]),
    ("sx8_compute_z", _I32, [_P, _I64, _I64, _P, _P, _I64, _P, _P]),
    ("sx8_gemv", _I32, [_P, _P, _P, _I32, _P, _P, _P, _P, _I64, _I64, _P, _P, _I64, _P]),
    ("sx8_gemv_group", _I32, [_P, _I32, _P, _P, _I32, _P, _P, _P, _P, _I64, _P, _P, _I64, _P]),
    ("sx8_gemv_workspace_bytes", _I64, [_I64]),
    ("sx8_gemm_prefill_workspace_bytes", _I64, [_I64, _I32, _P, _I64]),
    ("sx8_gemm_prefill_plan", _I32, [_I64, _I32, _P, _I64, _P]),
    ("sx8_gemm_reload_tuning", _I32, []),
    ("sx8_gemm_prefill", _I32, [_P, _I64, _I64, _I64, _P, _P, _I32, _P, _P, _I64, _I64, _P, _P, _I64, _P]),
    ("sx8_gemm_prefill_static", _I32, [_P, _I64, _I64, _I64, _P, _P, _I32, _P, _P, _I64, _I64, _P, _P]),
    ("sx8_gemm_prefill_split", _I32,
     [_P, _I64, _I64, _I64, _P, _P, _P, _P, _P, _P, _P, _P, _I64, _I64, _P, _P, _I64, _P]),
    ("sx8_gemm_prefill_z", _I32, [_P, _I64, _I64, _I64, _P, _P, _I32, _P, _I64, _I64, _P, _P, _I64, _P]),
    ("sx8_gemm_prefill_group", _I32,
     [_P, _I64, _I64, _I64, _I32, _P, _P, _I32, _P, _P, _P, _I64, _P, _P, _I64, _P]),
    ("sx8_gemm_prefill_group_deferred", _I32,
     [_P, _I64, _I64, _I64, _I32, _P, _P, _I32, _P, _P, _P, _I64, _P, _P, _I64, _P, _P, _P, _P]),
    ("sx8_gemm_prefill_packed", _I32,
     [_P, _P, _I64, _I64, _I32, _P, _P, _I32, _P, _I64, _P, _P, _I64, _P, _P, _P, _P]),
    ("sx8_gemm_prefill_packed_workspace_bytes", _I64, [_I64, _I32, _P, _I64]),
    ("sx8_dec_gemm_gateup_silu", _I32,
     [_P, _P, _P, _I64, _I64, _P, _P, _I32, _P, _P, _I64, _I64, _P, _P, _P, _P, _P, _I64, _P]),
    ("sx8_dec_add_rmsnorm_packed", _I32,
     [_P, _P, _P, _P, _I64, _I64, ctypes.c_float, _P, _I32, _I64, _I32, _P, _P, _P, _P, _P]),
    ("sx8_dec_gemm_gateup_silu_workspace_bytes", _I64, [_I64, _I64, _I64]),
    ("sx8_gemm_pca_z", _I32, [_P, _I64, _P, _I32, _I64, _I64, _P, _P]),
    ("sx8_gemm_prefill_core", _I32, [_P, _I64, _I64, _I64, _P, _P, _I32, _I64, _I64, _P, _P, _I64, _P]),
    # include/sx8_decoder.h
    ("sx8_dec_add_rmsnorm", _I32, [_P, _P, _P, _P, _P, _I64, _I64, ctypes.c_float, _P]),
    ("sx8_dec_add_rmsnorm_parts", _I32, [_P, _P, _P, _P, _P, _I64, _I64, ctypes.c_float, _P, _I32, _I64, _P]),
    ("sx8_dec_qk_rope_cache", _I32, [_P, _P, _P, _P, _P, _P, _P, _P, _P, _P, _P, _I32, _I32, _I32,
                                     _I64, ctypes.c_float, _P]),
    ("sx8_dec_qk_rope_cache_rows", _I32, [_P, _P, _P, _P, _P, _P, _P, _P, _I64, _P, _P, _P, _I32, _I32,
                                          _I32, _I64, ctypes.c_float, _P]),
    ("sx8_dec_qk_rope_cache_rows_parts", _I32, [_P, _P, _P, _P, _P, _P, _P, _P, _I64, _P, _P, _P, _I32, _I32,
                                                _I32, _I64, ctypes.c_float, _P, _I32, _I64, _P]),
    ("sx8_dec_attn", _I32, [_P, _P, _P, _P, _P, _I32, _I32, _I32, _I64, ctypes.c_float, _P]),
    ("sx8_dec_gemm_silu", _I32, [_P, _P, _I64, _I64, _P, _P, _I32, _P, _P, _I64, _I64, _P, _P, _I64, _P]),
    ("sx8_dec_gemm_silu_deferred", _I32,
     [_P, _P, _I64, _I64, _P, _P, _I32, _P, _P, _I64, _I64, _P, _P, _I64, _P, _P, _P, _P]),
    ("sx8_dec_attn_prefill", _I32, [_P, _P, _P, _P, _I64, _I64, _I32, _I32, _I32, _I64, ctypes.c_float, _P]),
    ("sx8_dec_attn_prefill_packed", _I32,
     [_P, _P, _P, _I64, _I64, _I32, _I32, _I32, _I64, ctypes.c_float, _P, _P, _P, _P, _P]),
    ("sx8_dec_attn_split", _I32, [_P, _P, _P, _P, _P, _I32, _I32, _I32, _I64, ctypes.c_float, _P, _I64,
                                  _P]),
    ("sx8_dec_attn_workspace_bytes", _I64, [_I32, _I32]),
    ("sx8_dec_attn_rope", _I32, [_P, _P, _P, _P, _P, _P, _P, _P, _P, _P, _P, _I32, _I32, _I32, _I64,
                                 ctypes.c_float, ctypes.c_float, _P, _I64, _P]),
    ("sx8_dec_silu_mul", _I32, [_P, _P, _P, _I64, _P]),
    ("sx8_dec_argmax_advance", _I32, [_P, _I64, _P, _P, _P]),
    ("sx8_dec_argmax_parts_bytes", _I64, [_I64, _I64]),
    ("sx8_dec_gemv_rmsnorm_argmax", _I32, [_P, _P, ctypes.c_float, _P, _P, _I32, _P, _P, _I64, _I64, _P, _P,
                                           _I64, _P, _P, _P]),
    ("sx8_dec_gemv_rmsnorm", _I32, [_P, _P, _P, _P, ctypes.c_float, _P, _I32, _P, _P, _I32, _P, _P, _P,
                                    _I64, _P, _P]),
    ("sx8_dec_gemv_silu", _I32, [_P, _P, _I32, _P, _P, _I32, _P, _P, _P, _I64, _P, _P]),
    ("sx8_dec_gemv_silu_add", _I32, [_P, _P, _I32, _P, _P, _I32, _P, _P, _P, _I64, _P, _P, _P]),
    ("sx8_dec_gemv_add", _I32, [_P, _I32, _P, _P, _I32, _P, _P, _P, _I64, _P, _P, _P]),
    ("sx8_dec_gemv_rmsnorm_pair", _I32, [_P, _P, ctypes.c_float, _P, _P, _I32, _P, _P, _P, _P, _P, _P, _I64, _I64,
                                         _P, _P, _P, _P]),
    ("sx8_dec_gemv_zp_add", _I32, [_P, _P, _P, _I32, _P, _P, _I64, _I64, _P, _P, _P]),
]
ABI_VERSION = 5

_lib = None
_lock = threading.Lock()


def build(verbose: bool = False) -> str:
    """Compile every HIP source for gfx950 with hipcc (one object per source, in parallel)
    and link LIB_PATH (always rebuilds)."""
    from concurrent.futures import ThreadPoolExecutor
    import tempfile
    with tempfile.TemporaryDirectory(prefix="sx8_build_") as d:
        def compile_one(name):
            obj = os.path.join(d, name + ".o")
            flags = [f for f in HIP_FLAGS if f != "-shared"] + SOURCE_FLAGS.get(name, [])
            cmd = [HIPCC, *flags, "-I", CSRC_DIR, "-I", INCLUDE_DIR, "-c", "-o", obj,
                   os.path.join(CSRC_DIR, name)]
            return obj, subprocess.run(cmd, capture_output=True, text=True)
        jobs = min(len(SOURCES), max(1, (os.cpu_count() or 1)), 8)
        with ThreadPoolExecutor(jobs) as ex:
            results = list(ex.map(compile_one, SOURCES))
        errs = [r.stdout + r.stderr for _, r in results if r.returncode != 0]
        if errs:
            raise RuntimeError("hipcc failed:\n" + "\n".join(errs))
        if verbose:
            for _, r in results:
                print(r.stderr)
        tmp = LIB_PATH + ".tmp"
        cmd = [HIPCC, "--offload-arch=gfx950", "-shared", "-fPIC", "-o", tmp, *[o for o, _ in results]]
        res = subprocess.run(cmd, capture_output=True, text=True)
        if res.returncode != 0:
            raise RuntimeError("hipcc link failed:\n" + res.stdout + res.stderr)
    os.replace(tmp, LIB_PATH)
    return LIB_PATH


def lib_path() -> str:
    return os.environ.get("SX8_HIP_LIB", LIB_PATH)


def _hip_runtimes_loaded():
    """Distinct libamdhip64 files mapped into this process."""
    try:
        with open("/proc/self/maps") as f:
            return sorted({ln.split()[-1] for ln in f if "libamdhip64" in ln})
    except OSError:
        return []


def lib():
    """Load the HIP library once; raise RuntimeError if it is missing or stale.

    torch is imported first: it maps its bundled HIP runtime (SONAME libamdhip64.so.7),
    and the dynamic linker then binds this library's libamdhip64.so.7 dependency to
    that same copy.  Two HIP runtimes in one process (torch's and /opt/rocm's) do not
    share devices, streams or allocations, so that case is refused outright."""
    global _lib
    if _lib is not None:
        return _lib
    with _lock:
        if _lib is None:
            import torch  # noqa: F401  (maps torch's HIP runtime before ours)
            path = lib_path()
            if not os.path.exists(path):
                raise RuntimeError(f"S-X8 HIP library not found at {path}; run "
                                   "__graft_entry__.build() (or _sx8lib.build()) first")
            L = ctypes.CDLL(path)
            runtimes = _hip_runtimes_loaded()
            if len(runtimes) > 1:
                raise RuntimeError("two HIP runtimes are loaded in this process: "
                                   + ", ".join(runtimes))
            for name, res, args in SIGNATURES:
                fn = getattr(L, name)
                fn.restype = res
                fn.argtypes = args
            if L.sx8_abi_version() != ABI_VERSION:
                raise RuntimeError(f"{path}: ABI version {L.sx8_abi_version()} != {ABI_VERSION}")
            _lib = L
    return _lib


def call(name: str, *args) -> None:
    """Call an entry point and raise RuntimeError with the library's message on error."""
    L = lib()
    rc = getattr(L, name)(*args)
    if rc != 0:
        msg = L.sx8_last_error().decode(errors="replace")
        raise RuntimeError(f"{name} failed (code {rc}): {msg}")


def ptr(t) -> ctypes.c_void_p:
    """Device pointer of a torch tensor (None -> NULL)."""
    if t is None:
        return ctypes.c_void_p(None)
    return ctypes.c_void_p(t.data_ptr())


def stream(device=None) -> ctypes.c_void_p:
    """The current torch stream on `device` as a hipStream_t."""
    import torch
    return ctypes.c_void_p(torch.cuda.current_stream(device).cuda_stream)


def gemm_workspace(M, Ns, n_cb, device):
    """A fresh workspace for a prefill call over matrices of Ns output columns sharing an
    (M, K) X (sx8_gemm_prefill_workspace_bytes), from torch's caching allocator on the
    current stream: stream-ordered, so calls on different streams never share it, and
    capture-safe (a graph keeps its own copy).  Returns (tensor, bytes)."""
    import torch
    n = len(Ns)
    nb = int(lib().sx8_gemm_prefill_workspace_bytes(int(M), n, (ctypes.c_int64 * n)(*[int(v) for v in Ns]),
                                                    int(n_cb)))
    if nb < 0:
        raise RuntimeError(f"sx8_gemm_prefill_workspace_bytes: bad shape M={M} Ns={list(Ns)} n_cb={n_cb}")
    return torch.empty(max(nb, 256), dtype=torch.uint8, device=device), nb


def gemm_plan(M, Ns, n_cb):
    """The plan a prefill call with these sizes runs: dict(tile, groups, k_ranges,
    kb_per_range, whole_tiles, split_tiles, workspace)."""
    n = len(Ns)
    desc = (ctypes.c_int64 * 8)()
    call("sx8_gemm_prefill_plan", int(M), n, (ctypes.c_int64 * n)(*[int(v) for v in Ns]), int(n_cb), desc)
    keys = ("tile", "groups", "k_ranges", "kb_per_range", "whole_tiles", "split_tiles", "workspace")
    return dict(zip(keys, (int(v) for v in desc[:7])))


GEMM_TUNING_VARS = ("SX8_GEMM_TILE", "SX8_GEMM_PLAN", "SX8_GEMM_W2")


class GemmTuning:
    """Prefill tuning variables set from Python (tuning runs and tests).  The library reads
    SX8_GEMM_TILE / SX8_GEMM_PLAN / SX8_GEMM_W2 once; set() changes them and makes the
    library read them again (sx8_gemm_reload_tuning), restore() puts back what was there."""

    def __init__(self):
        self._saved = {k: os.environ.get(k) for k in GEMM_TUNING_VARS}

    def set(self, **kv):
        for k, v in kv.items():
            name = "SX8_GEMM_" + k.upper()
            if name not in GEMM_TUNING_VARS:
                raise KeyError(name)
            if v is None:
                os.environ.pop(name, None)
            else:
                os.environ[name] = str(v)
        call("sx8_gemm_reload_tuning")

    def restore(self):
        for k, v in self._saved.items():
            if v is None:
                os.environ.pop(k, None)
            else:
                os.environ[k] = v
        call("sx8_gemm_reload_tuning")


def as_device(a, np_dtype, device):
    """numpy array / torch tensor -> contiguous 1-D torch tensor of np_dtype on device.
    A device tensor of the right dtype is used as is (no copy)."""
    import numpy as np
    import torch
    tdt = {np.uint8: torch.uint8, np.uint16: torch.int16, np.float16: torch.float16,
           np.float32: torch.float32, np.int64: torch.int64}[np_dtype]
    if isinstance(a, torch.Tensor):
        t = a.reshape(-1)
        if t.dtype != tdt:
            if np_dtype is np.uint16 and t.dtype == torch.float16:
                t = t.view(torch.int16)
            else:
                t = t.to(tdt)
        return t.to(device).contiguous()
    arr = np.ascontiguousarray(np.asarray(a).reshape(-1))
    if np_dtype is np.uint16 and arr.dtype == np.float16:
        arr = arr.view(np.uint16)
    arr = arr.astype(np_dtype, copy=False)
    if np_dtype is np.uint16:
        arr = arr.view(np.int16)
    return torch.from_numpy(arr).to(device)
