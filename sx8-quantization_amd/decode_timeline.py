"""Per-wave timeline of the decode step's GEMV launches (a profiling aid, GPU only).

Builds an instrumented copy of csrc/sx8_gemv.hip into a temporary directory: wave 0 of every
work-group of every k_gemv_panel / k_gemv_pair launch stamps the shader clock (s_memtime)
at fixed points of the kernel and stores one record.  Then it replays decode steps of the
36-layer decoder through that library (HIP graph, as bench.py's e2e) and prints, per launch
kind, the median work-group's phases in shader cycles:

  pre-tab          kernel start -> activation-table loads issued
  tab->rec         -> first record rounds issued
  build(a)         -> table build (RMSNorm forms: up to the norm's barrier)
  rms->build(b)    RMSNorm forms: norm barrier -> rest of the table build
  barrier          table barrier
  loop             the K loop
  red-barrier      loop end -> reduction barrier passed (waiting for the slowest wave)
  reduce+store     reduction, epilogue, stores

plus the launch span (first start to last end, 100 MHz clock), the median start skew and
the tail after the median work-group ends.  Usage: python3 decode_timeline.py [tokens].
The instrumentation is anchored on the source text; it fails loudly when the kernel code
it expects has changed.
"""
import collections
import ctypes
import os
import subprocess
import sys
import tempfile
from concurrent.futures import ThreadPoolExecutor

import numpy as np

PKG_DIR = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, PKG_DIR)
import _sx8lib as L  # noqa: E402

MAX_REC = 262144

HEADER = r'''
__device__ unsigned long long g_rec[262144 * 16];
__device__ unsigned int g_tick;
#define TS(i) do { __builtin_amdgcn_sched_barrier(0); ts[i] = __builtin_amdgcn_s_memtime(); __builtin_amdgcn_sched_barrier(0); } while (0)
extern "C" int sx8x_ts_reset() { unsigned int z = 0; return (int)hipMemcpyToSymbol(HIP_SYMBOL(g_tick), &z, 4); }
extern "C" int sx8x_ts_read(void* dst, size_t n, unsigned* tick) {
    int r = (int)hipMemcpyFromSymbol(dst, HIP_SYMBOL(g_rec), n);
    if (r) return r;
    return (int)hipMemcpyFromSymbol(tick, HIP_SYMBOL(g_tick), 4);
}
'''


def _record(tag):
    return f"""    TS(7);
    ts[11] = __builtin_amdgcn_s_memrealtime();
    if (tid < 64) {{
        unsigned tk = 0;
        if (tid == 0) tk = atomicAdd(&g_tick, 1u);
        tk = __builtin_amdgcn_readfirstlane(tk);
        if (tid == 0 && tk < 262144) {{
            unsigned long long* o = g_rec + (size_t)tk * 16;
            for (int i = 0; i < 12; ++i) o[i] = ts[i];
            o[12] = gridDim.x;
            o[13] = blockIdx.x;
            o[14] = (unsigned long long)({tag});
            o[15] = (unsigned long long)TP;
        }}
    }}
"""


def instrument(src):
    """The instrumented source text (asserts every anchor)."""
    def sub(old, new, count=1):
        nonlocal src
        if src.count(old) != count:
            raise SystemExit(f"decode_timeline: anchor found {src.count(old)} times, expected {count}: {old[:70]!r}")
        src = src.replace(old, new)

    sub("namespace {\n\nstruct KbInfo", HEADER + "namespace {\n\nstruct KbInfo")
    start = ("    extern __shared__ __align__(16) unsigned char smem[];\n"
             "    float* red = reinterpret_cast<float*>(smem);                 // 2 x 512 floats\n"
             "    KbInfo* info")
    sub(start, "    unsigned long long ts[12] = {};\n    TS(0);\n    ts[10] = __builtin_amdgcn_s_memrealtime();\n"
        + start, 2)
    sub("    asm volatile(\"\" ::: \"memory\");\n    __builtin_amdgcn_sched_barrier(0);\n",
        "    asm volatile(\"\" ::: \"memory\");\n    __builtin_amdgcn_sched_barrier(0);\n    TS(1);\n", 2)
    sub("        load(buf[i], i);\n        __builtin_amdgcn_sched_barrier(0);\n    }\n",
        "        load(buf[i], i);\n        __builtin_amdgcn_sched_barrier(0);\n    }\n    TS(2);\n", 2)
    sub("            const float inv = rms_inv<TP>(xr, h, red, n_units, n_cb * 32, xp.eps, tid);\n",
        "            const float inv = rms_inv<TP>(xr, h, red, n_units, n_cb * 32, xp.eps, tid);\n            TS(8);\n")
    sub("        const float inv = rms_inv<TP>(xr, h, red, n_units, n_cb * 32, pa.eps, tid);\n",
        "        const float inv = rms_inv<TP>(xr, h, red, n_units, n_cb * 32, pa.eps, tid);\n        TS(8);\n")
    sub("    __syncthreads();\n#pragma unroll\n    for (int i = kNR0; i < NR; ++i) load(buf[i], i);",
        "    TS(3);\n    __syncthreads();\n    TS(4);\n#pragma unroll\n    for (int i = kNR0; i < NR; ++i) load(buf[i], i);", 2)
    sub("    red[tid] = acc;\n    __syncthreads();\n    if (tid < 8 * CT) {",
        "    asm volatile(\"\" :: \"v\"(acc));\n    TS(6);\n    red[tid] = acc;\n    __syncthreads();\n    TS(9);\n"
        "    if (tid < 8 * CT) {")
    sub("    if (lane_ok) red[va] = acc;\n    __syncthreads();\n    const int NG = CT > 64 ? 4 : 8;",
        "    asm volatile(\"\" :: \"v\"(acc));\n    TS(6);\n    if (lane_ok) red[va] = acc;\n    __syncthreads();\n"
        "    TS(9);\n    const int NG = CT > 64 ? 4 : 8;")
    # end of k_gemv_panel (after the argmax partials) and of k_gemv_pair
    sub("                xp.amax[2 * panel + 1] = (uint32_t)idx;\n            }\n        }\n    }\n}\n",
        "                xp.amax[2 * panel + 1] = (uint32_t)idx;\n            }\n        }\n    }\n"
        + _record("kX * 100 + kMode * 10 + (kOne ? 1 : 0) + (kPre ? 1000 : 0) + (kResY ? 2000 : 0)") + "}\n")
    sub("                if (slot == 0 && min(32 * kb + 32, N) <= c1) pa.zp[((int64_t)kb * 2 + 1) * 2 + cc] = 0.f;\n"
        "            }\n        }\n    }\n}\n",
        "                if (slot == 0 && min(32 * kb + 32, N) <= c1) pa.zp[((int64_t)kb * 2 + 1) * 2 + cc] = 0.f;\n"
        "            }\n        }\n    }\n" + _record("9999") + "}\n")
    return src


def build(out_dir):
    """libsx8_hip.so with the instrumented GEMV source, in out_dir."""
    src = instrument(open(os.path.join(L.CSRC_DIR, "sx8_gemv.hip")).read())
    gemv = os.path.join(out_dir, "sx8_gemv_ts.hip")
    open(gemv, "w").write(src)
    flags = [f for f in L.HIP_FLAGS if f != "-shared"]

    def cc(name):
        path = gemv if name == "sx8_gemv.hip" else os.path.join(L.CSRC_DIR, name)
        obj = os.path.join(out_dir, name + ".o")
        r = subprocess.run([L.HIPCC, *flags, *L.SOURCE_FLAGS.get(name, []), "-I", L.CSRC_DIR, "-I",
                            L.INCLUDE_DIR, "-c", "-o", obj, path], capture_output=True, text=True)
        if r.returncode:
            raise SystemExit(r.stderr[-3000:])
        return obj

    with ThreadPoolExecutor(8) as ex:
        objs = list(ex.map(cc, L.SOURCES))
    lib = os.path.join(out_dir, "libsx8_hip.so")
    subprocess.run([L.HIPCC, "--offload-arch=gfx950", "-shared", "-fPIC", "-o", lib, *objs], check=True)
    return lib


def main():
    n_tok = int(sys.argv[1]) if len(sys.argv) > 1 else 4
    with tempfile.TemporaryDirectory() as d:
        lib = build(d)
        print("built", lib, flush=True)
        os.environ["SX8_HIP_LIB"] = lib
        import torch
        from e2e_decoder import QWEN3_4B, SX8Decoder
        L.lib()
        raw = ctypes.CDLL(L.lib_path())
        raw.sx8x_ts_read.argtypes = [ctypes.c_void_p, ctypes.c_size_t, ctypes.c_void_p]
        dec = SX8Decoder(QWEN3_4B, device="cuda", seed=7, max_len=1024)
        g = torch.Generator(device="cpu").manual_seed(11)
        ids = torch.randint(0, QWEN3_4B["vocab"], (512,), generator=g).cuda()
        dec.generate(ids, n_tok, use_graph=True)           # capture and warm-up
        torch.cuda.synchronize()
        raw.sx8x_ts_reset()
        dec.generate(ids, n_tok, use_graph=True)           # prefill + n_tok - 1 replays
        torch.cuda.synchronize()
        buf = np.zeros(MAX_REC * 16, np.uint64)
        tick = ctypes.c_uint(0)
        assert raw.sx8x_ts_read(buf.ctypes.data, buf.nbytes, ctypes.byref(tick)) == 0
    n = min(tick.value, MAX_REC)
    rec = buf.reshape(-1, 16)[:n].astype(np.int64)
    launches, i = [], 0
    while i < n:                                          # records of a launch are contiguous
        G = int(rec[i, 12])
        launches.append(rec[i:i + G])
        i += G
    print(f"records {n}, launches {len(launches)}")
    stats = collections.defaultdict(list)
    for lr in launches:
        G, tag, tp = int(lr[0, 12]), int(lr[0, 14]), int(lr[0, 15])
        kx = 1 if tag == 9999 else (tag % 1000) // 100
        key = (f"pair grid {G}" if tag == 9999 else
               f"grid {G} kX {kx} mode {(tag % 100) // 10} one {tag % 10} pre/resy {tag // 1000} TP {tp}")
        t = lr[:, :12]
        rt0, rt1 = t[:, 10], t[:, 11]
        ph = lambda a, b: np.median(t[:, b] - t[:, a])  # noqa: E731
        stats[key].append(((rt1.max() - rt0.min()) * 10 / 1e3, ph(0, 1), ph(1, 2),
                           ph(2, 3) if kx != 1 else ph(2, 8), ph(8, 3) if kx == 1 else 0, ph(3, 4), ph(4, 6),
                           ph(6, 9), ph(9, 7), np.median(t[:, 7] - t[:, 0]),
                           (np.median(rt0) - rt0.min()) * 10 / 1e3, (rt1.max() - np.median(rt1)) * 10 / 1e3))
    print("median work-group, wave 0, shader cycles: pre-tab | tab->rec | build(a) | rms->build(b) | barrier | "
          "loop | red-barrier | reduce+store | total ; start skew us ; tail us")
    for key, v in stats.items():
        a = np.median(np.array(v), axis=0)
        print(f"{key:44s} n={len(v):4d} span {a[0]:6.2f} us | " + " ".join(f"{x:.0f}" for x in a[1:10]) +
              f" | {a[10]:.2f} {a[11]:.2f}")


if __name__ == "__main__":
    main()
