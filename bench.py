"""S-X8 hot-path benchmark on one MI355X: decode GEMV sweep (headline, plus the same layer
as a decoder runs it with grouped launches), fused prefill GEMM at M = 128, 512, 2048, the
vocab-sized matrix (lm_head GEMV at M = 1, GEMM at M = 512, embedding gather of 512 ids),
the end-to-end 36-layer decoder, plus the CPU dequant+GEMV baseline.

Headline (BASELINE.json metric, configs[1]): one step = the M = 1 decode GEMV of every
linear of one synthetic Qwen3-4B-class layer (q 4096x2560, k/v 1024x2560,
o 2560x4096, gate/up 9728x2560, down 2560x9728), weights N(0, 0.02) per seed quantized
to S-X8 with 1% degenerate blocks, x ~ N(0, 1) fp16.  `value` = packed-weight bytes
(30 B per 32 weights) of the step / step time, in GB/s.  Inputs are resident in HBM
before timing; the step cycles through --copies distinct copies of the layer (>1 GB in
total by default) so the 256 MB Infinity Cache cannot serve repeats.

Timing: a GPU delay kernel is queued first so the host enqueues the whole timed
region ahead of the GPU.  The timed region (K steps back to back) is bracketed by two
HIP events on the launch stream (torch's current stream, which the kernels use).  A
second pass of the same K steps brackets every launch with an event pair; its mean is
the per-launch kernel duration used for the roofline.
"""
import argparse
import json
import os
import subprocess
import sys
import time
from concurrent.futures import ThreadPoolExecutor

import numpy as np

REPO = os.path.dirname(os.path.abspath(__file__))
PKG = os.path.join(REPO, "sx8-quantization_amd")
sys.path.insert(0, PKG)

LAYER = [  # (name, N, K)
    ("q_proj", 4096, 2560), ("k_proj", 1024, 2560), ("v_proj", 1024, 2560),
    ("o_proj", 2560, 4096), ("gate_proj", 9728, 2560), ("up_proj", 9728, 2560),
    ("down_proj", 2560, 9728),
]
HBM_PEAK_GBS = 8000.0          # MI355X HBM3E, vendor figure
# Counter figures measured with rocprofv3 on the GPU box (profiles/gemv_decode_layer.md,
# profiles/prefill_gemm_m2048.md).  Each holds for the kernel source it was measured on
# (sha256 prefix of the files listed in SRC_FILES for that kernel); with any other source
# the bench line reports null for it instead of a stale figure.
# HBM bytes per launch = FETCH_SIZE x 2.000 + WRITE_SIZE x 1.000 (KiB per dispatch, scaled by
# what the two counters read for a 512 MiB device copy, bench.py --only copy).
# (the prefill figures are k_gemm_w2's alone, which is built from sx8_gemm.hip and the device
# headers; the Z/pack pass in sx8_gemv.hip is a kernel of its own)
SRC_FILES = {"gemv": ("sx8_gemv.hip", "sx8_device.h", "sx8_buffer.h"),
             "gemm": ("sx8_gemm.hip", "sx8_device.h", "sx8_buffer.h")}
MEASURED = {
    # k_gemv_panel over the layer sweep: mean 6820.9 KiB fetched, 17.1 KiB written per launch
    "gemv_traffic": {"value": (6820.9 * 2.0 + 17.1) * 1024, "src": "gemv", "src_sha16": "81981aeb00e8fc2a",
                     "how": "rocprofv3 --pmc FETCH_SIZE / WRITE_SIZE, bench.py --only gemv --steps 10 "
                            "--warmup 2, first 12 x 7 single-matrix dispatches"},
    # rocprofv3 kernel-trace mean over the 140 timed k_gemv_panel dispatches (20 steps x 7);
    # bench.py's own figure in that traced run: 6.244 us per launch (timed region / launches)
    "gemv_traced_launch_us": {"value": 6.216, "src": "gemv", "src_sha16": "81981aeb00e8fc2a",
                              "how": "rocprofv3 --kernel-trace --stats, bench.py --only gemv --steps 20 "
                                     "(same-run event figure under the tracer: 6.244 us)"},
    # k_gemm_w2 on down_proj at M = 2048 (plan 80 tiles x 3 K ranges): 89776.6 KiB fetched,
    # 61690.7 KiB written per dispatch (Y 21 MB + two partial tiles per split tile 42 MB)
    "prefill_traffic": {"value": (89776.6 * 2.0 + 61690.7) * 1024, "src": "gemm", "src_sha16": "55cfed02a03c334a",
                        "how": "rocprofv3 --pmc FETCH_SIZE / WRITE_SIZE, bench.py --only gemm-one "
                               "--shape down_proj --m 2048 --iters 20, mean of 21 dispatches"},
    # 100 x sum SQ_VALU_MFMA_BUSY_CYCLES / (GRBM_GUI_ACTIVE per XCD x 1024 SIMDs)
    "prefill_mfma_busy_pct": {"value": 48.1, "src": "gemm", "src_sha16": "55cfed02a03c334a",
                              "how": "rocprofv3 --pmc SQ_INSTS_VALU_MFMA_MOPS_F16 SQ_INSTS_VALU_MFMA_F16 "
                                     "SQ_VALU_MFMA_BUSY_CYCLES GRBM_GUI_ACTIVE, bench.py --only gemm-one "
                                     "--shape down_proj --m 2048 --iters 50 (k_gemm_w2; gate: 43.0; 47.0-48.1 on down across boxes and builds)"},
}
MFMA_F16_PEAK_TFLOPS = 2500.0  # MI355X dense fp16 MFMA, vendor figure
# The streaming-read rate measured on the GPU boxes (bench.py --only readbw: best of the
# probe's grid sizes, 6.06-6.25 TB/s across runs): a second reference beside the vendor peak
READ_CEILING_GBS = 6250.0


def src_sha16(kind):
    """sha256 prefix of a kernel's source files (SRC_FILES[kind]): a change to them
    invalidates a counter figure measured on the old source."""
    import hashlib
    h = hashlib.sha256()
    for f in SRC_FILES[kind]:
        with open(os.path.join(PKG, "csrc", f), "rb") as fh:
            h.update(fh.read())
    return h.hexdigest()[:16]


def measured(key):
    """(value or None, note) of a MEASURED counter figure for the source of this tree."""
    m = MEASURED[key]
    sha = src_sha16(m["src"])
    if m["src_sha16"] == sha:
        return m["value"], f"{m['how']} (source {sha})"
    return None, f"not measured on this source ({sha})"


def packed_bytes(N, K):
    return N * ((K + 31) // 32) * 30


def parse():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=50)
    ap.add_argument("--warmup", type=int, default=5)
    ap.add_argument("--copies", type=int, default=12, help="distinct layer copies (cold cache)")
    ap.add_argument("--hdr-bytes", type=int, default=6, choices=[6, 8])
    ap.add_argument("--prefill-m", default="128,512,2048",
                    help="comma-separated M values of the prefill sweep (the last is the headline)")
    ap.add_argument("--no-prefill", action="store_true")
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--cpu-seconds", type=float, default=10.0)
    ap.add_argument("--only", default="", help="restrict to one part: gemv|prefill|vocab|container|quantizer|e2e|copy|"
                    "library|gemm-one|timeline|attn-timeline|readbw|handoff (copy: the 512 MiB device copy that calibrates the HBM byte "
                    "counters; library: torch's fp16 GEMM/GEMV and the copy on the layer's shapes; gemm-one: "
                    "--iters calls of one prefill shape, the counter workload; timeline: per-wave phases of the "
                    "decode step's GEMV launches from an instrumented build; attn-timeline: per-tile phases of the prompt "
                    "attention (--attn-t rows) from an instrumented build; readbw: the streaming-read rate of "
                    "the GPU, a 4 GiB buffer read by a hipcc-built probe; handoff: an in-kernel producer-to-consumer "
                    "handoff against a second launch, a hipcc-built probe)")
    ap.add_argument("--no-library", action="store_true", help="skip the same-run library baseline")
    ap.add_argument("--timeline-tokens", type=int, default=4, help="timeline: tokens generated per run")
    ap.add_argument("--attn-t", type=int, default=512, help="attn-timeline: prompt rows")
    ap.add_argument("--shape", default="gate_proj", help="gemm-one: layer shape name")
    ap.add_argument("--m", type=int, default=2048, help="gemm-one: rows of X")
    ap.add_argument("--iters", type=int, default=200,
                    help="calls per duration distribution (median/p10/p90), at least 200")
    ap.add_argument("--no-e2e", action="store_true")
    ap.add_argument("--e2e-prompt", type=int, default=512)
    ap.add_argument("--e2e-new", type=int, default=256)
    return ap.parse_args()


def log(*a):
    print(*a, file=sys.stderr, flush=True)


def gpu_delay(torch, ms):
    """Queue roughly `ms` of GPU work so the host can enqueue a timed region ahead of
    the GPU (a bounded clock spin; falls back to large fills)."""
    try:
        torch.cuda._sleep(int(ms * 2.0e6))
    except Exception:
        buf = torch.empty(64 << 20, dtype=torch.float32, device="cuda")
        for _ in range(max(1, int(ms / 0.1))):
            buf.fill_(1.0)


def build_layer(torch, dev, hdr_bytes):
    from prepare_v44 import to_v44_device
    from quantize_sx8 import quantize_tensor
    layer = []
    for i, (name, N, K) in enumerate(LAYER):
        seed = 1000 + i
        g = torch.Generator(device="cpu").manual_seed(seed)
        W = (torch.randn(N, K, generator=g) * 0.02).half()
        qt, bi = quantize_tensor(W, device=dev, degenerate_frac=0.01, seed=seed + 1)
        hdr, lvl, bas, sca = to_v44_device(qt, bi, hdr_aligned=(hdr_bytes == 8), device=dev)
        layer.append({"name": name, "N": N, "K": K, "n_cb": qt["n_cb"], "qt": qt, "bi": bi,
                      "hdr": hdr, "lvl": lvl, "bas": bas, "sca": sca})
        log(f"quantized {name} {N}x{K}")
    return layer


class HipEvents:
    """Timing events straight from the HIP runtime torch already loaded, created with
    hipEventDisableSystemFence so a record does not flush system-scope caches (torch's
    default events add several microseconds per record).  Records go to `stream`."""

    def __init__(self, n, stream):
        import ctypes
        self.hip = ctypes.CDLL("libamdhip64.so.7")        # binds to the loaded runtime
        self.hip.hipEventCreateWithFlags.argtypes = [ctypes.c_void_p, ctypes.c_uint]
        self.hip.hipEventRecord.argtypes = [ctypes.c_void_p, ctypes.c_void_p]
        self.hip.hipEventElapsedTime.argtypes = [ctypes.c_void_p, ctypes.c_void_p, ctypes.c_void_p]
        self.hip.hipEventDestroy.argtypes = [ctypes.c_void_p]
        self.stream = stream
        self.ev = []
        flags = 0x20000000                                 # hipEventDisableSystemFence
        for _ in range(n):
            e = ctypes.c_void_p()
            if self.hip.hipEventCreateWithFlags(ctypes.byref(e), flags) != 0:
                raise RuntimeError("hipEventCreateWithFlags failed")
            self.ev.append(e)
        self._f = ctypes.c_float()
        self._ctypes = ctypes

    def record(self, i):
        if self.hip.hipEventRecord(self.ev[i], self.stream) != 0:
            raise RuntimeError("hipEventRecord failed")

    def ms(self, a, b):
        if self.hip.hipEventElapsedTime(self._ctypes.byref(self._f), self.ev[a], self.ev[b]) != 0:
            raise RuntimeError("hipEventElapsedTime failed")
        return self._f.value

    def close(self):
        for e in self.ev:
            self.hip.hipEventDestroy(e)


def quantiles(us):
    """median, p10, p90 (and the sample count) of a list of durations in us."""
    a = np.asarray(us, dtype=np.float64)
    p10, p50, p90 = np.percentile(a, [10, 50, 90])
    return {"median_us": float(p50), "p10_us": float(p10), "p90_us": float(p90), "n": int(a.size)}


def call_series(torch, st, fn, n, delay_ms=10):
    """Durations (us) of n back-to-back calls fn(i): one HIP event (no system fence) on the
    launch stream before the first call and after each one, so call i's duration is the
    time between the events around it, the event packet included."""
    ev = HipEvents(n + 1, st)
    gpu_delay(torch, delay_ms)
    ev.record(0)
    for i in range(n):
        fn(i)
        ev.record(i + 1)
    torch.cuda.synchronize()
    out = [ev.ms(i, i + 1) * 1e3 for i in range(n)]
    ev.close()
    return out


def region_series(torch, st, fn, n, reps=10, delay_ms=10):
    """Per-call time (us) of n back-to-back calls fn(i) with one HIP event before the first
    and one after the last (nothing between the calls: the GEMV headline's method), `reps`
    such regions; returns the regions' per-call times."""
    out = []
    for _ in range(reps):
        ev = HipEvents(2, st)
        gpu_delay(torch, delay_ms)
        ev.record(0)
        for i in range(n):
            fn(i)
        ev.record(1)
        torch.cuda.synchronize()
        out.append(ev.ms(0, 1) * 1e3 / n)
        ev.close()
    return out


def bench_gemv(torch, L, layer, args):
    import ctypes
    dev = torch.device("cuda:0")
    R = max(1, args.copies)
    copies = [[(t["hdr"].clone(), t["lvl"].clone()) for t in layer] for _ in range(R)]
    copies[0] = [(t["hdr"], t["lvl"]) for t in layer]
    g = torch.Generator(device="cpu").manual_seed(2)
    xs = {K: torch.randn(K, generator=g).half().to(dev) for K in {t["K"] for t in layer}}
    ys = [torch.empty(t["N"], dtype=torch.float32, device=dev) for t in layer]
    zs = [torch.empty(t["n_cb"], 2, dtype=torch.float32, device=dev) for t in layer]
    wss = [torch.empty(L.lib().sx8_gemv_workspace_bytes(t["n_cb"]) // 4, dtype=torch.float32,
                       device=dev) for t in layer]
    st = L.stream(dev)
    calls = []
    for r in range(R):
        step = []
        for i, t in enumerate(layer):
            h, lv = copies[r][i]
            step.append((L.ptr(xs[t["K"]]), L.ptr(h), L.ptr(lv), args.hdr_bytes, L.ptr(t["bas"]),
                         L.ptr(t["sca"]), ctypes.c_void_p(None), ctypes.c_void_p(None), t["N"], t["n_cb"],
                         L.ptr(ys[i]), L.ptr(wss[i]), wss[i].numel() * 4, st))
        calls.append(step)
    fn = L.lib().sx8_gemv
    step_bytes = sum(packed_bytes(t["N"], t["K"]) for t in layer)
    log(f"gemv: {R} copies x {step_bytes / 1e6:.1f} MB = {R * step_bytes / 1e9:.2f} GB resident")
    nL = len(layer)
    K = args.steps
    ev = HipEvents(2, st)

    def run_step(s):
        for a in calls[s % R]:
            rc = fn(*a)
            if rc != 0:
                raise RuntimeError(L.lib().sx8_last_error().decode())

    for s in range(args.warmup):
        run_step(s)
    torch.cuda.synchronize()

    # timed region: K steps back to back, bracketed by two events (nothing in between)
    gpu_delay(torch, 50)                     # keep the GPU busy while the host enqueues
    ev.record(0)
    for s in range(K):
        run_step(s)
    ev.record(1)
    torch.cuda.synchronize()
    total_ms = ev.ms(0, 1)

    # distributions: args.iters steps with an event after each, and args.iters launches of
    # each shape alone (rotating copies) with an event after each
    nd = max(200, args.iters)
    step_us = call_series(torch, st, run_step, nd, delay_ms=50)
    per_shape = {}
    for i, t in enumerate(layer):
        def one(r, i=i):
            rc = fn(*calls[r % R][i])
            if rc != 0:
                raise RuntimeError(L.lib().sx8_last_error().decode())
        q = quantiles(call_series(torch, st, one, nd))
        q["gbs_at_median"] = packed_bytes(t["N"], t["K"]) / (q["median_us"] * 1e-6) / 1e9
        per_shape[t["name"]] = q
    step_q = quantiles(step_us)
    step_q["gbs_at_median"] = sum(packed_bytes(t["N"], t["K"]) for t in layer) / (step_q["median_us"] * 1e-6) / 1e9

    # the same layer as a decoder step runs it: q/k/v and gate/up share their input and
    # go out as one launch each (sx8_gemv_group), o and down alone -> 4 launches per step
    idx = {t["name"]: i for i, t in enumerate(layer)}
    groups = [["q_proj", "k_proj", "v_proj"], ["o_proj"], ["gate_proj", "up_proj"], ["down_proj"]]
    gfn = L.lib().sx8_gemv_group
    gcalls = []
    for r in range(R):
        step = []
        for grp in groups:
            ii = [idx[n] for n in grp if n in idx]
            if not ii:
                continue
            n = len(ii)
            P = ctypes.c_void_p * n
            t0 = layer[ii[0]]
            step.append((L.ptr(xs[t0["K"]]), n, P(*[copies[r][i][0].data_ptr() for i in ii]),
                         P(*[copies[r][i][1].data_ptr() for i in ii]), args.hdr_bytes,
                         P(*[layer[i]["bas"].data_ptr() for i in ii]),
                         P(*[layer[i]["sca"].data_ptr() for i in ii]), None,
                         (ctypes.c_int64 * n)(*[layer[i]["N"] for i in ii]), t0["n_cb"],
                         P(*[ys[i].data_ptr() for i in ii]), None, 0, st))
        gcalls.append(step)

    def run_group_step(s):
        for a in gcalls[s % R]:
            if gfn(*a) != 0:
                raise RuntimeError(L.lib().sx8_last_error().decode())

    for s in range(args.warmup):
        run_group_step(s)
    torch.cuda.synchronize()
    gpu_delay(torch, 50)
    ev.record(0)
    for s in range(K):
        run_group_step(s)
    ev.record(1)
    torch.cuda.synchronize()
    g_ms = ev.ms(0, 1)
    ev.close()
    gq = quantiles(call_series(torch, st, run_group_step, nd, delay_ms=50))
    grouped = {"launches_per_step": len(gcalls[0]), "ms_per_step": g_ms / K,
               "gbs": step_bytes * K / (g_ms * 1e-3) / 1e9, "step_us": gq,
               "groups": [g for g in groups]}

    # the same seven launches per step, replayed from a HIP graph (how a decode loop that
    # captures its step launches them): one graph holds the R rotated steps; the kernels are
    # the eager ones, only the host dispatch between them goes away
    graph = torch.cuda.CUDAGraph()
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        with torch.cuda.graph(graph, stream=side):
            cst = L.stream(dev)
            for r in range(R):
                for a in calls[r]:
                    if fn(*(a[:-1] + (cst,))) != 0:
                        raise RuntimeError(L.lib().sx8_last_error().decode())
    torch.cuda.current_stream().wait_stream(side)
    n_rep = max(1, K // R)
    graph.replay()
    torch.cuda.synchronize()
    ge0, ge1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    gpu_delay(torch, 50)
    ge0.record()
    for _ in range(n_rep):
        graph.replay()
    ge1.record()
    torch.cuda.synchronize()
    gr_ms = ge0.elapsed_time(ge1)
    del graph
    graph_res = {"steps": n_rep * R, "ms_per_step": gr_ms / (n_rep * R),
                 "gbs": step_bytes * n_rep * R / (gr_ms * 1e-3) / 1e9}
    out = {
        "ms_per_step": total_ms / K,
        "value_gbs": step_bytes * K / (total_ms * 1e-3) / 1e9,
        "launches": K * nL,
        "avg_launch_us": total_ms * 1e3 / (K * nL),
        "bytes_per_launch": step_bytes / nL,
        "achieved_gbs": step_bytes * K / (total_ms * 1e-3) / 1e9,
        "step_us": step_q,
        "per_shape": per_shape,
        "step_bytes": step_bytes,
        "grouped": grouped,
        "graph": graph_res,
    }
    return out


def bench_prefill_m(torch, L, layer, args, M):
    dev = torch.device("cuda:0")
    g = torch.Generator(device="cpu").manual_seed(12)
    xs = {K: torch.randn(M, K, generator=g).half().to(dev) for K in {t["K"] for t in layer}}
    ys = [torch.empty(M, t["N"], dtype=torch.float32, device=dev) for t in layer]
    wss = [L.gemm_workspace(M, (t["N"],), t["n_cb"], dev) for t in layer]
    st = L.stream(dev)
    fn = L.lib().sx8_gemm_prefill

    def one(i, t):
        rc = fn(L.ptr(xs[t["K"]]), M, t["K"], t["K"], L.ptr(t["hdr"]), L.ptr(t["lvl"]),
                args.hdr_bytes, L.ptr(t["bas"]), L.ptr(t["sca"]), t["N"], t["n_cb"],
                L.ptr(ys[i]), L.ptr(wss[i][0]), wss[i][1], st)
        if rc != 0:
            raise RuntimeError(L.lib().sx8_last_error().decode())

    for i, t in enumerate(layer):
        one(i, t)
    torch.cuda.synchronize()
    res = {}
    tot_flop, tot_us = 0.0, 0.0
    for i, t in enumerate(layer):
        q = quantiles(call_series(torch, st, lambda r, i=i, t=t: one(i, t), max(200, args.iters)))
        flop = 2.0 * M * t["N"] * t["K"]
        q["us"] = q["median_us"]
        q["tflops"] = flop / (q["median_us"] * 1e-6) / 1e12
        q["plan"] = L.gemm_plan(M, (t["N"],), t["n_cb"])
        res[t["name"]] = q
        tot_flop += flop
        tot_us += q["median_us"]
        log(f"prefill {t['name']} M={M}: {q['median_us']:.1f} us (p10 {q['p10_us']:.1f}, p90 {q['p90_us']:.1f}) "
            f"{q['tflops']:.1f} TFLOP/s")
    tf = tot_flop / (tot_us * 1e-6) / 1e12
    return {"M": M, "tflops": tf, "layer_us": tot_us, "layer_flop": tot_flop, "per_shape": res,
            "frac_of_mfma_peak": tf / MFMA_F16_PEAK_TFLOPS}


def bench_prefill_grouped(torch, L, layer, args, M):
    """The layer at M rows as a prompt pass runs it: q/k/v and gate/up each one
    sx8_gemm_prefill_group call, o and down alone (4 calls); TFLOP/s over the layer."""
    import ctypes
    dev = torch.device("cuda:0")
    g = torch.Generator(device="cpu").manual_seed(12)
    xs = {K: torch.randn(M, K, generator=g).half().to(dev) for K in {t["K"] for t in layer}}
    ys = [torch.empty(M, t["N"], dtype=torch.float32, device=dev) for t in layer]
    st = L.stream(dev)
    fn = L.lib().sx8_gemm_prefill_group
    by = {t["name"]: i for i, t in enumerate(layer)}
    groups = [["q_proj", "k_proj", "v_proj"], ["o_proj"], ["gate_proj", "up_proj"], ["down_proj"]]
    calls, keep = [], []
    for grp in groups:
        ii = [by[n] for n in grp]
        n = len(ii)
        P = ctypes.c_void_p * n
        t0 = layer[ii[0]]
        ws, nb = L.gemm_workspace(M, [layer[i]["N"] for i in ii], t0["n_cb"], dev)
        keep.append(ws)
        calls.append((L.ptr(xs[t0["K"]]), M, t0["K"], t0["K"], n, P(*[layer[i]["hdr"].data_ptr() for i in ii]),
                      P(*[layer[i]["lvl"].data_ptr() for i in ii]), args.hdr_bytes,
                      P(*[layer[i]["bas"].data_ptr() for i in ii]), P(*[layer[i]["sca"].data_ptr() for i in ii]),
                      (ctypes.c_int64 * n)(*[layer[i]["N"] for i in ii]), t0["n_cb"],
                      P(*[ys[i].data_ptr() for i in ii]), L.ptr(ws), nb, st))

    def step():
        for a in calls:
            if fn(*a) != 0:
                raise RuntimeError(L.lib().sx8_last_error().decode())

    step()
    torch.cuda.synchronize()
    q = quantiles(call_series(torch, st, lambda r: step(), max(200, args.iters)))
    flop = sum(2.0 * M * t["N"] * t["K"] for t in layer)
    tf = flop / (q["median_us"] * 1e-6) / 1e12
    log(f"prefill grouped M={M}: {q['median_us']:.1f} us (p10 {q['p10_us']:.1f}, p90 {q['p90_us']:.1f}) "
        f"{tf:.1f} TFLOP/s")
    return {"M": M, "calls_per_layer": len(calls), "us": q["median_us"], "us_dist": q, "tflops": tf,
            "frac_of_mfma_peak": tf / MFMA_F16_PEAK_TFLOPS, "groups": groups}


def bench_prefill(torch, L, layer, args):
    """Fused dequant + GEMM over the layer at every M of --prefill-m (config 2); the last M
    (2048 by default) is the headline.  Also the layer as a prompt pass runs it (grouped
    calls) at every M."""
    ms = [int(v) for v in str(args.prefill_m).split(",") if v.strip()]
    sweep = {M: bench_prefill_m(torch, L, layer, args, M) for M in ms}
    out = dict(sweep[ms[-1]])
    out["grouped"] = {str(M): bench_prefill_grouped(torch, L, layer, args, M) for M in ms}
    out["sweep"] = {str(M): {"tflops": r["tflops"], "frac_of_mfma_peak": r["frac_of_mfma_peak"],
                             "per_shape_tflops": {k: v["tflops"] for k, v in r["per_shape"].items()}}
                    for M, r in sweep.items()}
    return out


def bench_container(torch, L, layer, args):
    """§8f row 2: the layer written as an .sx8v43 container (v1.1, with a small-tensor
    section) and loaded straight into the v4.4 device layout (load_v44: file map, one
    host-to-device copy of each tensor's block payload, sx8_v43_to_v44 on the GPU), plus
    the layout kernel alone on device-resident payloads (30 B read + 30 B written per
    block)."""
    import tempfile
    import sx8_container_v43 as C
    dev = torch.device("cuda:0")
    wd = {t["name"] + ".weight": t["qt"] for t in layer}
    bd = {t["name"] + ".weight": t["bi"] for t in layer}
    small = {"norm.weight": {"shape": (2560,), "dtype": "fp16",
                             "data": np.ones(2560, dtype=np.float16)}}
    out = {}
    with tempfile.TemporaryDirectory() as d:
        path = os.path.join(d, "layer.sx8v43")
        t0 = time.time()
        C.write_sx43((wd, bd, {"bench": 1}), path, verbose=False, config={"hidden_size": 2560},
                     small=small)
        out["write_s"] = time.time() - t0
        out["file_bytes"] = os.path.getsize(path)
        C.load_v44(path, device=dev, hdr_bytes=args.hdr_bytes)     # warm the page cache
        torch.cuda.synchronize()
        t0 = time.time()
        t44 = C.load_v44(path, device=dev, hdr_bytes=args.hdr_bytes)
        torch.cuda.synchronize()
        out["load_s"] = time.time() - t0
        out["load_gbs"] = out["file_bytes"] / out["load_s"] / 1e9
    # the layout kernel alone
    lib = L.lib()
    st = L.stream(dev)
    jobs = []
    for t in layer:
        qt = t["qt"]
        nb = qt["n_blocks"]
        raw = torch.from_numpy(np.concatenate([np.asarray(qt[k]).reshape(-1).view(np.uint8) for k in
                                               ("dmin", "dmax", "config", "levels_hi", "levels_lo",
                                                "coeff")])).to(dev)
        hdr = torch.empty(nb, args.hdr_bytes, dtype=torch.uint8, device=dev)
        lvl = torch.empty(nb, 24, dtype=torch.uint8, device=dev)
        jobs.append((raw, hdr, lvl, qt["shape"][0], qt["n_cb"], nb))

    def run():
        for raw, hdr, lvl, out_f, n_cb, nb in jobs:
            b = raw.data_ptr()
            P = L.ctypes.c_void_p
            rc = lib.sx8_v43_to_v44(P(b), P(b + 2 * nb), P(b + 4 * nb), P(b + 29 * nb), P(b + 5 * nb),
                                    P(b + 21 * nb), out_f, n_cb, args.hdr_bytes, L.ptr(hdr), L.ptr(lvl), st)
            if rc != 0:
                raise RuntimeError(lib.sx8_last_error().decode())
    run()
    torch.cuda.synchronize()
    a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    gpu_delay(torch, 10)
    a.record()
    for _ in range(10):
        run()
    b.record()
    torch.cuda.synchronize()
    ms = a.elapsed_time(b) / 10
    blocks = sum(j[5] for j in jobs)
    out["layout_us"] = ms * 1e3
    out["layout_gbs"] = blocks * 60 / (ms * 1e-3) / 1e9
    ok = all(torch.equal(t44[t["name"] + ".weight"][0], t["hdr"]) and
             torch.equal(t44[t["name"] + ".weight"][1], t["lvl"]) for t in layer)
    out["matches_in_memory_layout"] = bool(ok)
    log(f"container: load {out['load_s'] * 1e3:.1f} ms ({out['load_gbs']:.2f} GB/s), "
        f"layout kernel {out['layout_us']:.1f} us ({out['layout_gbs']:.0f} GB/s)")

    # §8f row 4: the same layer as a GGUF (block_sx8 records), loaded into the v4.4 layout,
    # and the llama.cpp fork's no-PCA float32 dequant (R32-ggml) of all its blocks
    import sx8_gguf as G
    gg = {}
    with tempfile.TemporaryDirectory() as d:
        path = os.path.join(d, "layer.gguf")
        G.convert(wd, path)
        gg["file_bytes"] = os.path.getsize(path)
        G.load_v44(path, device=dev, hdr_bytes=args.hdr_bytes)
        torch.cuda.synchronize()
        t0 = time.time()
        g44 = G.load_v44(path, device=dev, hdr_bytes=args.hdr_bytes)
        torch.cuda.synchronize()
        gg["load_s"] = time.time() - t0
        gg["matches_container_layout"] = bool(all(
            torch.equal(g44[n][0], t44[n][0]) and torch.equal(g44[n][1], t44[n][1]) for n in wd))
    dq = []
    for t in layer:
        qt = t["qt"]
        blk = torch.from_numpy(G.blockify(qt).reshape(-1)).to(dev)
        dq.append((blk, qt["shape"][0], qt["n_cb"], torch.empty(qt["shape"][0], t["K"], dtype=torch.float32,
                                                                device=dev)))

    def run_dq():
        for blk, out_f, n_cb, y in dq:
            G.dequant_ggml(blk, out_f, n_cb, contract=True, out=y)
    run_dq()
    torch.cuda.synchronize()
    a.record()
    for _ in range(5):
        run_dq()
    b.record()
    torch.cuda.synchronize()
    ms = a.elapsed_time(b) / 5
    gg["r32_ggml_dequant_us"] = ms * 1e3
    gg["r32_ggml_gbs"] = blocks * (30 + 128) / (ms * 1e-3) / 1e9
    out["gguf"] = gg
    log(f"gguf: load {gg['load_s'] * 1e3:.1f} ms, R32-ggml dequant {gg['r32_ggml_dequant_us']:.0f} us "
        f"({gg['r32_ggml_gbs']:.0f} GB/s)")
    return out


def bench_quantizer(torch, L, args):
    """§8f row 3: the S-X8 quantizer on the GPU over one layer's shapes (weights already
    on the device): V6 encode + packing as one HIP kernel (timed alone with HIP events) and
    the whole quantize_tensor (V6 kernel + batched Gram/eigh PCA in torch + copies to host
    arrays), wall time.  weights/s and the time that rate gives for 4.0e9 weights."""
    from quantize_sx8 import quantize_tensor, v6_encode_hip
    dev = torch.device("cuda:0")
    g = torch.Generator(device=dev).manual_seed(9)
    Ws = [(torch.randn(N, K, generator=g, device=dev) * 0.02).half() for _, N, K in LAYER]
    n_w = sum(w.numel() for w in Ws)
    blocks = [w.reshape(-1, 32) for w in Ws]
    for b in blocks:
        v6_encode_hip(b)
    torch.cuda.synchronize()
    a, b_ = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    a.record()
    for b in blocks:
        v6_encode_hip(b)
    b_.record()
    torch.cuda.synchronize()
    v6_ms = a.elapsed_time(b_)
    quantize_tensor(Ws[1], device=dev)
    torch.cuda.synchronize()
    t0 = time.time()
    for w in Ws:
        quantize_tensor(w, device=dev)
    torch.cuda.synchronize()
    q_s = time.time() - t0
    out = {"weights": n_w, "v6_encode_ms": v6_ms, "v6_weights_per_s": n_w / (v6_ms * 1e-3),
           "quantize_s": q_s, "quantize_weights_per_s": n_w / q_s,
           "model_4b_s": 4.0e9 / (n_w / q_s)}
    log(f"quantizer: V6 kernel {v6_ms:.2f} ms for {n_w / 1e6:.0f} M weights; quantize_tensor "
        f"{q_s:.2f} s ({out['quantize_weights_per_s'] / 1e6:.0f} M weights/s, 4e9 weights in "
        f"{out['model_4b_s']:.0f} s)")
    return out


VOCAB = 151936


def bench_vocab(torch, L, args):
    """Config 3 on one vocab-sized S-X8 matrix (151936 x 2560, seeded N(0, 0.02), 1%
    degenerate blocks): the lm_head GEMV at M = 1 and the prefill GEMM at M = 512 through
    it, and the embedding row gather of 512 ids drawn uniformly from [0, 151936)."""
    from prepare_v44 import to_v44_device
    from quantize_sx8 import quantize_tensor
    dev = torch.device("cuda:0")
    N, K = VOCAB, 2560
    g = torch.Generator(device="cpu").manual_seed(4242)
    W = (torch.randn(N, K, generator=g) * 0.02).half()
    qt, bi = quantize_tensor(W, device=dev, degenerate_frac=0.01, seed=4243)
    del W
    hdr, lvl, bas, sca = to_v44_device(qt, bi, hdr_aligned=(args.hdr_bytes == 8), device=dev)
    n_cb = qt["n_cb"]
    st = L.stream(dev)
    lib = L.lib()
    out = {"shape": f"{N}x{K}", "packed_bytes": packed_bytes(N, K)}

    def timed(fn, reps):
        """median ms over 10 series of `reps` back-to-back calls, an event after each call and
        the same pause before each series as before each timed region (and the distribution);
        `region` gets the per-call time of timed regions of `reps` calls with events only
        around each region (the GEMV headline's method); `sustained` the distribution of one
        series of max(reps, --iters) calls.  (A long series of these 365 MB reads drifts: the
        lm_head GEMV runs ~65 us per call in its first 20 calls, then 70-88 us once the GPU
        has streamed from HBM for more than ~1.5 ms without a pause; the kernel is the same.)"""
        fn()
        torch.cuda.synchronize()
        q = quantiles([u for _ in range(10) for u in call_series(torch, st, lambda r: fn(), reps)])
        dist.append(q)
        region.append(quantiles(region_series(torch, st, lambda r: fn(), reps)))
        sustained.append(quantiles(call_series(torch, st, lambda r: fn(), max(reps, args.iters))))
        return q["median_us"] * 1e-3

    dist, region, sustained = [], [], []

    def ok(rc):
        if rc != 0:
            raise RuntimeError(lib.sx8_last_error().decode())

    # lm_head GEMV, M = 1
    x1 = torch.randn(K, generator=g).half().to(dev)
    y1 = torch.empty(N, dtype=torch.float32, device=dev)
    ws = torch.empty(int(lib.sx8_gemv_workspace_bytes(n_cb)) // 4 + 64, dtype=torch.float32, device=dev)
    ms = timed(lambda: ok(lib.sx8_gemv(L.ptr(x1), L.ptr(hdr), L.ptr(lvl), args.hdr_bytes, L.ptr(bas),
                                       L.ptr(sca), None, None, N, n_cb, L.ptr(y1), L.ptr(ws),
                                       ws.numel() * 4, st)), 20)
    rus = region[-1]["median_us"]
    out["gemv_m1"] = {"us": ms * 1e3, "gbs": packed_bytes(N, K) / (ms * 1e-3) / 1e9, "us_dist": dist[-1],
                      "region_us": rus, "region_gbs": packed_bytes(N, K) / (rus * 1e-6) / 1e9,
                      "region_dist": region[-1], "sustained_dist": sustained[-1],
                      "method": "us: median over 10 series of 20 back-to-back calls with an event after each "
                                "call; sustained_dist: one series of max(20, --iters) such calls",
                      "region_method": "median over 10 timed regions of 20 back-to-back calls, one event "
                                       "before and one after each region (as the layer sweep's avg_launch_us)"}
    log(f"vocab gemv M=1: {ms * 1e3:.1f} us {out['gemv_m1']['gbs']:.0f} GB/s (event after each call); "
        f"{rus:.1f} us {out['gemv_m1']['region_gbs']:.0f} GB/s (timed regions)")
    # lm_head prefill GEMM, M = 512
    M = 512
    xm = torch.randn(M, K, generator=g).half().to(dev)
    ym = torch.empty(M, N, dtype=torch.float32, device=dev)
    wsm, nbm = L.gemm_workspace(M, (N,), n_cb, dev)
    ms = timed(lambda: ok(lib.sx8_gemm_prefill(L.ptr(xm), M, K, K, L.ptr(hdr), L.ptr(lvl), args.hdr_bytes,
                                               L.ptr(bas), L.ptr(sca), N, n_cb, L.ptr(ym), L.ptr(wsm), nbm,
                                               st)), 5)
    out["gemm_m512"] = {"us": ms * 1e3, "tflops": 2.0 * M * N * K / (ms * 1e-3) / 1e12, "us_dist": dist[-1],
                        "region_us": region[-1]["median_us"],
                        "region_tflops": 2.0 * M * N * K / (region[-1]["median_us"] * 1e-6) / 1e12,
                        "sustained_dist": sustained[-1],
                        "plan": L.gemm_plan(M, (N,), n_cb)}
    log(f"vocab gemm M=512: {ms * 1e3:.1f} us {out['gemm_m512']['tflops']:.0f} TFLOP/s")
    del ym
    # embedding gather of 512 ids
    ids = torch.randint(0, N, (512,), generator=g).to(dev)
    rows = torch.empty(512, K, dtype=torch.float16, device=dev)
    ms = timed(lambda: ok(lib.sx8_embed_gather(L.ptr(ids), 512, L.ptr(hdr), L.ptr(lvl), args.hdr_bytes,
                                               L.ptr(bas), L.ptr(sca), K, N, n_cb, L.ptr(rows), st)), 20)
    rd, wr = 512 * n_cb * 30, 512 * K * 2
    out["embed"] = {"ids": 512, "us": ms * 1e3, "gbs": (rd + wr) / (ms * 1e-3) / 1e9, "us_dist": dist[-1],
                    "region_us": region[-1]["median_us"], "sustained_dist": sustained[-1]}
    log(f"vocab embed 512 ids: {ms * 1e3:.1f} us")
    return out


def bench_e2e(torch, args):
    """Config 5: 36-layer random-init Qwen3-4B-style decoder on S-X8 weights (every layer
    quantized separately), batch 1: a 512-token prefill of uniform-random ids, then 256
    greedy tokens, one decode step replayed from a HIP graph.  The whole generate() runs
    twice; the second (warm) run is reported, then once more with every decode step launched
    from the host (no graph).  Generation's prefill computes the lm_head
    for the last prompt row only (all it needs); the prefill with logits for every row --
    what a Hugging Face forward computes -- is timed separately."""
    from e2e_decoder import QWEN3_4B, SX8Decoder
    t0 = time.time()
    dec = SX8Decoder(QWEN3_4B, device="cuda", seed=7, max_len=1024)
    log(f"e2e: built in {time.time() - t0:.1f}s")
    g = torch.Generator(device="cpu").manual_seed(11)
    ids = torch.randint(0, QWEN3_4B["vocab"], (args.e2e_prompt,), generator=g).cuda()
    res = None
    out = None
    for _ in range(2):
        out, tp, td = dec.generate(ids, args.e2e_new, use_graph=True)
        res = {"prompt": args.e2e_prompt, "new_tokens": args.e2e_new,
               "prefill_ms": tp * 1e3, "prefill_tok_s": args.e2e_prompt / tp,
               "prefill_logits": "last row only (generation path)",
               "decode_ms_per_token": td * 1e3 / (args.e2e_new - 1),
               "decode_tok_s": (args.e2e_new - 1) / td,
               "weights_gb": sum(t.numel() for ly in dec.layers for lin in
                                 (ly.q, ly.k, ly.v, ly.o, ly.gate, ly.up, ly.down)
                                 for t in lin._t44[:2]) / 1e9 + sum(t.numel() for t in dec.head._t44[:2]) / 1e9}
        log("e2e", json.dumps(res))
    # the prompt pass alone, five more times (one pass is a few ms, so a single timing moves
    # with the box's state): the median is the reported prefill figure, generate()'s second
    # pass is kept beside it
    passes = []
    for _ in range(5):
        torch.cuda.synchronize()
        t1 = time.perf_counter()
        dec.prefill_fused(ids)
        torch.cuda.synchronize()
        passes.append(time.perf_counter() - t1)
    tp5 = float(np.median(passes))
    res["prefill_generate_ms"] = res["prefill_ms"]
    res["prefill_ms"] = tp5 * 1e3
    res["prefill_tok_s"] = args.e2e_prompt / tp5
    res["prefill_passes_ms"] = [round(t * 1e3, 3) for t in passes]
    res["prefill_method"] = ("median of 5 prompt passes (generation path: lm_head on the last row), each "
                             "between two device synchronizations; prefill_generate_ms is the second "
                             "generate()'s pass")
    log("e2e prompt passes", f"{tp5 * 1e3:.3f} ms median of {[round(t * 1e3, 3) for t in passes]}")
    # the same decode without the graph: every step's launches issued from the host (the
    # same kernels; the greedy tokens must not change)
    out_e, _, td_e = dec.generate(ids, args.e2e_new, use_graph=False)
    res["decode_eager_ms_per_token"] = td_e * 1e3 / (args.e2e_new - 1)
    res["decode_eager_tok_s"] = (args.e2e_new - 1) / td_e
    res["eager_tokens_equal_graph"] = bool(torch.equal(out_e, out))
    log("e2e eager decode", f"{res['decode_eager_ms_per_token']:.3f} ms/token, tokens equal: "
        f"{res['eager_tokens_equal_graph']}")
    times = []
    for _ in range(3):
        torch.cuda.synchronize()
        t1 = time.perf_counter()
        dec.prefill_fused(ids, all_logits=True)
        torch.cuda.synchronize()
        times.append(time.perf_counter() - t1)
    ta = min(times[1:])
    res["prefill_all_logits_ms"] = ta * 1e3
    res["prefill_all_logits_tok_s"] = args.e2e_prompt / ta
    log("e2e all-row logits prefill", f"{ta * 1e3:.2f} ms")
    del dec
    torch.cuda.empty_cache()
    return res


def bench_copy(torch, args):
    """Plain device copy of 512 MiB (torch's elementwise copy kernel), 10 launches: the
    known-size kernel that calibrates the FETCH_SIZE / WRITE_SIZE counters (each launch
    reads and writes exactly 512 MiB), and the achievable streaming rate of this GPU."""
    nbytes = 512 << 20
    src = torch.ones(nbytes // 4, dtype=torch.float32, device="cuda")
    dst = torch.empty_like(src)
    dst.copy_(src)
    torch.cuda.synchronize()
    a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    gpu_delay(torch, 10)
    a.record()
    for _ in range(10):
        dst.copy_(src)
    b.record()
    torch.cuda.synchronize()
    us = a.elapsed_time(b) * 1e3 / 10
    return {"bytes_read": nbytes, "bytes_written": nbytes, "us": us,
            "gbs": 2 * nbytes / (us * 1e-6) / 1e9}


def bench_library(torch, args):
    """Same-run library baseline on the layer's shapes, without any dequant: torch's fp16
    GEMM (hipBLASLt) Y (M, N) fp16 = X (M, K) . W^T at every M of --prefill-m (TFLOP/s per
    shape and over the layer, median of --iters calls), torch's fp16 GEMV at M = 1 over the
    layer with 6 rotated copies of the fp16 weights (1.2 GB, cold cache; GB/s of fp16 weight
    bytes per 7-launch step), and the 512 MiB device copy (the streaming rate)."""
    dev = torch.device("cuda:0")
    import _sx8lib as L
    st = L.stream(dev)
    g = torch.Generator(device="cpu").manual_seed(99)
    W = {name: (torch.randn(N, K, generator=g) * 0.02).half().to(dev) for name, N, K in LAYER}
    out = {"gemm_f16": {}, "library": "torch.mm fp16 (hipBLASLt), fp32 accumulation, fp16 output"}
    ms = [int(v) for v in str(args.prefill_m).split(",") if v.strip()]
    for M in ms:
        xs = {K: torch.randn(M, K, generator=g).half().to(dev) for K in {K for _, _, K in LAYER}}
        per, tot_flop, tot_us = {}, 0.0, 0.0
        for name, N, K in LAYER:
            Y = torch.empty(M, N, dtype=torch.float16, device=dev)
            Wt = W[name].t()
            torch.mm(xs[K], Wt, out=Y)
            torch.cuda.synchronize()
            q = quantiles(call_series(torch, st, lambda r, X=xs[K], Wt=Wt, Y=Y: torch.mm(X, Wt, out=Y),
                                      max(200, args.iters)))
            flop = 2.0 * M * N * K
            per[name] = {"us": q["median_us"], "p10_us": q["p10_us"], "p90_us": q["p90_us"],
                         "tflops": flop / (q["median_us"] * 1e-6) / 1e12}
            tot_flop += flop
            tot_us += q["median_us"]
        tf = tot_flop / (tot_us * 1e-6) / 1e12
        out["gemm_f16"][str(M)] = {"layer_tflops": tf, "frac_of_mfma_peak": tf / MFMA_F16_PEAK_TFLOPS,
                                   "layer_us": tot_us, "per_shape": per}
        log(f"library fp16 GEMM M={M}: layer {tf:.1f} TFLOP/s ({tot_us:.1f} us); " +
            ", ".join(f"{k} {v['tflops']:.0f}" for k, v in per.items()))
    # fp16 GEMV at M = 1, cold weights: 6 copies of the layer rotated
    copies = [{name: W[name].clone() for name, _, _ in LAYER} for _ in range(6)]
    xs = {K: torch.randn(K, generator=g).half().to(dev) for K in {K for _, _, K in LAYER}}
    ys = {name: torch.empty(N, dtype=torch.float16, device=dev) for name, N, _ in LAYER}

    def step(r):
        c = copies[r % len(copies)]
        for name, N, K in LAYER:
            torch.mv(c[name], xs[K], out=ys[name])

    for r in range(len(copies)):
        step(r)
    torch.cuda.synchronize()
    q = quantiles(call_series(torch, st, step, max(200, args.iters)))
    wbytes = sum(2 * N * K for _, N, K in LAYER)
    out["gemv_f16_m1"] = {"step_us": q, "weight_bytes": wbytes, "gbs": wbytes / (q["median_us"] * 1e-6) / 1e9,
                          "launches_per_step": len(LAYER), "copies": len(copies)}
    log(f"library fp16 GEMV M=1: {q['median_us']:.1f} us per layer step, "
        f"{out['gemv_f16_m1']['gbs']:.0f} GB/s of fp16 weights")
    del copies
    out["copy_512MiB"] = bench_copy(torch, args)
    log(f"device copy 512 MiB: {out['copy_512MiB']['gbs']:.0f} GB/s")
    return out


# ------------------------------------------------------------------ decode timeline
# Per-wave timeline of the decode step's GEMV launches (bench.py --only timeline, GPU only).
#
# Builds an instrumented copy of csrc/sx8_gemv.hip into a temporary directory: wave 0 of every
# work-group of every k_gemv_panel / k_gemv_pair launch stamps the shader clock (s_memtime)
# at fixed points of the kernel and stores one record.  Then it replays decode steps of the
# 36-layer decoder through that library (HIP graph, as bench.py's e2e) and prints, per launch
# kind, the median work-group's phases in shader cycles:
#
#   pre-tab          kernel start -> activation-table loads issued
#   tab->rec         -> first record rounds issued
#   build(a)         -> table build (RMSNorm forms: up to the norm's barrier)
#   rms->build(b)    RMSNorm forms: norm barrier -> rest of the table build
#   barrier          table barrier
#   loop             the K loop
#   red-barrier      loop end -> reduction barrier passed (waiting for the slowest wave)
#   reduce+store     reduction, epilogue, stores
#
# plus the launch span (first start to last end, 100 MHz clock), the median start skew and
# the tail after the median work-group ends.  Usage: python3 bench.py --only timeline [--timeline-tokens T].
# The instrumentation is anchored on the source text; it fails loudly when the kernel code
# it expects has changed.
TL_MAX_REC = 262144

TL_HEADER = r'''
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


def _tl_record(tag):
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


def timeline_instrument(src):
    """The GEMV source with the timeline stamps inserted (asserts every anchor)."""
    def sub(old, new, count=1):
        nonlocal src
        if src.count(old) != count:
            raise SystemExit(f"timeline: anchor found {src.count(old)} times, expected {count}: {old[:70]!r}")
        src = src.replace(old, new)

    sub("namespace {\n\nstruct KbInfo", TL_HEADER + "namespace {\n\nstruct KbInfo")
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
    sub("    red[tid] = acc;\n    __syncthreads();\n    const bool wide = CT > 64;",
        "    asm volatile(\"\" :: \"v\"(acc));\n    TS(6);\n    red[tid] = acc;\n    __syncthreads();\n    TS(9);\n"
        "    const bool wide = CT > 64;")
    sub("    if (lane_ok) red[va] = acc;\n    __syncthreads();\n    const int NG = CT > 64 ? 4 : 8;",
        "    asm volatile(\"\" :: \"v\"(acc));\n    TS(6);\n    if (lane_ok) red[va] = acc;\n    __syncthreads();\n"
        "    TS(9);\n    const int NG = CT > 64 ? 4 : 8;")
    # end of k_gemv_panel (after the argmax partials) and of k_gemv_pair
    sub("                xp.amax[2 * panel + 1] = (uint32_t)idx;\n            }\n        }\n    }\n}\n",
        "                xp.amax[2 * panel + 1] = (uint32_t)idx;\n            }\n        }\n    }\n"
        + _tl_record("kX * 100 + kMode * 10 + (kOne ? 1 : 0) + (kPre ? 1000 : 0) + (kResY ? 2000 : 0)") + "}\n")
    sub("                if (slot == 0 && min(32 * kb + 32, N) <= c1) pa.zp[((int64_t)kb * 2 + 1) * 2 + cc] = 0.f;\n"
        "            }\n        }\n    }\n}\n",
        "                if (slot == 0 && min(32 * kb + 32, N) <= c1) pa.zp[((int64_t)kb * 2 + 1) * 2 + cc] = 0.f;\n"
        "            }\n        }\n    }\n" + _tl_record("9999") + "}\n")
    return src


def timeline_build(L, out_dir, source="sx8_gemv.hip", instrument=None):
    """libsx8_hip.so in out_dir with `source` replaced by its instrumented copy (the GEMV's
    timeline stamps unless `instrument` is given)."""
    instrument = instrument or timeline_instrument
    src = instrument(open(os.path.join(L.CSRC_DIR, source)).read())
    gemv = os.path.join(out_dir, source.replace(".hip", "_ts.hip"))
    open(gemv, "w").write(src)
    flags = [f for f in L.HIP_FLAGS if f != "-shared"]

    def cc(name):
        path = gemv if name == source else os.path.join(L.CSRC_DIR, name)
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


def bench_timeline(args):
    """--only timeline: per-wave phases of the decode step's GEMV launches (the comment block above)."""
    import collections
    import ctypes
    import tempfile
    import _sx8lib as L
    n_tok = args.timeline_tokens
    with tempfile.TemporaryDirectory() as d:
        lib = timeline_build(L, d)
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
        buf = np.zeros(TL_MAX_REC * 16, np.uint64)
        tick = ctypes.c_uint(0)
        assert raw.sx8x_ts_read(buf.ctypes.data, buf.nbytes, ctypes.byref(tick)) == 0
    n = min(tick.value, TL_MAX_REC)
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


# ------------------------------------------------------------------ prompt-attention timeline
# bench.py --only attn-timeline [--attn-t T]: an instrumented copy of sx8_decoder.hip (built
# into a temporary directory, anchored on the source text; it refuses to run if the kernel
# moved) in which wave 0 of every k_attn_prefill work-group stamps the shader clock
# (s_memtime).  The packed prompt attention of 32/8 heads of 128 over T rows (synthetic
# fp16 q, K, V; random o-projection basis and scales) runs a few times; per query tile the
# median work-group's phases, shader cycles:
#   issue        entry -> query, block 0 and the first ring slot requested
#   stage0       -> block 0 staged (its loads waited for)
#   bar0         -> the first barrier passed (the slowest wave's block 0)
#   step0        -> step 0's barrier (query exchange, the second slot's request, step 0)
#   steps1..     -> the last step's barrier
#   ->merge-bar  -> the merge barrier
#   merge+emit   -> the end (the sets' merge and the packed operands' stores)
ATL_HEADER = r"""
__device__ unsigned long long g_rec[65536 * 16];
__device__ unsigned int g_tick;
#define TSN() ({ __builtin_amdgcn_sched_barrier(0); unsigned long long _t = __builtin_amdgcn_s_memtime(); __builtin_amdgcn_sched_barrier(0); _t; })
extern "C" int sx8x_ts_reset() { unsigned int z = 0; return (int)hipMemcpyToSymbol(HIP_SYMBOL(g_tick), &z, 4); }
extern "C" int sx8x_ts_read(void* dst, size_t n, unsigned* tick) {
    int r = (int)hipMemcpyFromSymbol(dst, HIP_SYMBOL(g_rec), n);
    if (r) return r;
    return (int)hipMemcpyFromSymbol(tick, HIP_SYMBOL(g_tick), 4);
}
"""


def attn_timeline_instrument(src):
    """sx8_decoder.hip with k_attn_prefill's timeline stamps inserted (asserts every anchor)."""
    def sub(old, new, count=1):
        nonlocal src
        if src.count(old) != count:
            raise SystemExit(f"attn-timeline: anchor found {src.count(old)} times, expected {count}: {old[:70]!r}")
        src = src.replace(old, new)

    sub("constexpr int kApVRow = 40;", ATL_HEADER + "constexpr int kApVRow = 40;")
    sub("    __shared__ __align__(16) unsigned char lds[Lds::kBytes];\n",
        "    __shared__ __align__(16) unsigned char lds[Lds::kBytes];\n"
        "    unsigned long long t0 = TSN(), t1 = 0, t2 = 0, t3 = 0, t4 = 0, t5 = 0, t6 = 0, t7 = 0;\n")
    sub("        stage(0, k0, v0);                        // (a set past the tile's blocks: zeros, unused)\n",
        "        t6 = TSN();\n        stage(0, k0, v0);\n        t7 = TSN();\n")
    sub("            aps[min(tid, GW * NT - 1)] = spre;\n        }\n        __syncthreads();\n",
        "            aps[min(tid, GW * NT - 1)] = spre;\n        }\n        __syncthreads();\n        t1 = TSN();\n")
    sub("        __syncthreads();      // step j + 1 staged; step j's buffers free for step j + 2\n    };\n",
        "        __syncthreads();      // step j + 1 staged; step j's buffers free for step j + 2\n"
        "        { const unsigned long long tt = TSN(); if (j == 0) t2 = tt; if (j == nstep - 1) t3 = tt; }\n    };\n")
    sub("    __syncthreads();\n    if (!kPack && qi >= T) return;\n    // set t's state",
        "    __syncthreads();\n    t4 = TSN();\n    if (!kPack && qi >= T) return;\n    // set t's state")
    sub("            v[r] = acc;\n        }\n        emit(n, v);\n    }\n}\n",
        "            v[r] = acc;\n        }\n        emit(n, v);\n    }\n"
        "    t5 = TSN();\n"
        "    if (tid < 64) {\n        unsigned tk = 0;\n        if (tid == 0) tk = atomicAdd(&g_tick, 1u);\n"
        "        tk = __builtin_amdgcn_readfirstlane(tk);\n        if (tid == 0 && tk < 65536) {\n"
        "            unsigned long long* o = g_rec + (size_t)tk * 16;\n"
        "            o[0] = t0; o[1] = t1; o[2] = t2; o[3] = t3; o[4] = t4; o[5] = t5; o[6] = t6; o[7] = t7;\n"
        "            o[8] = blockIdx.x; o[9] = blockIdx.y; o[10] = nstep; o[11] = NS;\n"
        "        }\n    }\n}\n")
    return src


def bench_attn_timeline(args):
    """--only attn-timeline: per-tile phases of the packed prompt attention (the comment block above)."""
    import ctypes
    import math
    import tempfile
    import _sx8lib as L
    T = args.attn_t
    with tempfile.TemporaryDirectory() as d:
        lib = timeline_build(L, d, "sx8_decoder.hip", attn_timeline_instrument)
        print("built", lib, flush=True)
        os.environ["SX8_HIP_LIB"] = lib
        import torch
        L.lib()
        raw = ctypes.CDLL(L.lib_path())
        raw.sx8x_ts_read.argtypes = [ctypes.c_void_p, ctypes.c_size_t, ctypes.c_void_p]
        cuda = torch.device("cuda")
        st = L.stream(cuda)
        P = L.ptr
        nh, nk, hd, Lc = 32, 8, 128, max(2048, T)
        n_cb = nh * hd // 32
        g = torch.Generator(device="cpu").manual_seed(5)
        q = torch.randn(T, nh, hd, generator=g).half().to(cuda)
        kc = torch.randn(nk, Lc, hd, generator=g).half().to(cuda)
        vc = torch.randn(nk, Lc, hd, generator=g).half().to(cuda)
        bas = (torch.randn(n_cb, 2, 32, generator=g) * 0.1).to(cuda)
        sca = torch.rand(n_cb, 2, generator=g).to(cuda)
        Xp = torch.empty((T + 31) // 32 * n_cb * 1024, dtype=torch.int16, device=cuda)
        Zhl = torch.empty(T * n_cb * 4, dtype=torch.int16, device=cuda)

        def run():
            L.call("sx8_dec_attn_prefill_packed", P(q), P(kc), P(vc), T, 0, nh, nk, hd, Lc, 1.0 / math.sqrt(hd),
                   P(bas), P(sca), P(Xp), P(Zhl), st)

        for _ in range(20):
            run()
        torch.cuda.synchronize()
        names = ["issue", "stage0", "bar0", "step0", "steps1..", "->merge-bar", "merge+emit", "total"]
        rows = []
        for _ in range(3):
            run()
            run()
            torch.cuda.synchronize()
            raw.sx8x_ts_reset()
            run()
            torch.cuda.synchronize()
            buf = np.zeros(65536 * 16, dtype=np.uint64)
            tick = ctypes.c_uint()
            assert raw.sx8x_ts_read(buf.ctypes.data, buf.nbytes, ctypes.byref(tick)) == 0
            r = buf[:tick.value * 16].reshape(-1, 16).astype(np.int64)
            multi = r[:, 10] > 1
            last = np.where(multi, r[:, 3], r[:, 2])
            rows.append(np.stack([r[:, 8], r[:, 10], r[:, 6] - r[:, 0], r[:, 7] - r[:, 6], r[:, 1] - r[:, 7],
                                  r[:, 2] - r[:, 1], np.where(multi, r[:, 3] - r[:, 2], 0), r[:, 4] - last,
                                  r[:, 5] - r[:, 4], r[:, 5] - r[:, 0]], 1))
        a = np.concatenate(rows)
        print(f"T {T}: {len(a) // 3} work-groups per call, 3 calls; median work-group per query tile, wave 0, "
              f"shader cycles: " + " | ".join(names))
        for tile in sorted(set(a[:, 0].tolist())):
            sel = a[a[:, 0] == tile]
            print(f"tile {tile:3d} steps {int(sel[0, 1])}: " + " ".join(f"{np.median(sel[:, i]):7.0f}"
                                                                   for i in range(2, 10)), flush=True)


# ------------------------------------------------------------------ read ceiling
# The streaming-read rate of this GPU (bench.py --only readbw): a 4 GiB buffer read with
# 16-byte loads by 256..4096 work-groups, each streaming a contiguous slice (8 loads in
# flight per thread, one store per work-group), 10 launches per grid size.  The GEMV is a
# read stream, so this -- not the 8 TB/s vendor figure, nor the read + write device copy --
# is the practical ceiling its streaming phase is compared with.  Built with hipcc into a
# temporary directory at run time.
READBW_SRC = r'''
#include <hip/hip_runtime.h>
#include <cstdio>
__global__ __launch_bounds__(256) void rd(const uint4* __restrict__ p, size_t n16, unsigned* out) {
    const size_t per = (n16 + gridDim.x - 1) / gridDim.x;
    const size_t b = (size_t)blockIdx.x * per, e = b + per < n16 ? b + per : n16;
    unsigned acc = 0;
    for (size_t i = b + threadIdx.x; i < e; i += 256 * 8) {
        uint4 v[8];
#pragma unroll
        for (int u = 0; u < 8; ++u) { size_t k = i + 256 * u; v[u] = k < e ? p[k] : make_uint4(0, 0, 0, 0); }
#pragma unroll
        for (int u = 0; u < 8; ++u) acc ^= v[u].x ^ v[u].y ^ v[u].z ^ v[u].w;
    }
    if (acc == 0x12345678u) out[blockIdx.x] = acc;
}
int main() {
    const size_t bytes = (size_t)4 << 30;
    uint4* p; unsigned* o;
    if (hipMalloc(&p, bytes) != hipSuccess || hipMalloc(&o, 1 << 20) != hipSuccess) return 1;
    if (hipMemset(p, 1, bytes) != hipSuccess) return 1;
    hipEvent_t a, b;
    if (hipEventCreate(&a) != hipSuccess || hipEventCreate(&b) != hipSuccess) return 1;
    for (int grid : {256, 512, 1024, 2048, 4096}) {
        rd<<<grid, 256>>>(p, bytes / 16, o);
        hipEventRecord(a);
        for (int i = 0; i < 10; ++i) rd<<<grid, 256>>>(p, bytes / 16, o);
        hipEventRecord(b);
        if (hipEventSynchronize(b) != hipSuccess) return 1;
        float ms = 0.f;
        hipEventElapsedTime(&ms, a, b);
        printf("{\"grid\": %d, \"gbs\": %.1f}\n", grid, bytes * 10.0 / (ms * 1e-3) / 1e9);
    }
    return hipFree(p) != hipSuccess || hipFree(o) != hipSuccess;
}
'''


def run_probe(name, source):
    """Build a stand-alone HIP probe with hipcc into a temporary directory, run it as a child
    process (it makes its own HIP context) and return the JSON objects it printed."""
    import tempfile
    sys.path.insert(0, PKG)
    import _sx8lib as L
    with tempfile.TemporaryDirectory() as d:
        src, exe = os.path.join(d, name + ".hip"), os.path.join(d, name)
        with open(src, "w") as f:
            f.write(source)
        r = subprocess.run([L.HIPCC, "--offload-arch=gfx950", "-O3", "-Xclang", "-target-feature", "-Xclang",
                            "-packed-fp32-ops", "-o", exe, src], capture_output=True, text=True)
        if r.returncode:
            raise SystemExit(r.stderr[-2000:])
        r = subprocess.run([exe], capture_output=True, text=True, timeout=120)
        if r.returncode:
            raise SystemExit(f"{name} probe failed ({r.returncode}): {r.stderr[-500:]} {r.stdout[-500:]}")
    return [json.loads(l) for l in r.stdout.splitlines() if l.startswith("{")]


def bench_readbw():
    """--only readbw: the streaming-read ceiling (the comment block above)."""
    rows = run_probe("readbw", READBW_SRC)
    best = max(x["gbs"] for x in rows)
    return {"per_grid": rows, "best_gbs": best, "frac_of_vendor_peak": best / HBM_PEAK_GBS}


# ------------------------------------------------------------------ handoff cost
# What it costs to pass data from the work-groups of one kernel to a consumer inside the
# same launch, against a second launch (bench.py --only handoff).  A producer of 256
# work-groups (8 groups of 32) each streams 64 KB, reduces it and writes a 2 KB partial;
# the 32 partials of a group are summed (fixed order) (a) by a second, 8-work-group launch;
# (b) by the group's last work-group to arrive, the partials stored and loaded as
# agent-scope relaxed atomics, each thread's stores acknowledged before one relaxed
# agent-scope ticket per work-group (no fences); (c) as (b) with a release fence before
# the ticket and an acquire fence in the last work-group.  Nothing waits on another
# work-group (the last to arrive does the sum), so every form ends; the three outputs are
# compared.  This is the pattern a fused decoder step would need between its phases.  Form
# (b) leans on the hardware (a store acknowledged at agent scope is visible to agent-scope
# loads) rather than on the language's memory model, which asks for (c)'s fences; it is
# timed as the cheapest handoff there could be, and checked against the other two outputs.
HANDOFF_SRC = r'''
#include <hip/hip_runtime.h>
#include <cstdio>
#include <vector>
constexpr int kG = 8, kC = 32, kP = 512;
__device__ float part_sum(const float4* __restrict__ src, int wg, int t) {
    const float4* p = src + (size_t)wg * 4096;
    float a = 0.f;
#pragma unroll
    for (int i = 0; i < 16; ++i) { const float4 v = p[i * 256 + t]; a += (v.x + v.y) + (v.z + v.w); }
    return a;
}
__device__ void group_sum(const float* part, float* out, int g, int t, bool atomic_loads) {
    float s0 = 0.f, s1 = 0.f;
    for (int c = 0; c < kC; ++c) {
        const float* q = part + (size_t)(g * kC + c) * kP;
        if (atomic_loads) {
            s0 += __hip_atomic_load(q + t, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            s1 += __hip_atomic_load(q + 256 + t, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        } else {
            s0 += q[t];
            s1 += q[256 + t];
        }
    }
    out[g * kP + t] = s0;
    out[g * kP + 256 + t] = s1;
}
__global__ __launch_bounds__(256) void k_produce(const float4* src, float* part) {
    const float a = part_sum(src, blockIdx.x, threadIdx.x);
    part[(size_t)blockIdx.x * kP + threadIdx.x] = a;
    part[(size_t)blockIdx.x * kP + 256 + threadIdx.x] = 0.5f * a;
}
__global__ __launch_bounds__(256) void k_consume(const float* part, float* out) {
    group_sum(part, out, blockIdx.x, threadIdx.x, false);
}
template <bool kFence>
__global__ __launch_bounds__(256) void k_fused(const float4* src, float* part, float* out, unsigned* ticket) {
    const int wg = blockIdx.x, t = threadIdx.x, g = wg / kC;
    const float a = part_sum(src, wg, t);
    float* pp = part + (size_t)wg * kP;
    if (kFence) {
        pp[t] = a;
        pp[256 + t] = 0.5f * a;
    } else {
        __hip_atomic_store(pp + t, a, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        __hip_atomic_store(pp + 256 + t, 0.5f * a, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        __builtin_amdgcn_s_waitcnt(0);
    }
    __shared__ unsigned last;
    __syncthreads();
    if (t == 0) {
        const unsigned old = kFence
            ? __hip_atomic_fetch_add(ticket + g, 1u, __ATOMIC_RELEASE, __HIP_MEMORY_SCOPE_AGENT)
            : __hip_atomic_fetch_add(ticket + g, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        last = old == kC - 1;
    }
    __syncthreads();
    if (!last) return;
    if (kFence) __atomic_thread_fence(__ATOMIC_ACQUIRE);
    group_sum(part, out, g, t, !kFence);
    if (t == 0) ticket[g] = 0u;
}
int main() {
    const int nwg = kG * kC, kSlices = 16;
    const size_t slice = (size_t)nwg * 4096;                     // float4s per launch (16 MB)
    float4* src; float* part; float* out; unsigned* ticket;
    if (hipMalloc(&src, kSlices * slice * sizeof(float4)) != hipSuccess || hipMalloc(&part, (size_t)nwg * kP * 4) != hipSuccess ||
        hipMalloc(&out, 3 * kG * kP * 4) != hipSuccess || hipMalloc(&ticket, 64) != hipSuccess) return 1;
    std::vector<float> h(kSlices * slice * 4);
    for (size_t i = 0; i < h.size(); ++i) h[i] = (float)((i * 2654435761u) % 1000) * 1e-3f;
    if (hipMemcpy(src, h.data(), h.size() * 4, hipMemcpyHostToDevice) != hipSuccess) return 1;
    if (hipMemset(ticket, 0, 64) != hipSuccess) return 1;
    hipEvent_t e0, e1;
    if (hipEventCreate(&e0) != hipSuccess || hipEventCreate(&e1) != hipSuccess) return 1;
    auto run = [&](int form, const float4* s) {
        if (form == 0) {
            k_produce<<<nwg, 256>>>(s, part);
            k_consume<<<kG, 256>>>(part, out);
        } else if (form == 1) {
            k_fused<false><<<nwg, 256>>>(s, part, out + kG * kP, ticket);
        } else if (form == 2) {
            k_fused<true><<<nwg, 256>>>(s, part, out + 2 * kG * kP, ticket);
        } else {
            k_produce<<<nwg, 256>>>(s, part);
        }
    };
    const char* names[4] = {"two launches", "one launch, atomic data, no fences", "one launch, release/acquire fences",
                            "producer alone"};
    for (int form = 0; form < 4; ++form) {
        for (int i = 0; i < 20; ++i) run(form, src + (i % kSlices) * slice);
        if (hipDeviceSynchronize() != hipSuccess) return 1;
        const int n = 200;
        if (hipEventRecord(e0) != hipSuccess) return 1;
        for (int i = 0; i < n; ++i) run(form, src + (i % kSlices) * slice);
        if (hipEventRecord(e1) != hipSuccess || hipEventSynchronize(e1) != hipSuccess) return 1;
        float ms = 0.f;
        if (hipEventElapsedTime(&ms, e0, e1) != hipSuccess) return 1;
        run(form, src);
        if (hipDeviceSynchronize() != hipSuccess) return 1;
        printf("{\"form\": \"%s\", \"us\": %.2f}\n", names[form], ms * 1e3f / n);
    }
    std::vector<float> r(3 * kG * kP);
    if (hipMemcpy(r.data(), out, r.size() * 4, hipMemcpyDeviceToHost) != hipSuccess) return 1;
    int bad = 0;
    for (int i = 0; i < kG * kP; ++i) bad += (r[i] != r[kG * kP + i]) + (r[i] != r[2 * kG * kP + i]);
    printf("{\"mismatches\": %d}\n", bad);
    return bad != 0;
}
'''


def bench_handoff():
    """--only handoff: one launch with an in-kernel handoff against two launches (the comment
    block above)."""
    rows = run_probe("handoff", HANDOFF_SRC)
    out = {r["form"]: r["us"] for r in rows if "form" in r}
    out["mismatches"] = next(r["mismatches"] for r in rows if "mismatches" in r)
    return out

def cpu_baseline(layer, seconds):
    """The oracle's C restatement (R64 dequant to fp16 + fp32 GEMV, OpenMP) on the host,
    over as many layer shapes as fit in about `seconds`: with every host thread OpenMP
    gives it (the reported `value`), then single-threaded for about a third of that."""
    import numpy as np
    sys.path.insert(0, os.path.join(REPO, "oracle"))
    import oracle as O
    O.build()
    lib = O.lib()

    def run(budget):
        threads = int(lib.sx8o_num_threads())
        done_bytes, t_dq, t_gv, names = 0, 0.0, 0.0, []
        rng = np.random.default_rng(2)
        # cycle through the layer's shapes until about `budget` seconds of CPU work is done
        for i in range(10000):
            t = layer[i % len(layer)]
            qt, bi = t["qt"], t["bi"]
            n_blk, dmin, dmax, cfg, cof, hi, lo = O._fields(qt)
            data, sc = O._bases(bi)
            w16 = np.empty(n_blk * 32, dtype=np.uint16)
            x = rng.standard_normal(t["K"]).astype(np.float16).view(np.uint16)
            y = np.empty(t["N"], dtype=np.float32)
            t0 = time.perf_counter()
            lib.sx8o_dequant_r64(n_blk, qt["n_cb"], O._ptr(dmin), O._ptr(dmax), O._ptr(cfg),
                                 O._ptr(cof), O._ptr(hi), O._ptr(lo), O._ptr(data), O._ptr(sc), 1,
                                 O._ptr(w16), None)
            t1 = time.perf_counter()
            lib.sx8o_gemv_f32(t["N"], t["K"], qt["n_cb"] * 32, O._ptr(w16), O._ptr(x), O._ptr(y))
            t2 = time.perf_counter()
            t_dq += t1 - t0
            t_gv += t2 - t1
            done_bytes += packed_bytes(t["N"], t["K"])
            names.append(t["name"])
            if t_dq + t_gv > budget:
                break
        tot = t_dq + t_gv
        return {"value": done_bytes / tot / 1e9, "unit": "GB/s", "cores": threads, "kind": "port",
                "sample": f"R64 dequant + fp32 GEMV, {len(names)} matrices cycling through the "
                          f"layer's shapes ({done_bytes / 1e6:.1f} MB packed) "
                          f"in {tot:.1f} s (dequant {t_dq:.1f} s, GEMV {t_gv:.1f} s)"}

    multi = run(seconds)
    lib.sx8o_set_num_threads(1)
    single = run(seconds / 3)
    multi["single_thread"] = {"value": single["value"], "cores": 1, "sample": single["sample"]}
    return multi


def bench_gemm_one(torch, L, layer, args):
    """One prefill GEMM shape (--shape) at M = --m, called --iters times back to back: the
    workload of the counter passes in profiles/prefill_gemm_m2048.md."""
    dev = torch.device("cuda:0")
    t = {x["name"]: x for x in layer}[args.shape]
    M = args.m
    g = torch.Generator(device="cpu").manual_seed(12)
    X = torch.randn(M, t["K"], generator=g).half().to(dev)
    Y = torch.empty(M, t["N"], dtype=torch.float32, device=dev)
    ws, nb = L.gemm_workspace(M, (t["N"],), t["n_cb"], dev)
    st = L.stream(dev)
    fn = L.lib().sx8_gemm_prefill

    def one(r):
        if fn(L.ptr(X), M, t["K"], t["K"], L.ptr(t["hdr"]), L.ptr(t["lvl"]), args.hdr_bytes, L.ptr(t["bas"]),
              L.ptr(t["sca"]), t["N"], t["n_cb"], L.ptr(Y), L.ptr(ws), nb, st) != 0:
            raise RuntimeError(L.lib().sx8_last_error().decode())
    one(0)
    torch.cuda.synchronize()
    q = quantiles(call_series(torch, st, one, max(1, args.iters)))
    q["tflops_at_median"] = 2.0 * M * t["N"] * t["K"] / (q["median_us"] * 1e-6) / 1e12
    q["plan"] = L.gemm_plan(M, (t["N"],), t["n_cb"])
    q["mfma_instructions_per_call"] = mfma_count(M, t["N"], t["K"], q["plan"])
    return q


def mfma_count(M, N, K, plan):
    """v_mfma_f32_32x32x16_f16 instructions one sx8_gemm_prefill call issues: every work-group
    runs, for each 32 x 32 output fragment of its tile (padded rows included), two per K
    block of its range plus one PCA k-step per started group of 4 K blocks."""
    tile = plan["tile"]
    n_cb = -(-K // 32)
    NB = -(-N // 128)
    frags = (tile // 32) * 4

    def per_range(nb):
        return frags * (2 * nb + -(-nb // 4))

    def ranges(S, kbs):
        return [min(kbs, n_cb - s * kbs) for s in range(S) if s * kbs < n_cb]

    if tile != 512:
        MB = -(-M // tile)
        return MB * NB * sum(per_range(nb) for nb in ranges(plan["k_ranges"], plan["kb_per_range"]))
    T = -(-M // 512) * NB
    n_split = plan["split_tiles"]
    whole = T - n_split
    return whole * per_range(n_cb) + n_split * sum(per_range(nb) for nb in ranges(plan["k_ranges"],
                                                                                  plan["kb_per_range"]))


def prefill_roofline(pf, lib=None):
    """The roofline block of the prefill GEMM at the headline M: the layer (7 calls, each
    with its Z/pack pass and any split-K sum) and its dominant call, median durations; the
    dominant kernel's MFMA busy % and HBM bytes per launch from the counter passes when the
    source and plan are the ones measured; the same-run library fp16 GEMM (no dequant) over
    the layer at that M for comparison.  The dominant call is the one with the most flops:
    gate, up and down tie (and run within a few microseconds of each other, in either order
    from run to run), so down -- the shape of the counter passes -- is taken; the run's
    slowest call is reported beside it."""
    if not pf:
        return None
    M = pf["M"]
    fl = dict((n, N * K) for n, N, K in LAYER)
    name = max(pf["per_shape"], key=lambda n: (fl[n], n == "down_proj"))
    q = pf["per_shape"][name]
    slowest = max(pf["per_shape"].items(), key=lambda kv: kv[1]["median_us"])
    flop = 2.0 * M * dict((n, N * K) for n, N, K in LAYER)[name]
    same = name == "down_proj" and M == 2048 and q["plan"]["tile"] == 512 and os.environ.get("SX8_GEMM_W2") != "0"
    busy, busy_src = measured("prefill_mfma_busy_pct") if same else (None, "measured for down_proj at M = 2048 only")
    traffic, traffic_src = measured("prefill_traffic") if same else (None, "measured for down_proj at M = 2048 only")
    lib_tf = None
    if lib and str(M) in lib.get("gemm_f16", {}):
        lib_tf = round(lib["gemm_f16"][str(M)]["layer_tflops"], 1)
    return {
        "bound": "mfma", "unit": "TFLOP/s", "peak": MFMA_F16_PEAK_TFLOPS, "M": M,
        "layer": {"flop": pf["layer_flop"], "us": pf["layer_us"], "achieved": round(pf["tflops"], 1),
                  "frac": round(pf["tflops"] / MFMA_F16_PEAK_TFLOPS, 4)},
        "dominant": {"shape": name,
                     "kernel": ("k_gemm_w1" if os.environ.get("SX8_GEMM_W2") == "0" else "k_gemm_w2")
                     if q["plan"]["tile"] == 512 else "k_gemm",
                     "flop_per_call": flop, "us": q["median_us"], "p10_us": q["p10_us"], "p90_us": q["p90_us"],
                     "achieved": round(q["tflops"], 1), "frac": round(q["tflops"] / MFMA_F16_PEAK_TFLOPS, 4),
                     "plan": q["plan"]},
        "slowest": {"shape": slowest[0], "us": slowest[1]["median_us"]},
        "mfma_busy_pct": busy,
        "mfma_busy_source": busy_src,
        "traffic": traffic,
        "traffic_unit": "HBM bytes per launch of the dominant call's GEMM kernel (FETCH_SIZE+WRITE_SIZE, "
                        "copy-calibrated)",
        "traffic_source": traffic_src,
        "library_layer_tflops": lib_tf,
        "vs_library": round(pf["tflops"] / lib_tf, 3) if lib_tf else None,
    }


def main():
    args = parse()
    if args.gpus != 1:
        print(f"bench.py measures one GPU only (got --gpus {args.gpus}); this build has no "
              "multi-GPU path: the value is one GPU's throughput", file=sys.stderr)
        sys.exit(2)
    import torch
    import _sx8lib as L
    if not torch.cuda.is_available():
        print("no GPU visible", file=sys.stderr)
        sys.exit(1)
    if args.only == "timeline":
        bench_timeline(args)                               # loads its own instrumented build
        return
    if args.only == "attn-timeline":
        bench_attn_timeline(args)                          # loads its own instrumented build
        return
    if args.only == "readbw":
        print(json.dumps({"readbw": bench_readbw()}), flush=True)   # a child process of its own
        return
    if args.only == "handoff":
        print(json.dumps({"handoff": bench_handoff()}), flush=True)
        return
    L.lib()
    dev = torch.device("cuda:0")
    torch.cuda.set_device(dev)
    if args.only == "copy":
        log("copy", json.dumps(bench_copy(torch, args)))
        return
    t0 = time.time()
    layer = build_layer(torch, dev, args.hdr_bytes)
    log(f"setup {time.time() - t0:.1f}s")
    res = {}
    if args.only == "gemm-one":
        log("gemm-one", json.dumps(bench_gemm_one(torch, L, layer, args)))
        return
    if args.only in ("", "gemv"):
        res["gemv"] = bench_gemv(torch, L, layer, args)
        log("gemv", json.dumps(res["gemv"]))
    if args.only in ("", "prefill") and not args.no_prefill:
        res["prefill"] = bench_prefill(torch, L, layer, args)
    if args.only in ("", "container"):
        res["container"] = bench_container(torch, L, layer, args)
        log("container", json.dumps(res["container"]))
    if args.only in ("", "quantizer"):
        res["quantizer"] = bench_quantizer(torch, L, args)
        log("quantizer", json.dumps(res["quantizer"]))
    if args.only in ("", "vocab", "embed"):
        res["vocab"] = bench_vocab(torch, L, args)
        log("vocab", json.dumps(res["vocab"]))
    if args.only in ("", "e2e") and not args.no_e2e:
        res["e2e"] = bench_e2e(torch, args)
    if args.only in ("", "library") and not args.no_library:
        res["library"] = bench_library(torch, args)
    cpu = None
    if not args.no_cpu:
        cpu = cpu_baseline(layer, args.cpu_seconds)
        log("cpu", json.dumps(cpu))
    gv = res.get("gemv", {})
    line = {
        "metric": "S-X8 decode GEMV GB/s (packed weights) @M=1, Qwen3-4B-class layer sweep",
        "value": round(gv.get("value_gbs", 0.0), 1),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(gv.get("ms_per_step", 0.0), 5),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f32 accumulate over fp16 activations x S-X8 (u8) weights",
        "data": "synthetic: N(0,0.02) weights quantized to S-X8 v4.3 (1% degenerate blocks), x~N(0,1)",
        "config": {
            "workload": "decode GEMV M=1 over one Qwen3-4B-class layer (q,k,v,o,gate,up,down), "
                        f"{args.copies} distinct copies rotated (cold cache), hdr_bytes={args.hdr_bytes}",
            "shapes": {n: f"{N}x{K}" for n, N, K in LAYER},
            "step_bytes": gv.get("step_bytes"),
            "per_shape": gv.get("per_shape"),
            "frac_of_hbm_peak": round(gv.get("value_gbs", 0.0) / HBM_PEAK_GBS, 4),
        },
        "roofline": {
            "kernel": f"k_gemv_panel<{args.hdr_bytes},1,ring,TP,plain,one> (sx8_gemv)",
            "bound": "hbm",
            "achieved": round(gv.get("achieved_gbs", 0.0), 1),
            "peak": HBM_PEAK_GBS,
            "unit": "GB/s",
            "frac": round(gv.get("achieved_gbs", 0.0) / HBM_PEAK_GBS, 4),
            "read_ceiling_gbs": READ_CEILING_GBS,
            "frac_of_read_ceiling": round(gv.get("achieved_gbs", 0.0) / READ_CEILING_GBS, 4),
            "read_ceiling_source": "bench.py --only readbw (streaming 16-byte reads of 4 GiB)",
            "traffic": measured("gemv_traffic")[0] if args.hdr_bytes == 6 else None,
            "traffic_unit": "bytes per launch (HBM, rocprofv3 FETCH_SIZE+WRITE_SIZE, copy-calibrated)",
            "traffic_source": measured("gemv_traffic")[1] if args.hdr_bytes == 6 else "measured for hdr_bytes=6 only",
            "avg_launch_us": round(gv.get("avg_launch_us", 0.0), 3),
            "traced_avg_launch_us": measured("gemv_traced_launch_us")[0] if args.hdr_bytes == 6 else None,
            "traced_avg_launch_source": measured("gemv_traced_launch_us")[1],
            "avg_launch_source": "timed region / launches (two HIP events on the launch stream, "
                                 "nothing between the launches); traced_avg_launch_us is the rocprofv3 "
                                 "kernel-trace mean of the same launches (profiles/gemv_decode_layer.md)",
            "bytes_per_launch": gv.get("bytes_per_launch"),
            "step_us": gv.get("step_us"),
        },
        "prefill_roofline": prefill_roofline(res.get("prefill"), res.get("library")),
        "cpu_baseline": cpu,
        "gemv_grouped": gv.get("grouped"),
        "gemv_graph": gv.get("graph"),
        "prefill": res.get("prefill"),
        "vocab": res.get("vocab"),
        "container": res.get("container"),
        "quantizer": res.get("quantizer"),
        "e2e": res.get("e2e"),
        "library_baseline": res.get("library"),
    }
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
