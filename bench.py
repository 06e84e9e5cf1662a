#!/usr/bin/env python3
"""Benchmark of libbwpp_hip on one MI355X.

Headline workload ("C2"): the fp32 bandwidth-bound
row operators on X[8192 x 4096] ~ N(0,1) -- row softmax, LayerNorm
(eps 1e-5, gamma ~ U[0.5,1.5], beta ~ N(0,0.1)), RMSNorm (eps 1e-6, same
gamma), reduce_max forward (max + int32 argmax) and reduce_max grad
(X, dy -> dX one-hot).  One step = one launch of each of the five over one
batch.  Inputs are generated on the host from --seed, copied to HBM before
timing, and rotated over several buffer sets whose total (>= 768 MB) exceeds
the 256 MB Infinity Cache, so every launch streams from HBM.

`value` = algorithmic bytes of one step / wall-clock time per step (GB/s).
`roofline` = the kernel with the largest share of step time: its algorithmic
bytes per launch / its average launch time, measured with HIP events on the
stream the kernels run on.  `cpu_baseline` = the oracle (this repo's C
restatement of runtime/cpu/bwpp_cpu_ref.c) timed for the same five operators
on one host core, at full size.

The contraction configs run in the same invocation and are reported under
"extras" (not part of `value`): C3 bf16 SiLU(X W + b) 4096 x 4096 x 11008
and its fp32 2048^3 variant (TFLOP/s vs dense MFMA peak), C4 attention
B8 H32 S2048 d128 bf16 unmasked and causal (causal FLOPs counted as half),
the bf16 attention backward at that shape, C1's 256^3 fp32 GEMM latency
and the C5 fp32 transformer-block training step.  C3 and C4 carry a CPU
oracle timing on a bounded slice (rows or heads are independent, so the
rate extrapolates).
"""
from __future__ import annotations

import argparse
import json
import os
import platform
import sys
import time

import numpy as np

ROOT = os.path.dirname(os.path.abspath(__file__))
PKG = os.path.join(ROOT, "bluewolf-plus-plus_amd")
sys.path.insert(0, PKG)

METRIC = "fused matmul & attention TFLOP/s, norm/softmax GB/s on 1 MI355X; % of roofline"
HBM_PEAK_GBS = 8000.0
BF16_PEAK_TFLOPS = 2516.6
F32_PEAK_TFLOPS = 157.3
ROWS, COLS = 8192, 4096
F = 4  # bytes per fp32

# Algorithmic bytes per launch (read inputs once, write outputs once).
C2_BYTES = {
    "softmax": 2 * ROWS * COLS * F,
    "layernorm": 2 * ROWS * COLS * F + 2 * COLS * F,
    "rmsnorm": 2 * ROWS * COLS * F + COLS * F,
    "reduce_max": ROWS * COLS * F + ROWS * F + ROWS * 4,
    "reduce_max_grad": ROWS * COLS * F + ROWS * F + ROWS * COLS * F,
}
C2_KERNEL = {}  # kernel symbol each op launched (filled by time_c2_ops from the library)


def host_info():
    model = platform.processor() or "unknown"
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    model = line.split(":", 1)[1].strip()
                    break
    except OSError:
        pass
    return {"cpu_model": model, "nproc": os.cpu_count()}


def load_traffic():
    """HBM bytes per launch measured by rocprofv3 --pmc (FETCH_SIZE +
    WRITE_SIZE, copy-kernel calibrated), committed under profiles/."""
    path = os.path.join(ROOT, "profiles", "traffic.json")
    try:
        with open(path) as f:
            return json.load(f)
    except (OSError, ValueError):
        return {}


class C2Bench:
    def __init__(self, be, torch, seed, nbuf):
        from bwpp import synth
        self.be = be
        self.torch = torch
        self.nbuf = nbuf
        g = synth.uniform((COLS,), seed, 1, 0.5, 1.5)
        b = synth.normal((COLS,), seed, 2, 0.0, 0.1)
        self.gamma = torch.from_numpy(g).cuda()
        self.beta = torch.from_numpy(b).cuda()
        self.x, self.y, self.dy = [], [], []
        for i in range(nbuf):
            x = synth.normal((ROWS, COLS), seed + i, 0)
            self.x.append(torch.from_numpy(x).cuda())
            self.y.append(torch.empty((ROWS, COLS), dtype=torch.float32, device="cuda"))
            self.dy.append(torch.from_numpy(synth.normal((ROWS,), seed + i, 3)).cuda())
        self.maxv = torch.empty(ROWS, dtype=torch.float32, device="cuda")
        self.argmax = torch.empty(ROWS, dtype=torch.int32, device="cuda")
        import bwpp
        self.sp = bwpp.SoftmaxParams(ROWS, COLS, COLS)
        self.lp = bwpp.RmsnormParams(ROWS, COLS, COLS, 1e-5)
        self.rp = bwpp.RmsnormParams(ROWS, COLS, COLS, 1e-6)
        self.mp = bwpp.ReduceParams(ROWS, COLS, COLS, 1)
        self.host_x0 = None

    def launch(self, op, i):
        be, x, y = self.be, self.x[i], self.y[i]
        if op == "softmax":
            be.dispatch_softmax(x, y, self.sp)
        elif op == "layernorm":
            be.dispatch_layernorm(x, self.gamma, self.beta, y, self.lp)
        elif op == "rmsnorm":
            be.dispatch_rmsnorm(x, self.gamma, None, y, self.rp)
        elif op == "reduce_max":
            be.dispatch_reduce_max(x, self.maxv, self.argmax, self.mp)
        elif op == "reduce_max_grad":
            be.dispatch_reduce_max_grad_argmax(x, None, self.dy[i], y, self.mp)
        else:
            raise KeyError(op)


def time_c2(bench, steps, warmup):
    """The timed region: `steps` passes of the five operators, back to back
    on one stream, bracketed by synchronizations and HIP events."""
    torch = bench.torch
    ops = list(C2_BYTES)
    stream = torch.cuda.current_stream()
    k = 0
    for _ in range(warmup):
        for op in ops:
            bench.launch(op, k % bench.nbuf)
            k += 1
    s = torch.cuda.Event(enable_timing=True)
    e = torch.cuda.Event(enable_timing=True)
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    s.record(stream)
    for _ in range(steps):
        for op in ops:
            bench.launch(op, k % bench.nbuf)
            k += 1
    e.record(stream)
    torch.cuda.synchronize()
    wall = time.perf_counter() - t0
    return wall, s.elapsed_time(e) * 1e-3


WARM_MS = 40.0  # sustained work before any extras timing starts


def _launch_times_ms(torch, fn, iters, group=5):
    """Per-launch durations (ms) of `iters` back-to-back launches of fn, as
    the mean over consecutive groups of `group` launches: an event on the
    launch stream before the first launch and after every group, so the
    stream is never drained and the events add no gap inside a group (an
    event between every two launches adds ~2 us to a 45 us kernel)."""
    stream = torch.cuda.current_stream()
    ng = max(1, iters // group)
    ev = [torch.cuda.Event(enable_timing=True) for _ in range(ng + 1)]
    ev[0].record(stream)
    i = 0
    for g in range(ng):
        for _ in range(group):
            fn(i)
            i += 1
        ev[g + 1].record(stream)
    torch.cuda.synchronize()
    return [ev[g].elapsed_time(ev[g + 1]) / group for g in range(ng)]


def time_c2_ops(bench, reps):
    """Median (over groups of 10 back-to-back launches) and mean launch
    duration per operator (ms), over `reps` launches on the rotating
    buffer sets."""
    torch = bench.torch
    out = {}
    for op in C2_BYTES:
        for i in range(bench.nbuf):
            bench.launch(op, i)
        C2_KERNEL[op] = bench.be.last_kernel
        t = _launch_times_ms(torch, lambda i: bench.launch(op, i % bench.nbuf), reps, group=10)
        out[op] = (float(np.median(t)), float(np.mean(t)))
    return out


def copy_calibration(bench, launches):
    """A plain copy of known size (X -> Y, 128 MiB each way) through the
    elementwise kernel, for scaling the FETCH_SIZE / WRITE_SIZE counters."""
    import bwpp
    p = bwpp.ElementwiseParams(ROWS, COLS, COLS, 4, 0)
    for i in range(launches):
        j = i % bench.nbuf
        bench.be.dispatch_elementwise(None, bench.x[j], bench.y[j], p)
    bench.torch.cuda.synchronize()


def traffic_from_pmc(fetch_dir, write_dir):
    """HBM bytes per launch from two rocprofv3 --pmc runs (FETCH_SIZE, then
    WRITE_SIZE, in KiB per dispatch).  Each counter is scaled by what it
    reads for the copy calibration (bwpp_elementwise moving a known
    134,217,728 bytes each way).  Returns {kernel: record}."""
    import csv
    import glob

    def per_kernel(d, counter):
        vals = {}
        for f in glob.glob(os.path.join(d, "**", "*counter_collection.csv"), recursive=True):
            with open(f, newline="") as fh:
                for row in csv.DictReader(fh):
                    if row["Counter_Name"] != counter:
                        continue
                    name = row["Kernel_Name"]
                    if name.startswith("bwpp_"):
                        vals.setdefault(name, []).append(float(row["Counter_Value"]))
        return {k: float(np.median(v)) for k, v in vals.items()}

    fetch = per_kernel(fetch_dir, "FETCH_SIZE")
    write = per_kernel(write_dir, "WRITE_SIZE")
    known = ROWS * COLS * 4
    f_scale = known / (fetch["bwpp_elementwise"] * 1024.0)
    w_scale = known / (write["bwpp_elementwise"] * 1024.0)
    out = {"_calibration": {"kernel": "bwpp_elementwise (copy)", "bytes_each_way": known,
                            "fetch_kib": fetch["bwpp_elementwise"], "write_kib": write["bwpp_elementwise"],
                            "fetch_scale": round(f_scale, 4), "write_scale": round(w_scale, 4)}}
    for k in sorted(set(fetch) & set(write)):
        if k == "bwpp_elementwise":
            continue
        fb = fetch[k] * 1024.0 * f_scale
        wb = write[k] * 1024.0 * w_scale
        out[k] = {"fetch_bytes": int(fb), "write_bytes": int(wb), "traffic": int(fb + wb)}
    return out


def pmc_summary(dirs):
    """Per-kernel counter table (markdown) from rocprofv3 output dirs: every
    *counter_collection.csv (--pmc runs) and *kernel_stats.csv (--stats
    runs) found under them.  Counters are summed over a dispatch's rows and
    then averaged over the kernel's dispatches.  Derived columns, with
    XCDS = 8, SIMDS = 4 per CU and CUS from the agent info:
      clock GHz   = GRBM_GUI_ACTIVE / XCDS / duration of the same dispatch
                    in the counter run (its Start/End timestamps)
      MFMA busy   = SQ_VALU_MFMA_BUSY_CYCLES / (CUS * SIMDS * GRBM_GUI_ACTIVE / XCDS)
      VALU / MFMA = SQ_INSTS_VALU / SQ_INSTS_MFMA
    (SQ_VALU_MFMA_BUSY_CYCLES counts SIMD cycles with the matrix pipe busy,
    summed over SIMDs; GRBM_GUI_ACTIVE counts GPU-busy cycles, summed over
    the XCDs.)"""
    import csv
    import glob
    counters, dur, cus, pmc_ns = {}, {}, 256, {}
    for d in dirs:
        for f in glob.glob(os.path.join(d, "**", "*agent_info.csv"), recursive=True):
            with open(f, newline="") as fh:
                for row in csv.DictReader(fh):
                    n = int(row.get("Cu_Count", 0) or 0)
                    if n > 0:
                        cus = n
        for f in glob.glob(os.path.join(d, "**", "*counter_collection.csv"), recursive=True):
            per = {}
            with open(f, newline="") as fh:
                for row in csv.DictReader(fh):
                    k = row["Kernel_Name"]
                    if not k.startswith("bwpp_"):
                        continue
                    key = (k, row["Dispatch_Id"])
                    per.setdefault(key, {}).setdefault(row["Counter_Name"], 0.0)
                    per[key][row["Counter_Name"]] += float(row["Counter_Value"])
            for (k, _), cv in per.items():
                for c, v in cv.items():
                    counters.setdefault(k, {}).setdefault(c, []).append(v)
            with open(f, newline="") as fh:
                seen = set()
                for row in csv.DictReader(fh):
                    key = (row["Kernel_Name"], row["Dispatch_Id"])
                    if key[0].startswith("bwpp_") and key not in seen:
                        seen.add(key)
                        pmc_ns.setdefault(key[0], []).append(
                            float(row["End_Timestamp"]) - float(row["Start_Timestamp"]))
        for f in glob.glob(os.path.join(d, "**", "*kernel_stats.csv"), recursive=True):
            with open(f, newline="") as fh:
                for row in csv.DictReader(fh):
                    if row["Name"].startswith("bwpp_"):
                        dur[row["Name"]] = float(row["AverageNs"])
    cols = ["GRBM_GUI_ACTIVE", "SQ_BUSY_CYCLES", "SQ_VALU_MFMA_BUSY_CYCLES", "SQ_INSTS_MFMA", "SQ_INSTS_VALU",
            "SQ_INSTS_LDS", "SQ_LDS_BANK_CONFLICT", "SQ_WAVES"]
    lines = ["| kernel | trace avg ns | pmc-run ns | clock GHz | MFMA busy | VALU/MFMA | " + " | ".join(cols) + " |",
             "|---" * (len(cols) + 6) + "|"]
    for k in sorted(set(counters) | set(dur)):
        c = {n: float(np.mean(v)) for n, v in counters.get(k, {}).items()}
        ns = dur.get(k)
        pns = float(np.mean(pmc_ns[k])) if k in pmc_ns else None
        g = c.get("GRBM_GUI_ACTIVE")
        clock = f"{g / 8 / pns:.2f}" if g and pns else ""
        busy = f"{c['SQ_VALU_MFMA_BUSY_CYCLES'] / (cus * 4 * g / 8):.3f}" if g and "SQ_VALU_MFMA_BUSY_CYCLES" in c else ""
        ratio = (f"{c['SQ_INSTS_VALU'] / c['SQ_INSTS_MFMA']:.2f}"
                 if c.get("SQ_INSTS_MFMA") and "SQ_INSTS_VALU" in c else "")
        vals = [f"{c[n]:.4g}" if n in c else "" for n in cols]
        lines.append((f"| {k} | {ns:.0f} | " if ns else f"| {k} | | ") + (f"{pns:.0f} | " if pns else " | "))
        lines[-1] += f"{clock} | {busy} | {ratio} | " + " | ".join(vals) + " |"
    return "\n".join(lines)


def stream_ceiling(torch, nbuf=3, reps=20, kind="copy", final_reps=70):
    """The box's HBM ceiling for the C2 byte pattern: plain non-temporal
    128-bit copies of X[8192 x 4096] fp32 (the bytes one read+write row
    operator moves; kind "read": the same loads without stores,
    reduce_max's pattern) from tests/hip/stream.hip, loaded through HIP's
    module API.  A sweep over float4-per-thread x block x grid (each shape
    the median of `reps` launches in groups of 10 over `nbuf` rotating
    buffer pairs) picks the fastest shape; that shape is then timed again
    over `final_reps` launches, the same count and statistic as each C2
    operator, and that median is the ceiling (the sweep's best, a maximum
    over ~50 noisy medians, is reported beside it as sweep_best_GB_s)."""
    import ctypes
    path = os.path.join(ROOT, "tests", "hip", "bwpp_stream.hsaco")
    if not os.path.exists(path):
        return None
    hip = ctypes.CDLL("libamdhip64.so.7")
    mod = ctypes.c_void_p()
    if hip.hipModuleLoad(ctypes.byref(mod), path.encode()) != 0:
        return None

    class Args(ctypes.Structure):
        _fields_ = [("x", ctypes.c_void_p), ("y", ctypes.c_void_p), ("n", ctypes.c_uint64)]

    n16 = ROWS * COLS // 4
    xs = [torch.empty(ROWS * COLS, dtype=torch.float32, device="cuda").normal_() for _ in range(nbuf)]
    ys = [torch.empty_like(x) for x in xs]
    hip.hipModuleLaunchKernel.argtypes = [ctypes.c_void_p] + [ctypes.c_uint] * 7 + [ctypes.c_void_p] * 3
    stream = torch.cuda.current_stream().cuda_stream
    cus = torch.cuda.get_device_properties(0).multi_processor_count
    best = None
    for v in (1, 2, 4, 8):
        fn = ctypes.c_void_p()
        if hip.hipModuleGetFunction(ctypes.byref(fn), mod, f"bwpp_stream_{kind}_v{v}".encode()) != 0:
            continue
        for block in (256, 512, 1024):
            full = (n16 + block * v - 1) // (block * v)
            for grid in sorted({cus, 2 * cus, 4 * cus, 8 * cus, full}):
                if grid > full:
                    continue
                args = [Args(xs[i].data_ptr(), ys[i].data_ptr(), n16) for i in range(nbuf)]
                params = [(ctypes.c_void_p * 1)(ctypes.addressof(a)) for a in args]

                def launch(i):
                    rc = hip.hipModuleLaunchKernel(fn, grid, 1, 1, block, 1, 1, 0, ctypes.c_void_p(stream),
                                                   params[i % nbuf], None)
                    if rc != 0:
                        raise RuntimeError(f"stream launch failed ({rc})")

                for i in range(nbuf * 2):
                    launch(i)
                t = _launch_times_ms(torch, launch, reps, group=10)
                us = float(np.median(t)) * 1e3
                gbs = (2 if kind == "copy" else 1) * ROWS * COLS * F / us / 1e3
                if best is None or gbs > best["GB_s"]:
                    best = {"GB_s": round(gbs, 1), "us_per_launch": round(us, 2), "frac_hbm_peak": round(gbs / HBM_PEAK_GBS, 4),
                            "config": {"float4_per_thread": v, "block": block, "grid": grid},
                            "_fn": fn, "_params": params, "_args": args}  # args: the structs params point at
    if best is None:
        return None
    fn, params, keep, cfg = best.pop("_fn"), best.pop("_params"), best.pop("_args"), best["config"]

    def launch_best(i):
        rc = hip.hipModuleLaunchKernel(fn, cfg["grid"], 1, 1, cfg["block"], 1, 1, 0, ctypes.c_void_p(stream),
                                       params[i % nbuf], None)
        if rc != 0:
            raise RuntimeError(f"stream launch failed ({rc})")

    t = _launch_times_ms(torch, launch_best, final_reps, group=10)
    del keep
    us = float(np.median(t)) * 1e3
    gbs = (2 if kind == "copy" else 1) * ROWS * COLS * F / us / 1e3
    best["sweep_best_GB_s"] = best["GB_s"]
    best.update({"GB_s": round(gbs, 1), "us_per_launch": round(us, 2), "frac_hbm_peak": round(gbs / HBM_PEAK_GBS, 4)})
    torch.cuda.synchronize()
    hip.hipModuleUnload(mod)
    best["kernel"] = f"tests/hip/stream.hip bwpp_stream_{kind}_v*"
    return best


def cpu_baseline_c2(seed, reps):
    """The oracle on one host core over the five C2 operators at full size."""
    sys.path.insert(0, ROOT)
    from bwpp import synth
    from oracle.oracle import Oracle
    orc = Oracle()
    x = synth.normal((ROWS, COLS), seed, 0)
    g = synth.uniform((COLS,), seed, 1, 0.5, 1.5)
    b = synth.normal((COLS,), seed, 2, 0.0, 0.1)
    dy = synth.normal((ROWS,), seed, 3)
    t = 0.0
    for _ in range(reps):
        t0 = time.perf_counter()
        orc.softmax(x)
        orc.layernorm(x, g, b, 1e-5)
        orc.rmsnorm(x, g, None, 1e-6)
        orc.reduce_max(x, 1)
        orc.reduce_max_grad(dy, x.shape, x=x, axis=1)
        t += time.perf_counter() - t0
    step_s = t / reps
    return {
        "value": round(sum(C2_BYTES.values()) / step_s / 1e9, 3),
        "unit": "GB/s",
        "cores": 1,
        "kind": "port",
        "sample": f"full C2 step (5 ops on X[{ROWS}x{COLS}]) x {reps}, oracle/bwpp_oracle.c, "
                  f"1 thread; {step_s * 1e3:.1f} ms/step",
    }


def regress_json(args):
    """The reference's CPU bench workload (bench/bench_cpu.c: ramp inputs
    x[i][j] = (i*cols + j + 1) * scale, fp32 matmul without epilogue,
    softmax, RMSNorm with gamma = 1 and eps 1e-5, `iters` back-to-back calls)
    run through libbwpp_hip, written in the reference's JSON layout
    (bench_cpu.c:142-157, read by bench/bench_regress.py:93-111): time_s is
    the wall time of all iterations.  Each group also carries the GPU rate,
    its roofline fraction and the oracle's time on one core (cpu_time_s)."""
    import torch
    import bwpp
    from bwpp import synth
    be = bwpp.HipBackend(0)
    be.set_stream(torch.cuda.current_stream())
    M, N, K, rows, cols, iters = args.m, args.n, args.k, args.rows, args.cols, args.iters
    a = torch.from_numpy(synth.ramp(M, K, 0.01)).cuda()
    b = torch.from_numpy(synth.ramp(K, N, 0.02)).cuda()
    c = torch.empty((M, N), device="cuda")
    x = torch.from_numpy(synth.ramp(rows, cols, 0.01)).cuda()
    y = torch.empty_like(x)
    z = torch.empty_like(x)
    gamma = torch.ones(cols, device="cuda")

    def timed(fn):
        fn()
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        for _ in range(iters):
            fn()
        torch.cuda.synchronize()
        return time.perf_counter() - t0

    mp = bwpp.MatmulParams(M, N, K, K, N, N)
    sp = bwpp.SoftmaxParams(rows, cols, cols)
    rp = bwpp.RmsnormParams(rows, cols, cols, 1e-5)
    t_mm = timed(lambda: be.dispatch_matmul(a, b, c, None, mp))
    t_sm = timed(lambda: be.dispatch_softmax(x, y, sp))
    t_rn = timed(lambda: be.dispatch_rmsnorm(x, gamma, None, z, rp))
    be.close()
    flops = 2.0 * M * N * K * iters
    nb = 2.0 * rows * cols * 4 * iters
    out = {
        "matmul": {"M": M, "N": N, "K": K, "iters": iters, "time_s": round(t_mm, 9),
                   "gflops": round(flops / t_mm / 1e9, 3),
                   "gpu_frac_f32_peak": round(flops / t_mm / 1e12 / F32_PEAK_TFLOPS, 5)},
        "softmax": {"rows": rows, "cols": cols, "iters": iters, "time_s": round(t_sm, 9),
                    "gpu_GB_s": round(nb / t_sm / 1e9, 2), "gpu_frac_hbm_peak": round(nb / t_sm / 1e9 / HBM_PEAK_GBS, 5)},
        "rmsnorm": {"rows": rows, "cols": cols, "iters": iters, "time_s": round(t_rn, 9),
                    "gpu_GB_s": round(nb / t_rn / 1e9, 2), "gpu_frac_hbm_peak": round(nb / t_rn / 1e9 / HBM_PEAK_GBS, 5)},
        "device": "MI355X (libbwpp_hip)",
    }
    if not args.no_cpu:
        # CPU baseline: the oracle (bit-identical to the reference's C) on one core.
        sys.path.insert(0, ROOT)
        from oracle.oracle import Oracle
        orc = Oracle()
        ah, bh, xh = a.cpu().numpy(), b.cpu().numpy(), x.cpu().numpy()
        gh = np.ones(cols, np.float32)
        for key, fn in (("matmul", lambda: orc.matmul(ah, bh)), ("softmax", lambda: orc.softmax(xh)),
                        ("rmsnorm", lambda: orc.rmsnorm(xh, gh, None, 1e-5))):
            t0 = time.perf_counter()
            for _ in range(iters):
                fn()
            out[key]["cpu_time_s"] = round(time.perf_counter() - t0, 9)
    return out


_WARM_MS = WARM_MS  # set by extras() from --warm-ms


def _events_us(torch, fn, iters, warm_ms=None, stats=None):
    """Median launch time (us) of fn over `iters` back-to-back launches,
    after at least warm_ms of the same work: the MI355X clock ramps up over
    the first ~35 ms of sustained matrix work (a C3 GEMM goes from ~1035 to
    ~1180 TFLOP/s), and the figure wanted is the steady state.  `stats`, if
    given, also receives the mean."""
    warm_ms = _WARM_MS if warm_ms is None else warm_ms
    t = _launch_times_ms(torch, lambda i: fn(), 3, group=3)
    est_us = max(float(np.mean(t)) * 1e3, 1.0)
    for _ in range(min(4000, int(warm_ms * 1e3 / est_us) + 1) if warm_ms > 0 else 0):
        fn()
    t = _launch_times_ms(torch, lambda i: fn(), iters, group=max(1, min(5, iters // 3)))
    if stats is not None:
        stats["us_mean"] = round(float(np.mean(t)) * 1e3, 2)
    return float(np.median(t)) * 1e3


def _bf16(torch, x):
    from bwpp import synth
    return torch.from_numpy(synth.to_bf16_bits(x).view(np.int16)).cuda().view(torch.bfloat16)


EXTRA_GROUPS = ("c3", "c3f32", "c4", "c5")


def library_baseline(be, torch, seed, iters):
    """The same contractions through the vendor libraries torch uses on
    ROCm, timed the same way (steady state, median of grouped launches):
    C3 as hipBLASLt GEMM alone and GEMM + bias + SiLU (torch.addmm, silu),
    C3-fp32 as torch.mm, C4 forward and backward through
    scaled_dot_product_attention restricted to its flash backend (no
    fallback to the math path).  Next to each, this library's time."""
    import bwpp
    from bwpp import synth
    out = {}
    M, K, N = 4096, 4096, 11008
    x = _bf16(torch, synth.normal((M, K), seed, 0, 0.0, 0.02))
    w = _bf16(torch, synth.normal((K, N), seed, 1, 0.0, 0.02))
    b = _bf16(torch, synth.normal((N,), seed, 2, 0.0, 0.02))
    y = torch.empty((M, N), dtype=torch.bfloat16, device="cuda")
    fl = 2.0 * M * N * K
    t_lib = _events_us(torch, lambda: torch.matmul(x, w, out=y), iters)
    t_fused = _events_us(torch, lambda: torch.nn.functional.silu(torch.addmm(b, x, w)), iters)
    p = bwpp.MatmulParams(M, N, K, K, N, N, int(bwpp.DType.BF16), 3, 0, 0)
    t_ours = _events_us(torch, lambda: be.dispatch_matmul(x, w, y, b, p), iters)
    out["c3_gemm_bf16"] = {"torch_matmul_us": round(t_lib, 1), "torch_matmul_TFLOP_s": round(fl / t_lib / 1e6, 1),
                           "torch_addmm_silu_us": round(t_fused, 1),
                           "bwpp_gemm_bias_silu_us": round(t_ours, 1),
                           "bwpp_TFLOP_s": round(fl / t_ours / 1e6, 1)}
    del x, w, y
    n = 2048
    xf = torch.from_numpy(synth.uniform((n, n), seed, 0, -1, 1)).cuda()
    wf = torch.from_numpy(synth.uniform((n, n), seed, 1, -1, 1)).cuda()
    yf = torch.empty((n, n), device="cuda")
    fl = 2.0 * n ** 3
    t_lib = _events_us(torch, lambda: torch.mm(xf, wf, out=yf), iters)
    p = bwpp.MatmulParams(n, n, n, n, n, n, int(bwpp.DType.F32), 0, 0, 0)
    t_ours = _events_us(torch, lambda: be.dispatch_matmul(xf, wf, yf, None, p), iters)
    out["c3_gemm_f32_2048"] = {"torch_mm_us": round(t_lib, 1), "torch_TFLOP_s": round(fl / t_lib / 1e6, 1),
                               "bwpp_us": round(t_ours, 1), "bwpp_TFLOP_s": round(fl / t_ours / 1e6, 1)}
    del xf, wf, yf
    B, H, S, d = 8, 32, 2048, 128
    q, k, v = (_bf16(torch, synth.normal((B, H, S, d), seed, i)) for i in range(3))
    o = torch.empty_like(q)
    full = 4.0 * B * H * S * S * d
    try:
        from torch.nn.attention import SDPBackend, sdpa_kernel
        for causal in (0, 1):
            p = bwpp.AttentionParams(M=S, N=S, K=d, D=d, ldq=d, ldk=d, ldv=d, ldo=d, batch=B, heads=H,
                                     scale=d ** -0.5, causal=causal, dtype=int(bwpp.DType.BF16))
            fl = full / 2 if causal else full
            with sdpa_kernel([SDPBackend.FLASH_ATTENTION]):
                f = lambda: torch.nn.functional.scaled_dot_product_attention(q, k, v, is_causal=bool(causal))
                t_lib = _events_us(torch, f, iters)
                qg, kg, vg = (t.detach().clone().requires_grad_(True) for t in (q, k, v))
                og = torch.nn.functional.scaled_dot_product_attention(qg, kg, vg, is_causal=bool(causal))
                go = torch.ones_like(og)
                t_lib_bwd = _events_us(torch, lambda: torch.autograd.grad(og, (qg, kg, vg), go, retain_graph=True),
                                       max(3, iters // 3))
            t_ours = _events_us(torch, lambda: be.dispatch_attention(q, k, v, o, p), iters)
            lse = torch.empty((B, H, S), device="cuda")
            be.dispatch_attention_lse(q, k, v, o, lse, p)
            dq, dk, dv = torch.empty_like(q), torch.empty_like(k), torch.empty_like(v)
            t_ours_bwd = _events_us(torch, lambda: be.dispatch_attention_grad(q, k, v, o, go, lse, dq, dk, dv, p),
                                    max(3, iters // 3))
            out["c4_attention" + ("_causal" if causal else "")] = {
                "torch_sdpa_flash_fwd_us": round(t_lib, 1), "torch_sdpa_flash_bwd_us": round(t_lib_bwd, 1),
                "bwpp_fwd_us": round(t_ours, 1), "bwpp_bwd_us": round(t_ours_bwd, 1),
                "torch_fwd_TFLOP_s": round(fl / t_lib / 1e6, 1), "bwpp_fwd_TFLOP_s": round(fl / t_ours / 1e6, 1)}
    except Exception as e:  # no flash backend: report, do not fall back to the math path
        out["c4_attention"] = {"error": f"{type(e).__name__}: {e}"}
    return out


def extras(be, torch, seed, iters, with_cpu, warm_ms=WARM_MS, only=EXTRA_GROUPS):
    """Contraction configs C3, C3-fp32 (with C1), C4 (both masks, and the
    C4-shape attention backward) and C5; `only` selects groups."""
    import bwpp
    from bwpp import synth
    global _WARM_MS
    _WARM_MS = warm_ms
    out = {}
    orc = None
    if with_cpu:
        sys.path.insert(0, ROOT)
        from oracle.oracle import Oracle
        orc = Oracle()
    if "c3" in only:
        _extras_c3(be, torch, seed, iters, orc, out)
    if "c3f32" in only:
        _extras_c3f32(be, torch, seed, iters, orc, out)
    if "c4" in only:
        _extras_c4(be, torch, seed, iters, orc, out)
    if "c5" in only:
        out["c5_block_train_f32"] = block_train(be, torch, seed, max(3, iters // 4), with_cpu=orc is not None)
    return out


def _extras_c3(be, torch, seed, iters, orc, out):
    import bwpp
    from bwpp import synth
    # C3: Y = SiLU(X W + b), bf16 ~ N(0, 0.02), fp32 accumulation
    M, K, N = 4096, 4096, 11008
    xh = synth.normal((M, K), seed, 0, 0.0, 0.02)
    wh = synth.normal((K, N), seed, 1, 0.0, 0.02)
    bh = synth.normal((N,), seed, 2, 0.0, 0.02)
    x, w, b = _bf16(torch, xh), _bf16(torch, wh), _bf16(torch, bh)
    y = torch.empty((M, N), dtype=torch.bfloat16, device="cuda")
    p = bwpp.MatmulParams(M, N, K, K, N, N, int(bwpp.DType.BF16), 3, 0, 0)
    st = {}
    us = _events_us(torch, lambda: be.dispatch_matmul(x, w, y, b, p), iters, stats=st)
    fl = 2.0 * M * N * K
    c3 = {"kernel": be.last_kernel, "us_per_launch": round(us, 1), **st,
          "TFLOP_s": round(fl / us / 1e6, 1), "frac_bf16_peak": round(fl / us / 1e6 / BF16_PEAK_TFLOPS, 4)}
    if orc is not None:
        rows = 32
        xr = synth.bf16_bits_to_f32(synth.to_bf16_bits(xh[:rows]))
        wr = synth.bf16_bits_to_f32(synth.to_bf16_bits(wh))
        br = synth.bf16_bits_to_f32(synth.to_bf16_bits(bh))
        t0 = time.perf_counter()
        orc.matmul(xr, wr, br, apply_silu=True, apply_bias=True)
        dt = time.perf_counter() - t0
        c3["cpu"] = {"GFLOP_s": round(2.0 * rows * N * K / dt / 1e9, 3), "cores": 1, "kind": "port",
                     "sample": f"first {rows} rows (exact rows; extrapolated rate)"}
    out["c3_gemm_bf16_bias_silu"] = c3


def _extras_c3f32(be, torch, seed, iters, orc, out):
    import bwpp
    from bwpp import synth
    # C3 fp32 variant: 2048^3, U[-1, 1]
    n = 2048
    xf = torch.from_numpy(synth.uniform((n, n), seed, 0, -1, 1)).cuda()
    wf = torch.from_numpy(synth.uniform((n, n), seed, 1, -1, 1)).cuda()
    bf = torch.from_numpy(synth.uniform((n,), seed, 2, -1, 1)).cuda()
    yf = torch.empty((n, n), device="cuda")
    p = bwpp.MatmulParams(n, n, n, n, n, n, int(bwpp.DType.F32), 3, 0, 0)
    st = {}
    us = _events_us(torch, lambda: be.dispatch_matmul(xf, wf, yf, bf, p), iters, stats=st)
    fl = 2.0 * n ** 3
    # 256 tiles of 128 x 128: the dispatcher's cost model picks the 4-stage
    # LDS-DMA ring kernel (one block per CU) without a K split.
    c3f = {"kernel": be.last_kernel,
           "us_per_launch": round(us, 1), **st,
           "TFLOP_s": round(fl / us / 1e6, 1),
           "frac_f32_peak": round(fl / us / 1e6 / F32_PEAK_TFLOPS, 4)}
    if orc is not None:
        rows = 256
        xr, wr, br = xf[:rows].cpu().numpy(), wf.cpu().numpy(), bf.cpu().numpy()
        t0 = time.perf_counter()
        orc.matmul(xr, wr, br, apply_silu=True, apply_bias=True)
        dt = time.perf_counter() - t0
        c3f["cpu"] = {"GFLOP_s": round(2.0 * rows * n * n / dt / 1e9, 3), "cores": 1, "kind": "port",
                      "sample": f"first {rows} rows (exact rows; extrapolated rate)"}
    out["c3_gemm_f32_2048"] = c3f
    # C1: 256^3 fp32 (latency)
    a1, b1 = xf[:256, :256].contiguous(), wf[:256, :256].contiguous()
    c1 = torch.empty((256, 256), device="cuda")
    p = bwpp.MatmulParams(256, 256, 256, 256, 256, 256)
    us = _events_us(torch, lambda: be.dispatch_matmul(a1, b1, c1, None, p), iters)
    # 4 output tiles: the cost model splits K, so one call is the split-K
    # ring GEMM and the reduce that sums its partials (the last kernel).
    c1k = be.last_kernel
    if c1k == "bwpp_gemm_f32_splitk_reduce":
        c1k = be.recent_kernel(1) + " + " + c1k
    c1e = {"kernel": c1k, "us_per_call": round(us, 2),
           "TFLOP_s": round(2.0 * 256 ** 3 / us / 1e6, 2)}
    if orc is not None:
        ah, bh = a1.cpu().numpy(), b1.cpu().numpy()
        reps, t0 = 0, time.perf_counter()
        while reps < 3 or time.perf_counter() - t0 < 0.5:
            orc.matmul(ah, bh)
            reps += 1
        dt = (time.perf_counter() - t0) / reps
        c1e["cpu"] = {"GFLOP_s": round(2.0 * 256 ** 3 / dt / 1e9, 3), "us_per_call": round(dt * 1e6, 1),
                      "cores": 1, "kind": "port", "sample": f"the whole 256^3 product, {reps} calls"}
    out["c1_gemm_f32_256"] = c1e


def _extras_c4(be, torch, seed, iters, orc, out):
    import bwpp
    from bwpp import synth
    # C4: attention B 8, H 32, S 2048, d 128, bf16 ~ N(0, 1)
    B, H, S, d = 8, 32, 2048, 128
    qh = synth.normal((B, H, S, d), seed, 0)
    kh = synth.normal((B, H, S, d), seed, 1)
    vh = synth.normal((B, H, S, d), seed, 2)
    q, k, v = _bf16(torch, qh), _bf16(torch, kh), _bf16(torch, vh)
    o = torch.empty_like(q)
    full = 4.0 * B * H * S * S * d
    for causal in (0, 1):
        p = bwpp.AttentionParams(M=S, N=S, K=d, D=d, ldq=d, ldk=d, ldv=d, ldo=d, batch=B, heads=H,
                                 scale=d ** -0.5, causal=causal, dtype=int(bwpp.DType.BF16))
        st = {}
        us = _events_us(torch, lambda: be.dispatch_attention(q, k, v, o, p), iters, stats=st)
        fl = full / 2 if causal else full
        entry = {"kernel": be.last_kernel,
                 "us_per_launch": round(us, 1), **st, "TFLOP_s": round(fl / us / 1e6, 1),
                 "frac_bf16_peak": round(fl / us / 1e6 / BF16_PEAK_TFLOPS, 4)}
        if orc is not None:
            sl = lambda t: synth.bf16_bits_to_f32(synth.to_bf16_bits(t[:1, :1]))
            t0 = time.perf_counter()
            orc.attention_bh(sl(qh), sl(kh), sl(vh), d ** -0.5, bool(causal))
            dt = time.perf_counter() - t0
            entry["cpu"] = {"GFLOP_s": round(fl / (B * H) / dt / 1e9, 3), "cores": 1, "kind": "port",
                            "sample": "one (batch, head) slice (extrapolated rate)"}
        out["c4_attention_causal" if causal else "c4_attention"] = entry
    # Attention backward at the C4 shape (bf16 matrix-core passes after a
    # forward that saves lse): 5 products of 2*S*S*d per slice (S, dP, dV,
    # dK, dQ) = 2.5x the forward FLOP.  The default stored-dS scheme runs
    # exactly these (D_m pass; dK/dV pass that also stores dS; dQ = dS K
    # pass); with it off, the dQ pass recomputes S and dP (7 products).
    dout = _bf16(torch, synth.normal((B, H, S, d), seed, 3))
    lse = torch.empty((B, H, S), device="cuda")
    dq, dk, dv = torch.empty_like(q), torch.empty_like(k), torch.empty_like(v)
    for causal in (0, 1):
        p = bwpp.AttentionParams(M=S, N=S, K=d, D=d, ldq=d, ldk=d, ldv=d, ldo=d, batch=B, heads=H,
                                 scale=d ** -0.5, causal=causal, dtype=int(bwpp.DType.BF16))
        be.dispatch_attention_lse(q, k, v, o, lse, p)
        st = {}
        us = _events_us(torch, lambda: be.dispatch_attention_grad(q, k, v, o, dout, lse, dq, dk, dv, p),
                        max(3, iters // 3), stats=st)
        fl = 2.5 * (full / 2 if causal else full)
        cs = "_causal" if causal else ""
        last = be.last_kernel
        if last.endswith("_dq_ds"):  # stored dS: D_m, 8-wave dK/dV + dS, dQ = dS K
            kern = f"bwpp_attn_bwd_bf16_d128_dsum + bwpp_attn_bwd_bf16_mfma_d128{cs}_dkdv_w8_ds + {last}"
        else:
            kern = f"bwpp_attn_bwd_bf16_mfma_d128{cs}_dq + {last}"
        entry = {"kernel": kern,
                 "us_per_launch": round(us, 1), **st, "TFLOP_s": round(fl / us / 1e6, 1),
                 "frac_bf16_peak": round(fl / us / 1e6 / BF16_PEAK_TFLOPS, 4)}
        if orc is not None:
            sl = lambda t: synth.bf16_bits_to_f32(synth.to_bf16_bits(t[:1, :1]))
            g1 = synth.bf16_bits_to_f32(synth.to_bf16_bits(synth.normal((1, 1, S, d), seed, 3)))
            t0 = time.perf_counter()
            orc.attention_grad(sl(qh), sl(kh), sl(vh), g1, d ** -0.5, bool(causal))
            dt = time.perf_counter() - t0
            entry["cpu"] = {"GFLOP_s": round(fl / (B * H) / dt / 1e9, 3), "cores": 1, "kind": "port",
                            "sample": "one (batch, head) slice (extrapolated rate)"}
        out["c4_attention_grad_bf16" + ("_causal" if causal else "")] = entry


# FLOP of one C5 step: forward GEMMs 2*BT*D*(3D + D + 2F), backward twice
# that; causal attention 4*B*H*T*T*dh/2 forward, twice that backward
# (dV, dP, dQ, dK; the recomputed scores are not counted).
def block_train_flop(B, T, D, H, F):
    BT = B * T
    gemm = 2.0 * BT * D * (3 * D + D + 2 * F)
    attn = 4.0 * B * H * T * T * (D // H) / 2
    return 3.0 * gemm + 3.0 * attn


def block_inputs(seed, B, T, D, F):
    """C5's synthetic inputs from the repo's SplitMix64 generator: x ~ N(0,1),
    gamma ~ U[0.5,1.5], weights ~ N(0,0.02) (the plan's parameter names:
    F is the DSL's MLP width H)."""
    from bwpp import synth
    w = lambda shape, st: synth.normal(shape, seed, st, 0.0, 0.02)
    return {"x": synth.normal((B * T, D), seed, 0), "g1": synth.uniform((D,), seed, 1, 0.5, 1.5),
            "g2": synth.uniform((D,), seed, 2, 0.5, 1.5), "wq": w((D, D), 3), "wk": w((D, D), 4),
            "wv": w((D, D), 5), "wo": w((D, D), 6), "w1": w((D, F), 7), "w2": w((F, D), 8)}


def block_train(be, torch, seed, iters, B=8, T=512, D=1024, H=16, F=4096, with_cpu=False):
    """C5: one forward + backward step of examples/tiny_model.bwpp's `block`
    (16 causal heads, loss mean(out^2)) in fp32: the plan bwppc-hip lowers
    from the DSL and its autodiff (plans/block_train.plan), run by the
    launch-plan executor over one mem-planned device arena.  The CPU leg
    runs the same plan text for one sample (B = 1) on the oracle
    (oracle/plan_cpu.py), one core."""
    from bwpp import plan
    dims = dict(BATCH=B, T=T, D=D, H=F, HEADS=H)
    text = plan.load_text("block_train", **dims)
    p = plan.Plan(be, text)
    p.allocate()
    for name, a in block_inputs(seed, B, T, D, F).items():
        p.bind(name, torch.from_numpy(a).cuda())
    st = {}
    us = _events_us(torch, p.run, iters, stats=st)
    fl = block_train_flop(B, T, D, H, F)
    res = {"workload": f"B{B} T{T} D{D} H{H} F{F} fp32 fwd+bwd", "plan": "plans/block_train.plan",
           "us_per_step": round(us, 1), "us_mean": st.get("us_mean"),
           "TFLOP_s": round(fl / us / 1e6, 1), "frac_f32_peak": round(fl / us / 1e6 / F32_PEAK_TFLOPS, 4),
           "arena_bytes": p.arena_bytes, "ops_per_step": sum(1 for ln in text.splitlines() if ln.startswith("op "))}
    p.close()
    if with_cpu:
        sys.path.insert(0, ROOT)
        from oracle.plan_cpu import CpuPlan
        cp = CpuPlan(plan.load_text("block_train", **dict(dims, BATCH=1)))
        for name, a in block_inputs(seed, 1, T, D, F).items():
            cp.bind(name, a)
        t0 = time.perf_counter()
        cp.run()
        dt = time.perf_counter() - t0
        res["cpu"] = {"GFLOP_s": round(block_train_flop(1, T, D, H, F) / dt / 1e9, 3), "cores": 1, "kind": "port",
                      "sample": f"one sample (B=1) fwd+bwd through the same plan on the oracle, {dt:.1f} s "
                                "(extrapolated rate)"}
    return res


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=50)
    ap.add_argument("--warmup", type=int, default=100,
                    help="untimed C2 steps first (~20 ms: the clock ramps up under sustained load)")
    ap.add_argument("--seed", type=int, default=0)
    ap.add_argument("--nbuf", type=int, default=3, help="rotating input/output buffer sets")
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline leg")
    ap.add_argument("--cpu-reps", type=int, default=3)
    ap.add_argument("--no-extras", action="store_true", help="skip the C1/C3/C4 contraction configs")
    ap.add_argument("--op-reps", type=int, default=70, help="launches per operator for per-kernel timing")
    ap.add_argument("--copy-calibration", type=int, default=0, metavar="N",
                    help="also run N plain copies of known size (for scaling --pmc byte counters)")
    ap.add_argument("--traffic-from", nargs=2, metavar=("FETCH_DIR", "WRITE_DIR"),
                    help="no GPU: turn two rocprofv3 --pmc output dirs into profiles/traffic.json")
    ap.add_argument("--regress-json", metavar="PATH",
                    help="run the reference bench workload (bench_cpu.c) and write its JSON layout to PATH")
    ap.add_argument("--m", type=int, default=256)
    ap.add_argument("--n", type=int, default=256)
    ap.add_argument("--k", type=int, default=256)
    ap.add_argument("--rows", type=int, default=256)
    ap.add_argument("--cols", type=int, default=256)
    ap.add_argument("--iters", type=int, default=10)
    ap.add_argument("--no-c2", action="store_true",
                    help="skip the C2 headline (with --no-extras off: time the contractions only)")
    ap.add_argument("--extras-iters", type=int, default=30, help="timed launches per contraction config")
    ap.add_argument("--extras-only", default=",".join(EXTRA_GROUPS),
                    help="comma list of contraction groups to run: " + ", ".join(EXTRA_GROUPS))
    ap.add_argument("--warm-ms", type=float, default=WARM_MS,
                    help="sustained work before each contraction is timed (0 for counter runs)")
    ap.add_argument("--vs-library", action="store_true",
                    help="also time C3, C3-fp32 and C4 through torch's vendor-library paths (hipBLASLt, SDPA flash)")
    ap.add_argument("--pmc-summary", nargs="+", metavar="DIR",
                    help="no GPU: print a markdown table of per-kernel counters from rocprofv3 --pmc "
                         "(and --kernel-trace) output dirs")
    args = ap.parse_args()

    if args.pmc_summary:
        print(pmc_summary(args.pmc_summary))
        return

    if args.regress_json:
        out = regress_json(args)
        with open(args.regress_json, "w") as f:
            json.dump(out, f, indent=2)
            f.write("\n")
        print(json.dumps(out))
        return

    if args.traffic_from:
        t = traffic_from_pmc(*args.traffic_from)
        with open(os.path.join(ROOT, "profiles", "traffic.json"), "w") as f:
            json.dump(t, f, indent=1, sort_keys=True)
            f.write("\n")
        print(json.dumps(t, indent=1, sort_keys=True))
        return

    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) > 1:
        print("bench.py: this build measures one GPU only (single-GPU kernels; "
              "multi-GPU sharding is design-only). Run with --gpus 1.", file=sys.stderr)
        sys.exit(2)

    import torch
    import bwpp
    if not torch.cuda.is_available():
        print("bench.py: no GPU visible", file=sys.stderr)
        sys.exit(1)
    be = bwpp.HipBackend(0)
    be.set_stream(torch.cuda.current_stream())
    only = tuple(g.strip() for g in args.extras_only.split(",") if g.strip())
    bad = [g for g in only if g not in EXTRA_GROUPS]
    if bad:
        print(f"bench.py: unknown --extras-only group(s) {bad}; choose from {list(EXTRA_GROUPS)}", file=sys.stderr)
        sys.exit(2)

    if args.no_c2:
        out = {"metric": METRIC, "config": {"workload": "contractions only (no headline)"},
               "extras": extras(be, torch, args.seed, args.extras_iters, not args.no_cpu, args.warm_ms, only)}
        if args.vs_library:
            out["library"] = library_baseline(be, torch, args.seed, args.extras_iters)
        be.close()
        print(json.dumps(out))
        return

    bench = C2Bench(be, torch, args.seed, args.nbuf)
    torch.cuda.synchronize()
    wall, gpu_s = time_c2(bench, args.steps, args.warmup)
    per_op_ms = time_c2_ops(bench, args.op_reps)
    if args.copy_calibration:
        copy_calibration(bench, args.copy_calibration)
    step_bytes = sum(C2_BYTES.values())
    ms_per_step = wall / args.steps * 1e3
    value = step_bytes / (wall / args.steps) / 1e9

    dom = max(per_op_ms, key=lambda op: per_op_ms[op][0])
    achieved = C2_BYTES[dom] / (per_op_ms[dom][0] * 1e-3) / 1e9
    tr = load_traffic().get(C2_KERNEL[dom])
    traffic = tr["traffic"] if tr else None
    ops = {}
    for op, (ms, mean_ms) in per_op_ms.items():
        gbs = C2_BYTES[op] / (ms * 1e-3) / 1e9
        ops[op] = {"kernel": C2_KERNEL[op], "us_per_launch": round(ms * 1e3, 2),
                   "us_mean": round(mean_ms * 1e3, 2),
                   "algorithmic_bytes": C2_BYTES[op], "GB_s": round(gbs, 1),
                   "frac_hbm_peak": round(gbs / HBM_PEAK_GBS, 4)}
        t = load_traffic().get(C2_KERNEL[op])
        if t:
            ops[op]["traffic"] = t["traffic"]

    out = {
        "metric": METRIC,
        "value": round(value, 2),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms_per_step, 4),
        "gpu_ms_per_step": round(gpu_s / args.steps * 1e3, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f32",
        "data": "synthetic",
        "config": {"workload": "C2: fp32 row ops on X[8192x4096] ~ N(0,1): softmax, LayerNorm, "
                               "RMSNorm, reduce_max fwd (max+argmax), reduce_max grad (X,dy->dX)",
                   "rows": ROWS, "cols": COLS, "seed": args.seed, "rotating_buffer_sets": args.nbuf,
                   "step_algorithmic_bytes": step_bytes},
        "roofline": {"bound": "hbm", "kernel": C2_KERNEL[dom], "op": dom,
                     "us_per_launch": round(per_op_ms[dom][0] * 1e3, 2), "timing": "median",
                     "achieved": round(achieved, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": round(achieved / HBM_PEAK_GBS, 4), "traffic": traffic},
        "ops": ops,
        "host": host_info(),
    }
    ceil = stream_ceiling(torch, final_reps=args.op_reps)
    rceil = stream_ceiling(torch, kind="read", final_reps=args.op_reps)
    if ceil:
        out["stream_ceiling"] = ceil
        if rceil:
            out["read_ceiling"] = rceil
        for name, op in ops.items():
            # reduce_max reads X and writes 64 KB: its ceiling is the read stream
            c = rceil if (name == "reduce_max" and rceil) else ceil
            op["frac_of_stream_ceiling"] = round(op["GB_s"] / c["GB_s"], 4)
    if not args.no_cpu:
        out["cpu_baseline"] = cpu_baseline_c2(args.seed, args.cpu_reps)
    else:
        out["cpu_baseline"] = None
    del bench
    if not args.no_extras:
        torch.cuda.empty_cache()
        out["extras"] = extras(be, torch, args.seed, args.extras_iters, not args.no_cpu, args.warm_ms, only)
    be.close()
    print(json.dumps(out))


if __name__ == "__main__":
    main()
