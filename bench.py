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

Extra contraction configs (C3 GEMM, C4 attention) are reported under "ops"
once their kernels exist; they are not part of `value`.
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
C2_KERNEL = {  # kernel symbol each op launches at this shape (rowops.hip)
    "softmax": "bwpp_row_softmax_v2_w8_f",
    "layernorm": "bwpp_row_layernorm_v4_w4_f",
    "rmsnorm": "bwpp_row_rmsnorm_v4_w4_f",
    "reduce_max": "bwpp_row_max_v4_w4_f",
    "reduce_max_grad": "bwpp_row_maxgrad_v4_w4_f",
}


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
    torch = bench.torch
    ops = list(C2_BYTES)
    stream = torch.cuda.current_stream()
    k = 0
    for _ in range(warmup):
        for op in ops:
            bench.launch(op, k % bench.nbuf)
            k += 1
    ev = {op: [] for op in ops}
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for _ in range(steps):
        for op in ops:
            s = torch.cuda.Event(enable_timing=True)
            e = torch.cuda.Event(enable_timing=True)
            s.record(stream)
            bench.launch(op, k % bench.nbuf)
            e.record(stream)
            ev[op].append((s, e))
            k += 1
    torch.cuda.synchronize()
    wall = time.perf_counter() - t0
    per_op_ms = {op: float(np.mean([s.elapsed_time(e) for s, e in ev[op]])) for op in ops}
    return wall, per_op_ms


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


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=50)
    ap.add_argument("--warmup", type=int, default=5)
    ap.add_argument("--seed", type=int, default=0)
    ap.add_argument("--nbuf", type=int, default=3, help="rotating input/output buffer sets")
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline leg")
    ap.add_argument("--cpu-reps", type=int, default=3)
    args = ap.parse_args()

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

    bench = C2Bench(be, torch, args.seed, args.nbuf)
    torch.cuda.synchronize()
    wall, per_op_ms = time_c2(bench, args.steps, args.warmup)
    step_bytes = sum(C2_BYTES.values())
    ms_per_step = wall / args.steps * 1e3
    value = step_bytes / (wall / args.steps) / 1e9

    dom = max(per_op_ms, key=per_op_ms.get)
    achieved = C2_BYTES[dom] / (per_op_ms[dom] * 1e-3) / 1e9
    traffic = load_traffic().get(C2_KERNEL[dom])
    ops = {}
    for op, ms in per_op_ms.items():
        gbs = C2_BYTES[op] / (ms * 1e-3) / 1e9
        ops[op] = {"kernel": C2_KERNEL[op], "us_per_launch": round(ms * 1e3, 2),
                   "algorithmic_bytes": C2_BYTES[op], "GB_s": round(gbs, 1),
                   "frac_hbm_peak": round(gbs / HBM_PEAK_GBS, 4)}

    out = {
        "metric": METRIC,
        "value": round(value, 2),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms_per_step, 4),
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
                     "achieved": round(achieved, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": round(achieved / HBM_PEAK_GBS, 4), "traffic": traffic},
        "ops": ops,
        "host": host_info(),
    }
    if not args.no_cpu:
        out["cpu_baseline"] = cpu_baseline_c2(args.seed, args.cpu_reps)
    else:
        out["cpu_baseline"] = None
    be.close()
    print(json.dumps(out))


if __name__ == "__main__":
    main()
