"""Regenerate tests/golden/ref_vectors.npz from the reference's own CPU code.

Runs in the build container only, where /root/reference exists:
    make -C oracle ref            # compiles runtime/cpu/bwpp_cpu_ref.c as is
    python tests/golden/make_golden.py

Every case stores its inputs and the outputs of the compiled reference
(oracle/_ref/libbwpp_cpu_ref.so).  Fixtures are the reference tests' own ramp
inputs (runtime/cpu/test_matmul.c:7-13, test_norm.c, test_reduce_max.c,
test_metal_parity.c) plus small seeded inputs and special values.  The file
is data only: inputs and expected outputs.
"""
from __future__ import annotations

import os
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(os.path.dirname(HERE))
sys.path.insert(0, ROOT)

from oracle.oracle import RefLib  # noqa: E402

OUT = os.path.join(HERE, "ref_vectors.npz")


def ramp(rows, cols, scale):
    """(i*cols + j + 1) * scale with the reference's uint32 -> float cast."""
    i = np.arange(rows * cols, dtype=np.uint32) + np.uint32(1)
    return (i.astype(np.float32) * np.float32(scale)).reshape(rows, cols)


def seeded(shape, seed, lo=-1.0, hi=1.0):
    rng = np.random.default_rng(seed)
    return rng.uniform(lo, hi, size=shape).astype(np.float32)


def main():
    ref = RefLib()
    out = {}

    def put(name, **arrays):
        for k, v in arrays.items():
            out[f"{name}/{k}"] = np.asarray(v)

    # --- matmul: test_matmul.c / test_metal_parity.c fixture (4x4x4 ramp)
    a = ramp(4, 4, 0.1)
    b = ramp(4, 4, 0.05)
    bias = (np.float32(0.01) * (np.arange(4, dtype=np.float32) + 1)).astype(np.float32)
    for tag, silu, add in (("none", 0, 0), ("add", 0, 1), ("silu", 1, 0), ("add_silu", 1, 1)):
        bb = bias if add else np.zeros(4, np.float32)
        c = ref.matmul(a, b, bb, apply_silu=silu, apply_bias=add)
        put(f"matmul_ramp4_{tag}", a=a, b=b, bias=bb, silu=silu, add=add, c=c)
    # seeded, odd sizes, all epilogues
    a = seeded((17, 29), 1)
    b = seeded((29, 23), 2)
    bias = seeded((23,), 3)
    for tag, silu, add in (("none", 0, 0), ("add", 0, 1), ("silu", 1, 0), ("add_silu", 1, 1)):
        c = ref.matmul(a, b, bias, apply_silu=silu, apply_bias=add)
        put(f"matmul_seed_{tag}", a=a, b=b, bias=bias, silu=silu, add=add, c=c)
    # bwpp_bench default fixture (bench_cpu.c:82-83) at a reduced 32^3
    a = ramp(32, 32, 0.01)
    b = ramp(32, 32, 0.02)
    put("matmul_bench32", a=a, b=b, bias=np.zeros(32, np.float32), silu=0, add=0,
        c=ref.matmul(a, b, None))

    # --- softmax
    x = ramp(2, 4, 0.1)
    put("softmax_ramp", x=x, y=ref.softmax(x))
    x = seeded((7, 33), 4, -4, 4)
    put("softmax_seed", x=x, y=ref.softmax(x))
    xs = np.zeros((5, 12), np.float32)
    xs[:, :10] = seeded((5, 10), 5, -3, 3)
    put("softmax_ld", xfull=xs, cols=10, yfull=np.asarray(ref.softmax(xs[:, :10]).base))
    x = np.array([[0.0, np.inf, 1.0, -1.0],
                  [-np.inf, -np.inf, -np.inf, -np.inf],
                  [np.nan, 1.0, 2.0, 3.0],
                  [-np.inf, 0.5, -np.inf, 0.25],
                  [np.inf, np.inf, 0.0, 1.0],
                  [3.0, 3.0, 3.0, 3.0]], np.float32)
    put("softmax_special", x=x, y=ref.softmax(x))

    # --- rmsnorm
    x = ramp(2, 4, 0.1)
    put("rmsnorm_ramp", x=x, gamma=np.ones(4, np.float32), eps=np.float32(1e-5),
        y=ref.rmsnorm(x, np.ones(4, np.float32), None, 1e-5))
    x = seeded((6, 40), 6, -2, 2)
    g = seeded((40,), 7, 0.5, 1.5)
    bt = seeded((40,), 8, -0.1, 0.1)
    put("rmsnorm_seed_gb", x=x, gamma=g, beta=bt, eps=np.float32(1e-6),
        y=ref.rmsnorm(x, g, bt, 1e-6))
    put("rmsnorm_seed_g", x=x, gamma=g, eps=np.float32(1e-5), y=ref.rmsnorm(x, g, None, 1e-5))
    put("rmsnorm_seed_none", x=x, eps=np.float32(1e-5), y=ref.rmsnorm(x, None, None, 1e-5))

    # --- attention: test_metal_parity.c:237-248 fixture and a seeded case
    q = ramp(2, 4, 0.03)
    k = ramp(3, 4, 0.04)
    v = ramp(3, 5, 0.02)
    put("attention_ramp", q=q, k=k, v=v, o=ref.attention(q, k, v))
    q = seeded((9, 8), 9)
    k = seeded((11, 8), 10)
    v = seeded((11, 6), 11)
    put("attention_seed", q=q, k=k, v=v, o=ref.attention(q, k, v))

    # --- reduce_max mask / grad: test_reduce_max.c fixture (x[r][c] = r*cols+c)
    x = np.arange(6, dtype=np.float32).reshape(2, 3)
    dy = np.array([1.0, 2.0], np.float32)
    m1 = ref.reduce_max_mask(x, 1)
    put("rmax_ramp_axis1", x=x, mask=m1, dy=dy, dx=ref.reduce_max_grad_mask(m1, dy, 1))
    # ties (small integer values), both axes
    rng = np.random.default_rng(12)
    x = rng.integers(0, 4, size=(6, 7)).astype(np.float32)
    x[2, :] = -np.inf
    x[3, 1] = np.nan
    dyr = seeded((6,), 13)
    dyc = seeded((7,), 14)
    m1 = ref.reduce_max_mask(x, 1)
    m0 = ref.reduce_max_mask(x, 0)
    put("rmax_ties_axis1", x=x, mask=m1, dy=dyr, dx=ref.reduce_max_grad_mask(m1, dyr, 1))
    put("rmax_ties_axis0", x=x, mask=m0, dy=dyc, dx=ref.reduce_max_grad_mask(m0, dyc, 0))

    np.savez_compressed(OUT, **out)
    print(f"wrote {OUT}: {len(out)} arrays")


if __name__ == "__main__":
    main()
