#!/usr/bin/env python3
"""Lowers the reference's example programs to launch plans with bwppc-hip
and writes them to bluewolf-plus-plus_amd/plans/.

The compiler links the reference's front end from its source tree, so this
runs where /root/reference exists (the build container); the committed
plans are what the library, the tests and bench.py load, and
tests/test_lowering.py checks that they are exactly what this emits.

    python bluewolf-plus-plus_amd/compiler/emit_plans.py [--check]
"""
from __future__ import annotations

import argparse
import os
import subprocess
import sys
import tempfile

HERE = os.path.dirname(os.path.abspath(__file__))
PKG = os.path.dirname(HERE)
PLANS = os.path.join(PKG, "plans")
REFERENCE = os.environ.get("REFERENCE", "/root/reference")
EXAMPLES = os.path.join(REFERENCE, "examples")
BWPPC = os.path.join(HERE, "_build", "bwppc-hip")

C5 = ["--dim", "T=512", "--dim", "D=1024", "--dim", "H=4096", "--batch", "8", "--heads", "16", "--causal",
      "--attn-scale", "auto"]

# plan file -> (example, arguments)
TABLE = {
    # config 5: the block of tiny_model, 8 samples of 512 tokens, 16 causal
    # heads of 64, trained on loss = mean(out^2) through the DSL's autodiff
    "block_train.plan": ("tiny_model.bwpp", ["--entry", "block", *C5, "--train", "mean_square"]),
    "block_fwd.plan": ("tiny_model.bwpp", ["--entry", "block", *C5]),
    "tiny_model_fwd.plan": ("tiny_model.bwpp", ["--entry", "tiny_model", *C5, "--dim", "V=8192"]),
    # rank-4 [B, H, T, D] attention and its gradients (seeded by dO): fp32,
    # and bf16 at config 4's size
    "attention_train.plan": ("attention.bwpp", ["--dim", "B=2", "--dim", "H=4", "--dim", "T=256", "--dim", "D=64",
                                                "--attn-scale", "auto", "--train", "seed"]),
    "attention_train_bf16.plan": ("attention.bwpp", ["--dim", "B=8", "--dim", "H=32", "--dim", "T=2048",
                                                     "--dim", "D=128", "--attn-scale", "auto", "--dtype", "bf16",
                                                     "--train", "seed"]),
    "attention_causal_bf16.plan": ("attention.bwpp", ["--dim", "B=8", "--dim", "H=32", "--dim", "T=2048",
                                                      "--dim", "D=128", "--attn-scale", "auto", "--causal",
                                                      "--dtype", "bf16"]),
    # config 3 as a DSL program: bias + SiLU fused into the bf16 GEMM
    "matmul_add_silu.plan": ("matmul_add_silu.bwpp", ["--dim", "M=4096", "--dim", "K=4096", "--dim", "N=11008",
                                                      "--dtype", "bf16"]),
    "matmul_add_bias_reshape.plan": ("matmul_add_bias_reshape.bwpp",
                                     ["--dim", "M=2048", "--dim", "K=2048", "--dim", "N=2048"]),
    "multi_fn_bias.plan": ("multi_fn_bias.bwpp", ["--entry", "block_b", "--dim", "M=2048", "--dim", "K=2048",
                                                  "--dim", "N=2048"]),
    # config 1
    "matmul.plan": ("matmul.bwpp", ["--dim", "M=256", "--dim", "K=256", "--dim", "N=256"]),
    "norms.plan": ("norms.bwpp", ["--dim", "B=8192", "--dim", "N=4096"]),
}

# Programs of this repository's tests (tests/golden/bwpp/), lowered next to
# their sources: plan file -> (program, arguments).
TESTS = os.path.join(os.path.dirname(PKG), "tests", "golden", "bwpp")
TEST_TABLE = {
    # reduce_max along rows at config 2's shape, and its DSL autodiff
    "reduce_max.plan": ("reduce_max.bwpp", ["--dim", "M=8192", "--dim", "K=1024", "--dim", "N=4096"]),
    "reduce_max_train.plan": ("reduce_max.bwpp", ["--dim", "M=8192", "--dim", "K=1024", "--dim", "N=4096",
                                                  "--train", "seed"]),
}


def build():
    subprocess.run(["make", "-C", HERE, "-s"], check=True)


def emit(name, out_path):
    """Runs bwppc-hip for one table entry (the plan records its command
    line, with the two file arguments reduced to their names)."""
    if name in TABLE:
        src_dir, (example, args) = EXAMPLES, TABLE[name]
    else:
        src_dir, (example, args) = TESTS, TEST_TABLE[name]
    cmd = [BWPPC, os.path.join(src_dir, example), out_path, *args]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"{name}: {' '.join(cmd)}\n{r.stderr}")
    return out_path


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--check", action="store_true", help="compare with the committed plans, write nothing")
    args = ap.parse_args()
    if not os.path.isdir(EXAMPLES):
        sys.exit(f"{EXAMPLES} not found: the plans are emitted where the reference tree exists")
    build()
    bad = []
    with tempfile.TemporaryDirectory() as td:
        for name in [*TABLE, *TEST_TABLE]:
            path = emit(name, os.path.join(td, name))
            text = open(path).read()
            committed = os.path.join(PLANS if name in TABLE else TESTS, name)
            if args.check:
                if not os.path.exists(committed) or open(committed).read() != text:
                    bad.append(name)
            else:
                with open(committed, "w") as f:
                    f.write(text)
                print("wrote", committed)
    if bad:
        sys.exit("plans differ from the lowering: " + ", ".join(bad))


if __name__ == "__main__":
    main()
