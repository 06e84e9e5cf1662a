"""bench.py's regression mode writes the reference's bench JSON
(bench/bench_cpu.c:142-157): the three groups and the fields
bench/bench_regress.py:93-111 compares (time_s per group), measured on the
GPU through libbwpp_hip."""
import argparse
import json
import os
import sys

import pytest

pytestmark = pytest.mark.gpu

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def test_regress_json_layout(tmp_path):
    sys.path.insert(0, ROOT)
    import bench
    args = argparse.Namespace(m=64, n=48, k=80, rows=33, cols=200, iters=3, no_cpu=False)
    out = bench.regress_json(args)
    path = tmp_path / "cur.json"
    path.write_text(json.dumps(out, indent=2))
    data = json.loads(path.read_text())
    assert {"M": 64, "N": 48, "K": 80, "iters": 3}.items() <= data["matmul"].items()
    for group in ("softmax", "rmsnorm"):
        assert {"rows": 33, "cols": 200, "iters": 3}.items() <= data[group].items()
    for group in ("matmul", "softmax", "rmsnorm"):
        assert float(data[group]["time_s"]) > 0.0
        assert float(data[group]["cpu_time_s"]) > 0.0
    assert data["matmul"]["gflops"] > 0.0
