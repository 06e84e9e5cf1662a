"""Pins the gfx950 MFMA operand and accumulator lane layouts that the GEMM
and attention kernels are written against (probes in tests/hip/probe.hip,
built by tests/hip/Makefile).  Small integers make every product exact, so any
mismatch between the hardware and the assumed layout shows as a wrong
entry."""
import ctypes
import os

import numpy as np
import pytest

from hipmod import Module

pytestmark = pytest.mark.gpu

PROBE = os.path.join(os.path.dirname(os.path.abspath(__file__)), "hip", "bwpp_probe.hsaco")


class ProbeArgs(ctypes.Structure):
    _fields_ = [("a", ctypes.c_void_p), ("b", ctypes.c_void_p), ("c", ctypes.c_void_p)]


def _maps(shape):
    """(a_map, b_map, c_map): dicts from matrix index to (lane, element)."""
    if shape in ("32x32x16_bf16", "32x32x2_f32"):
        n, kdim, per = 32, (16 if shape.endswith("bf16") else 2), (8 if shape.endswith("bf16") else 1)
    else:
        n, kdim, per = 16, (32 if shape.endswith("bf16") else 4), (8 if shape.endswith("bf16") else 1)
    a = {(i, k): (i + n * (k // per), k % per) for i in range(n) for k in range(kdim)}
    b = {(k, j): (j + n * (k // per), k % per) for k in range(kdim) for j in range(n)}
    if n == 32:
        c = {(i, j): (j + 32 * ((i // 4) % 2), (i // 8) * 4 + i % 4) for i in range(32) for j in range(32)}
    else:
        c = {(i, j): (j + 16 * (i // 4), i % 4) for i in range(16) for j in range(16)}
    return n, kdim, per, a, b, c


@pytest.mark.parametrize("shape", ["32x32x16_bf16", "16x16x32_bf16", "32x32x2_f32", "16x16x4_f32"])
def test_mfma_layout(shape):
    import torch
    n, kdim, per, amap, bmap, cmap = _maps(shape)
    nacc = 16 if n == 32 else 4
    rng = np.random.default_rng(hash(shape) % 1000)
    areg = rng.integers(-4, 5, (64, per)).astype(np.float32)
    breg = rng.integers(-4, 5, (64, per)).astype(np.float32)
    dt = torch.bfloat16 if shape.endswith("bf16") else torch.float32
    a = torch.from_numpy(areg).to(dt).cuda()
    b = torch.from_numpy(breg).to(dt).cuda()
    c = torch.zeros(64 * nacc, dtype=torch.float32, device="cuda")
    mod = Module(PROBE)
    args = ProbeArgs(a.data_ptr(), b.data_ptr(), c.data_ptr())
    mod.launch("probe_mfma_" + shape, (1, 1, 1), (64, 1, 1), args,
               stream=torch.cuda.current_stream().cuda_stream)
    torch.cuda.synchronize()
    creg = c.cpu().numpy().reshape(64, nacc)
    mod.close()
    A = np.zeros((n, kdim), np.float32)
    B = np.zeros((kdim, n), np.float32)
    for (i, k), (l, e) in amap.items():
        A[i, k] = areg[l, e]
    for (k, j), (l, e) in bmap.items():
        B[k, j] = breg[l, e]
    C = A @ B
    got = np.zeros_like(C)
    for (i, j), (l, r) in cmap.items():
        got[i, j] = creg[l, r]
    assert np.array_equal(got, C), shape
