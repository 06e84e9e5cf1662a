"""Tensor-level operators (bwpp_hip_tensor_*) on the GPU: each derives its
params struct from BwppHipTensor metadata and runs the same kernel as the
dispatch form, so results must be bit-identical to the dispatch call with
the params written out by hand -- including column-major (transposed)
GEMM operands, padded rows and rank-3/4 tensors.  The plain-C caller
(tests/c/caller.c) runs end to end against host-computed results."""
import os
import subprocess

import numpy as np
import pytest

import bwpp
from bwpp import synth, tensor_of
from conftest import rel_max_err

pytestmark = pytest.mark.gpu

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def _t():
    import torch
    return torch


def dev(a):
    return _t().from_numpy(np.ascontiguousarray(a, np.float32)).cuda()


@pytest.mark.parametrize("ta,tb", [(False, False), (True, False), (False, True), (True, True)])
def test_tensor_matmul_orientations(be, oracle, ta, tb):
    torch = _t()
    M, N, K = 192, 160, 96
    a = synth.normal((M, K), 1, 0)
    b = synth.normal((K, N), 1, 1)
    bias = synth.normal((N,), 1, 2)
    # A column-major [M, K] is a row-major [K, M] buffer seen through .t()
    ad = dev(a.T).t() if ta else dev(a)
    bd = dev(b.T).t() if tb else dev(b)
    c1 = torch.full((M, N), 3.0, device="cuda")
    be.tensor_matmul(tensor_of(ad, 1 if ta else 0), tensor_of(bd, 1 if tb else 0), tensor_of(dev(bias)),
                     tensor_of(c1), 3)
    c2 = torch.full((M, N), 3.0, device="cuda")
    p = bwpp.MatmulParams(M, N, K, M if ta else K, K if tb else N, N, 0, 3, int(ta), int(tb))
    be.dispatch_matmul(dev(a.T) if ta else ad, dev(b.T) if tb else bd, c2, dev(bias), p)
    torch.cuda.synchronize()
    assert torch.equal(c1, c2)
    want = oracle.matmul(a, b, bias, apply_silu=True, apply_bias=True)
    assert rel_max_err(c1.cpu().numpy(), want) <= 1e-4


def test_tensor_matmul_bf16(be):
    torch = _t()
    M, N, K = 256, 256, 64
    a = torch.randn(M, K, device="cuda").bfloat16()
    b = torch.randn(K, N, device="cuda").bfloat16()
    c1, c2 = (torch.empty(M, N, device="cuda", dtype=torch.bfloat16) for _ in range(2))
    be.tensor_matmul(tensor_of(a), tensor_of(b), None, tensor_of(c1), 0)
    be.dispatch_matmul(a, b, c2, None, bwpp.MatmulParams(M, N, K, K, N, N, 1, 0, 0, 0))
    torch.cuda.synchronize()
    assert torch.equal(c1, c2)


def test_tensor_row_ops_rank3_padded(be):
    torch = _t()
    B, R, C, LD = 3, 50, 300, 320
    base = torch.from_numpy(synth.normal((B, R, LD), 2, 0)).cuda()
    x = base[:, :, :C]  # padded rows, batches stacked at R * LD
    g = torch.from_numpy(synth.uniform((C,), 2, 1, 0.5, 1.5)).cuda()
    bt = torch.from_numpy(synth.normal((C,), 2, 2)).cuda()
    for op in ("softmax", "rmsnorm", "layernorm"):
        y1 = torch.full((B, R, LD), 9.0, device="cuda")
        y2 = torch.full((B, R, LD), 9.0, device="cuda")
        if op == "softmax":
            be.tensor_softmax(tensor_of(x), tensor_of(y1[:, :, :C]))
            be.dispatch_softmax(base, y2, bwpp.SoftmaxParams(B * R, C, LD))
        elif op == "rmsnorm":
            be.tensor_rmsnorm(tensor_of(x), tensor_of(g), None, tensor_of(y1[:, :, :C]), 1e-6)
            be.dispatch_rmsnorm(base, g, None, y2, bwpp.RmsnormParams(B * R, C, LD, 1e-6))
        else:
            be.tensor_layernorm(tensor_of(x), tensor_of(g), tensor_of(bt), tensor_of(y1[:, :, :C]), 1e-5)
            be.dispatch_layernorm(base, g, bt, y2, bwpp.RmsnormParams(B * R, C, LD, 1e-5))
        torch.cuda.synchronize()
        assert torch.equal(y1, y2), op
        assert torch.all(y1[:, :, C:] == 9.0), op  # padding untouched


def test_tensor_attention_rank4(be):
    torch = _t()
    B, H, S, d = 2, 3, 100, 64
    q, k, v = (torch.from_numpy(synth.normal((B, H, S, d), 3, i)).cuda() for i in range(3))
    o1, o2 = torch.empty_like(q), torch.empty_like(q)
    be.tensor_attention(tensor_of(q), tensor_of(k), tensor_of(v), tensor_of(o1), 0.125, 1)
    be.dispatch_attention(q, k, v, o2, bwpp.AttentionParams(M=S, N=S, K=d, D=d, ldq=d, ldk=d, ldv=d, ldo=d,
                                                            batch=B, heads=H, scale=0.125, causal=1))
    torch.cuda.synchronize()
    assert torch.equal(o1, o2)


def test_tensor_errors(be):
    torch = _t()
    x = torch.zeros(4, 8, device="cuda")
    with pytest.raises(bwpp.BwppError) as e:
        be.tensor_matmul(tensor_of(x), tensor_of(x), None, tensor_of(x), 0)  # shapes do not chain
    assert e.value.status == bwpp.Status.INVALID_ARG
    with pytest.raises(bwpp.BwppError):
        be.tensor_softmax(tensor_of(x), tensor_of(torch.zeros(4, 9, device="cuda")))


def test_c_caller_runs():
    exe = os.path.join(ROOT, "tests", "c", "bwpp_caller")
    assert os.path.exists(exe), "tests/c/bwpp_caller not built (__graft_entry__.build())"
    r = subprocess.run([exe], capture_output=True, text=True, timeout=120)
    print(r.stdout)
    assert r.returncode == 0, r.stdout + r.stderr
    assert r.stdout.strip().endswith("OK")


# ------------------------------------------------------ missing code objects
def _lib_dir():
    return os.path.join(ROOT, "bluewolf-plus-plus_amd", "lib")


def test_create_with_missing_code_objects(tmp_path):
    """bwpp_hip_create loads six code objects and resolves every kernel
    before it returns (the reference's dispatch returns silently on a
    missing pipeline, dispatch_stub.m:74-79): an empty directory, a
    directory lacking one object, and an object holding other kernels each
    give NO_KERNEL naming what is missing, and the library stays usable."""
    import shutil
    names = sorted(f for f in os.listdir(_lib_dir()) if f.endswith(".hsaco"))
    assert len(names) == 6, names
    empty = tmp_path / "empty"
    empty.mkdir()
    with pytest.raises(bwpp.BwppError) as e:
        bwpp.HipBackend(0, code_object_dir=str(empty))
    assert e.value.status == bwpp.Status.NO_KERNEL and "hipModuleLoad" in str(e.value)
    part = tmp_path / "part"
    part.mkdir()
    for n in names:
        if n != "bwpp_attention.hsaco":
            shutil.copy(os.path.join(_lib_dir(), n), part / n)
    with pytest.raises(bwpp.BwppError) as e:
        bwpp.HipBackend(0, code_object_dir=str(part))
    assert e.value.status == bwpp.Status.NO_KERNEL and "bwpp_attention.hsaco" in str(e.value)
    # a loadable object with the wrong kernels: the load succeeds, resolution fails
    shutil.copy(os.path.join(_lib_dir(), "bwpp_grad.hsaco"), part / "bwpp_attention.hsaco")
    with pytest.raises(bwpp.BwppError) as e:
        bwpp.HipBackend(0, code_object_dir=str(part))
    assert e.value.status == bwpp.Status.NO_KERNEL and "not found" in str(e.value)
    be = bwpp.HipBackend(0)  # the real objects still load
    be.close()
