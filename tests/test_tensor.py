"""Tensor metadata layer of libbwpp_hip (host side, no GPU): the device
twin of runtime/core/tensor.h's BwppTensor keeps its layout, the dtype
mappers agree with the three enums they join (runtime/core/tensor.h:7-11,
compiler/include/graph_ir.h:18-23, BwppHipDType), and shapes, strides,
byte spans and matrix views come out as the row operators need them.  The
plain-C caller (tests/c/caller.c) builds warning-free against the header."""
import ctypes
import os
import subprocess

import pytest

import bwpp
from bwpp import _lib

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


class RefTensor(ctypes.Structure):
    """runtime/core/tensor.h:18-25 as a C compiler lays it out (enums are int)."""
    _fields_ = [("dtype", ctypes.c_int), ("layout", ctypes.c_int), ("rank", ctypes.c_uint32),
                ("shape", ctypes.c_uint64 * 4), ("stride", ctypes.c_uint64 * 4), ("buffer", ctypes.c_void_p)]


def test_layout_matches_reference_tensor():
    assert ctypes.sizeof(bwpp.Tensor) == ctypes.sizeof(RefTensor) == 88
    for name, *_ in RefTensor._fields_:
        assert getattr(bwpp.Tensor, name).offset == getattr(RefTensor, name).offset, name


def test_dtype_mappers():
    lib = _lib.load()
    # runtime/core: F16 0, BF16 1, F32 2; compiler: UNKNOWN 0, F16 1, BF16 2, F32 3;
    # BwppHipDType: F32 0, BF16 1.
    assert [lib.bwpp_hip_dtype_from_core(d) for d in (0, 1, 2, 3, -1)] == [-1, 1, 0, -1, -1]
    assert [lib.bwpp_hip_dtype_from_graph(d) for d in (0, 1, 2, 3, 4)] == [-1, -1, 1, 0, -1]
    assert [lib.bwpp_hip_dtype_to_core(d) for d in (0, 1, 2)] == [2, 1, -1]
    assert [lib.bwpp_hip_dtype_to_graph(d) for d in (0, 1, 2)] == [3, 2, -1]
    for hip in (0, 1):  # round trips
        assert lib.bwpp_hip_dtype_from_core(lib.bwpp_hip_dtype_to_core(hip)) == hip
        assert lib.bwpp_hip_dtype_from_graph(lib.bwpp_hip_dtype_to_graph(hip)) == hip
    assert [lib.bwpp_hip_core_dtype_size(d) for d in (0, 1, 2, 7)] == [2, 2, 4, 0]


def _init(shape, dtype=2, layout=0, buf=None):
    lib = _lib.load()
    t = bwpp.Tensor()
    sh = (ctypes.c_uint64 * max(4, len(shape)))(*shape)
    st = lib.bwpp_hip_tensor_init(ctypes.byref(t), dtype, layout, len(shape),
                                  ctypes.cast(sh, ctypes.POINTER(ctypes.c_uint64)), buf)
    return st, t


def test_init_strides_and_bytes():
    lib = _lib.load()
    st, t = _init((2, 3, 5))
    assert st == 0 and list(t.stride)[:3] == [15, 5, 1] and t.rank == 3
    assert lib.bwpp_hip_tensor_bytes(ctypes.byref(t)) == 2 * 3 * 5 * 4
    st, t = _init((4, 6), dtype=1, layout=1)  # column-major rank 2
    assert st == 0 and list(t.stride)[:2] == [1, 4]
    assert lib.bwpp_hip_tensor_bytes(ctypes.byref(t)) == 4 * 6 * 2
    # strided: bytes span the last element
    t.stride[1] = 10
    assert lib.bwpp_hip_tensor_bytes(ctypes.byref(t)) == (3 + 5 * 10 + 1) * 2
    assert _init((0, 4))[0] == 0 and lib.bwpp_hip_tensor_bytes(ctypes.byref(_init((0, 4))[1])) == 0
    assert _init((2, 2, 2), layout=1)[0] == bwpp.Status.INVALID_ARG  # col-major needs rank 2
    assert _init((2,) * 5)[0] == bwpp.Status.INVALID_ARG
    assert _init((2, 2), dtype=9)[0] == bwpp.Status.INVALID_ARG


def _matrix(t):
    lib = _lib.load()
    r, c, ld = ctypes.c_uint32(), ctypes.c_uint32(), ctypes.c_uint32()
    st = lib.bwpp_hip_tensor_matrix(ctypes.byref(t), ctypes.byref(r), ctypes.byref(c), ctypes.byref(ld))
    return st, (r.value, c.value, ld.value)


def test_matrix_view():
    _, t = _init((2, 3, 8))
    assert _matrix(t) == (0, (6, 8, 8))
    t.stride[1], t.stride[0] = 12, 36  # padded rows, stacked batches
    assert _matrix(t) == (0, (6, 8, 12))
    t.stride[0] = 40  # batches not at one row stride
    assert _matrix(t)[0] == bwpp.Status.UNSUPPORTED
    _, t = _init((4, 6), layout=1)
    assert _matrix(t)[0] == bwpp.Status.UNSUPPORTED
    _, t = _init((7,))
    assert _matrix(t) == (0, (1, 7, 7))


def test_alloc_from_arena_is_aligned_and_bounded():
    """bwpp_hip_tensor_alloc only does the arena's pointer arithmetic, so a
    host-side arena record stands in for device memory here."""
    lib = _lib.load()
    arena = _lib.Arena(buffer=0x100000, capacity=4096, offset=3, device=0)
    t = bwpp.Tensor()
    sh = (ctypes.c_uint64 * 4)(10, 10)
    assert lib.bwpp_hip_tensor_alloc(ctypes.byref(arena), ctypes.byref(t), 2, 0, 2, sh) == 0
    assert t.buffer == 0x100000 + 256 and arena.offset == 256 + 400
    sh = (ctypes.c_uint64 * 4)(100, 100)
    assert lib.bwpp_hip_tensor_alloc(ctypes.byref(arena), ctypes.byref(t), 2, 0, 2, sh) == \
        bwpp.Status.OUT_OF_MEMORY
    assert arena.offset == 656


def test_tensor_ops_reject_null_handle():
    lib = _lib.load()
    _, t = _init((4, 4))
    assert lib.bwpp_hip_tensor_softmax(None, ctypes.byref(t), ctypes.byref(t)) == bwpp.Status.INVALID_ARG
    assert lib.bwpp_hip_tensor_matmul(None, None, None, None, None, 0) == bwpp.Status.INVALID_ARG


def test_c_caller_builds_and_reports_no_device():
    """The header compiles as C11 with -Wall -Wextra -Wpedantic -Werror and
    the caller links; without a GPU it stops at bwpp_hip_create with
    NO_DEVICE (exit 2)."""
    import torch
    subprocess.run(["make", "-C", os.path.join(ROOT, "tests", "c"), "-B"], check=True,
                   capture_output=True)
    if torch.cuda.is_available():
        pytest.skip("a GPU is visible: tests/test_gpu_tensor.py runs the caller")
    r = subprocess.run([os.path.join(ROOT, "tests", "c", "bwpp_caller")], capture_output=True, text=True)
    assert r.returncode == 2, r.stdout + r.stderr
    assert "no device" in r.stdout
