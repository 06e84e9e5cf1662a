"""libbwpp_hip's C ABI without a GPU: the library loads, exports every
function include/bwpp_hip.h declares, rejects bad calls with a status, and its
host-side synthetic-input generator is deterministic and subset-stable."""
import ctypes
import re

import numpy as np
import pytest

import bwpp
from bwpp import _lib


def _header_functions():
    src = open(_lib.HEADER_PATH).read()
    src = re.sub(r"/\*.*?\*/", "", src, flags=re.S)
    src = re.sub(r"//[^\n]*", "", src)
    return sorted(set(re.findall(r"\b(bwpp_[a-z0-9_]+)\s*\(", src)))


def test_header_declares_expected_surface():
    names = _header_functions()
    for must in ("bwpp_hip_create", "bwpp_hip_dispatch_matmul", "bwpp_hip_dispatch_softmax",
                 "bwpp_hip_dispatch_rmsnorm", "bwpp_hip_dispatch_layernorm",
                 "bwpp_hip_dispatch_attention", "bwpp_hip_dispatch_reduce_max",
                 "bwpp_hip_dispatch_reduce_max_grad", "bwpp_hip_arena_alloc"):
        assert must in names


def test_library_exports_every_declared_function():
    lib = _lib.load()
    missing = [n for n in _header_functions() if not hasattr(lib, n)]
    assert not missing, missing
    # and the binding declares a prototype for each of them
    assert set(_header_functions()) <= set(_lib.SIGNATURES)


def test_struct_layouts_match_header():
    """Sizes of the ctypes mirrors equal the C structs' (natural alignment)."""
    assert ctypes.sizeof(bwpp.MatmulParams) == 40
    assert ctypes.sizeof(bwpp.SoftmaxParams) == 12
    assert ctypes.sizeof(bwpp.RmsnormParams) == 16
    assert ctypes.sizeof(bwpp.ReduceParams) == 16
    assert ctypes.sizeof(bwpp.AttentionParams) == 4 * 10 + 8 * 8 + 4 * 3 + 4  # tail padding
    assert bwpp.AttentionParams.scale.offset == 104


def test_status_strings():
    lib = _lib.load()
    for s in bwpp.Status:
        assert lib.bwpp_hip_status_string(int(s))
    assert lib.bwpp_hip_status_string(0) == b"ok"


def test_null_handle_is_rejected():
    lib = _lib.load()
    p = bwpp.SoftmaxParams(2, 4, 4)
    assert lib.bwpp_hip_dispatch_softmax(None, None, None, p) == bwpp.Status.INVALID_ARG
    assert lib.bwpp_hip_sync(None) == bwpp.Status.INVALID_ARG
    assert lib.bwpp_hip_set_stream(None, None) == bwpp.Status.INVALID_ARG
    arena = bwpp._lib.Arena()
    assert lib.bwpp_hip_arena_init(None, ctypes.byref(arena), 1024) == bwpp.Status.INVALID_ARG
    assert lib.bwpp_hip_arena_alloc(ctypes.byref(arena), 16, 16) is None


def test_create_without_device_fails_loudly():
    import torch
    if torch.cuda.is_available():
        pytest.skip("a GPU is visible")
    with pytest.raises(bwpp.BwppError) as e:
        bwpp.HipBackend(0)
    assert e.value.status == bwpp.Status.NO_DEVICE


def test_create_out_null():
    lib = _lib.load()
    assert lib.bwpp_hip_create(None, 0, None) == bwpp.Status.INVALID_ARG


def test_synth_deterministic_and_subset_stable():
    from bwpp import synth
    a = synth.normal((1000,), seed=3, stream=1)
    b = synth.normal((1000,), seed=3, stream=1)
    c = synth.normal((10,), seed=3, stream=1)
    d = synth.normal((1000,), seed=3, stream=2)
    assert np.array_equal(a, b) and np.array_equal(a[:10], c)
    assert not np.array_equal(a, d)
    big = synth.normal((200000,), seed=0, stream=0)
    assert abs(big.mean()) < 0.01 and abs(big.std() - 1) < 0.01
    u = synth.uniform((200000,), seed=0, stream=5, lo=-1, hi=1)
    assert u.min() >= -1 and u.max() < 1 and abs(u.mean()) < 0.01


def test_synth_ramp_matches_reference_fixture():
    from bwpp import synth
    r = synth.ramp(2, 3, 0.5)
    assert np.array_equal(r, np.array([[0.5, 1, 1.5], [2, 2.5, 3]], np.float32))


def test_bf16_conversion_matches_torch(oracle):
    import torch
    from bwpp import synth
    x = np.concatenate([np.random.default_rng(0).normal(size=5000).astype(np.float32),
                        np.array([0x3F808000, 0x3F818000, 0x7F7F8000], np.uint32).view(np.float32),
                        np.array([np.inf, -np.inf, 0.0, -0.0, 1e-40], np.float32)])
    bits = synth.to_bf16_bits(x)
    want = torch.from_numpy(x).to(torch.bfloat16).view(torch.int16).numpy().view(np.uint16)
    assert np.array_equal(bits, want)
    back = synth.bf16_bits_to_f32(bits)
    assert np.array_equal(back, oracle.round_bf16(x))
