"""ctypes binding of libbwpp_hip (include/bwpp_hip.h).

The structures mirror the C params structs field for field; their leading
fields are the reference's Metal params structs
(runtime/metal/dispatch_stub.h:9-40), in the same order.
"""
from __future__ import annotations

import ctypes
import enum
import os
from ctypes import (POINTER, Structure, byref, c_char_p, c_float, c_int,
                    c_int32, c_size_t, c_uint16, c_uint32, c_uint64, c_void_p)

PKG_DIR = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
LIB_DIR = os.path.join(PKG_DIR, "lib")
LIB_PATH = os.path.join(LIB_DIR, "libbwpp_hip.so")
REPO_ROOT = os.path.dirname(PKG_DIR)
HEADER_PATH = os.path.join(REPO_ROOT, "include", "bwpp_hip.h")


class Status(enum.IntEnum):
    OK = 0
    ERR = 1
    INVALID_ARG = 2
    HIP = 3
    NO_KERNEL = 4
    ALIAS = 5
    OUT_OF_MEMORY = 6
    UNSUPPORTED = 7
    NO_DEVICE = 8


class DType(enum.IntEnum):
    F32 = 0
    BF16 = 1


class Epilogue(enum.IntEnum):
    NONE = 0
    ADD = 1
    SILU = 2
    ADD_SILU = 3


class MatmulParams(Structure):
    _fields_ = [("M", c_uint32), ("N", c_uint32), ("K", c_uint32),
                ("lda", c_uint32), ("ldb", c_uint32), ("ldc", c_uint32),
                ("dtype", c_uint32), ("epilogue", c_uint32),
                ("trans_a", c_uint32), ("trans_b", c_uint32)]


class Fusion(enum.IntEnum):
    NONE = 0
    RESIDUAL = 1
    DUAL_SILU = 2
    SILU_GRAD = 3


class FusionParams(Structure):
    _fields_ = [("kind", c_uint32), ("ld_aux", c_uint32), ("ld_c2", c_uint32)]


class SoftmaxParams(Structure):
    _fields_ = [("rows", c_uint32), ("cols", c_uint32), ("ld", c_uint32)]


class RmsnormParams(Structure):
    _fields_ = [("rows", c_uint32), ("cols", c_uint32), ("ld", c_uint32),
                ("eps", c_float)]


class MeanSquareParams(Structure):
    _fields_ = [("rows", c_uint32), ("cols", c_uint32), ("ld", c_uint32)]


class AttentionParams(Structure):
    _fields_ = [("M", c_uint32), ("N", c_uint32), ("K", c_uint32),
                ("D", c_uint32), ("ldq", c_uint32), ("ldk", c_uint32),
                ("ldv", c_uint32), ("ldo", c_uint32),
                ("batch", c_uint32), ("heads", c_uint32),
                ("q_batch_stride", c_uint64), ("q_head_stride", c_uint64),
                ("k_batch_stride", c_uint64), ("k_head_stride", c_uint64),
                ("v_batch_stride", c_uint64), ("v_head_stride", c_uint64),
                ("o_batch_stride", c_uint64), ("o_head_stride", c_uint64),
                ("scale", c_float), ("causal", c_uint32), ("dtype", c_uint32)]


class ReduceParams(Structure):
    _fields_ = [("rows", c_uint32), ("cols", c_uint32), ("ld", c_uint32),
                ("axis", c_int32)]


class ElementwiseParams(Structure):
    _fields_ = [("rows", c_uint32), ("cols", c_uint32), ("ld", c_uint32),
                ("op", c_uint32), ("bmode", c_uint32)]


class Arena(Structure):
    _fields_ = [("buffer", c_void_p), ("capacity", c_size_t),
                ("offset", c_size_t), ("device", c_int)]


class CoreDType(enum.IntEnum):
    """runtime/core/tensor.h:7-11 numbering, carried by Tensor.dtype."""
    F16 = 0
    BF16 = 1
    F32 = 2


class Tensor(Structure):
    """BwppHipTensor: runtime/core/tensor.h:18-25 over device memory."""
    _fields_ = [("dtype", ctypes.c_int32), ("layout", ctypes.c_int32), ("rank", c_uint32),
                ("shape", c_uint64 * 4), ("stride", c_uint64 * 4), ("buffer", c_void_p)]


_P = c_void_p
# name -> (restype, argtypes); every function include/bwpp_hip.h declares.
SIGNATURES = {
    "bwpp_hip_create": (c_int, [POINTER(c_void_p), c_int, c_char_p]),
    "bwpp_hip_destroy": (None, [_P]),
    "bwpp_hip_set_stream": (c_int, [_P, _P]),
    "bwpp_hip_get_stream": (_P, [_P]),
    "bwpp_hip_sync": (c_int, [_P]),
    "bwpp_hip_last_error": (c_char_p, [_P]),
    "bwpp_hip_status_string": (c_char_p, [c_int]),
    "bwpp_hip_device_cus": (c_int, [_P]),
    "bwpp_hip_last_kernel": (c_char_p, [_P]),
    "bwpp_hip_recent_kernel": (c_char_p, [_P, c_int]),
    "bwpp_hip_arena_init": (c_int, [_P, POINTER(Arena), c_size_t]),
    "bwpp_hip_arena_reset": (None, [POINTER(Arena)]),
    "bwpp_hip_arena_alloc": (_P, [POINTER(Arena), c_size_t, c_size_t]),
    "bwpp_hip_arena_destroy": (None, [POINTER(Arena)]),
    "bwpp_hip_dtype_from_core": (ctypes.c_int32, [ctypes.c_int32]),
    "bwpp_hip_dtype_from_graph": (ctypes.c_int32, [ctypes.c_int32]),
    "bwpp_hip_dtype_to_core": (ctypes.c_int32, [ctypes.c_int32]),
    "bwpp_hip_dtype_to_graph": (ctypes.c_int32, [ctypes.c_int32]),
    "bwpp_hip_core_dtype_size": (c_size_t, [ctypes.c_int32]),
    "bwpp_hip_tensor_init": (c_int, [POINTER(Tensor), ctypes.c_int32, ctypes.c_int32, c_uint32,
                                     POINTER(c_uint64), _P]),
    "bwpp_hip_tensor_bytes": (c_size_t, [POINTER(Tensor)]),
    "bwpp_hip_tensor_alloc": (c_int, [POINTER(Arena), POINTER(Tensor), ctypes.c_int32, ctypes.c_int32,
                                      c_uint32, POINTER(c_uint64)]),
    "bwpp_hip_tensor_matrix": (c_int, [POINTER(Tensor), POINTER(c_uint32), POINTER(c_uint32),
                                       POINTER(c_uint32)]),
    "bwpp_hip_tensor_matmul": (c_int, [_P, POINTER(Tensor), POINTER(Tensor), POINTER(Tensor),
                                       POINTER(Tensor), c_uint32]),
    "bwpp_hip_tensor_softmax": (c_int, [_P, POINTER(Tensor), POINTER(Tensor)]),
    "bwpp_hip_tensor_rmsnorm": (c_int, [_P, POINTER(Tensor), POINTER(Tensor), POINTER(Tensor),
                                        POINTER(Tensor), c_float]),
    "bwpp_hip_tensor_layernorm": (c_int, [_P, POINTER(Tensor), POINTER(Tensor), POINTER(Tensor),
                                          POINTER(Tensor), c_float]),
    "bwpp_hip_tensor_attention": (c_int, [_P, POINTER(Tensor), POINTER(Tensor), POINTER(Tensor),
                                          POINTER(Tensor), c_float, c_uint32]),
    "bwpp_hip_copy_to_device": (c_int, [_P, _P, _P, c_size_t]),
    "bwpp_hip_copy_to_host": (c_int, [_P, _P, _P, c_size_t]),
    "bwpp_hip_plan_create": (c_int, [_P, c_char_p, POINTER(c_void_p)]),
    "bwpp_hip_plan_destroy": (None, [_P]),
    "bwpp_hip_plan_last_error": (c_char_p, [_P]),
    "bwpp_hip_plan_arena_bytes": (c_size_t, [_P]),
    "bwpp_hip_plan_allocate": (c_int, [_P]),
    "bwpp_hip_plan_bind": (c_int, [_P, c_char_p, _P]),
    "bwpp_hip_plan_value_ptr": (_P, [_P, c_char_p]),
    "bwpp_hip_plan_run": (c_int, [_P]),
    "bwpp_hip_plan_capture": (c_int, [_P]),
    "bwpp_hip_plan_replay": (c_int, [_P]),
    "bwpp_hip_plan_report": (c_size_t, [_P, c_char_p, c_size_t]),
    "bwpp_hip_dispatch_matmul": (c_int, [_P, _P, _P, _P, _P, MatmulParams]),
    "bwpp_hip_dispatch_matmul_fused": (c_int, [_P, _P, _P, _P, _P, _P, _P, MatmulParams, FusionParams]),
    "bwpp_hip_dispatch_softmax": (c_int, [_P, _P, _P, SoftmaxParams]),
    "bwpp_hip_dispatch_rmsnorm": (c_int, [_P, _P, _P, _P, _P, RmsnormParams]),
    "bwpp_hip_dispatch_layernorm": (c_int, [_P, _P, _P, _P, _P, RmsnormParams]),
    "bwpp_hip_dispatch_attention": (c_int, [_P, _P, _P, _P, _P, AttentionParams]),
    "bwpp_hip_dispatch_attention_lse": (c_int, [_P, _P, _P, _P, _P, _P, AttentionParams]),
    "bwpp_hip_dispatch_attention_grad": (c_int, [_P, _P, _P, _P, _P, _P, _P, _P, _P, _P, AttentionParams]),
    "bwpp_hip_dispatch_attention_grad_noalloc": (c_int, [_P, _P, _P, _P, _P, _P, _P, _P, _P, _P,
                                                         AttentionParams]),
    "bwpp_hip_dispatch_reduce_max": (c_int, [_P, _P, _P, _P, ReduceParams]),
    "bwpp_hip_dispatch_reduce_max_mask": (c_int, [_P, _P, _P, ReduceParams]),
    "bwpp_hip_dispatch_reduce_max_grad": (c_int, [_P, _P, _P, _P, ReduceParams]),
    "bwpp_hip_dispatch_reduce_max_grad_argmax": (c_int, [_P, _P, _P, _P, _P, ReduceParams]),
    "bwpp_hip_dispatch_silu_grad": (c_int, [_P, _P, _P, _P, c_uint64]),
    "bwpp_hip_dispatch_softmax_grad": (c_int, [_P, _P, _P, _P, SoftmaxParams]),
    "bwpp_hip_dispatch_rmsnorm_grad": (c_int, [_P, _P, _P, _P, _P, _P, _P, RmsnormParams]),
    "bwpp_hip_dispatch_rmsnorm_grad_acc": (c_int, [_P, _P, _P, _P, _P, _P, _P, _P, RmsnormParams]),
    "bwpp_hip_dispatch_mean_square": (c_int, [_P, _P, _P, _P, _P, _P, MeanSquareParams]),
    "bwpp_hip_dispatch_reduce_sum": (c_int, [_P, _P, _P, ReduceParams]),
    "bwpp_hip_dispatch_elementwise": (c_int, [_P, _P, _P, _P, ElementwiseParams]),
    "bwpp_synth_uniform_f32": (None, [_P, c_uint64, c_uint64, c_uint64, c_float, c_float]),
    "bwpp_synth_normal_f32": (None, [_P, c_uint64, c_uint64, c_uint64, c_float, c_float]),
    "bwpp_synth_ramp_f32": (None, [_P, c_uint32, c_uint32, c_float]),
    "bwpp_f32_to_bf16": (None, [_P, _P, c_uint64]),
    "bwpp_bf16_to_f32": (None, [_P, _P, c_uint64]),
}

_lib = None


class LibraryMissing(RuntimeError):
    pass


def load():
    """Load libbwpp_hip.so from the package's lib/ directory (no fallback)."""
    global _lib
    if _lib is not None:
        return _lib
    try:
        # torch ships its own HIP runtime under the same soname; loading torch
        # first makes libbwpp_hip bind to that one, so device pointers and
        # streams from torch are valid in the library.
        import torch  # noqa: F401
    except ImportError:
        pass
    if not os.path.exists(LIB_PATH):
        raise LibraryMissing(
            f"{LIB_PATH} is not built; run `make -C {PKG_DIR}` or "
            "__graft_entry__.build()")
    lib = ctypes.CDLL(LIB_PATH)
    for name, (res, args) in SIGNATURES.items():
        fn = getattr(lib, name, None)
        if fn is None:
            continue  # reported by the export test; not fatal for loading
        fn.restype = res
        fn.argtypes = args
    _lib = lib
    return lib


__all__ = ["Status", "DType", "Epilogue", "MatmulParams", "Fusion", "FusionParams", "SoftmaxParams",
           "RmsnormParams", "MeanSquareParams", "AttentionParams", "ReduceParams", "ElementwiseParams", "Arena",
           "CoreDType", "Tensor",
           "SIGNATURES", "load", "LIB_PATH", "LIB_DIR", "HEADER_PATH",
           "LibraryMissing", "byref", "c_void_p", "c_uint16"]
