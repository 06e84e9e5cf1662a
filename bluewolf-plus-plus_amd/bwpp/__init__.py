"""bwpp -- Python host side of libbwpp_hip, the MI355X backend of BW++.

The compute path is the C library libbwpp_hip.so and its gfx950 code
objects (lib/); this package only binds them.  There is no CPU fallback:
if the library or a code object is missing, HipBackend() raises.
"""
from . import _lib, plan, synth
from ._lib import (AttentionParams, CoreDType, DType, ElementwiseParams, Epilogue, Fusion,
                   FusionParams, LibraryMissing, MatmulParams, MeanSquareParams, ReduceParams,
                   RmsnormParams, SoftmaxParams, Status, Tensor)
from .backend import BwppError, HipBackend, tensor_of

__all__ = ["HipBackend", "BwppError", "LibraryMissing", "Status", "DType",
           "Epilogue", "Fusion", "FusionParams", "MatmulParams", "SoftmaxParams", "RmsnormParams",
           "MeanSquareParams",
           "AttentionParams", "ReduceParams", "ElementwiseParams", "CoreDType", "Tensor",
           "tensor_of", "synth", "plan",
           "load_library"]


def load_library():
    return _lib.load()
