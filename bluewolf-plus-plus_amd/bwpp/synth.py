"""Seeded synthetic inputs (host numpy arrays) from libbwpp_hip's generator.

Element i of (seed, stream) depends only on (seed, stream, i), so a subset
drawn here equals the same slice of a full-size draw.
"""
from __future__ import annotations

import numpy as np

from . import _lib


def _out(n: int, dtype=np.float32) -> np.ndarray:
    return np.empty(n, dtype=dtype)


def uniform(shape, seed: int, stream: int, lo: float = 0.0, hi: float = 1.0) -> np.ndarray:
    lib = _lib.load()
    n = int(np.prod(shape))
    a = _out(n)
    lib.bwpp_synth_uniform_f32(a.ctypes.data, n, seed, stream, lo, hi)
    return a.reshape(shape)


def normal(shape, seed: int, stream: int, mean: float = 0.0, std: float = 1.0) -> np.ndarray:
    lib = _lib.load()
    n = int(np.prod(shape))
    a = _out(n)
    lib.bwpp_synth_normal_f32(a.ctypes.data, n, seed, stream, mean, std)
    return a.reshape(shape)


def ramp(rows: int, cols: int, scale: float) -> np.ndarray:
    """x[i][j] = (i*cols + j + 1) * scale (runtime/cpu/test_matmul.c:7-13)."""
    lib = _lib.load()
    a = _out(rows * cols)
    lib.bwpp_synth_ramp_f32(a.ctypes.data, rows, cols, scale)
    return a.reshape(rows, cols)


def to_bf16_bits(x: np.ndarray) -> np.ndarray:
    """fp32 -> bf16 bit patterns (uint16), round to nearest even."""
    lib = _lib.load()
    x = np.ascontiguousarray(x, dtype=np.float32)
    out = np.empty(x.shape, dtype=np.uint16)
    lib.bwpp_f32_to_bf16(x.ctypes.data, out.ctypes.data, x.size)
    return out


def bf16_bits_to_f32(h: np.ndarray) -> np.ndarray:
    lib = _lib.load()
    h = np.ascontiguousarray(h, dtype=np.uint16)
    out = np.empty(h.shape, dtype=np.float32)
    lib.bwpp_bf16_to_f32(h.ctypes.data, out.ctypes.data, h.size)
    return out
