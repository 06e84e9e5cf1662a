"""Python binding of the CPU parity oracle.

TEST INFRASTRUCTURE ONLY: imported by tests/, __graft_entry__.smoke() and the
cpu_baseline leg of bench.py, as the checker or the timed CPU baseline.  The
shipped library never loads it.

Two shared libraries are wrapped:
  * libbwpp_oracle.so -- this repo's C restatement (bwpp_oracle.c);
  * _ref/libbwpp_cpu_ref.so -- the reference's runtime/cpu/bwpp_cpu_ref.c
    compiled as is by `make -C oracle ref` (absent if it was never built).
All arrays are numpy float32 (int32 for indices), row-major; a 2-D array
may have a row stride larger than its width (passed as ld).
"""
from __future__ import annotations

import ctypes
import os
from ctypes import c_float, c_int, c_uint16, c_uint32, c_uint64, c_void_p

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
ORACLE_SO = os.path.join(HERE, "libbwpp_oracle.so")
REF_SO = os.path.join(HERE, "_ref", "libbwpp_cpu_ref.so")

_P = c_void_p
_U = c_uint32

_ORACLE_SIGS = {
    "oracle_matmul_f32": [_P, _P, _P, _U, _U, _U, _U, _U, _U, _P, c_int, c_int],
    "oracle_matmul_ex_f32": [_P, _P, _P, _U, _U, _U, _U, _U, _U, c_int, c_int, _P, c_int, c_int],
    "oracle_softmax_f32": [_P, _P, _U, _U, _U],
    "oracle_rmsnorm_f32": [_P, _P, _P, _P, _U, _U, _U, c_float],
    "oracle_layernorm_f32": [_P, _P, _P, _P, _U, _U, _U, c_float],
    "oracle_attention_f32": [_P, _P, _P, _P, _U, _U, _U, _U, _U, _U, _U, _U],
    "oracle_attention_lse_f32": [_P, _P, _P, _U, _U, _U, _U, _U, ctypes.c_float, ctypes.c_int],
    "oracle_attention_grad_f32": [_P, _P, _P, _P, _P, _P, _P, _U, _U, _U, _U, _U, _U, ctypes.c_float,
                                  ctypes.c_int],
    "oracle_attention_bh_f32": [_P, _P, _P, _P, _U, _U, _U, _U, _U, _U, _U, _U, _U, _U,
                                c_uint64, c_uint64, c_uint64, c_uint64, c_uint64, c_uint64,
                                c_uint64, c_uint64, c_float, c_int],
    "oracle_reduce_max_mask_f32": [_P, _P, _U, _U, c_int],
    "oracle_reduce_max_grad_mask_f32": [_P, _P, _P, _U, _U, c_int],
    "oracle_reduce_max_f32": [_P, _P, _P, _U, _U, _U, c_int],
    "oracle_reduce_max_grad_f32": [_P, _P, _P, _P, _U, _U, _U, c_int],
    "oracle_silu_grad_f32": [_P, _P, _P, c_uint64],
    "oracle_softmax_grad_f32": [_P, _P, _P, _U, _U, _U],
    "oracle_rmsnorm_grad_f32": [_P, _P, _P, _P, _P, _P, _U, _U, _U, c_float],
    "oracle_reduce_sum_f32": [_P, _P, _U, _U, _U, c_int],
    "oracle_round_bf16_f32": [_P, _P, c_uint64],
}

_REF_SIGS = {
    "bwpp_cpu_matmul_f32": [_P, _P, _P, _U, _U, _U, _U, _U, _U, _P, c_int, c_int],
    "bwpp_cpu_softmax_f32": [_P, _P, _U, _U, _U],
    "bwpp_cpu_rmsnorm_f32": [_P, _P, _P, _P, _U, _U, _U, c_float],
    "bwpp_cpu_attention_f32": [_P, _P, _P, _P, _U, _U, _U, _U, _U, _U, _U, _U],
    "bwpp_cpu_reduce_max_mask_f32": [_P, _P, _U, _U, c_int],
    "bwpp_cpu_reduce_max_grad_f32": [_P, _P, _P, _U, _U, c_int],
}


def _load(path, sigs, ret):
    lib = ctypes.CDLL(path)
    for name, args in sigs.items():
        fn = getattr(lib, name)
        fn.argtypes = args
        fn.restype = ret
    return lib


def _p(a):
    return None if a is None else a.ctypes.data


def _f32(a):
    return None if a is None else np.ascontiguousarray(a, dtype=np.float32)


def _ld(a: np.ndarray) -> int:
    """Row stride in elements of a 2-D float32 array with unit inner stride."""
    assert a.ndim == 2 and a.dtype == np.float32 and a.strides[1] == 4
    return a.strides[0] // 4


def _base(a: np.ndarray) -> np.ndarray:
    assert a.flags.c_contiguous or (a.ndim == 2 and a.strides[1] == 4)
    return a


def _like(a: np.ndarray) -> np.ndarray:
    """Output with the same shape and row stride as `a` (2-D)."""
    if a.flags.c_contiguous:
        return np.zeros_like(a)
    ld = _ld(a)
    buf = np.zeros((a.shape[0], ld), dtype=np.float32)
    return buf[:, : a.shape[1]]


class Oracle:
    """This repo's C restatement (bit-identical to the reference where it
    restates it)."""

    def __init__(self, path: str = ORACLE_SO):
        if not os.path.exists(path):
            raise FileNotFoundError(f"{path} not built; run `make -C {HERE}`")
        self.lib = _load(path, _ORACLE_SIGS, c_int)
        self.lib.oracle_f32_to_bf16.argtypes = [c_float]
        self.lib.oracle_f32_to_bf16.restype = c_uint16
        self.lib.oracle_bf16_to_f32.argtypes = [c_uint16]
        self.lib.oracle_bf16_to_f32.restype = c_float

    # -- restatements ------------------------------------------------------
    def matmul(self, a, b, bias=None, apply_silu=False, apply_bias=False,
               trans_a=False, trans_b=False):
        a = _base(a)
        b = _base(b)
        M = a.shape[1] if trans_a else a.shape[0]
        K = a.shape[0] if trans_a else a.shape[1]
        N = b.shape[0] if trans_b else b.shape[1]
        c = np.zeros((M, N), dtype=np.float32)
        rc = self.lib.oracle_matmul_ex_f32(
            _p(a), _p(b), _p(c), M, N, K, _ld(a), _ld(b), N, int(trans_a),
            int(trans_b), _p(_f32(bias)), int(apply_silu), int(apply_bias))
        assert rc == 0
        return c

    def softmax(self, x):
        y = _like(x)
        assert self.lib.oracle_softmax_f32(_p(x), _p(y), x.shape[0], x.shape[1], _ld(x)) == 0
        return y

    def rmsnorm(self, x, gamma=None, beta=None, eps=1e-5):
        y = _like(x)
        assert self.lib.oracle_rmsnorm_f32(_p(x), _p(y), _p(_f32(gamma)), _p(_f32(beta)),
                                           x.shape[0], x.shape[1], _ld(x), eps) == 0
        return y

    def layernorm(self, x, gamma=None, beta=None, eps=1e-5):
        y = _like(x)
        assert self.lib.oracle_layernorm_f32(_p(x), _p(y), _p(_f32(gamma)), _p(_f32(beta)),
                                             x.shape[0], x.shape[1], _ld(x), eps) == 0
        return y

    def attention(self, q, k, v):
        """Reference single-head attention, bwpp_cpu_ref.c:92-144."""
        M, K = q.shape
        N, D = v.shape
        o = np.zeros((M, D), dtype=np.float32)
        assert self.lib.oracle_attention_f32(_p(q), _p(k), _p(v), _p(o), M, N, K, D,
                                             _ld(q), _ld(k), _ld(v), D) == 0
        return o

    def attention_bh(self, q, k, v, scale=1.0, causal=False):
        """q [B,H,M,K], k [B,H,N,K], v [B,H,N,D] contiguous float32."""
        q, k, v = (np.ascontiguousarray(t, dtype=np.float32) for t in (q, k, v))
        B, H, M, K = q.shape
        N, D = v.shape[2], v.shape[3]
        o = np.zeros((B, H, M, D), dtype=np.float32)
        rc = self.lib.oracle_attention_bh_f32(
            _p(q), _p(k), _p(v), _p(o), B, H, M, N, K, D, K, K, D, D,
            H * M * K, M * K, H * N * K, N * K, H * N * D, N * D, H * M * D, M * D,
            scale, int(causal))
        assert rc == 0
        return o

    def attention_lse(self, q, k, scale=1.0, causal=False):
        """Per-query natural-log LSE of the scaled scores, [B,H,M]."""
        q, k = (np.ascontiguousarray(t, dtype=np.float32) for t in (q, k))
        B, H, M, K = q.shape
        N = k.shape[2]
        lse = np.zeros((B, H, M), dtype=np.float32)
        assert self.lib.oracle_attention_lse_f32(_p(q), _p(k), _p(lse), B, H, M, N, K, scale, int(causal)) == 0
        return lse

    def attention_grad(self, q, k, v, dout, scale=1.0, causal=False):
        """(dq, dk, dv) of attention_bh for upstream gradient dout."""
        q, k, v, dout = (np.ascontiguousarray(t, dtype=np.float32) for t in (q, k, v, dout))
        B, H, M, K = q.shape
        N, D = v.shape[2], v.shape[3]
        dq, dk, dv = np.zeros_like(q), np.zeros_like(k), np.zeros_like(v)
        assert self.lib.oracle_attention_grad_f32(_p(q), _p(k), _p(v), _p(dout), _p(dq), _p(dk), _p(dv),
                                                  B, H, M, N, K, D, scale, int(causal)) == 0
        return dq, dk, dv

    def reduce_max_mask(self, x, axis=1):
        x = np.ascontiguousarray(x, dtype=np.float32)
        m = np.zeros_like(x)
        assert self.lib.oracle_reduce_max_mask_f32(_p(x), _p(m), x.shape[0], x.shape[1], axis) == 0
        return m

    def reduce_max_grad_mask(self, mask, dy, axis=1):
        mask = np.ascontiguousarray(mask, dtype=np.float32)
        dx = np.zeros_like(mask)
        assert self.lib.oracle_reduce_max_grad_mask_f32(
            _p(mask), _p(_f32(dy)), _p(dx), mask.shape[0], mask.shape[1], axis) == 0
        return dx

    # -- extensions ---------------------------------------------------------
    def reduce_max(self, x, axis=1):
        rows, cols = x.shape
        n = cols if axis == 0 else rows
        mv = np.zeros(n, dtype=np.float32)
        ix = np.zeros(n, dtype=np.int32)
        assert self.lib.oracle_reduce_max_f32(_p(x), _p(mv), _p(ix), rows, cols, _ld(x), axis) == 0
        return mv, ix

    def reduce_max_grad(self, dy, shape, x=None, argmax=None, axis=1):
        rows, cols = shape
        dx = np.zeros((rows, cols), dtype=np.float32)
        ld = _ld(x) if x is not None else cols
        if x is not None and ld != cols:
            dx = np.zeros((rows, ld), dtype=np.float32)[:, :cols]
        ix = None if argmax is None else np.ascontiguousarray(argmax, dtype=np.int32)
        assert self.lib.oracle_reduce_max_grad_f32(_p(x), _p(ix), _p(_f32(dy)), _p(dx),
                                                   rows, cols, ld, axis) == 0
        return dx

    def silu_grad(self, x, dy):
        x = _f32(x)
        dy = _f32(dy)
        dx = np.zeros_like(x)
        assert self.lib.oracle_silu_grad_f32(_p(x), _p(dy), _p(dx), x.size) == 0
        return dx

    def softmax_grad(self, y, dy):
        y = _f32(y)
        dy = _f32(dy)
        dx = np.zeros_like(y)
        assert self.lib.oracle_softmax_grad_f32(_p(y), _p(dy), _p(dx), y.shape[0], y.shape[1],
                                                y.shape[1]) == 0
        return dx

    def rmsnorm_grad(self, x, gamma, dy, eps=1e-5):
        x = _f32(x)
        dy = _f32(dy)
        rows, cols = x.shape
        dx = np.zeros_like(x)
        dg = np.zeros(cols, dtype=np.float32)
        db = np.zeros(cols, dtype=np.float32)
        assert self.lib.oracle_rmsnorm_grad_f32(_p(x), _p(_f32(gamma)), _p(dy), _p(dx), _p(dg),
                                                _p(db), rows, cols, cols, eps) == 0
        return dx, dg, db

    def reduce_sum(self, x, axis):
        x = _f32(x)
        rows, cols = x.shape
        out = np.zeros(cols if axis == 0 else rows, dtype=np.float32)
        assert self.lib.oracle_reduce_sum_f32(_p(x), _p(out), rows, cols, cols, axis) == 0
        return out

    def round_bf16(self, x):
        x = _f32(x)
        y = np.empty_like(x)
        self.lib.oracle_round_bf16_f32(_p(x), _p(y), x.size)
        return y

    def f32_to_bf16(self, v: float) -> int:
        return self.lib.oracle_f32_to_bf16(v)


class RefLib:
    """The reference's own bwpp_cpu_ref.c, compiled unchanged into oracle/_ref."""

    def __init__(self, path: str = REF_SO):
        if not os.path.exists(path):
            raise FileNotFoundError(path)
        self.lib = _load(path, _REF_SIGS, None)

    @staticmethod
    def available(path: str = REF_SO) -> bool:
        return os.path.exists(path)

    def matmul(self, a, b, bias=None, apply_silu=False, apply_bias=False):
        M, K = a.shape
        N = b.shape[1]
        c = np.zeros((M, N), dtype=np.float32)
        self.lib.bwpp_cpu_matmul_f32(_p(a), _p(b), _p(c), M, N, K, _ld(a), _ld(b), N,
                                     _p(_f32(bias)), int(apply_silu), int(apply_bias))
        return c

    def softmax(self, x):
        y = _like(x)
        self.lib.bwpp_cpu_softmax_f32(_p(x), _p(y), x.shape[0], x.shape[1], _ld(x))
        return y

    def rmsnorm(self, x, gamma=None, beta=None, eps=1e-5):
        y = _like(x)
        self.lib.bwpp_cpu_rmsnorm_f32(_p(x), _p(y), _p(_f32(gamma)), _p(_f32(beta)),
                                      x.shape[0], x.shape[1], _ld(x), eps)
        return y

    def attention(self, q, k, v):
        M, K = q.shape
        N, D = v.shape
        o = np.zeros((M, D), dtype=np.float32)
        self.lib.bwpp_cpu_attention_f32(_p(q), _p(k), _p(v), _p(o), M, N, K, D,
                                        _ld(q), _ld(k), _ld(v), D)
        return o

    def reduce_max_mask(self, x, axis=1):
        x = np.ascontiguousarray(x, dtype=np.float32)
        m = np.zeros_like(x)
        self.lib.bwpp_cpu_reduce_max_mask_f32(_p(x), _p(m), x.shape[0], x.shape[1], axis)
        return m

    def reduce_max_grad_mask(self, mask, dy, axis=1):
        mask = np.ascontiguousarray(mask, dtype=np.float32)
        dx = np.zeros_like(mask)
        self.lib.bwpp_cpu_reduce_max_grad_f32(_p(mask), _p(_f32(dy)), _p(dx),
                                              mask.shape[0], mask.shape[1], axis)
        return dx
