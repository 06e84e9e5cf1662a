"""Python host mirror of libbwpp_hip's operator interface.

`HipBackend.dispatch_*` keep the argument order of the reference's Metal
dispatch functions (runtime/metal/dispatch_stub.h:42-74): buffers first, then
the params struct.  The Metal device/queue pair becomes the backend handle and
the MSL source argument disappears (kernels are prebuilt code objects).
Buffers are torch tensors on the GPU or raw device addresses (int); None is
NULL.  Every call raises BwppError on a non-OK status instead of returning
silently as the Metal stub does (dispatch_stub.m:66-79).
"""
from __future__ import annotations

import ctypes

from . import _lib
from ._lib import (AttentionParams, ElementwiseParams, MatmulParams, ReduceParams,
                   RmsnormParams, SoftmaxParams, Status)


class BwppError(RuntimeError):
    def __init__(self, status: int, message: str):
        self.status = Status(status) if status in Status._value2member_map_ else status
        super().__init__(f"{self.status!s}: {message}")


def _ptr(buf) -> int | None:
    if buf is None:
        return None
    if isinstance(buf, int):
        return buf
    if hasattr(buf, "data_ptr"):
        if not buf.is_cuda:
            raise ValueError("libbwpp_hip operators take device buffers")
        return buf.data_ptr()
    raise TypeError(f"cannot pass {type(buf)!r} as a device buffer")


def tensor_of(t, layout: int = 0) -> "_lib.Tensor":
    """BwppHipTensor describing a torch CUDA tensor (f32 or bf16, its own
    shape and element strides).  layout 1 (column-major) marks a rank-2
    tensor whose storage is the transpose (e.g. `x.t()` of a row-major x)."""
    import torch
    dt = {torch.float32: _lib.CoreDType.F32, torch.bfloat16: _lib.CoreDType.BF16}[t.dtype]
    r = _lib.Tensor()
    r.dtype = int(dt)
    r.layout = layout
    r.rank = t.dim()
    for i in range(t.dim()):
        r.shape[i] = t.shape[i]
        r.stride[i] = t.stride(i)
    r.buffer = t.data_ptr()
    return r


class HipBackend:
    """One libbwpp_hip handle (device, loaded code objects, stream)."""

    def __init__(self, device: int = 0, code_object_dir: str | None = None,
                 stream=None):
        self.lib = _lib.load()
        h = ctypes.c_void_p()
        st = self.lib.bwpp_hip_create(
            ctypes.byref(h), device,
            code_object_dir.encode() if code_object_dir else None)
        if st != 0:
            raise BwppError(st, self.lib.bwpp_hip_last_error(None).decode())
        self._h = h
        self.device = device
        if stream is not None:
            self.set_stream(stream)

    # ------------------------------------------------------------ handle
    def close(self):
        if getattr(self, "_h", None):
            self.lib.bwpp_hip_destroy(self._h)
            self._h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    def _check(self, st: int):
        if st != 0:
            raise BwppError(st, self.lib.bwpp_hip_last_error(self._h).decode())

    def set_stream(self, stream):
        """stream: torch.cuda.Stream, a raw hipStream_t (int) or None."""
        raw = getattr(stream, "cuda_stream", stream)
        self._check(self.lib.bwpp_hip_set_stream(self._h, raw or None))

    def stream(self) -> int:
        return self.lib.bwpp_hip_get_stream(self._h) or 0

    def sync(self):
        self._check(self.lib.bwpp_hip_sync(self._h))

    @property
    def cus(self) -> int:
        return self.lib.bwpp_hip_device_cus(self._h)

    @property
    def last_kernel(self) -> str:
        """Symbol of the last kernel this handle launched ('' if none)."""
        return self.lib.bwpp_hip_last_kernel(self._h).decode()

    def recent_kernel(self, back: int) -> str:
        """Symbol of the launch `back` launches before the last (0..3; '' if none)."""
        return self.lib.bwpp_hip_recent_kernel(self._h, back).decode()

    # --------------------------------------------------------- operators
    def dispatch_matmul(self, a, b, c, bias, params: MatmulParams):
        self._check(self.lib.bwpp_hip_dispatch_matmul(
            self._h, _ptr(a), _ptr(b), _ptr(c), _ptr(bias), params))

    def dispatch_matmul_fused(self, a, b, c, bias, aux, c2, params: MatmulParams, fusion):
        self._check(self.lib.bwpp_hip_dispatch_matmul_fused(
            self._h, _ptr(a), _ptr(b), _ptr(c), _ptr(bias), _ptr(aux), _ptr(c2), params, fusion))

    def dispatch_softmax(self, x, y, params: SoftmaxParams):
        self._check(self.lib.bwpp_hip_dispatch_softmax(
            self._h, _ptr(x), _ptr(y), params))

    def dispatch_rmsnorm(self, x, gamma, beta, y, params: RmsnormParams):
        self._check(self.lib.bwpp_hip_dispatch_rmsnorm(
            self._h, _ptr(x), _ptr(gamma), _ptr(beta), _ptr(y), params))

    def dispatch_layernorm(self, x, gamma, beta, y, params: RmsnormParams):
        self._check(self.lib.bwpp_hip_dispatch_layernorm(
            self._h, _ptr(x), _ptr(gamma), _ptr(beta), _ptr(y), params))

    def dispatch_attention(self, q, k, v, o, params: AttentionParams):
        self._check(self.lib.bwpp_hip_dispatch_attention(
            self._h, _ptr(q), _ptr(k), _ptr(v), _ptr(o), params))

    def dispatch_attention_lse(self, q, k, v, o, lse, params: AttentionParams):
        self._check(self.lib.bwpp_hip_dispatch_attention_lse(
            self._h, _ptr(q), _ptr(k), _ptr(v), _ptr(o), _ptr(lse), params))

    def dispatch_attention_grad(self, q, k, v, o, dout, lse, dq, dk, dv, params: AttentionParams):
        self._check(self.lib.bwpp_hip_dispatch_attention_grad(
            self._h, _ptr(q), _ptr(k), _ptr(v), _ptr(o), _ptr(dout), _ptr(lse),
            _ptr(dq), _ptr(dk), _ptr(dv), params))

    def dispatch_attention_grad_noalloc(self, q, k, v, o, dout, lse, dq, dk, dv, params: AttentionParams):
        self._check(self.lib.bwpp_hip_dispatch_attention_grad_noalloc(
            self._h, _ptr(q), _ptr(k), _ptr(v), _ptr(o), _ptr(dout), _ptr(lse),
            _ptr(dq), _ptr(dk), _ptr(dv), params))

    def dispatch_reduce_max(self, x, maxv, argmax, params: ReduceParams):
        self._check(self.lib.bwpp_hip_dispatch_reduce_max(
            self._h, _ptr(x), _ptr(maxv), _ptr(argmax), params))

    def dispatch_reduce_max_mask(self, x, mask, params: ReduceParams):
        self._check(self.lib.bwpp_hip_dispatch_reduce_max_mask(
            self._h, _ptr(x), _ptr(mask), params))

    def dispatch_reduce_max_grad(self, mask, dy, dx, params: ReduceParams):
        self._check(self.lib.bwpp_hip_dispatch_reduce_max_grad(
            self._h, _ptr(mask), _ptr(dy), _ptr(dx), params))

    def dispatch_reduce_max_grad_argmax(self, x, argmax, dy, dx,
                                        params: ReduceParams):
        self._check(self.lib.bwpp_hip_dispatch_reduce_max_grad_argmax(
            self._h, _ptr(x), _ptr(argmax), _ptr(dy), _ptr(dx), params))

    # ------------------------------------------------------ grad ops / glue
    def dispatch_silu_grad(self, x, dy, dx, n: int):
        self._check(self.lib.bwpp_hip_dispatch_silu_grad(self._h, _ptr(x), _ptr(dy), _ptr(dx), n))

    def dispatch_softmax_grad(self, y, dy, dx, params: SoftmaxParams):
        self._check(self.lib.bwpp_hip_dispatch_softmax_grad(self._h, _ptr(y), _ptr(dy), _ptr(dx), params))

    def dispatch_rmsnorm_grad(self, x, gamma, dy, dx, dgamma, dbeta, params: RmsnormParams):
        self._check(self.lib.bwpp_hip_dispatch_rmsnorm_grad(
            self._h, _ptr(x), _ptr(gamma), _ptr(dy), _ptr(dx), _ptr(dgamma), _ptr(dbeta), params))

    def dispatch_rmsnorm_grad_acc(self, x, gamma, dy, acc, dx, dgamma, dbeta, params: RmsnormParams):
        """dx = acc + rmsnorm_grad(x, gamma, dy); acc may be dx itself."""
        self._check(self.lib.bwpp_hip_dispatch_rmsnorm_grad_acc(
            self._h, _ptr(x), _ptr(gamma), _ptr(dy), _ptr(acc), _ptr(dx), _ptr(dgamma), _ptr(dbeta), params))

    def dispatch_mean_square(self, x, loss_scale, grad_scale, loss, dx, params):
        """loss[0] = loss_scale * sum(x^2); dx = grad_scale * x (scales: device scalars or None = 1)."""
        self._check(self.lib.bwpp_hip_dispatch_mean_square(
            self._h, _ptr(x), _ptr(loss_scale), _ptr(grad_scale), _ptr(loss), _ptr(dx), params))

    def dispatch_reduce_sum(self, x, out, params: ReduceParams):
        self._check(self.lib.bwpp_hip_dispatch_reduce_sum(self._h, _ptr(x), _ptr(out), params))

    # ------------------------------------------------------ tensor forms
    def tensor_matmul(self, a, b, bias, c, epilogue: int = 0):
        ref = lambda t: ctypes.byref(t) if t is not None else None
        self._check(self.lib.bwpp_hip_tensor_matmul(self._h, ref(a), ref(b), ref(bias), ref(c), epilogue))

    def tensor_softmax(self, x, y):
        self._check(self.lib.bwpp_hip_tensor_softmax(self._h, ctypes.byref(x), ctypes.byref(y)))

    def tensor_rmsnorm(self, x, gamma, beta, y, eps: float):
        ref = lambda t: ctypes.byref(t) if t is not None else None
        self._check(self.lib.bwpp_hip_tensor_rmsnorm(self._h, ref(x), ref(gamma), ref(beta), ref(y), eps))

    def tensor_layernorm(self, x, gamma, beta, y, eps: float):
        ref = lambda t: ctypes.byref(t) if t is not None else None
        self._check(self.lib.bwpp_hip_tensor_layernorm(self._h, ref(x), ref(gamma), ref(beta), ref(y), eps))

    def tensor_attention(self, q, k, v, o, scale: float, causal: int):
        self._check(self.lib.bwpp_hip_tensor_attention(self._h, ctypes.byref(q), ctypes.byref(k),
                                                       ctypes.byref(v), ctypes.byref(o), scale, causal))

    def dispatch_elementwise(self, a, b, out, params: ElementwiseParams):
        self._check(self.lib.bwpp_hip_dispatch_elementwise(self._h, _ptr(a), _ptr(b), _ptr(out), params))
