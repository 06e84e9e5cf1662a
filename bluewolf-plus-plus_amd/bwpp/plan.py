"""Launch plans: the executor of lowered BW++ graphs in libbwpp_hip.

A plan (text; format in csrc/runtime/bwpp_plan.cpp) names tensors over bound
dims and lists operator launches.  `Plan` parses it, builds the memory plan
(one device arena, liveness-based buffer reuse) and runs it; inputs and
params are bound to caller device memory, outputs read back by name.
"""
from __future__ import annotations

import ctypes
import os
import re

from . import _lib

PLAN_DIR = os.path.join(os.path.dirname(os.path.dirname(os.path.abspath(__file__))), "plans")


def load_text(name_or_path: str, **dims) -> str:
    """Plan text from plans/<name>.plan (or a path), with `dim` lines
    overridden by the keyword arguments (e.g. B=2, T=64)."""
    path = name_or_path if os.path.sep in name_or_path else os.path.join(PLAN_DIR, name_or_path + ".plan")
    with open(path) as f:
        text = f.read()
    for k, v in dims.items():
        text, n = re.subn(rf"(?m)^dim {re.escape(k)} .*$", f"dim {k} {v}", text)
        if n != 1:
            raise KeyError(f"plan has no single 'dim {k}' line")
    return text


class PlanError(RuntimeError):
    pass


class Plan:
    def __init__(self, backend, text: str):
        """backend: a HipBackend, or None to parse and plan only."""
        self.lib = _lib.load()
        self.backend = backend
        h = ctypes.c_void_p()
        hb = backend._h if backend is not None else None
        st = self.lib.bwpp_hip_plan_create(hb, text.encode(), ctypes.byref(h))
        self._p = h
        if st != 0:
            msg = self.error()
            self.close()
            raise PlanError(f"plan rejected ({st}): {msg}")

    def error(self) -> str:
        return self.lib.bwpp_hip_plan_last_error(self._p).decode() if self._p else ""

    def _check(self, st):
        if st != 0:
            raise PlanError(f"status {st}: {self.error()}")

    @property
    def arena_bytes(self) -> int:
        return self.lib.bwpp_hip_plan_arena_bytes(self._p)

    def report(self) -> str:
        n = self.lib.bwpp_hip_plan_report(self._p, None, 0)
        buf = ctypes.create_string_buffer(n)
        self.lib.bwpp_hip_plan_report(self._p, buf, n)
        return buf.value.decode()

    def allocate(self):
        self._check(self.lib.bwpp_hip_plan_allocate(self._p))

    def bind(self, name: str, tensor):
        self._keep = getattr(self, "_keep", {})
        self._keep[name] = tensor
        self._check(self.lib.bwpp_hip_plan_bind(self._p, name.encode(), tensor.data_ptr()))

    def ptr(self, name: str) -> int:
        p = self.lib.bwpp_hip_plan_value_ptr(self._p, name.encode())
        if not p:
            raise KeyError(name)
        return p

    def host(self, name: str, shape, dtype=None):
        """Copy of a placed value in host memory (numpy; waits for the stream)."""
        import numpy as np
        dtype = np.dtype(dtype or np.float32)
        out = np.empty(shape, dtype=dtype)
        st = self.lib.bwpp_hip_copy_to_host(self.backend._h, out.ctypes.data, self.ptr(name), out.nbytes)
        self._check(st)
        return out

    def run(self):
        self._check(self.lib.bwpp_hip_plan_run(self._p))

    def capture(self):
        """Record one run as a HIP graph (the handle's stream must not be
        the default stream); replay() launches it."""
        self._check(self.lib.bwpp_hip_plan_capture(self._p))

    def replay(self):
        self._check(self.lib.bwpp_hip_plan_replay(self._p))

    def close(self):
        if getattr(self, "_p", None):
            self.lib.bwpp_hip_plan_destroy(self._p)
            self._p = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass
