"""CPU executor of launch-plan text over the oracle.

TEST INFRASTRUCTURE ONLY: imported by tests/ (as the checker of plans run on
the GPU) and by bench.py's cpu_baseline legs (the oracle composing config
5's block step for one sample).  The shipped library never loads it.

It reads the same text libbwpp_hip's executor runs (format documented in
bluewolf-plus-plus_amd/csrc/runtime/bwpp_plan.cpp: `dim`, `value`, `view`,
`op` lines) and computes every op with this repo's C restatement of the
reference's CPU kernels (oracle/bwpp_oracle.c, following
runtime/cpu/bwpp_cpu_ref.c) or, for the graph's elementwise glue
(graph_ir.c:697-770, 1585-1654), numpy float32 arithmetic, which rounds each
add / sub / mul / div exactly as IEEE single precision.  Nothing is fused or
reordered: each op is one oracle call in plan order.
"""
from __future__ import annotations

import numpy as np
from numpy.lib.stride_tricks import as_strided

from .oracle import Oracle


class PlanTextError(ValueError):
    pass


def _tokens(line):
    out, cur, depth = [], "", 0
    for c in line:
        if c == "[":
            depth += 1
        if c == "]":
            depth -= 1
        if c in " \t" and depth == 0:
            if cur:
                out.append(cur)
            cur = ""
        else:
            cur += c
    if cur:
        out.append(cur)
    return out


class CpuPlan:
    """Parses plan text; bind() inputs and params as numpy arrays, run(),
    then get() any value as a [rows, cols] float32 matrix."""

    def __init__(self, text: str, oracle: Oracle | None = None):
        self.orc = oracle or Oracle()
        self.dims: dict[str, int] = {}
        self.vals: dict[str, dict] = {}
        self.ops: list[tuple[str, list[str], list[str], dict, int]] = []
        self.store: dict[str, np.ndarray] = {}
        self._parse(text)

    # -- parsing -----------------------------------------------------------
    def _eval(self, e: str) -> int:
        n = 1
        for t in e.split("*"):
            t = t.strip()
            if t.isdigit():
                n *= int(t)
            elif t in self.dims:
                n *= self.dims[t]
            else:
                raise PlanTextError(f"unknown dim '{t}'")
        return n

    def _num(self, s: str) -> float:
        """An attribute: a product of integers and dims, else a float."""
        try:
            return float(self._eval(s))
        except PlanTextError:
            return float(s)

    def _parse(self, text):
        header = False
        for ln, raw in enumerate(text.splitlines(), 1):
            line = raw.split("#", 1)[0].strip()
            if not line:
                continue
            t = _tokens(line)
            if not header:
                if t != ["bwpp.plan", "1"]:
                    raise PlanTextError(f"line {ln}: expected 'bwpp.plan 1'")
                header = True
                continue
            if t[0] == "dim":
                self.dims[t[1]] = self._eval(t[2])
            elif t[0] == "value":
                name, dt, shape, kind = t[1], t[2], t[3], t[4]
                if dt != "f32":
                    raise PlanTextError(f"line {ln}: the CPU executor runs f32 plans only")
                inner = shape[1:-1].strip()
                dims = [self._eval(d) for d in inner.split(",")] if inner else []
                v = {"dims": dims, "kind": kind}
                if kind.startswith("const="):
                    c = kind[6:]
                    num, _, den = c.partition("/")
                    v["const"] = float(num) / (self._eval(den) if den else 1)
                    v["kind"] = "const"
                self.vals[name] = v
            elif t[0] == "view":
                kv = dict(x.split("=", 1) for x in t[2:])
                inner = kv["shape"][1:-1]
                self.vals[t[1]] = {"kind": "view", "of": kv["of"], "offset": self._eval(kv["offset"]),
                                   "ld": self._eval(kv["ld"]), "dims": [self._eval(d) for d in inner.split(",")]}
            elif t[0] == "op":
                kv = dict(x.split("=", 1) for x in t[2:])
                outs = kv.pop("out").split(",")
                ins = kv.pop("in").split(",")
                self.ops.append((t[1], outs, ins, kv, ln))
            else:
                raise PlanTextError(f"line {ln}: unknown statement '{t[0]}'")
        for name, v in self.vals.items():
            if v["kind"] in ("temp", "output", "const"):
                n = int(np.prod(v["dims"])) if v["dims"] else 1
                self.store[name] = np.full(n, v.get("const", 0.0), dtype=np.float32)

    # -- storage -----------------------------------------------------------
    def bind(self, name: str, array: np.ndarray):
        v = self.vals[name]
        if v["kind"] not in ("input", "param"):
            raise PlanTextError(f"'{name}' is not an input or param")
        a = np.ascontiguousarray(array, dtype=np.float32).reshape(-1)
        n = int(np.prod(v["dims"])) if v["dims"] else 1
        if a.size != n:
            raise PlanTextError(f"'{name}' needs {n} elements, got {a.size}")
        self.store[name] = a

    def mat(self, name: str) -> np.ndarray:
        """[rows, cols] float32 view of a value (cols = last dim); writes go
        through to the value's storage."""
        v = self.vals[name]
        dims = v["dims"]
        cols = dims[-1] if dims else 1
        rows = int(np.prod(dims)) // cols if dims else 1
        if v["kind"] == "view":
            base = self.store[v["of"]]
            need = v["offset"] + (rows - 1) * v["ld"] + cols
            if need > base.size:
                raise PlanTextError(f"view '{name}' runs past '{v['of']}'")
            return as_strided(base[v["offset"]:], shape=(rows, cols), strides=(v["ld"] * 4, 4))
        return self.store[name].reshape(rows, cols)

    def get(self, name: str) -> np.ndarray:
        return np.array(self.mat(name))

    # -- execution ---------------------------------------------------------
    def run(self):
        for kind, outs, ins, kv, ln in self.ops:
            try:
                self._op(kind, outs, ins, kv)
            except PlanTextError:
                raise
            except Exception as e:  # name the line that failed
                raise PlanTextError(f"line {ln} ({kind}): {e}") from e

    def _op(self, k, outs, ins, kv):
        o, m = self.orc, self.mat
        X = [m(n) for n in ins]
        if k == "matmul":
            ta, tb = int(kv.get("ta", 0)), int(kv.get("tb", 0))
            epi = kv.get("epi", "none")
            fuse = kv.get("fuse", "none")
            has_bias = epi in ("add", "add_silu") if fuse != "none" else len(X) > 2
            bias = X[2].reshape(-1) if has_bias else None
            r = o.matmul(X[0], X[1], bias, apply_silu=epi in ("silu", "add_silu"),
                         apply_bias=epi in ("add", "add_silu"), trans_a=bool(ta), trans_b=bool(tb))
            # fused tails, each the separate op it replaces
            if fuse == "residual":
                r = np.add(r, X[-1], dtype=np.float32)
            elif fuse == "silu_grad":
                r = o.silu_grad(np.ascontiguousarray(X[-1]), r).reshape(r.shape)
            elif fuse == "dual_silu":
                with np.errstate(all="ignore"):
                    m(outs[1])[...] = (r / (np.float32(1) + np.exp(-r))).astype(np.float32)
            elif fuse != "none":
                raise PlanTextError(f"unknown fuse '{fuse}'")
            m(outs[0])[...] = r
        elif k == "softmax":
            m(outs[0])[...] = o.softmax(np.ascontiguousarray(X[0]))
        elif k in ("rmsnorm", "layernorm"):
            g = X[1].reshape(-1) if len(X) > 1 else None
            b = X[2].reshape(-1) if len(X) > 2 else None
            fn = o.rmsnorm if k == "rmsnorm" else o.layernorm
            m(outs[0])[...] = fn(np.ascontiguousarray(X[0]), g, b, float(kv.get("eps", 1e-5)))
        elif k == "copy" and len(outs) > 1:  # pair i: in[i] -> out[i]
            assert len(X) == len(outs) <= 4 and kv.get("bcast", "full") == "full"
            for i, o_name in enumerate(outs):
                m(o_name)[...] = X[i].reshape(m(o_name).shape)
        elif k in ("add", "sub", "mul", "div", "copy", "silu"):
            out = m(outs[0])
            bv = X[-1]
            bm = kv.get("bcast", "full")
            if bm == "row":
                bv = bv.reshape(1, -1)
            elif bm == "col":
                bv = bv.reshape(-1, 1)
            elif bm == "scalar":
                bv = bv.reshape(-1)[:1].reshape(1, 1)
            with np.errstate(all="ignore"):
                if k == "copy":
                    out[...] = bv
                elif k == "silu":
                    out[...] = (bv / (np.float32(1) + np.exp(-bv))).astype(np.float32)
                else:
                    a = X[0]
                    f = {"add": np.add, "sub": np.subtract, "mul": np.multiply, "div": np.divide}[k]
                    out[...] = f(a, bv, dtype=np.float32)
        elif k == "reduce_sum":
            axis = int(kv.get("axis", 1))
            r = o.reduce_sum(np.ascontiguousarray(X[0]), 0 if axis == 0 else 1)
            m(outs[0]).reshape(-1)[...] = r
        elif k in ("reduce_max", "reduce_max_mask"):
            axis = int(kv.get("axis", 1))
            x = np.ascontiguousarray(X[0])
            if k == "reduce_max":
                m(outs[0]).reshape(-1)[...] = o.reduce_max(x, 0 if axis == 0 else 1)[0]
            else:
                m(outs[0])[...] = o.reduce_max_mask(x, 0 if axis == 0 else 1)
        elif k == "mean_square":  # loss = s_l * sum(x^2) (fp64 sum), dX = s_g * x (fp32 product)
            x = np.ascontiguousarray(X[0], np.float32)
            sl = float(X[1].reshape(-1)[0]) if len(X) > 1 else 1.0
            sg = np.float32(X[2].reshape(-1)[0]) if len(X) > 2 else np.float32(1.0)
            m(outs[0]).reshape(-1)[0] = np.float32(np.sum(x.astype(np.float64) ** 2) * sl)
            if len(outs) > 1:
                m(outs[1])[...] = (x * sg).reshape(m(outs[1]).shape)
        elif k == "silu_grad":
            m(outs[0])[...] = o.silu_grad(X[0], X[1]).reshape(m(outs[0]).shape)
        elif k == "softmax_grad":
            m(outs[0])[...] = o.softmax_grad(X[0], X[1])
        elif k == "rmsnorm_grad":
            dx, dg, db = o.rmsnorm_grad(X[0], X[1].reshape(-1), X[2], float(kv.get("eps", 1e-5)))
            if len(X) > 3:  # residual gradient added in the same pass
                dx = np.add(X[3].reshape(dx.shape), dx, dtype=np.float32)
            m(outs[0])[...] = dx
            if len(outs) > 1:
                m(outs[1]).reshape(-1)[...] = dg
            if len(outs) > 2:
                m(outs[2]).reshape(-1)[...] = db
        elif k in ("attention", "attention_grad"):
            B, H = int(self._num(kv.get("batch", "1"))), int(self._num(kv.get("heads", "1")))
            causal = bool(int(kv.get("causal", 0)))
            bhsd = kv.get("layout", "bshd") == "bhsd"
            if kv.get("scale") == "auto":  # 1/sqrt(head dim)
                d = X[0].shape[1] if bhsd else X[0].shape[1] // H
                scale = float(np.float32(1.0 / np.sqrt(d)))
            else:
                scale = float(kv.get("scale", 0.0)) or 1.0

            def split(a):  # [B*T, H*d] (bshd) or [B*H*T, d] (bhsd) -> [B, H, T, d]
                if bhsd:
                    return np.ascontiguousarray(a.reshape(B, H, a.shape[0] // (B * H), a.shape[1]))
                T, C = a.shape[0] // B, a.shape[1] // H
                return np.ascontiguousarray(a.reshape(B, T, H, C).transpose(0, 2, 1, 3))

            def merge(a):  # inverse of split
                if bhsd:
                    return a.reshape(-1, a.shape[3])
                return a.transpose(0, 2, 1, 3).reshape(a.shape[0] * a.shape[2], -1)

            q, kk, v = split(X[0]), split(X[1]), split(X[2])
            if k == "attention":
                m(outs[0])[...] = merge(o.attention_bh(q, kk, v, scale, causal))
                if len(outs) > 1:
                    m(outs[1]).reshape(-1)[...] = o.attention_lse(q, kk, scale, causal).reshape(-1)
            else:
                dq, dk, dv = o.attention_grad(q, kk, v, split(X[4]), scale, causal)
                for name, g in zip(outs, (dq, dk, dv)):
                    m(name)[...] = merge(g)
        else:
            raise PlanTextError(f"unknown op '{k}'")
