"""A numpy interpreter of hawk_amd's IR, vectorised over samples — TEST
INFRASTRUCTURE (the shape of reference tests/_eval.py).  It evaluates a
program's per-sample sinks so the derivative transforms can be checked against
central differences and the emitter's operation order against the oracle
without a GPU.  Tensors are numpy arrays of shape (*value_shape, n)."""

from __future__ import annotations

import numpy as np

from hawk_amd import ir


def _fold(terms):
    acc = terms[0]
    for t in terms[1:]:
        acc = acc + t
    return acc


class Evaluator:
    def __init__(self, env: dict, n: int, deps=None):
        self.env = env
        self.n = n
        self.memo: dict = {}
        self.tapes: dict = {}
        self.exits: dict = {}
        self.deps = deps if deps is not None else ir.Deps()

    def value(self, node):
        hit = self.memo.get(node.uid)
        if hit is not None:
            return hit
        for m in ir.level_order([node], self.deps):
            if m.uid in self.memo:
                continue
            if m.kind in ("carry", "loop_index"):
                continue                      # bound by the loop being evaluated
            self.memo[m.uid] = self._eval(m)
        return self.memo[node.uid]

    def _op(self, m, i):
        return self.memo[m.operands[i].uid]

    def _eval(self, m):
        k = m.kind
        n = self.n
        if k == "leaf":
            role, name = m.literal
            x = self.env[name]
            if role == "uniform":
                return np.full(n, float(x))
            if role == "terminated":
                return np.asarray(x, dtype=bool)
            return np.asarray(x, dtype=np.float64 if m.ttype.dtype != "i32" else np.int32)
        if k == "const":
            return np.full(n, m.literal)
        if k == "iconst":
            return np.full(n, m.literal)
        if k == "sample_count":
            return np.full(n, float(self.env.get("__n_samples__", n)))
        if k == "real":
            return self._op(m, 0).astype(np.float64)
        if k in ("add", "sub", "mul", "div"):
            a, b = self._op(m, 0), self._op(m, 1)
            a, b = self._bc(a, m.operands[0], m), self._bc(b, m.operands[1], m)
            return {"add": np.add, "sub": np.subtract, "mul": np.multiply, "div": np.divide}[k](a, b)
        if k == "neg":
            return -self._op(m, 0)
        if k in ("exp", "sin", "cos", "tanh", "sqrt", "log", "abs"):
            return {"exp": np.exp, "sin": np.sin, "cos": np.cos, "tanh": np.tanh, "sqrt": np.sqrt,
                    "log": np.log, "abs": np.abs}[k](self._op(m, 0))
        if k in ("lt", "le", "gt", "ge", "eq", "ne"):
            return {"lt": np.less, "le": np.less_equal, "gt": np.greater, "ge": np.greater_equal,
                    "eq": np.equal, "ne": np.not_equal}[k](self._op(m, 0), self._op(m, 1))
        if k == "select":
            c, a, b = self._op(m, 0), self._op(m, 1), self._op(m, 2)
            return np.where(c, a, b)
        if k == "dot":
            a, b = self._op(m, 0), self._op(m, 1)
            return _fold([a[i] * b[i] for i in range(a.shape[0])])
        if k == "norm":
            a = self._op(m, 0)
            return np.sqrt(_fold([a[i] * a[i] for i in range(a.shape[0])]))
        if k == "sum":
            a = self._op(m, 0)
            flat = a.reshape(-1, n)
            return _fold([flat[i] for i in range(flat.shape[0])])
        if k == "splat":
            return np.broadcast_to(self._op(m, 0), tuple(m.literal) + (n,)).copy()
        if k == "component":
            idx = m.literal if isinstance(m.literal, tuple) else (m.literal,)
            return self._op(m, 0)[idx]
        if k == "vec":
            parts = [self.memo[o.uid] for o in m.operands]
            return np.stack(parts).reshape(tuple(m.literal) + (n,))
        if k == "transpose":
            return np.ascontiguousarray(np.swapaxes(self._op(m, 0), 0, 1))
        if k == "mv":
            M, v = self._op(m, 0), self._op(m, 1)
            return np.stack([_fold([M[i, j] * v[j] for j in range(M.shape[1])]) for i in range(M.shape[0])])
        if k == "mm":
            A, B = self._op(m, 0), self._op(m, 1)
            return np.stack([np.stack([_fold([A[i, q] * B[q, j] for q in range(A.shape[1])])
                                       for j in range(B.shape[1])]) for i in range(A.shape[0])])
        if k == "outer":
            a, b = self._op(m, 0), self._op(m, 1)
            return a[:, None, :] * b[None, :, :]
        if k == "chol":
            return self._chol(self._op(m, 0))
        if k == "chol_info":
            return self.memo[m.operands[0].uid][1]
        if k == "cho_solve":
            (L, info), b = self.memo[m.operands[0].uid], self._op(m, 1)
            return self._cho_solve(L, info, b)
        if k == "lane_axis":
            div, mod = m.literal
            idx = np.arange(n, dtype=np.int64)
            if mod == 0:
                return idx
            q = idx // div
            return (q if mod is None else q % mod).astype(np.int32)
        if k in ("floordiv", "mod"):
            a, b = self._op(m, 0), self._op(m, 1)
            return (np.floor_divide if k == "floordiv" else np.mod)(a, b)
        if k in ("gather", "table_index") and m.literal is not None:
            table = np.asarray(self._op(m, 0)).reshape(-1)
            keys = [np.broadcast_to(np.asarray(self._op(m, j), dtype=np.int64), (n,)) for j in range(1, len(m.operands))]
            extents = list(m.literal[1])
            rest = int(np.prod([e for e in extents[1:]] or [1]))
            if extents[0] is None:
                extents[0] = table.shape[0] // rest
            flat = np.zeros(n, dtype=np.int64)
            for j, (key, e) in enumerate(zip(keys, extents)):
                stride = int(np.prod(extents[j + 1:] or [1]))
                flat = flat + np.clip(key, 0, e - 1) * stride
            return flat if k == "table_index" else table[flat]
        if k == "gather":
            table, key = self._op(m, 0), self._op(m, 1)
            ok = (key >= 0) & (key < table.shape[0])
            if table.shape[0] == 0:
                return np.zeros(n)
            return np.where(ok, table[np.where(ok, key, 0)], 0.0)
        if k == "loop":
            return self._loop(m)
        if k == "loop_value":
            return self.memo[m.operands[0].uid][m.literal]
        if k == "loop_exit":
            return self.exits[m.operands[0].uid]
        if k == "tape_read":
            loop, index = m.operands
            kval = int(self.memo[index.uid][0])
            info = loop.literal
            return self.tapes[loop.uid][m.literal][(kval - info.start) // info.step]
        raise NotImplementedError(k)

    def _bc(self, x, node, out):
        if node.ttype.shape == out.ttype.shape:
            return x
        return np.broadcast_to(x, tuple(out.ttype.shape) + (self.n,))

    @staticmethod
    def _chol(a):
        size = a.shape[0]
        n = a.shape[-1]
        L = np.zeros_like(a)
        info = np.zeros(n, dtype=np.int32)
        for j in range(size):
            live = info == 0
            d = (0.5 * a[j, j]) + (0.5 * a[j, j])
            for k in range(j):
                d = d - (L[j, k] * L[j, k])
            ok = live & (d > 0)
            ljj = np.sqrt(np.where(ok, d, 1.0))
            L[j, j] = np.where(ok, ljj, L[j, j])
            for i in range(j + 1, size):
                acc = (0.5 * a[i, j]) + (0.5 * a[j, i])
                for k in range(j):
                    acc = acc - (L[i, k] * L[j, k])
                L[i, j] = np.where(ok, acc / ljj, L[i, j])
            info = np.where(live & ~ok, j + 1, info)
        return L, info

    @staticmethod
    def _cho_solve(L, info, b):
        size = b.shape[0]
        x = np.zeros_like(b)
        for i in range(size):
            acc = b[i].copy()
            for j in range(i):
                acc = acc - (L[i, j] * x[j])
            x[i] = acc / L[i, i]
        for r in range(size):
            i = size - 1 - r
            acc = x[i].copy()
            for j in range(i + 1, size):
                acc = acc - (L[j, i] * x[j])
            x[i] = acc / L[i, i]
        return np.where(info == 0, x, 0.0)

    def _loop(self, m):
        info = m.literal
        carries = [np.array(self.memo[o.uid], copy=True) for o in m.operands]
        tape = [[] for _ in carries]
        done = np.zeros(self.n, dtype=bool)       # lanes that took the loop's exit
        trips = range(info.start, info.stop(), info.step)
        if info.count is not None:                # the launch's word: that many trips
            trips = range(0, max(0, int(np.asarray(self.env[info.count]).reshape(-1)[0])))
        for kval in trips:
            if info.exit is not None and done.all():
                break
            for j, c in enumerate(carries):
                tape[j].append(c)
            inner = Evaluator(self.env, self.n, self.deps)
            inner.memo = dict(self.memo)
            inner.tapes = self.tapes
            inner.exits = self.exits
            inner.memo[info.index.uid] = np.full(self.n, kval)
            for c, val in zip(info.carries, carries):
                inner.memo[c.uid] = val
            nexts = [np.array(inner.value(x), copy=True) for x in info.nexts]
            if info.exit is None:
                carries = nexts
                continue
            # a tail break: a lane still in the loop keeps this trip's values,
            # then leaves if its exit holds
            leave = np.asarray(inner.value(info.exit), dtype=bool)
            carries = [np.where(done, c, nx) for c, nx in zip(carries, nexts)]
            done = done | leave
        self.tapes[m.uid] = tape
        self.exits[m.uid] = done
        return carries


def evaluate(program, env: dict, n: int) -> dict:
    """``{sink name: value}`` of the per-sample sinks of ``program``; a
    ``hawk.sum`` sink gives its per-sample terms (the caller sums them), a
    ``hawk.scatter`` sink its per-sample payloads (the caller adds them at
    the keys)."""
    ev = Evaluator(env, n)
    out = {}
    for s in program.sinks:
        if hasattr(s, "cells"):        # an ordered fold: (contributions, cells) per slot
            out[s.name] = ([ev.value(v) for v in s.values], [ev.value(c) for c in s.cells])
            continue
        out[s.name] = ev.value(s.value)
    return out
