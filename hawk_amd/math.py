"""``hawk.math``: the numpy-named functions a kernel body calls.

The subset of reference ``hawk/math.py`` the gfx950 target builds: the
elementwise transcendentals, ``dot``/``norm``/``outer``/``transpose``,
constructors ``vec``/``mat``, ``where``, and the Cholesky pair
``cholesky``/``cho_solve`` (reference ``hawk/trace/linalg.py:165-199``).
"""

from __future__ import annotations

from typing import Any


from .ir import HawkError, make
from .trace import Value, _projected, node_of


def _unary(kind: str, x: Any) -> Value:
    return Value(make(kind, (_projected(node_of(x)),)))


def exp(x): return _unary("exp", x)
def sin(x): return _unary("sin", x)
def cos(x): return _unary("cos", x)
def tanh(x): return _unary("tanh", x)
def sqrt(x): return _unary("sqrt", x)
def log(x): return _unary("log", x)
def abs(x): return _unary("abs", x)  # noqa: A001 - numpy's spelling


def dot(a, b) -> Value:
    """``sum_i a_i * b_i``, added in component order."""
    return Value(make("dot", (_projected(node_of(a)), _projected(node_of(b)))))


def norm(a) -> Value:
    """``sqrt(dot(a, a))``."""
    return Value(make("norm", (_projected(node_of(a)),)))


def outer(a, b) -> Value:
    return Value(make("outer", (_projected(node_of(a)), _projected(node_of(b)))))


def transpose(m) -> Value:
    return Value(make("transpose", (_projected(node_of(m)),)))


def sum(x) -> Value:  # noqa: A001 - numpy's spelling
    """The sum of a vector's or matrix's components (of ONE sample)."""
    return Value(make("sum", (_projected(node_of(x)),)))


def vec(*components) -> Value:
    """A vector of traced scalars."""
    return Value(make("vec", tuple(node_of(c) for c in components)))


def mat(rows) -> Value:
    """A matrix from rows of traced scalars: ``mat([[a, b], [c, d]])``."""
    rows = [list(r) for r in rows]
    if not rows or any(len(r) != len(rows[0]) for r in rows):
        raise HawkError("mat takes equal-length rows")
    flat = tuple(node_of(x) for r in rows for x in r)
    return Value(make("vec", flat, (len(rows), len(rows[0]))))


def where(cond, a, b) -> Value:
    """``a`` where ``cond`` holds, else ``b`` (both sides are evaluated)."""
    c = node_of(cond)
    if c.ttype.dtype != "bool":
        raise HawkError("where(cond, a, b): cond is a comparison")
    return Value(make("select", (c, _projected(node_of(a)), _projected(node_of(b)))))


def cholesky(a) -> tuple:
    """``L, info = cholesky(A)``: ``L L^T`` is the symmetric part of ``A``; ``info``
    is 0, or the 1-based column whose pivot was not positive (then the factor
    is zeros and a solve against it gives zeros)."""
    f = make("chol", (_projected(node_of(a)),))
    return Value(f), Value(make("chol_info", (f,)))


def cho_solve(factor, b) -> Value:
    """``A x = b`` from :func:`cholesky`'s factor."""
    f = node_of(factor)
    return Value(make("cho_solve", (f, _projected(node_of(b)))))


__all__ = ["abs", "cho_solve", "cholesky", "cos", "dot", "exp", "log", "mat", "norm", "outer",
           "sin", "sqrt", "sum", "tanh", "transpose", "vec", "where"]


