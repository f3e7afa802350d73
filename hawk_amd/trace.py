"""The authoring surface: ``@hawk.kernel``, traced values, ``hawk.sum`` and
``hawk.scatter``.

A kernel is a plain Python function for ONE sample.  Tracing runs it once over
:class:`Value` objects (operator overloading builds IR nodes), after a small
``ast`` rewrite (reference ``hawk/trace/astpass.py``):

* ``for k in range(...)`` becomes ONE rolled ``loop`` node: the names the body
  assigns that were bound before the loop are its carried slots;
* every ``return`` (and the end of the body) reports the final value of each
  ``Mutable`` parameter, so ``y = expr`` commits ``expr`` into the plane ``y``
  (reference ``hawk/trace/kernel.py:480-525``), and a returned value commits
  into a synthesised slot named ``out``.

A ``Mutable`` read before it is assigned reads the value the plane held when
the launch began (a prior read, refused by ``vjp``/``jvp`` as in reference
``hawk/diff/transform.py:169-192``).

A kernel that declares ``terminated: Terminated`` runs only the samples its
mask has not finished; ``terminated = cond`` (one statement, a traced bool)
finishes a sample, and :func:`steps` makes a finishing kernel take up to K
steps a launch (reference ``hawk/trace/steps.py``).
"""

from __future__ import annotations

import ast
import inspect
import textwrap
from typing import Any

from . import ir
from .ir import (FINISHED_PLANE, GUARD_MASK, AccumWrite, Assign, Decl, Finish, HawkError, Node, Program, SampleSum,
                 make)
from .types import FinishRefusal, GridDecl, MutableDecl, TableDecl, TensorType, _ParamDecl, _TerminatedDecl, role_of

SUM_POLICIES = ("auto", "compensated", "ordered")
SCATTER_POLICIES = ("ordered",)


# --------------------------------------------------------------------------
# values


def node_of(x: Any) -> Node:
    """The IR node of a traced value or a Python number."""
    if isinstance(x, Value):
        return x.node
    if isinstance(x, bool):
        raise HawkError("a Python bool is not a number in a kernel body")
    if isinstance(x, int):
        return ir.const(float(x))
    if isinstance(x, float):
        return ir.const(x)
    try:
        import numpy as np
        if isinstance(x, np.floating | np.integer):
            return ir.const(float(x))
    except ImportError:       # pragma: no cover - numpy is a test dependency only
        pass
    if isinstance(x, Reduced):
        raise HawkError("a value reduced over every sample (hawk.sum) is read back in the body: "
                        "that needs a stage boundary this build does not cut; assign it to a "
                        "Mutable (or return it) instead")
    raise HawkError(f"{x!r} ({type(x).__name__}) is not a traced value or a number")


def _projected(n: Node) -> Node:
    """A Cholesky factor used as a matrix reads its lower triangle."""
    return make("chol_factor", (n,)) if n.ttype.tag == "chol_factor" else n


def _is_index(x: Any) -> bool:
    return isinstance(x, Value) and x.node.ttype.dtype in ("i32", "i64") and not x.node.ttype.shape


def _operand(x: Any, other: Any) -> Node:
    """``x`` as an operand beside ``other``: a Python int beside an Index is
    an integer constant (index arithmetic), otherwise a number."""
    if isinstance(x, int) and not isinstance(x, bool) and _is_index(other):
        return ir.index_const(x)
    return _projected(node_of(x))


def _bin(kind: str, a: Any, b: Any) -> Value:
    return Value(make(kind, (_operand(a, b), _operand(b, a))))


class Value:
    """One traced value (scalar, vector or matrix) of the current sample."""

    __slots__ = ("node",)
    __array_priority__ = 1000      # numpy scalars defer to these operators

    def __init__(self, node: Node):
        self.node = node

    @property
    def ttype(self) -> TensorType:
        return self.node.ttype

    @property
    def shape(self) -> tuple:
        return self.node.ttype.shape

    def __add__(self, o): return _bin("add", self, o)
    def __radd__(self, o): return _bin("add", o, self)
    def __sub__(self, o): return _bin("sub", self, o)
    def __rsub__(self, o): return _bin("sub", o, self)
    def __mul__(self, o): return _bin("mul", self, o)
    def __rmul__(self, o): return _bin("mul", o, self)
    def __floordiv__(self, o): return _bin("floordiv", self, o)
    def __rfloordiv__(self, o): return _bin("floordiv", o, self)
    def __mod__(self, o): return _bin("mod", self, o)
    def __rmod__(self, o): return _bin("mod", o, self)
    def __truediv__(self, o): return _bin("div", self, o)
    def __rtruediv__(self, o): return _bin("div", o, self)
    def __neg__(self): return Value(make("neg", (_projected(self.node),)))
    def __pos__(self): return self
    def __abs__(self): return Value(make("abs", (_projected(self.node),)))

    def __pow__(self, p):
        if isinstance(p, int) and not isinstance(p, bool) and 1 <= p <= 8:
            out = self
            for _ in range(p - 1):
                out = out * self
            return out
        raise HawkError("x ** p is written for a literal integer 1 <= p <= 8 in this build "
                        "(repeated products); use hawk.math.exp/log for other powers")

    def __lt__(self, o): return _bin("lt", self, o)
    def __le__(self, o): return _bin("le", self, o)
    def __gt__(self, o): return _bin("gt", self, o)
    def __ge__(self, o): return _bin("ge", self, o)

    def __matmul__(self, o):
        a, b = _projected(self.node), _projected(node_of(o))
        kind = "mm" if len(b.ttype.shape) == 2 else "mv"
        return Value(make(kind, (a, b)))

    def __rmatmul__(self, o):
        return Value(node_of(o)) @ self

    @property
    def T(self) -> Value:
        return Value(make("transpose", (_projected(self.node),)))

    def __getitem__(self, k) -> Value:
        n = _projected(self.node)
        if isinstance(k, Value):
            raise HawkError("a component read at a runtime index is not in this build; "
                            "index with a literal int")
        if isinstance(k, tuple) and all(isinstance(i, int) for i in k):
            return Value(make("component", (n,), tuple(k)))
        if isinstance(k, int):
            if len(n.ttype.shape) == 2:
                r, c = n.ttype.shape
                return Value(make("vec", tuple(make("component", (n,), (k, j)) for j in range(c))))
            return Value(make("component", (n,), k))
        raise HawkError(f"index {k!r}: a value is indexed by literal ints")

    def __len__(self) -> int:
        if not self.shape:
            raise HawkError("a scalar has no length")
        return self.shape[0]

    def __bool__(self):
        raise HawkError("a traced value has no Python truth value: a branch on a per-sample value "
                        "is written hawk.math.where(cond, a, b)")

    def __iter__(self):
        if not self.shape:
            raise HawkError("a scalar is not iterable")
        return (self[i] for i in range(self.shape[0]))

    def __repr__(self) -> str:
        return f"Value({self.node!r})"


class MutableRef(Value):
    """A ``Mutable`` parameter before it is assigned: reading it reads the
    value the plane held when the launch began."""

    __slots__ = ("name",)

    def __init__(self, name: str, ttype: TensorType):
        super().__init__(ir.leaf("mutable", name, ttype))
        self.name = name


class Reduced:
    """The result of ``hawk.sum``: one value for the whole run, or with
    ``over=`` one per coordinate of the kept lane axes (``group`` consecutive
    samples each).  It can be committed (assigned to a ``Mutable`` or
    returned), not read back."""

    def __init__(self, node: Node, policy: str, group: int | None = None, kept: tuple = (), op: str = "sum"):
        self.node = node
        self.policy = policy
        self.group = group
        self.kept = kept
        self.op = op

    def _refuse(self, *_):
        raise HawkError("a value reduced over every sample (hawk.sum) is read back in the body: "
                        "that needs a stage boundary this build does not cut; assign it to a "
                        "Mutable (or return it) instead")

    __add__ = __radd__ = __sub__ = __rsub__ = __mul__ = __rmul__ = _refuse
    __truediv__ = __rtruediv__ = __neg__ = __getitem__ = _refuse


# --------------------------------------------------------------------------
# cross-sample vocabulary


class TableRef:
    """A ``Table`` parameter: ``t.at(i)`` / ``t[i]`` reads the flat cell i;
    ``t.at(row=r, col=c)`` / ``t[r, c]`` reads one index per declared axis in
    declared order.  Each index is clamped into its axis, so a read outside the
    table reads its edge (reference tests/test_table_clamp.py:1-8,
    tests/test_table_positional.py:1-9)."""

    def __init__(self, name: str, decl: TableDecl):
        self._name, self._decl = name, decl
        self._leaf = ir.leaf("lookup", name, TensorType((), "f64"))

    def _key(self, x: Any) -> Node:
        if isinstance(x, int) and not isinstance(x, bool):
            return ir.index_const(x)
        if _is_index(x):
            return x.node
        raise HawkError(f"{self._name!r}: a table index is an Index (an integer), got {x!r}")

    def _read(self, keys: list, extents: tuple) -> Value:
        return Value(make("gather", (self._leaf, *[self._key(k) for k in keys]), ("clamp", tuple(extents))))

    def at(self, *positional: Any, **named: Any) -> Value:
        axes = self._decl.axes
        labels = [a for a, _ in axes]
        if named:
            if positional or set(named) != set(labels):
                raise HawkError(f"{self._name!r}.at(...) names every axis {labels} once, got "
                                f"{list(named)} with {len(positional)} positional")
            return self._read([named[a] for a in labels], tuple(e for _, e in axes))
        if len(positional) == 1:
            return self._read([positional[0]], (None,))          # the flat read over every cell
        if len(positional) == len(axes):
            return self._read(list(positional), tuple(e for _, e in axes))
        raise HawkError(f"{self._name!r}: {self._name}.at(...) takes one flat index or one index per declared "
                        f"axis {labels}, got {len(positional)}")

    def __getitem__(self, idx: Any) -> Value:
        items = idx if isinstance(idx, tuple) else (idx,)
        labels = [a for a, _ in self._decl.axes]
        if len(items) not in (1, len(labels)):
            raise HawkError(f"{self._name!r}: {self._name}[...] takes one index per declared axis {labels}, "
                            f"got {len(items)}")
        return self.at(*items)

    def _refuse(self, *_):
        raise HawkError(f"{self._name!r} is a Table: read it with {self._name}.at(...) or {self._name}[...]")

    __add__ = __radd__ = __sub__ = __rsub__ = __mul__ = __rmul__ = __truediv__ = __neg__ = _refuse


class LaneRef:
    """The ``Grid`` parameter: the lane's coordinates, as Index values.
    ``lane.<axis>`` or ``lane[i]`` (0 the slowest axis, -1 the fastest) is
    ``(sample // stride) % extent`` with the stride the product of the later
    axes' extents; ``lane.flat`` is the flat lane index (reference
    ``hawk/trace/decl.py:135-145``)."""

    def __init__(self, grid: GridDecl):
        object.__setattr__(self, "_grid", grid)

    def _axis(self, pos: int) -> Value:
        axes = self._grid.axes
        stride = 1
        for _, e in axes[pos + 1:]:
            stride *= e
        return Value(make("lane_axis", (), (stride, axes[pos][1])))

    def __getattr__(self, label: str) -> Value:
        if label == "flat":
            return Value(make("lane_axis", (), (1, 0)))
        for pos, (name, _) in enumerate(self._grid.axes):
            if name == label:
                return self._axis(pos)
        raise HawkError(f"the Grid has no axis {label!r} (its axes: {[a for a, _ in self._grid.axes]})")

    def __getitem__(self, pos: int) -> Value:
        axes = self._grid.axes
        if not isinstance(pos, int) or not -len(axes) <= pos < len(axes):
            raise HawkError(f"lane[{pos!r}]: the Grid has {len(axes)} axes")
        return self._axis(pos % len(axes))


class _Trace:
    """The sinks a kernel body records while it is traced, and the Grid of
    its lanes (if declared)."""

    stack: list = []

    def __init__(self, grid: GridDecl | None = None):
        self.sinks: list = []
        self.grid = grid

    def __enter__(self):
        _Trace.stack.append(self)
        return self

    def __exit__(self, *exc):
        _Trace.stack.pop()

    @classmethod
    def current(cls, where: str) -> _Trace:
        if not cls.stack:
            raise HawkError(f"{where} is written inside a @hawk.kernel body")
        return cls.stack[-1]


_IDENTITY = {"sum": 0.0, "max": float("-inf"), "min": float("inf")}


def _reduce(op: str, x: Any, over: Any, where: Any, policy: str) -> Reduced:
    """The reductions' common front (reference ``hawk/trace/reduce.py:234-271``):
    the policy, ``where=`` (a masked lane contributes the op's identity), the
    mean's division by the sample count (over every sample) or by the reduced
    axes' extent (over some), and the lane axes ``over`` names."""
    call = f"hawk.{op}(x, over={over!r})" if over is not None else f"hawk.{op}(x)"
    if policy not in SUM_POLICIES:
        raise HawkError(f"{call}: policy={policy!r} is not one of {SUM_POLICIES}")
    base = "sum" if op == "mean" else op
    n = _projected(node_of(x))
    if n.ttype.dtype == "bool" and not n.ttype.shape:
        n = make("select", (n, ir.const(1.0), ir.const(0.0)))   # hawk.sum(mask): the count of true lanes
    if where is not None:
        mask = _projected(node_of(where))
        if mask.ttype.dtype != "bool" or mask.ttype.shape:
            raise HawkError(f"{call}: where= is this lane's bool mask, got {mask.ttype!r}")
        if op == "mean":
            raise HawkError(f"{call}: the mean of the masked lanes needs their count, a second reduction: "
                            "hawk.sum(x, where=mask) / hawk.sum(mask)")
        n = make("select", (mask, n, ir.const(_IDENTITY[base])))
    if over is None:
        if op == "mean":
            n = make("div", (n, make("sample_count", ())))
        return Reduced(n, policy, op=base)
    if n.ttype.shape:
        raise HawkError(f"{call}: a reduction over some lane axes takes a scalar in this build; reduce each "
                        "component")
    grid = _Trace.current(f"hawk.{op}").grid
    if grid is None:
        raise HawkError(f"{call} names lane axes: declare the kernel's lanes with a Grid parameter, e.g. "
                        'lane: Grid["key", "sample":1024]')
    labels = [a for a, _ in grid.axes]
    items = over if isinstance(over, tuple) else (over,)
    reduced = set()
    for item in items:
        if isinstance(item, str) and item in labels:
            reduced.add(labels.index(item))
        elif isinstance(item, int) and not isinstance(item, bool) and -len(labels) <= item < len(labels):
            reduced.add(item % len(labels))
        else:
            raise HawkError(f"{call}: {item!r} is not an axis of the Grid {labels}")
    if len(reduced) == len(labels):
        if op == "mean":
            n = make("div", (n, make("sample_count", ())))
        return Reduced(n, policy, op=base)
    if base != "sum":
        raise HawkError(f"{call}: a {op} over some of the lane axes is in the next release; hawk.{op}(x) "
                        f"(one value for the run) and hawk.sum/mean(x, over=...) work now")
    spelled = f"over={over!r}"
    if reduced != set(range(len(labels) - len(reduced), len(labels))):
        raise HawkError(f"hawk.{op}(x, {spelled}, policy={policy!r}): policy={policy!r} sums over the trailing "
                        f"lane axes only (the Grid's axes are {labels}): each key's samples are one run")
    group = 1
    for pos in reduced:
        group *= grid.axes[pos][1]
    if op == "mean":
        n = make("div", (n, ir.const(float(group))))
    kept = tuple(labels[:len(labels) - len(reduced)])
    return Reduced(n, policy, group, kept, op="sum")


def sum(x: Any, over: Any = None, where: Any = None, policy: str = "auto") -> Reduced:  # noqa: A001
    """The sum of ``x`` over every sample of the run, or over the lane axes
    ``over`` names (a label, a position, or a tuple of them) of the kernel's
    ``Grid`` (reference ``hawk/trace/reduce.py:277-301``).  A masked lane
    (``where=`` false) adds nothing.  A vector or matrix ``x`` sums each entry
    into its own cell entry (one row plane per entry).

    ``policy="ordered"`` adds in a fixed tree that depends on the sample count
    only: 65536 virtual lanes, each adding its rows in order, folded in groups
    of 1024 by a halving tree and the 64 group results by the same tree — the
    same bits on every launch.  Over some axes it sums over the TRAILING ones
    only: each coordinate of the kept leading axes is a run of consecutive
    samples, and each run takes that tree.  The default policies (``"auto"``,
    ``"compensated"``) sum each row of 32 samples as a compensated
    (hi, comp) pair and fold the rows in the canonical ordered tree of
    reference ``hawk/_cells.py``; over some axes each key's run is such a sum
    of its own (the reference commits keys atomically, in launch-dependent
    order once a key spans three warps)."""
    return _reduce("sum", x, over, where, policy)


def max(x: Any, over: Any = None, where: Any = None, policy: str = "auto") -> Reduced:  # noqa: A001
    """The maximum of ``x`` over every sample (reference
    ``hawk/trace/reduce.py:304-307``): each row of 32 samples by a butterfly
    that ignores a NaN operand, then the rows in the canonical tree of
    ``hawk/_cells.py`` (``a > b ? a : b``); exact.  A masked lane
    (``where=`` false) is -inf."""
    return _reduce("max", x, over, where, policy)


def min(x: Any, over: Any = None, where: Any = None, policy: str = "auto") -> Reduced:  # noqa: A001
    """The minimum of ``x`` over every sample, as :func:`max` with ``<``; a
    masked lane is +inf (reference ``hawk/trace/reduce.py:310-313``)."""
    return _reduce("min", x, over, where, policy)


def mean(x: Any, over: Any = None, where: Any = None, policy: str = "auto") -> Reduced:
    """The mean of ``x`` over the samples ``over`` names: the sum of each term
    divided by the count of reduced samples (the run's sample count over
    every sample; the reduced axes' extent over some), reference
    ``hawk/trace/reduce.py:263-273``, ``:316-320``."""
    return _reduce("mean", x, over, where, policy)


class _Stored:
    """What ``hawk.scatter(y)[key] += v`` leaves in the statement's target."""


class _ScatterSlot:
    def __init__(self, target: _ScatterTarget, key: Any):
        self.target, self.key = target, key

    def __iadd__(self, value: Any) -> _Stored:
        t = self.target
        key = node_of(self.key) if isinstance(self.key, Value) else None
        if key is None or key.ttype.dtype != "i32" or key.kind != "leaf":
            raise HawkError(f"hawk.scatter({t.name})[key] += v: the key is an Index plane in this build")
        v = _projected(node_of(value))
        if v.ttype.shape:
            raise HawkError(f"hawk.scatter({t.name}, policy='ordered') adds a scalar payload in this build")
        _Trace.current("hawk.scatter").sinks.append(AccumWrite(t.name, v, key, t.policy))
        return _Stored()


class _ScatterTarget:
    def __init__(self, ref: MutableRef, policy: str):
        self.name, self.policy = ref.name, policy

    def __getitem__(self, key) -> _ScatterSlot:
        return _ScatterSlot(self, key)

    def __setitem__(self, key, value) -> None:
        if not isinstance(value, _Stored):
            raise HawkError(f"hawk.scatter({self.name})[key] = v (a keyed store) is not in this build; "
                            "hawk.scatter(y, policy='ordered')[key] += v is")


def scatter(sink: Any, policy: str = "auto") -> _ScatterTarget:
    """``hawk.scatter(sink, policy="ordered")[key] += v`` adds ``v`` into the
    plane ``sink`` at ``key`` with no atomics: lanes are cut into chunks
    (``clamp(N // cells, 1, 256)``), each chunk adds its lanes in order into
    its own partial of every key, and each cell adds its partials in chunk
    order (reference ``hawk/trace/reduce.py:383-402``).  Key -1 adds nothing;
    another key outside the plane is reported by name after the run."""
    if not isinstance(sink, MutableRef):
        raise HawkError("hawk.scatter(y): y is a Mutable parameter of the kernel")
    if policy not in SCATTER_POLICIES:
        raise HawkError(f"hawk.scatter({sink.name}, policy={policy!r}): the hip target builds "
                        "policy='ordered' (no atomics, the serial walk's bits)")
    return _ScatterTarget(sink, policy)


# --------------------------------------------------------------------------
# loops


def _for(bounds: tuple, body, inits: tuple, names: tuple):
    """The rolled loop the ast pass made of ``for k in range(*bounds)``."""
    if not all(isinstance(b, int) and not isinstance(b, bool) for b in bounds):
        raise HawkError(f"for ... in range{bounds!r}: a loop's trip count is a literal int "
                        "(the body is emitted once, rolled)")
    rng = range(*bounds)
    if len(rng) == 0:
        return tuple(inits)
    init_nodes = []
    for name, x in zip(names, inits):
        if isinstance(x, Reduced):
            raise HawkError(f"{name!r}: a hawk.sum result cannot be carried through a loop")
        if isinstance(x, MutableRef):
            init_nodes.append(x.node)
        else:
            init_nodes.append(_projected(node_of(x)))
    marker = len(_Trace.current("a for loop").sinks)

    def traced(index: Node, *carries: Node):
        out = body(Value(index), *[Value(c) for c in carries])
        return tuple(_projected(node_of(v)) for v in out)

    loop = ir.new_loop(len(rng), rng.start, rng.step, tuple(init_nodes), traced, tuple(names))
    if len(_Trace.current("a for loop").sinks) != marker:
        raise HawkError("hawk.scatter inside a for loop is not in this build")
    return tuple(Value(ir.loop_value(loop, j)) for j in range(len(names)))


def _exit(ret, finals: dict):
    return ret, finals


# --------------------------------------------------------------------------
# the ast pass


def _stored_names(nodes) -> list:
    """Names bound by the statements ``nodes`` (nested defs excluded), in order."""
    out = []

    class V(ast.NodeVisitor):
        def visit_Name(self, n):
            if isinstance(n.ctx, ast.Store) and n.id not in out:
                out.append(n.id)

        def visit_FunctionDef(self, n):
            pass

        visit_AsyncFunctionDef = visit_FunctionDef
        visit_Lambda = visit_FunctionDef

    for st in nodes:
        V().visit(st)
    return out


class _Rewriter:
    def __init__(self, mutables: tuple):
        self.mutables = mutables
        self.count = 0

    def exit_call(self, value) -> ast.expr:
        finals = ast.Dict(keys=[ast.Constant(m) for m in self.mutables],
                          values=[ast.Name(m, ast.Load()) for m in self.mutables])
        return ast.Call(ast.Name("__hawk_exit__", ast.Load()), [value or ast.Constant(None), finals], [])

    def block(self, stmts: list, defined: set, in_loop: bool) -> list:
        out = []
        for st in stmts:
            if isinstance(st, ast.For):
                out.extend(self.loop(st, defined))
                defined |= set(_stored_names([st]))
                continue
            if isinstance(st, ast.Return):
                if in_loop:
                    raise HawkError("return inside a for loop of a kernel body")
                out.append(ast.Return(self.exit_call(st.value)))
                continue
            if isinstance(st, (ast.While, ast.Break, ast.Continue)):
                raise HawkError(f"{type(st).__name__.lower()} is not in this build's kernel language; "
                                "loops are for ... in range(<int>)")
            if isinstance(st, ast.If):
                st.body = self.block(st.body, set(defined), in_loop)
                st.orelse = self.block(st.orelse, set(defined), in_loop)
            out.append(st)
            defined |= set(_stored_names([st]))
        return out

    def loop(self, st: ast.For, defined: set) -> list:
        it = st.iter
        if not (isinstance(it, ast.Call) and isinstance(it.func, ast.Name) and it.func.id == "range"):
            st.body = self.block(st.body, set(defined), True)
            return [st]           # a Python-level loop over a static sequence: unrolled at trace
        if st.orelse:
            raise HawkError("for ... else is not in the kernel language")
        if not isinstance(st.target, ast.Name):
            raise HawkError("a rolled loop binds one index name: for k in range(...)")
        index = st.target.id
        carried = [n for n in _stored_names(st.body) if n in defined and n != index]
        body = self.block(st.body, set(defined) | {index}, True)
        self.count += 1
        fname = f"__hawk_body_{self.count}"
        fdef = ast.FunctionDef(
            name=fname,
            args=ast.arguments(posonlyargs=[], args=[ast.arg(index)] + [ast.arg(c) for c in carried],
                               vararg=None, kwonlyargs=[], kw_defaults=[], kwarg=None, defaults=[]),
            body=body + [ast.Return(ast.Tuple([ast.Name(c, ast.Load()) for c in carried], ast.Load()))],
            decorator_list=[], returns=None, type_comment=None)
        call = ast.Call(ast.Name("__hawk_for__", ast.Load()),
                        [ast.Tuple(list(it.args), ast.Load()), ast.Name(fname, ast.Load()),
                         ast.Tuple([ast.Name(c, ast.Load()) for c in carried], ast.Load()),
                         ast.Tuple([ast.Constant(c) for c in carried], ast.Load())], [])
        if carried:
            assign = ast.Assign(targets=[ast.Tuple([ast.Name(c, ast.Store()) for c in carried], ast.Store())],
                                value=call)
        else:
            assign = ast.Expr(call)
        return [ast.copy_location(fdef, st), ast.copy_location(assign, st)]


def _finish_checks(fdef: ast.FunctionDef, finishes: tuple) -> None:
    """The static rules of ``terminated = cond`` (reference
    ``tests/test_finish_own_sample.py:125-178``): one statement a mask, not
    inside a ``for``, not a Python literal."""
    seen: dict = {}

    def walk(stmts, in_for: bool):
        for st in stmts:
            if isinstance(st, (ast.FunctionDef, ast.AsyncFunctionDef, ast.ClassDef)):
                continue
            targets = []
            if isinstance(st, ast.Assign):
                targets = st.targets
            elif isinstance(st, (ast.AugAssign, ast.AnnAssign)):
                targets = [st.target]
            for t in targets:
                for node in ast.walk(t):
                    if isinstance(node, ast.Name) and isinstance(node.ctx, ast.Store) and node.id in finishes:
                        if in_for:
                            raise FinishRefusal(f"finishes {node.id!r} inside a `for`: a sample finishes once, "
                                                 "after its step (finish after the loop)")
                        seen[node.id] = seen.get(node.id, 0) + 1
                        if seen[node.id] > 1:
                            raise FinishRefusal(f"{node.id!r} is finished twice: a kernel finishes its sample "
                                                 "in ONE statement (combine the conditions with where or |)")
                        value = getattr(st, "value", None)
                        if isinstance(value, ast.Constant) and isinstance(value.value, bool):
                            raise FinishRefusal(f"{node.id!r} = {value.value}: a Python literal is no per-sample "
                                                 "condition; finish on a traced comparison")
            if isinstance(st, (ast.For, ast.AsyncFor, ast.While)):
                walk(st.body, True)
                walk(st.orelse, True)
            elif isinstance(st, ast.If):
                walk(st.body, in_for)
                walk(st.orelse, in_for)
            elif isinstance(st, ast.With):
                walk(st.body, in_for)

    walk(fdef.body, False)


def _rewritten(fn, mutables: tuple, finishes: tuple = ()):
    try:
        source = textwrap.dedent(inspect.getsource(fn))
    except (OSError, TypeError) as exc:
        raise HawkError(f"@hawk.kernel needs the source of {fn.__name__!r} to trace it: {exc}") from None
    tree = ast.parse(source)
    fdef = tree.body[0]
    if not isinstance(fdef, ast.FunctionDef):
        raise HawkError("@hawk.kernel decorates a def")
    fdef.decorator_list = []
    fdef.returns = None
    for a in fdef.args.args:
        a.annotation = None
    _finish_checks(fdef, finishes)
    rw = _Rewriter(mutables + finishes)
    params = {a.arg for a in fdef.args.args}
    fdef.body = rw.block(fdef.body, set(params), False) + [ast.Return(rw.exit_call(None))]
    ast.fix_missing_locations(tree)
    first = fn.__code__.co_firstlineno
    ast.increment_lineno(tree, first - 1)
    code = compile(tree, inspect.getsourcefile(fn) or "<kernel>", "exec")
    ns = dict(fn.__globals__)
    if fn.__closure__:
        for name, cell in zip(fn.__code__.co_freevars, fn.__closure__):
            ns[name] = cell.cell_contents
    ns["__hawk_for__"] = _for
    ns["__hawk_exit__"] = _exit
    exec(code, ns)
    return ns[fdef.name]


def _annotation(fn, raw, ns):
    if isinstance(raw, str):
        try:
            return eval(raw, ns)  # noqa: S307 - the kernel author's own annotation text
        except Exception as exc:
            raise HawkError(f"{fn.__name__}: cannot read the annotation {raw!r}: {exc}") from None
    return raw


def trace(fn, scope: dict | None = None) -> Program:
    """Trace ``fn`` into a :class:`~hawk_amd.ir.Program`.  ``scope`` holds the
    names visible where the kernel was defined (a function's locals), so a
    string annotation resolves as it would at the definition."""
    ns = dict(fn.__globals__)
    if scope:
        ns.update(scope)
    if fn.__closure__:
        for name, cell in zip(fn.__code__.co_freevars, fn.__closure__):
            ns[name] = cell.cell_contents
    sig = inspect.signature(fn)
    program = Program()
    args, mutables, finishes = [], [], []
    axes_of = {}                     # a Mutable declared with lane axes -> its axes
    for p in sig.parameters.values():
        if p.kind not in (p.POSITIONAL_ONLY, p.POSITIONAL_OR_KEYWORD):
            raise HawkError(f"{fn.__name__}: parameter {p.name!r} must be a plain positional parameter")
        ann = _annotation(fn, p.annotation, ns)
        if ann is inspect.Parameter.empty:
            raise HawkError(f"{fn.__name__}: parameter {p.name!r} has no declaration "
                            "(Scalar, Vector[n], Matrix[r, c], Index, Param, Mutable[...])")
        if isinstance(ann, TableDecl):
            program.decls[p.name] = Decl(p.name, "lookup", TensorType((), "f64"))
            program.tables[p.name] = ann.axes
            args.append(TableRef(p.name, ann))
        elif isinstance(ann, GridDecl):
            if program.grid is not None:
                raise HawkError(f"{fn.__name__}: one Grid parameter declares the lanes; {p.name!r} is a second")
            program.grid = ann
            args.append(LaneRef(ann))
        elif isinstance(ann, MutableDecl):
            program.decls[p.name] = Decl(p.name, "mutable", ann.ttype)
            if ann.axes:
                axes_of[p.name] = ann.axes
            args.append(MutableRef(p.name, ann.ttype))
            mutables.append(p.name)
        elif isinstance(ann, _TerminatedDecl):
            ttype = TensorType((), "bool")
            program.decls[p.name] = Decl(p.name, "terminated", ttype)
            args.append(Value(ir.leaf("terminated", p.name, ttype)))
            finishes.append(p.name)
        elif isinstance(ann, _ParamDecl):
            program.decls[p.name] = Decl(p.name, "uniform", TensorType((), "f64"))
            args.append(Value(ir.leaf("uniform", p.name, TensorType((), "f64"))))
        elif isinstance(ann, TensorType):
            role = role_of(ann)
            program.decls[p.name] = Decl(p.name, role, ann)
            args.append(Value(ir.leaf(role, p.name, ann)))
        else:
            raise HawkError(f"{fn.__name__}: parameter {p.name!r} is declared {ann!r}, which is not "
                            "Scalar, Vector[n], Matrix[r, c], Index, Param or Mutable[...]")
    try:
        body = _rewritten(fn, tuple(mutables), tuple(finishes))
        with _Trace(program.grid) as tr:
            ret, finals = body(*args)
    except FinishRefusal as exc:
        raise HawkError(f"kernel {fn.__name__!r}: {exc}") from None

    def keyed(name: str, red: Reduced):
        """The SampleSum committing ``red`` into ``name`` (a Mutable declared
        with the kept axes, or the returned ``out``)."""
        axes = axes_of.get(name)
        if red.group is None:
            if axes:
                raise HawkError(f"{name!r} is declared with lane axes {[a for a, _ in axes]} but assigned a sum "
                                "over every sample (one cell); declare Mutable[Scalar]")
            shape = red.node.ttype.shape
            if not shape:
                return [SampleSum(name, red.node, red.policy, op=red.op)]
            # a vector or matrix cell: one scalar reduction per entry, row-major
            count = 1
            for e in shape:
                count *= e
            idx = [divmod(k, shape[1]) if len(shape) == 2 else k for k in range(count)]
            return [SampleSum(name, make("component", (red.node,), i), red.policy, op=red.op, column=k)
                    for k, i in enumerate(idx)]
        grid_axes = dict(program.grid.axes)
        if axes is not None:
            if tuple(a for a, _ in axes) != red.kept or any(
                    e is not None and grid_axes[a] is not None and e != grid_axes[a] for a, e in axes):
                raise HawkError(f"{name!r} is declared with lane axes {list(axes)} but holds the sum over the "
                                f"other axes, one value per {list(red.kept)} coordinate")
        return [SampleSum(name, red.node, red.policy, red.group)]
    sinks = list(tr.sinks)
    for name in mutables:
        final = finals[name]
        decl = program.decls[name]
        if isinstance(final, MutableRef) and final.name == name:
            continue                      # never assigned per lane (a scatter target, or unused)
        if isinstance(final, Reduced):
            if decl.ttype.shape != final.node.ttype.shape:
                raise HawkError(f"{name!r}: hawk.{final.op} of a value of shape {final.node.ttype.shape or 'scalar'} "
                                f"commits a cell of that shape; {name!r} is declared "
                                f"{decl.ttype.shape or 'scalar'}")
            if final.group is not None and name not in axes_of:
                raise HawkError(f"{name!r} holds hawk.sum over some lane axes, one value per "
                                f"{list(final.kept)} coordinate: declare it Mutable[{', '.join(repr(k) for k in final.kept)}]")
            sinks.extend(keyed(name, final))
            continue
        if name in axes_of:
            raise HawkError(f"{name!r} is declared with lane axes: it holds hawk.sum(x, over=...), "
                            "not a per-sample value")
        node = _projected(node_of(final))
        if node.ttype.shape != decl.ttype.shape:
            if node.ttype.shape == ():
                node = make("splat", (node,), decl.ttype.shape)
            else:
                raise HawkError(f"{name!r} is declared {decl.ttype.shape or 'scalar'} but assigned a value "
                                f"of shape {node.ttype.shape}")
        sinks.append(Assign(name, ir.as_real(node), "mutable"))
    if ret is not None:
        ret_ann = _annotation(fn, sig.return_annotation, ns)
        if isinstance(ret, Reduced):
            program.decls["out"] = Decl("out", "mutable", TensorType(ret.node.ttype.shape, "f64"))
            sinks.extend(keyed("out", ret))
        else:
            node = ir.as_real(_projected(node_of(ret)))
            if isinstance(ret_ann, TensorType) and ret_ann.shape != node.ttype.shape:
                if node.ttype.shape == ():
                    node = make("splat", (node,), ret_ann.shape)
                else:
                    raise HawkError(f"{fn.__name__} returns shape {node.ttype.shape}, annotated {ret_ann.shape}")
            program.decls["out"] = Decl("out", "out", node.ttype)
            sinks.append(Assign("out", node, "out"))
    for name, arg in zip(sig.parameters, args):
        if name not in finishes or finals[name] is arg:
            continue                      # a mask read, never finished
        final = finals[name]
        if isinstance(final, bool):
            raise HawkError(f"kernel {fn.__name__!r}: {name!r} = {final}: a Python literal is no per-sample "
                            "condition; finish on a traced comparison")
        node = node_of(final)
        if node.ttype != TensorType((), "bool"):
            raise HawkError(f"kernel {fn.__name__!r}: {name!r} is finished with a {node.ttype}; a sample "
                            "finishes on a traced rank-0 bool")
        if name != GUARD_MASK:
            raise HawkError(f"kernel {fn.__name__!r}: finishes the mask {name!r}, which the guard does not gate "
                            f"on ([{GUARD_MASK!r}]); a kernel finishes only the mask its guard skips")
        program.decls[FINISHED_PLANE] = Decl(FINISHED_PLANE, "lookup", TensorType((), "u32"))
        sinks.append(Finish(name, node))
    if not sinks:
        raise HawkError(f"{fn.__name__}: the kernel commits nothing (assign a Mutable, return a value, "
                        "or hawk.scatter into one)")
    names = [s.name for s in sinks if not isinstance(s, AccumWrite) and not (isinstance(s, SampleSum) and s.column)]
    dup = sorted({n for n in names if names.count(n) > 1})
    if dup:
        raise HawkError(f"{fn.__name__}: {dup} are committed twice")
    program.sinks = sinks
    return program


class Kernel:
    """A traced kernel (or a derivative of one): a name and its
    :class:`~hawk_amd.ir.Program`.  ``Kernel("energy_vjp", vjp(energy, wrt=("v",)))``
    names a derivative, as the reference spells it (``README.md:75``)."""

    def __init__(self, name: str, program):
        if callable(program) and not isinstance(program, Program):
            program = trace(program)
        if not isinstance(program, Program):
            raise HawkError(f"Kernel({name!r}, ...) takes a traced program (vjp/jvp's result) or a function")
        if not name.isidentifier():
            raise HawkError(f"kernel name {name!r} is not an identifier")
        self.name = name
        self.program = program

    @property
    def decls(self) -> dict:
        return self.program.decls

    @property
    def sinks(self) -> list:
        return self.program.sinks

    @property
    def arg_spec(self) -> list:
        """``[(role, name)]`` of the planes the kernel binds, in the ABI's role order."""
        return ir.arg_spec(self.program, ir.used_names(self.program))

    def __repr__(self) -> str:
        return f"<hawk kernel {self.name}: {[type(s).__name__ + ':' + s.name for s in self.sinks]}>"


def steps(kernel: Kernel, K) -> Kernel:
    """``kernel`` stepping up to ``K`` times a launch, named ``<name>_x<K>``
    (reference ``hawk/trace/steps.py:81-99``).

    ``kernel`` finishes its own sample (``terminated = cond``) and commits
    only ``Mutable`` planes.  The step becomes one rolled loop of ``K`` trips
    whose carries are those planes (each launch-start read becomes the carry,
    each commit its next value) and whose exit is the finish condition,
    evaluated after the step (a tail break: a sample finishing at trip ``j``
    keeps step ``j``'s values).  After the loop the carries commit and the
    finish fires with the loop's exit.  Each trip evaluates the same DAG as
    one launch of ``kernel``, so K launches of ``kernel`` and one of the
    result give the same bits (the build does not contract multiply-adds).
    A sample may run up to ``K - 1`` steps past a caller's own step cap.

    ``K="auto"`` names the result ``<name>_xauto``: its trip count is read at
    launch from the one-cell ``fused_steps`` word, which the runtime sets
    (``hawk.run(..., steps=W)``, default 1; a word below 0 runs none), and it
    also builds the ``_range`` and ``_persist`` entries that report the
    steps taken (reference ``hawk/trace/steps.py:27-44``)."""
    if not isinstance(kernel, Kernel):
        raise HawkError("hawk.steps(kernel, K) takes a traced kernel")
    kernel = default_step(kernel)
    name = kernel.name
    auto = K == "auto"
    if not auto and (isinstance(K, bool) or not isinstance(K, int) or K < 1):
        raise HawkError(f"hawk.steps({name!r}, {K!r}): K is an int >= 1 or 'auto'")
    if auto and ir.FUSED_STEPS_PLANE in kernel.decls:
        raise HawkError(f"hawk.steps({name!r}, 'auto'): {ir.FUSED_STEPS_PLANE!r} is reserved for the trip "
                        "count of an automatic kernel; rename that parameter")
    program = kernel.program
    finishes = [s for s in program.sinks if isinstance(s, Finish)]
    if not finishes:
        raise HawkError(f"hawk.steps({name!r}): the kernel never finishes its sample -- K steps with no exit "
                        "is a plain `for` the author can write; finish with `terminated = cond`")
    finish = finishes[0]
    if finish.steps != 1:
        raise HawkError(f"hawk.steps({name!r}): the kernel already takes {finish.steps} steps a launch; "
                        "derive from the single step")
    commits = [s for s in program.sinks if s is not finish]
    for s in commits:
        if not (isinstance(s, Assign) and s.role == "mutable"):
            raise HawkError(f"hawk.steps({name!r}): a {type(s).__name__} into {s.name!r} is not a step "
                            "kernel's commit; a step kernel commits Mutable planes and finishes -- an "
                            "out, a sum or a scatter has no per-sample state to carry from one step to the next")
    if not commits:
        raise HawkError(f"hawk.steps({name!r}): the kernel commits no Mutable plane, so there is no state "
                        "to step")
    carried = {s.name for s in commits}
    roots = [s.value for s in commits] + [finish.value]
    reads = [n for n in ir.leaves_of(roots) if n.literal[0] == "mutable" and n.literal[1] in carried]
    read_ids = {n.uid for n in reads}
    for loop in (n for n in ir.topo(roots) if n.kind == "loop"):
        if any(m.uid in read_ids for m in ir.topo([loop])):
            raise HawkError(f"hawk.steps({name!r}): a loop of the step reads the carried state; carry it "
                            "through a step without inner loops over it")
    slot = {s.name: j for j, s in enumerate(commits)}
    inits = []
    for s in commits:
        decl = program.decls[s.name]
        inits.append(ir.leaf("mutable", s.name, decl.ttype))

    def body(index, *carries):
        mapping = {n.uid: carries[slot[n.literal[1]]] for n in reads}
        return tuple(ir.substitute(roots, mapping))

    loop = ir.new_loop(ir.AUTO_K_MAX if auto else K, 0, 1, tuple(inits), body, tuple(s.name for s in commits),
                       exits=True)
    decls = dict(program.decls)
    if auto:
        loop.literal.count = ir.FUSED_STEPS_PLANE
        decls[ir.FUSED_STEPS_PLANE] = Decl(ir.FUSED_STEPS_PLANE, "lookup", TensorType((), "i32"))
    sinks = [Assign(s.name, ir.loop_value(loop, j), "mutable") for j, s in enumerate(commits)]
    sinks.append(Finish(finish.name, ir.loop_exit(loop), steps=K))
    stepped = Kernel(f"{name}_x{K}", Program(decls, sinks, program.grid, dict(program.tables)))
    stepped.step = kernel
    return stepped


def admits_auto(kernel: Kernel) -> bool:
    """Whether ``kernel`` is a single step that ``hawk.steps(kernel, "auto")``
    admits (reference ``hawk/trace/steps.py:119-132``): it finishes its own
    sample once, commits at least one Mutable plane and nothing else, and
    declares no ``fused_steps`` plane."""
    sinks = list(kernel.sinks)
    finishes = [s for s in sinks if isinstance(s, Finish)]
    if len(finishes) != 1 or finishes[0].steps != 1:
        return False
    commits = [s for s in sinks if s is not finishes[0]]
    if not commits or not all(isinstance(s, Assign) and s.role == "mutable" for s in commits):
        return False
    return ir.FUSED_STEPS_PLANE not in kernel.decls


def default_step(kernel: Kernel) -> Kernel:
    """The single step a default automatic kernel stands for (its ``.step``,
    under the same name), else ``kernel`` (reference ``hawk/trace/steps.py:101-109``)."""
    step = getattr(kernel, "step", None)
    return step if step is not None and step.name == kernel.name else kernel


def kernel(fn=None, *, name: str | None = None, steps=None):
    """``@hawk.kernel``: trace a per-sample function into a :class:`Kernel`.

    A kernel that finishes its own sample and commits only Mutable planes is
    built, with no ``steps=``, as its automatic kernel under its own name (its
    trip count read at launch, ``.step`` the single step; reference
    ``hawk/trace/steps.py:39-44``); ``steps=1`` keeps the single step and
    ``steps=K`` is ``hawk.steps(kernel, K)``.  A step whose loop
    :func:`steps` refuses (an inner loop over the carried state) stays a
    single step."""
    def wrap(f, scope):
        k = Kernel(name or f.__name__, trace(f, scope))
        if steps == 1:
            return k
        if steps is not None:
            return globals()["steps"](k, steps)
        if not admits_auto(k):
            return k
        try:
            auto = globals()["steps"](k, "auto")
        except HawkError:
            return k                  # a step the loop cannot carry stays a single step
        auto.name = k.name
        return auto
    caller = inspect.currentframe().f_back
    scope = dict(caller.f_locals) if caller is not None else None
    if fn is not None:
        return wrap(fn, scope)
    return lambda f: wrap(f, scope)
