"""The tensor-typed IR of hawk's gfx950 target.

One node family (:class:`Node`): a ``kind``, its ``operands``, a static
:class:`~hawk_amd.types.TensorType` and an optional ``literal``.  Scalars,
vectors and matrices are all nodes; the emitter scalarises them.  A rolled
``for`` is one ``loop`` node whose body is the ``nexts`` of its carried slots
(reference ``hawk/ir/loops.py``), read back through ``loop_value``; a reversed
loop reads the forward loop's per-iteration carries through ``tape_read``
(reference ``hawk/diff/loops.py:484-540``).

Sinks are what a kernel commits: a per-sample :class:`Assign`, an
over-every-sample :class:`SampleSum` (``hawk.sum``) and a keyed
:class:`AccumWrite` (``hawk.scatter``), as reference ``hawk/ir/nodes.py``;
a VJP adds :class:`OrderedFold`, a table's gradient under an ordered keyed sum.
"""

from __future__ import annotations

import itertools
from dataclasses import dataclass, field

from .types import HawkError, TensorType   # noqa: F401 - HawkError is re-exported


#: Canonical role order of ``arg_spec`` == the entry-signature order
#: (reference ``hawk/ir/nodes.py:51-52``).
#: ``rows_out`` is this target's own: the per-32-sample compensated row
#: partials of a default-policy ``hawk.sum``, which the reference keeps as
#: runtime-owned scratch rather than kernel arguments.
ROLE_ORDER = ("mutable", "out", "wide_out", "key_out", "accum_out", "fold_scratch", "rows_out", "vec_in",
              "mat_in", "wide_in", "per_sample", "lookup", "terminated", "uniform", "nsamples")

UNARY = ("neg", "exp", "sin", "cos", "tanh", "sqrt", "abs", "log", "real")
BINARY = ("add", "sub", "mul", "div")
COMPARE = ("lt", "le", "gt", "ge", "eq", "ne")
ELEMENTWISE = UNARY + BINARY + COMPARE + ("select",)

_uid = itertools.count(1)


class Node:
    """One IR node.  Identity is the object: two structurally equal nodes are
    two values (the emitter and the compiler fold duplicates)."""

    __slots__ = ("kind", "operands", "ttype", "literal", "uid")

    def __init__(self, kind: str, operands: tuple, ttype: TensorType, literal=None):
        self.kind = kind
        self.operands = tuple(operands)
        self.ttype = ttype
        self.literal = literal
        self.uid = next(_uid)

    def __repr__(self) -> str:
        lit = "" if self.literal is None else f" {self.literal!r}"
        return f"<{self.kind}#{self.uid}{lit} {self.ttype.shape}{self.ttype.dtype}>"


@dataclass
class LoopInfo:
    """The static half of a ``loop`` node: trip, index and carried slots."""

    trip: int
    start: int
    step: int
    index: Node                      # kind "loop_index"
    carries: tuple                   # kind "carry" placeholders, one per slot
    nexts: tuple                     # the body's value of each slot
    names: tuple = ()                # the authored names of the slots (diagnostics)
    unroll: bool | None = None       # True: #pragma unroll; False: kept rolled; None: the compiler's choice
    exit: Node | None = None         # a bool over the trip's inputs: when true, the trip's nexts stand and the loop ends
    count: str | None = None         # a one-cell int32 plane read at launch: the trips run (start 0, step 1)

    def stop(self) -> int:
        return self.start + self.trip * self.step


# --------------------------------------------------------------------------
# constructors


def const(value: float, dtype: str = "f64") -> Node:
    return Node("const", (), TensorType((), dtype), float(value))


def index_const(value: int) -> Node:
    return Node("iconst", (), TensorType((), "i64"), int(value))


def leaf(role: str, name: str, ttype: TensorType) -> Node:
    return Node("leaf", (), ttype, (role, name))


def _broadcast(a: TensorType, b: TensorType, kind: str) -> tuple:
    if a.shape == b.shape:
        return a.shape
    if a.shape == ():
        return b.shape
    if b.shape == ():
        return a.shape
    raise HawkError(f"{kind}: operands of shapes {a.shape} and {b.shape} do not broadcast "
                    "(a scalar broadcasts; two tensors must have one shape)")


def _real_dtype(*nodes: Node) -> str:
    for n in nodes:
        if n.ttype.dtype in ("f64", "f32"):
            return n.ttype.dtype
    return "f64"


def as_real(n: Node) -> Node:
    """An integer value (a loop index, an int constant) as a real."""
    if n.ttype.dtype in ("f64", "f32"):
        return n
    if n.ttype.dtype == "bool":
        raise HawkError("a bool mask is not a number; use hawk.math.where(mask, a, b)")
    if n.kind == "iconst":
        return const(float(n.literal))
    return Node("real", (n,), TensorType(n.ttype.shape, "f64"))


_INTS = ("i32", "i64")


def make(kind: str, operands: tuple, literal=None) -> Node:
    """Build a node of ``kind``, typing it from its operands."""
    ops = tuple(operands)
    if kind in ("add", "sub", "mul", "floordiv", "mod") and all(
            o.ttype.dtype in _INTS and not o.ttype.shape for o in ops):
        # index arithmetic stays integer (64-bit when either side is); floordiv
        # and mod round toward minus infinity, as Python's // and %
        dt = "i64" if any(o.ttype.dtype == "i64" for o in ops) else "i32"
        return Node(kind, ops, TensorType((), dt))
    if kind in ("floordiv", "mod"):
        raise HawkError(f"{'//' if kind == 'floordiv' else '%'} takes two Index values (integers)")
    if kind in BINARY:
        a, b = (as_real(o) for o in ops)
        return Node(kind, (a, b), TensorType(_broadcast(a.ttype, b.ttype, kind), _real_dtype(a, b)))
    if kind in UNARY:
        (a,) = ops
        if kind == "real":
            return as_real(a)
        a = as_real(a)
        return Node(kind, (a,), TensorType(a.ttype.shape, a.ttype.dtype))
    if kind in COMPARE:
        a, b = (as_real(o) for o in ops)
        shape = _broadcast(a.ttype, b.ttype, kind)
        if shape:
            raise HawkError(f"{kind}: comparisons are per scalar in this build")
        return Node(kind, (a, b), TensorType((), "bool"))
    if kind == "select":
        cond, a, b = ops
        a, b = as_real(a), as_real(b)
        shape = _broadcast(a.ttype, b.ttype, "select")
        if a.ttype.shape != shape:
            a = make("splat", (a,), shape)
        if b.ttype.shape != shape:
            b = make("splat", (b,), shape)
        return Node(kind, (cond, a, b), TensorType(shape, _real_dtype(a, b)))
    if kind == "splat":
        (a,) = ops
        a = as_real(a)
        if a.ttype.shape:
            raise HawkError("splat widens a scalar")
        return Node(kind, (a,), TensorType(tuple(literal), a.ttype.dtype), tuple(literal))
    if kind == "dot":
        a, b = ops
        if len(a.ttype.shape) != 1 or a.ttype.shape != b.ttype.shape:
            raise HawkError(f"dot takes two vectors of one width, got {a.ttype.shape} and {b.ttype.shape}")
        return Node(kind, (a, b), TensorType((), _real_dtype(a, b)))
    if kind == "norm":
        (a,) = ops
        if len(a.ttype.shape) != 1:
            raise HawkError("norm takes a vector")
        return Node(kind, (a,), TensorType((), a.ttype.dtype))
    if kind == "sum":
        (a,) = ops
        return Node(kind, (a,), TensorType((), a.ttype.dtype))
    if kind == "sample_count":
        # the run's sample count (the entry's nSamples: every sample of the
        # run, not only this launch's partition), as a real
        return Node(kind, (), TensorType((), "f64"))
    if kind == "component":
        (a,) = ops
        shape = a.ttype.shape
        idx = literal if isinstance(literal, tuple) else (literal,)
        if len(idx) != len(shape) or any(not (0 <= i < e) for i, e in zip(idx, shape)):
            raise HawkError(f"index {literal!r} is outside a value of shape {shape}")
        return Node(kind, (a,), TensorType((), a.ttype.dtype), idx if len(idx) > 1 else idx[0])
    if kind == "vec":
        parts = tuple(as_real(o) for o in ops)
        if any(p.ttype.shape for p in parts):
            raise HawkError("vec/mat take scalar entries")
        shape = tuple(literal) if literal is not None else (len(parts),)
        count = 1
        for e in shape:
            count *= e
        if count != len(parts):
            raise HawkError(f"{len(parts)} entries do not fill shape {shape}")
        return Node(kind, parts, TensorType(shape, _real_dtype(*parts) if parts else "f64"), shape)
    if kind == "transpose":
        (a,) = ops
        if len(a.ttype.shape) != 2:
            raise HawkError("transpose takes a matrix")
        r, c = a.ttype.shape
        return Node(kind, (a,), TensorType((c, r), a.ttype.dtype))
    if kind == "mv":
        m, v = ops
        if len(m.ttype.shape) != 2 or len(v.ttype.shape) != 1 or m.ttype.shape[1] != v.ttype.shape[0]:
            raise HawkError(f"matrix @ vector: shapes {m.ttype.shape} and {v.ttype.shape} disagree")
        return Node(kind, (m, v), TensorType((m.ttype.shape[0],), _real_dtype(m, v)))
    if kind == "mm":
        a, b = ops
        if len(a.ttype.shape) != 2 or len(b.ttype.shape) != 2 or a.ttype.shape[1] != b.ttype.shape[0]:
            raise HawkError(f"matrix @ matrix: shapes {a.ttype.shape} and {b.ttype.shape} disagree")
        return Node(kind, (a, b), TensorType((a.ttype.shape[0], b.ttype.shape[1]), _real_dtype(a, b)))
    if kind == "outer":
        a, b = ops
        if len(a.ttype.shape) != 1 or len(b.ttype.shape) != 1:
            raise HawkError("outer takes two vectors")
        return Node(kind, (a, b), TensorType((a.ttype.shape[0], b.ttype.shape[0]), _real_dtype(a, b)))
    if kind == "chol":
        (a,) = ops
        if len(a.ttype.shape) != 2 or a.ttype.shape[0] != a.ttype.shape[1]:
            raise HawkError("cholesky takes a square matrix")
        return Node(kind, (a,), TensorType(a.ttype.shape, a.ttype.dtype, "chol_factor"))
    if kind == "chol_factor":
        (f,) = ops
        return Node(kind, (f,), TensorType(f.ttype.shape, f.ttype.dtype))
    if kind == "chol_info":
        (f,) = ops
        return Node(kind, (f,), TensorType((), "i32"))
    if kind == "cho_solve":
        f, b = ops
        if f.ttype.tag != "chol_factor":
            raise HawkError("cho_solve reads the factor that cholesky() returned, not a matrix "
                            f"built or changed since (got {f.ttype!r})")
        if len(b.ttype.shape) != 1 or b.ttype.shape[0] != f.ttype.shape[0]:
            raise HawkError(f"cho_solve: a right-hand side of shape {b.ttype.shape} for a "
                            f"{f.ttype.shape[0]}x{f.ttype.shape[0]} factor (a vector is supported)")
        return Node(kind, (f, b), TensorType(b.ttype.shape, _real_dtype(b)))
    if kind == "lane_axis":
        # a coordinate of the lane on its Grid: (sample // div) % mod (no mod
        # for the first axis), an Index; mod == 0 and div == 1 is the flat index
        div, mod = literal
        if mod == 0:
            return Node(kind, (), TensorType((), "i64"), (1, 0))
        return Node(kind, (), TensorType((), "i32"), (int(div), None if mod is None else int(mod)))
    if kind == "gather":
        # table[key] of a 1-D plane of cells (role "lookup").  literal None: a
        # key outside [0, cells) — the skip key -1 of hawk.scatter among them —
        # reads 0.  literal ("clamp", extents): the key is one index per axis
        # of a table of those extents (None: the first axis's, from the bound
        # cells), each clamped into [0, extent), read at their row-major flat
        # position (a Table read, reference tests/test_table_clamp.py:1-8).
        table, *keys = ops
        if table.kind != "leaf" or table.literal[0] != "lookup" or table.ttype.shape:
            raise HawkError("gather reads a scalar lookup plane (a 1-D plane of cells)")
        if any(k.ttype.dtype not in _INTS or k.ttype.shape for k in keys):
            raise HawkError(f"gather: a key is an Index (an integer), got {[k.ttype for k in keys]}")
        if literal is None and len(keys) != 1:
            raise HawkError("gather: one key")
        if literal is not None and (literal[0] != "clamp" or len(literal[1]) != len(keys)):
            raise HawkError("gather: one key per table axis")
        return Node(kind, (table, *keys), TensorType((), table.ttype.dtype), literal)
    if kind == "table_index":
        # the flat cell a clamped table read reads (the key of its gradient's
        # scatter, an Index): the same clamp and row-major flattening as the gather
        table, *keys = ops
        return Node(kind, (table, *keys), TensorType((), "i32"), literal)
    raise HawkError(f"no IR kind {kind!r}")


def zero_like(t: TensorType) -> Node:
    z = const(0.0)
    return z if t.shape == () else make("splat", (z,), t.shape)


def is_zero(n: Node) -> bool:
    if n.kind == "const":
        return n.literal == 0.0
    if n.kind == "splat":
        return is_zero(n.operands[0])
    return False


def new_loop(trip: int, start: int, step: int, inits: tuple, body, names: tuple = (),
             exits: bool = False) -> Node:
    """A rolled loop: ``body(index, *carries) -> nexts`` traced once over
    placeholders typed like ``inits``.  With ``exits`` the body gives one more
    value, a bool: a lane for which it is true keeps that trip's nexts and
    leaves the loop (a tail break)."""
    uid = next(_uid)
    index = Node("loop_index", (), TensorType((), "i64"), uid)
    carries = tuple(Node("carry", (), as_real(x).ttype if x.ttype.dtype != "i64" else x.ttype, (uid, j))
                    for j, x in enumerate(inits))
    nexts = tuple(body(index, *carries))
    exit = None
    if exits:
        nexts, exit = nexts[:-1], nexts[-1]
        if exit.ttype != TensorType((), "bool"):
            raise HawkError(f"a loop's exit is a rank-0 bool, got {exit.ttype}")
    return loop_node(uid, trip, start, step, index, carries, tuple(inits), nexts, names, exit=exit)


def loop_node(uid: int, trip: int, start: int, step: int, index: Node, carries: tuple,
              inits: tuple, nexts: tuple, names: tuple = (), exit: Node | None = None) -> Node:
    if len(nexts) != len(carries):
        raise HawkError("a loop body must give one value per carried slot")
    fixed = []
    for j, (c, x) in enumerate(zip(carries, nexts)):
        if x.ttype.shape != c.ttype.shape:
            if x.ttype.shape and not c.ttype.shape:
                raise HawkError(f"loop slot {names[j] if j < len(names) else j!r} changes shape in the body: "
                                f"{c.ttype.shape} before, {x.ttype.shape} after")
            x = make("splat", (as_real(x),), c.ttype.shape)
        fixed.append(as_real(x) if c.ttype.dtype in ("f64", "f32") else x)
    info = LoopInfo(trip, start, step, index, tuple(carries), tuple(fixed), tuple(names), exit=exit)
    node = Node("loop", tuple(as_real(x) if c.ttype.dtype in ("f64", "f32") else x
                              for c, x in zip(carries, inits)), TensorType((), "tuple"), info)
    node.uid = uid
    return node


def loop_value(loop: Node, j: int) -> Node:
    return Node("loop_value", (loop,), loop.literal.carries[j].ttype, j)


def loop_exit(loop: Node) -> Node:
    """Whether ``loop`` ended on its exit condition (rather than its trip count)."""
    return Node("loop_exit", (loop,), TensorType((), "bool"))


def body_roots(info: LoopInfo) -> tuple:
    """The nodes a loop's body computes each trip: its nexts and its exit."""
    return tuple(info.nexts) + ((info.exit,) if info.exit is not None else ())


def tape_read(loop: Node, j: int, index: Node) -> Node:
    """Carry ``j`` of the forward ``loop`` as it stood at the START of the
    iteration whose index value ``index`` holds."""
    return Node("tape_read", (loop, index), loop.literal.carries[j].ttype, j)


# --------------------------------------------------------------------------
# loop structure (shared by the emitter and autodiff)


class Deps:
    """Which loops (by the uid of their index node) each node depends on."""

    def __init__(self):
        self.memo: dict = {}
        self.owner: dict = {}          # carry/index uid -> loop index uid

    def register(self, loop: Node) -> None:
        info = loop.literal
        key = info.index.uid
        self.owner[info.index.uid] = key
        for c in info.carries:
            self.owner[c.uid] = key

    def of(self, n: Node) -> frozenset:
        hit = self.memo.get(n.uid)
        if hit is not None:
            return hit
        order = topo([n])
        for m in order:             # every loop first: a carry is reached before its loop
            if m.kind == "loop":
                self.register(m)
        for m in order:
            if m.uid in self.memo:
                continue
            if m.kind in ("carry", "loop_index"):
                own = self.owner.get(m.uid)
                self.memo[m.uid] = frozenset() if own is None else frozenset((own,))
                continue
            deps = set()
            for o in m.operands:
                deps |= self.memo[o.uid]
            if m.kind == "loop":
                inner = set()
                for x in body_roots(m.literal):
                    inner |= self.memo[x.uid]
                inner.discard(m.literal.index.uid)
                deps |= inner
            self.memo[m.uid] = frozenset(deps)
        return self.memo[n.uid]


def free_inputs(loop: Node, deps: Deps) -> list:
    """The nodes outside ``loop`` its body reads, in first-reach order: a walk
    from the body's values that stops at every node not depending on the loop
    and sees a nested loop as one node whose operands are its inits and its own
    free inputs (never the nodes inside the nested body)."""
    deps.register(loop)
    for n in topo(body_roots(loop.literal)):    # a body can reach other loops (a tape read's loop)
        if n.kind == "loop":
            deps.register(n)
    key = loop.literal.index.uid
    out, seen, expanded = [], set(), set()
    stack = list(reversed(body_roots(loop.literal)))
    while stack:
        n = stack.pop()
        if key not in deps.of(n):
            if n.uid not in seen and n.kind not in ("const", "iconst"):
                seen.add(n.uid)
                out.append(n)
            continue
        if n.uid in expanded:
            continue
        expanded.add(n.uid)
        kids = list(n.operands)
        if n.kind == "loop" and n is not loop:
            kids += free_inputs(n, deps)
        stack.extend(reversed(kids))
    return out


def level_order(roots, deps: Deps, stops=frozenset()) -> list:
    """Nodes reachable from ``roots`` at this level: a loop is opaque, its
    operands being its inits and its body's free inputs.  Nodes in ``stops``
    are reached but not expanded."""
    order, seen = [], set()
    stack = [(r, False) for r in reversed(list(roots))]
    while stack:
        node, expanded = stack.pop()
        if expanded:
            order.append(node)
            continue
        if node.uid in seen:
            continue
        seen.add(node.uid)
        stack.append((node, True))
        if node.uid in stops:
            continue
        kids = list(node.operands)
        if node.kind == "loop":
            kids += free_inputs(node, deps)
        for k in reversed(kids):
            if k.uid not in seen:
                stack.append((k, False))
    return order


def fresh_placeholders(loop: Node) -> tuple:
    """New index and carry placeholders for a copy of ``loop``'s body, and the
    substitution map from the old ones."""
    info = loop.literal
    uid = next(_uid)
    index = Node("loop_index", (), info.index.ttype, uid)
    carries = tuple(Node("carry", (), c.ttype, (uid, j)) for j, c in enumerate(info.carries))
    mapping = {info.index.uid: index, **{c.uid: nc for c, nc in zip(info.carries, carries)}}
    return uid, index, carries, mapping


# --------------------------------------------------------------------------
# sinks


@dataclass
class Assign:
    """The per-sample commit of ``value`` into the plane ``name``."""

    name: str
    value: Node
    role: str = "mutable"


@dataclass
class SampleSum:
    """``name = hawk.sum(value, policy=...)``: one cell over every sample; with
    ``group`` (``hawk.sum(value, over=<trailing lane axes>)``), one cell per
    run of ``group`` consecutive samples (one per coordinate of the kept
    leading axes).  ``op`` is the reduction: "sum" (``hawk.mean`` is the sum
    of each term over the sample count), "max" or "min" (reference
    ``hawk/trace/reduce.py:304-334``).  ``column`` is the flat entry of a
    vector or matrix cell this scalar reduction commits (one row plane per
    column, reference ``hawk/_cells.py:33-35``); None for a scalar cell."""

    name: str
    value: Node
    policy: str = "ordered"
    group: int | None = None
    op: str = "sum"
    column: int | None = None


@dataclass
class AccumWrite:
    """``hawk.scatter(name, policy=...)[key] += value``."""

    name: str
    value: Node
    key: Node
    policy: str = "ordered"


@dataclass
class Finish:
    """``terminated = cond``: the kernel finishes its own sample (reference
    ``hawk/ir/nodes.py:848-870``): the mask ``name`` becomes ``mask | cond``
    and each newly finished sample adds one to the ``finished_count`` cell."""

    name: str
    value: Node
    steps: int | str = 1             # the steps one launch takes (hawk.steps): 1 as authored, K, or "auto"


#: The one-cell counter a finishing kernel adds its newly finished samples to
#: (reference ``hawk/ir/nodes.py:839``).
FINISHED_PLANE = "finished_count"
#: The only mask a kernel's guard gates on: the ``Terminated`` parameter of this name.
GUARD_MASK = "terminated"
#: The one-cell int32 word a ``steps="auto"`` kernel reads its trip count
#: from (reference ``hawk/ir/nodes.py:841-845``): set by the runtime, never
#: bound by the caller.
FUSED_STEPS_PLANE = "fused_steps"
#: The static bound an automatic kernel records (reference ``hawk/trace/steps.py:70``).
AUTO_K_MAX = 64


@dataclass
class OrderedFold:
    """The gradient of a table read by key under an ordered keyed sum
    (reference ``hawk/diff/ordered.py``): ``values[e]`` is a lane's e-th
    contribution and ``cells[e]`` the table cell it adds to, one cell per key
    (a run of ``group`` consecutive samples).  For each key and slot the key's
    contributions are added in lane order, starting from +0, and the sum is
    stored into that cell."""

    name: str
    values: tuple
    cells: tuple
    group: int


@dataclass
class Decl:
    """One declared plane or uniform of a kernel."""

    name: str
    role: str            # per_sample / vec_in / mat_in / uniform / mutable / out
    ttype: TensorType


@dataclass
class Program:
    """What a kernel is: its declarations and its sinks (a traced kernel, or a
    derivative of one)."""

    decls: dict = field(default_factory=dict)     # name -> Decl, declaration order
    sinks: list = field(default_factory=list)
    grid: object = None                           # the GridDecl of the launch's lane axes, if declared
    tables: dict = field(default_factory=dict)    # a Table plane's name -> its axes ((label, extent|None), ...)


# --------------------------------------------------------------------------
# walks


def sink_roots(sinks) -> list:
    roots = []
    for s in sinks:
        if isinstance(s, OrderedFold):
            roots += list(s.values) + list(s.cells)
            continue
        roots.append(s.value)
        if isinstance(s, AccumWrite):
            roots.append(s.key)
    return roots


def topo(roots) -> list:
    """Every node reachable from ``roots`` (through operands and loop bodies),
    operands first.  Iterative, so deep chains do not hit Python's recursion limit."""
    order, seen = [], set()
    stack = [(r, False) for r in reversed(list(roots))]
    while stack:
        node, expanded = stack.pop()
        if expanded:
            order.append(node)
            continue
        if node.uid in seen:
            continue
        seen.add(node.uid)
        stack.append((node, True))
        kids = list(node.operands)
        if node.kind == "loop":
            kids += list(body_roots(node.literal))
        for k in reversed(kids):
            if k.uid not in seen:
                stack.append((k, False))
    return order


def leaves_of(roots) -> list:
    """The ``leaf`` nodes reachable from ``roots``, first reach first."""
    return [n for n in topo(roots) if n.kind == "leaf"]


def substitute(roots, mapping: dict) -> list:
    """Copies of ``roots`` with every node whose uid is in ``mapping`` replaced;
    nodes that reach no replaced node are shared, not copied."""
    memo = dict(mapping)
    order = topo(roots)
    for n in order:
        if n.uid in memo:
            continue
        kids = n.operands
        new_kids = tuple(memo.get(k.uid, k) for k in kids)
        if n.kind == "loop":
            info = n.literal
            new_nexts = tuple(memo.get(x.uid, x) for x in info.nexts)
            new_exit = memo.get(info.exit.uid, info.exit) if info.exit is not None else None
            if any(a is not b for a, b in zip(new_kids, kids)) or new_exit is not info.exit or \
                    any(a is not b for a, b in zip(new_nexts, info.nexts)):
                copy = loop_node(next(_uid), info.trip, info.start, info.step, info.index,
                                 info.carries, new_kids, new_nexts, info.names, exit=new_exit)
                copy.literal.unroll = info.unroll
                copy.literal.count = info.count
                memo[n.uid] = copy
            continue
        if any(a is not b for a, b in zip(new_kids, kids)):
            copy = Node(n.kind, new_kids, n.ttype, n.literal)
            memo[n.uid] = copy
    return [memo.get(r.uid, r) for r in roots]


#: The most iterations :func:`unroll_reading` writes out for one loop.
UNROLL_MAX = 256


def unroll_reading(roots, reads) -> list:
    """``roots`` with every loop whose body reaches a node ``n`` with
    ``reads(n)`` written out iteration by iteration: iteration t's body over
    index ``start + t * step`` and the previous iteration's carries.  The
    operations and their order do not change, so neither do the bits; each
    iteration's nodes are then values of their own (a table read's gradient
    needs one log slot per iteration)."""
    roots = list(roots)
    while True:
        loop = next((n for n in topo(roots) if n.kind == "loop"
                     and any(reads(m) for m in topo(n.literal.nexts))), None)
        if loop is None:
            return roots
        info = loop.literal
        if info.trip > UNROLL_MAX:
            raise HawkError(f"a for loop of {info.trip} iterations reads a differentiated table; its gradient "
                            f"keeps one slot per read and iteration, written out for at most {UNROLL_MAX} "
                            "iterations")
        vals = list(loop.operands)
        for t in range(info.trip):
            mapping = {info.index.uid: index_const(info.start + t * info.step)}
            mapping.update({c.uid: v for c, v in zip(info.carries, vals)})
            vals = substitute(info.nexts, mapping)
        finals = {m.uid: vals[m.literal] for m in topo(roots)
                  if m.kind == "loop_value" and m.operands[0] is loop}
        roots = substitute(roots, finals)


def key_only(n: Node, group: int) -> bool:
    """Whether ``n`` takes one value per key (a run of ``group`` consecutive
    samples): it reads constants, uniforms, table planes and lane coordinates
    of the kept (leading) axes, and nothing per sample."""
    for m in topo([n]):
        if m.kind in ("const", "iconst"):
            continue
        if m.kind == "leaf":
            if m.literal[0] in ("uniform", "lookup"):
                continue
            return False
        if m.kind == "lane_axis":
            div, mod = m.literal
            if (mod == 0 and group != 1) or (mod != 0 and div % group):
                return False
            continue
        if m.kind in ("loop", "loop_value", "carry", "loop_index", "tape_read"):
            return False
    return True


#: Kinds whose presence makes a repeated subexpression worth a carried slot.
_COSTLY = frozenset(("sqrt", "div", "exp", "sin", "cos", "tanh", "log", "norm", "chol", "cho_solve"))


def _literal_key(lit):
    try:
        hash(lit)
        return lit
    except TypeError:
        return repr(lit)


def _carry_repeats_of(loop: Node, deps: Deps):
    """The loop with each costly body value that the next iteration would
    compute again carried instead, or ``None`` if there is none.

    A body node X that reads the carries (and not the loop index) is computed
    again by iteration k+1 exactly when the body also computes Y = X with every
    carry replaced by its next value: the same operations on the values that
    become iteration k+1's carries.  X then becomes a carried slot, initialised
    by X over the inits and advanced by Y, so iteration k+1 reads the value
    iteration k computed.  The bits do not change: every value is produced by
    the same operations, in the same order, from the same operands (the kernel
    is compiled without contraction)."""
    info = loop.literal
    if info.exit is not None:
        return None                           # a stepped loop's trips end on its exit
    key_of = info.index.uid
    deps.register(loop)
    carry_slot = {c.uid: j for j, c in enumerate(info.carries)}
    body = [m for m in topo(info.nexts) if key_of in deps.of(m)]
    if any(m.kind in ("loop", "loop_value", "tape_read") for m in body):
        return None                           # innermost loops without tapes only
    outside: dict = {}

    def ext(n: Node):
        # a value the body reads from outside the loop, keyed by structure so
        # that two equal computations (two `-mu` nodes) are one key
        hit = outside.get(n.uid)
        if hit is None:
            for m in topo([n]):
                if m.uid not in outside:
                    if m.kind in ("loop", "carry", "loop_index", "loop_value", "tape_read"):
                        outside[m.uid] = ("x", m.uid)
                    else:
                        outside[m.uid] = ("x", m.kind, _literal_key(m.literal), m.ttype,
                                          tuple(outside[o.uid] for o in m.operands))
            hit = outside[n.uid]
        return hit

    keys: dict = {}
    shifted: dict = {}
    costly: dict = {}
    for m in body:
        if m.uid in carry_slot:
            keys[m.uid] = ("c", carry_slot[m.uid])
            shifted[m.uid] = None             # filled below, once every next has a key
            costly[m.uid] = False
            continue
        if m is info.index:
            keys[m.uid] = ("i",)
            costly[m.uid] = False
            continue
        ops = []
        for o in m.operands:
            ops.append(keys[o.uid] if o.uid in keys else ext(o))
        keys[m.uid] = (m.kind, _literal_key(m.literal), m.ttype, tuple(ops))
        costly[m.uid] = m.kind in _COSTLY or any(costly.get(o.uid, False) for o in m.operands)
    for c in info.carries:
        x = info.nexts[carry_slot[c.uid]]
        shifted[c.uid] = keys[x.uid] if x.uid in keys else ext(x)
    by_key = {}
    for m in body:
        by_key.setdefault(keys[m.uid], m)
    for m in body:
        if m.uid in shifted or m is info.index:
            continue
        ops = []
        for o in m.operands:
            if o is info.index or (o.uid in keys and shifted.get(o.uid, 0) is None):
                ops = None
                break
            ops.append(shifted[o.uid] if o.uid in shifted else ext(o))
        shifted[m.uid] = None if ops is None else (m.kind, _literal_key(m.literal), m.ttype, tuple(ops))
    found = {}
    for m in body:
        if m.uid in carry_slot or m is info.index or not costly[m.uid]:
            continue
        s = shifted.get(m.uid)
        y = by_key.get(s) if s is not None else None
        if y is not None and y is not m:
            found[m.uid] = (m, y)
    if not found:
        return None
    users: dict = {}
    for m in body:
        for o in m.operands:
            users.setdefault(o.uid, set()).add(m.uid)
    roots = {x.uid for x in info.nexts}
    chosen = [(x, y) for u, (x, y) in found.items()
              if u in roots or any(v not in found for v in users.get(u, ()))]
    if not chosen:
        return None
    slot0 = len(info.carries)
    places = tuple(Node("carry", (), x.ttype, (loop.uid, slot0 + i)) for i, (x, _) in enumerate(chosen))
    to_init = {c.uid: init for c, init in zip(info.carries, loop.operands)}
    inits = tuple(substitute([x for x, _ in chosen], to_init))
    body_map = {x.uid: p for (x, _), p in zip(chosen, places)}
    new_nexts = substitute(list(info.nexts) + [y for _, y in chosen], body_map)
    copy = loop_node(loop.uid, info.trip, info.start, info.step, info.index, info.carries + places,
                     tuple(loop.operands) + inits, tuple(new_nexts),
                     tuple(info.names) + tuple(f"hk_reuse{i}" for i in range(len(places))))
    copy.literal.unroll = info.unroll
    return copy


def carry_repeats(roots) -> list:
    """``roots`` with :func:`_carry_repeats_of` applied to every innermost loop
    that no tape reads (the two-body leapfrog's closing half-kick acceleration
    is the next substep's opening one)."""
    nodes = topo(roots)
    loops = [n for n in nodes if n.kind == "loop"]
    if not loops:
        return list(roots)
    taped = {n.operands[0].uid for n in nodes if n.kind == "tape_read"}
    deps = Deps()
    mapping = {}
    for lp in loops:
        if lp.uid in taped:
            continue
        copy = _carry_repeats_of(lp, deps)
        if copy is not None:
            mapping[lp.uid] = copy
    return substitute(roots, mapping) if mapping else list(roots)


def used_names(program: Program) -> set:
    """The planes a kernel binds: the ones its sinks read or write, the guard's
    mask when it declares one, and the finish counter when it finishes."""
    used = {n.literal[1] for n in leaves_of(sink_roots(program.sinks))} | {s.name for s in program.sinks}
    if GUARD_MASK in program.decls and program.decls[GUARD_MASK].role == "terminated":
        used.add(GUARD_MASK)
    if any(isinstance(s, Finish) for s in program.sinks):
        used.add(FINISHED_PLANE)
    used |= {n.literal.count for n in topo(sink_roots(program.sinks)) if n.kind == "loop" and n.literal.count}
    return used


def arg_spec(program: Program, used: set) -> list:
    """``[(role, name)]`` of the planes a kernel binds, in :data:`ROLE_ORDER`,
    declaration order within a role; ``used`` holds the names the body reads
    or writes (an unused declaration gets no slot)."""
    decls = [d for d in program.decls.values() if d.name in used]
    return [(d.role, d.name) for role in ROLE_ORDER for d in decls if d.role == role]
