"""``hawk.diff``: IR -> IR reverse (``vjp``) and forward (``jvp``) mode.

The rules are the reference's rule table, op for op, so a derivative kernel
computes the reference's expressions in the reference's order:

* elementwise and shaped rules: reference ``hawk/diff/rules.py`` (``_BIN_VJP``,
  ``_BIN_JVP``, ``_UNARY_D``, ``_SHAPED``);
* ``chol`` is an identity carrier and ``cho_solve`` reverses to
  ``lam = cho_solve(L, g); bar_b = lam; bar_A = -sym(outer(lam, x))``
  (reference ``hawk/diff/linalg_rules.py:230-241``);
* a rolled recurrence reverses into a rolled loop that runs backwards over the
  forward loop's per-iteration carries, read through ``tape_read``, replaying
  one iteration of the forward body to pull each adjoint back (reference
  ``hawk/diff/loops.py:484-540``); forward mode carries each slot's tangent
  beside its primal in one augmented loop (reference ``hawk/diff/transform.py:551-556``).

Names follow reference ``hawk/diff/transform.py:989-1022``: the adjoint seed
of a sink ``y`` is the plane ``bar_y`` and the gradient of an input ``x`` the
plane ``bar_x``; a tangent input is ``dot_x`` and a tangent output ``dot_y``.
"""

from __future__ import annotations

from . import ir
from .ir import (GUARD_MASK, AccumWrite, Assign, Decl, Deps, Finish, HawkError, Node, OrderedFold, Program,
                 SampleSum, fresh_placeholders, free_inputs, level_order, make, zero_like)
from .trace import Kernel
from .types import TensorType, role_of

__all__ = ["jvp", "vjp"]


# --------------------------------------------------------------------------
# small constructors


def _o(kind, *args, literal=None):
    return make(kind, args, literal)


def _c(x: float) -> Node:
    return ir.const(x)


def _sym(m: Node) -> Node:
    return _o("mul", _o("add", m, _o("transpose", m)), _c(0.5))


def _vec_like(parts: list, shape: tuple) -> Node:
    return make("vec", tuple(parts), shape)


def _entries(shape: tuple) -> list:
    if len(shape) == 1:
        return list(range(shape[0]))
    return [(i, j) for i in range(shape[0]) for j in range(shape[1])]


def _sum(terms) -> Node | None:
    live = [t for t in terms if t is not None]
    if not live:
        return None
    out = live[0]
    for t in live[1:]:
        out = _o("add", out, t)
    return out


def _ge_sign(x: Node) -> Node:
    one, minus = _c(1.0), _c(-1.0)
    if not x.ttype.shape:
        return _o("select", _o("ge", x, _c(0.0)), one, minus)
    parts = [_o("select", _o("ge", _o("component", x, literal=k), _c(0.0)), one, minus)
             for k in _entries(x.ttype.shape)]
    return _vec_like(parts, x.ttype.shape)


#: d(node)/d(x) of the unary kinds (reference hawk/diff/rules.py _UNARY_D).
_UNARY_D = {
    "neg": lambda n, x: _c(-1.0),
    "abs": lambda n, x: _ge_sign(x),
    "sqrt": lambda n, x: _o("div", _c(0.5), n),
    "exp": lambda n, x: n,
    "log": lambda n, x: _o("div", _c(1.0), x),
    "sin": lambda n, x: _o("cos", x),
    "cos": lambda n, x: _o("neg", _o("sin", x)),
    "tanh": lambda n, x: _o("sub", _c(1.0), _o("mul", n, n)),
}

_TERMINAL = ("leaf", "const", "iconst", "loop_index", "carry", "tape_read", "lane_axis", "gather", "sample_count")
_NO_DERIVATIVE = ("lt", "le", "gt", "ge", "eq", "ne", "chol_info", "real")


# --------------------------------------------------------------------------
# reverse mode


def _vjp_rule(n: Node, g: Node) -> list:
    k, ops = n.kind, n.operands
    if k == "add":
        return [(ops[0], g), (ops[1], g)]
    if k == "sub":
        return [(ops[0], g), (ops[1], _o("neg", g))]
    if k == "mul":
        a, b = ops
        return [(a, _o("mul", g, b)), (b, _o("mul", g, a))]
    if k == "div":
        a, b = ops
        return [(a, _o("div", g, b)), (b, _o("neg", _o("div", _o("mul", g, n), b)))]
    if k in _UNARY_D:
        x = ops[0]
        return [(x, _o("mul", g, _UNARY_D[k](n, x)))]
    if k == "dot":
        a, b = ops
        return [(a, _o("mul", g, b)), (b, _o("mul", g, a))]
    if k == "norm":
        a = ops[0]
        return [(a, _o("mul", _o("div", g, n), a))]
    if k == "sum":
        return [(ops[0], make("splat", (g,), ops[0].ttype.shape))]
    if k == "splat":
        return [(ops[0], _o("sum", g))]
    if k == "component":
        v = ops[0]
        z = _c(0.0)
        key = n.literal
        return [(v, _vec_like([g if e == key else z for e in _entries(v.ttype.shape)], v.ttype.shape))]
    if k == "vec":
        return [(c, _o("component", g, literal=e)) for e, c in zip(_entries(n.ttype.shape), ops)]
    if k == "mv":
        m, v = ops
        return [(m, _o("outer", g, v)), (v, _o("mv", _o("transpose", m), g))]
    if k == "mm":
        a, b = ops
        return [(a, _o("mm", g, _o("transpose", b))), (b, _o("mm", _o("transpose", a), g))]
    if k == "outer":
        a, b = ops
        return [(a, _o("mv", g, b)), (b, _o("mv", _o("transpose", g), a))]
    if k == "transpose":
        return [(ops[0], _o("transpose", g))]
    if k == "select":
        c, a, b = ops
        z = zero_like(g.ttype)
        return [(a, _o("select", c, g, z)), (b, _o("select", c, z, g))]
    if k == "chol":
        return [(ops[0], g)]              # the factor is an identity carrier of A
    if k == "cho_solve":
        f, b = ops
        lam = _o("cho_solve", f, g)
        return [(b, lam), (f, _o("neg", _sym(_o("outer", lam, n))))]
    if k == "chol_factor":
        raise HawkError("the derivative of a Cholesky factor read as a matrix is not in this build; "
                        "differentiate through cho_solve")
    if k in _NO_DERIVATIVE:
        return []
    raise HawkError(f"no reverse-mode rule for the IR kind {k!r}")


class _Reverse:
    def __init__(self, active_targets: set):
        self.deps = Deps()
        self.targets = active_targets      # uids of the leaves being differentiated
        self.active_memo: dict = {}
        self.scatters: list = []           # (table name, contribution, flat cell) of table reads
        self.depth = 0                     # loop bodies being reversed

    def active(self, n: Node) -> bool:
        hit = self.active_memo.get(n.uid)
        if hit is not None:
            return hit
        for m in ir.topo([n]):
            if m.uid in self.active_memo:
                continue
            if m.ttype.dtype not in ("f64", "f32", "tuple"):
                self.active_memo[m.uid] = False
                continue
            if m.kind == "leaf":
                self.active_memo[m.uid] = m.uid in self.targets
                continue
            kids = list(m.operands)
            if m.kind == "loop":
                kids += list(m.literal.nexts)
            self.active_memo[m.uid] = any(self.active_memo.get(k.uid, False) for k in kids)
        return self.active_memo[n.uid]

    @staticmethod
    def _accumulate(store: dict, child: Node, g: Node) -> None:
        if child.ttype.shape == () and g.ttype.shape != ():
            g = _o("sum", g)                      # un-broadcast a scalar operand
        held = store.get(child.uid)
        store[child.uid] = g if held is None else _o("add", held, g)

    def pullback(self, roots, seeds: list, stops=frozenset()) -> dict:
        """Adjoints (uid -> node) of everything at this level reachable from
        ``roots``, seeded by ``seeds`` [(node, adjoint)]; ``stops`` collect an
        adjoint but pass nothing back."""
        store: dict = {}
        loop_seeds: dict = {}
        for node, g in seeds:
            self._accumulate(store, node, g)
        order = level_order(roots, self.deps, stops)
        for n in reversed(order):
            if n.uid in stops or not self.active(n):
                continue
            if n.kind == "loop_value":
                g = store.get(n.uid)
                if g is not None:
                    loop_seeds.setdefault(n.operands[0].uid, {})[n.literal] = g
                continue
            if n.kind == "loop":
                seeds_j = loop_seeds.get(n.uid)
                if seeds_j:
                    for child, g in self._reverse_loop(n, seeds_j):
                        if self.active(child):
                            self._accumulate(store, child, g)
                continue
            g = store.get(n.uid)
            if g is None:
                continue
            if n.kind == "gather" and n.literal is not None and n.operands[0].uid in self.targets:
                # the reverse of a table read is a scatter-add into the table's
                # adjoint at the cell it read (reference hawk/diff/transform.py:695-705)
                if self.depth:          # vjp writes such loops out first (ir.unroll_reading)
                    raise HawkError(f"the gradient of a read of the table {n.operands[0].literal[1]!r} inside a "
                                    "rolled loop")
                self.scatters.append((n.operands[0].literal[1], g, make("table_index", n.operands, n.literal)))
                continue
            if n.kind in _TERMINAL:
                continue
            for child, contribution in _vjp_rule(n, g):
                if self.active(child):
                    self._accumulate(store, child, contribution)
        return store

    def _reverse_loop(self, loop: Node, seeds: dict) -> list:
        segmented = _strip_mined(loop, self.deps)
        if segmented is not None:
            loop = segmented
        info = loop.literal
        m = len(info.carries)
        free = [f for f in free_inputs(loop, self.deps) if self.active(f)]
        uid, index, _carries, _mapping = fresh_placeholders(loop)
        tapes = [ir.tape_read(loop, j, index) for j in range(m)]
        body = ir.substitute(info.nexts, {info.index.uid: index,
                                          **{c.uid: t for c, t in zip(info.carries, tapes)}})
        bars = tuple(Node("carry", (), c.ttype, (uid, j)) for j, c in enumerate(info.carries))
        accs = tuple(Node("carry", (), f.ttype, (uid, m + i)) for i, f in enumerate(free))
        stops = frozenset(t.uid for t in tapes) | frozenset(f.uid for f in free)
        live = [(b, bar) for b, bar in zip(body, bars)]
        self.depth += 1
        try:
            inner = self.pullback(body, live, stops)
        finally:
            self.depth -= 1
        nexts = tuple(inner.get(t.uid) if inner.get(t.uid) is not None else zero_like(c.ttype)
                      for t, c in zip(tapes, info.carries))
        nexts += tuple(_o("add", acc, inner[f.uid]) if inner.get(f.uid) is not None else acc
                       for acc, f in zip(accs, free))
        inits = tuple(seeds.get(j) if seeds.get(j) is not None else zero_like(c.ttype)
                      for j, c in enumerate(info.carries))
        inits += tuple(zero_like(f.ttype) for f in free)
        names = tuple(f"bar_{n}" for n in info.names) + tuple(f"bar_free{i}" for i in range(len(free)))
        reverse = ir.loop_node(uid, info.trip, info.start + (info.trip - 1) * info.step, -info.step,
                               index, bars + accs, inits, nexts, names)
        reverse.literal.unroll = info.unroll
        out = [(info_init, ir.loop_value(reverse, j)) for j, info_init in enumerate(loop.operands)]
        out += [(f, ir.loop_value(reverse, m + i)) for i, f in enumerate(free)]
        return out


#: The longest recurrence reversed with a single tape: a longer one is cut into
#: segments of this many iterations first (see :func:`_strip_mined`).
CHECKPOINT_SEGMENT = 4


def _strip_mined(loop: Node, deps: Deps):
    """``loop`` (trip T) as an outer loop of T/S iterations whose body is an inner
    loop of S iterations, S = :data:`CHECKPOINT_SEGMENT`, or None when it does
    not apply (T <= S, T not a multiple of S, or a body reading its index).

    The two compute the same operations in the same order, so the primal bits
    do not change.  Reversing the nested form tapes only the T/S segment starts
    and, per segment, replays the segment forward with an S-entry tape before
    reversing it: checkpointing by construction, which keeps the live tape at
    T/S + S carried values instead of T (the reference tapes every iteration,
    hawk/diff/loops.py:484-540, in local memory; a gfx950 lane keeps its tape
    in registers, so the tape's size sets the occupancy)."""
    info = loop.literal
    seg = CHECKPOINT_SEGMENT
    if info.trip <= seg or info.trip % seg:
        return None
    if any(n is info.index for n in ir.topo(info.nexts)):
        return None
    _, outer_index, outer_carries, _ = fresh_placeholders(loop)
    inner_uid, inner_index, inner_carries, mapping = fresh_placeholders(loop)
    outer_uid = next(ir._uid)
    outer_index.literal = outer_uid
    outer_carries = tuple(Node("carry", (), c.ttype, (outer_uid, j)) for j, c in enumerate(outer_carries))
    inner_nexts = ir.substitute(info.nexts, mapping)
    inner = ir.loop_node(inner_uid, seg, 0, 1, inner_index, inner_carries, outer_carries, tuple(inner_nexts),
                         info.names)
    outer_nexts = tuple(ir.loop_value(inner, j) for j in range(len(info.carries)))
    outer = ir.loop_node(outer_uid, info.trip // seg, 0, 1, outer_index, outer_carries, loop.operands,
                         outer_nexts, info.names)
    inner.literal.unroll = outer.literal.unroll = info.unroll
    deps.register(inner)
    deps.register(outer)
    return outer


def _refuse_prior_reads(program: Program, what: str) -> None:
    for n in ir.topo(ir.sink_roots(program.sinks)):
        if n.kind == "leaf" and n.literal[0] == "mutable":
            raise HawkError(f"{what}: the kernel reads {n.literal[1]!r} before it writes it (the value "
                            "the plane held when the launch began); that recurrence across launches has "
                            "no tape, so it cannot be differentiated — differentiate the per-launch term")


def _program_of(kernel) -> Program:
    """The program a derivative is taken of: a finishing kernel's without its
    finish (a derived kernel reads the mask through its guard and never
    finishes, reference ``tests/test_finish_own_sample.py:111-120``)."""
    if isinstance(kernel, Kernel):
        step = getattr(kernel, "step", None)
        if step is not None and step.name == kernel.name:
            kernel = step                  # a default automatic kernel: its single step
        program = kernel.program
    elif isinstance(kernel, Program):
        program = kernel
    else:
        raise HawkError("vjp/jvp take a @hawk.kernel (or a Kernel)")
    finishes = [s for s in program.sinks if isinstance(s, Finish)]
    if not finishes:
        return program
    if any(f.steps != 1 for f in finishes):
        raise HawkError(f"vjp/jvp of a kernel taking {finishes[0].steps} steps a launch (hawk.steps): "
                        "differentiate the single step (its .step)")
    return Program(dict(program.decls), [s for s in program.sinks if not isinstance(s, Finish)], program.grid,
                   dict(program.tables))


def _keep_guard(program: Program, out: Program) -> None:
    """A derived kernel of a guarded kernel is guarded by the same mask, read only."""
    d = program.decls.get(GUARD_MASK)
    if d is not None and d.role == "terminated":
        out.decls[GUARD_MASK] = d


def _namer(program: Program, prefix: str):
    taken = set(program.decls)

    def name(x: str) -> str:
        out = f"{prefix}_{x}"
        if out in taken:
            raise HawkError(f"the derived plane name {out!r} collides with a declared plane")
        return out
    return name


def _differentiable_inputs(program: Program, wrt, params: bool = False) -> list:
    """The inputs ``wrt`` names (default: every real input plane).  With
    ``params``, a ``Param`` may be named too (a reverse-mode gradient of a
    parameter is a cell summed over samples)."""
    inputs = [d for d in program.decls.values()
              if (d.role in ("per_sample", "vec_in", "mat_in") or d.name in program.tables)
              and d.ttype.dtype in ("f64", "f32")]
    if wrt is None:
        return inputs
    wrt = (wrt,) if isinstance(wrt, str) else tuple(wrt)
    by_name = {d.name: d for d in inputs}
    if params:
        by_name.update({d.name: d for d in program.decls.values() if d.role == "uniform"})
    missing = [w for w in wrt if w not in by_name]
    if missing:
        raise HawkError(f"wrt={missing}: not differentiable inputs of this kernel "
                        f"(those are {sorted(by_name)})")
    return [by_name[w] for w in wrt]


def param_planes(kernel):
    """The reference's spelling for differentiating a kernel's parameters
    (reference ``hawk/diff/transform.py:443-456``): ``vjp(param_planes(k),
    wrt=(..., "mu"))``.  On this target ``vjp`` takes a ``Param`` in ``wrt``
    directly, so this returns the kernel unchanged."""
    return kernel


def _seed(sink, seed_name: str) -> tuple:
    """``(node, role)``: the incoming adjoint of one primal sink, as reference
    ``hawk/diff/transform.py:989-1000`` derives it.  An assigned plane's adjoint
    is a plane of the same shape; the reverse of a sum over samples is a
    broadcast of the cell's adjoint (a uniform); the transpose of a keyed add
    ``acc[key] += v`` is a gather of the cells' adjoint, ``bar_acc[key]``."""
    t = sink.value.ttype
    if isinstance(sink, SampleSum) and sink.group is not None:
        # a sum over the trailing lane axes: each lane reads its key's adjoint
        # (key = flat lane // group), a gather from a plane of keys
        table = ir.leaf("lookup", seed_name, TensorType((), "f64"))
        return make("gather", (table, make("lane_axis", (), (sink.group, None)))), "lookup"
    if isinstance(sink, SampleSum):
        return ir.leaf("uniform", seed_name, t), "uniform"
    if isinstance(sink, AccumWrite):
        table = ir.leaf("lookup", seed_name, TensorType((), "f64"))
        return make("gather", (table, sink.key)), "lookup"
    return ir.leaf(role_of(t), seed_name, t), role_of(t)


def _refuse_extremes(program: Program, transform: str) -> None:
    """A max or a min over the samples has no derivative to take (reference
    ``tests/test_reduce_samples.py``: "subgradient is ambiguous at a tie");
    the reverse of a vector cell's sum would seed a vector uniform, which this
    build does not declare."""
    for s in program.sinks:
        if isinstance(s, SampleSum) and s.op != "sum":
            raise HawkError(f"{transform}: {s.name!r} is hawk.{s.op} over the samples; its subgradient is "
                            "ambiguous at a tie (two samples holding the extreme), so it has no derivative")
        if transform == "vjp" and isinstance(s, SampleSum) and s.column is not None:
            raise HawkError(f"vjp: {s.name!r} is hawk.sum of a vector over the samples; its adjoint is not "
                            "taken in this build: store each component's hawk.sum in a Scalar cell of its own")


def vjp(kernel, wrt=None) -> Program:
    """The reverse-mode derivative: a program reading the primal inputs and an
    adjoint seed plane ``bar_<sink>`` per per-sample sink, and writing
    ``bar_<x>`` for each input ``x`` of ``wrt`` (default: every real input
    plane).  A ``Param`` named in ``wrt`` gets a cell ``bar_<param>``: the
    sum over samples of each sample's contribution, by ``hawk.sum``'s default
    policy."""
    program = _program_of(kernel)
    _refuse_prior_reads(program, "vjp")
    _refuse_extremes(program, "vjp")
    name = _namer(program, "bar")
    targets = _differentiable_inputs(program, wrt, params=True)
    roots = [s.value for s in program.sinks]
    read_tables = {d.name for d in targets if d.name in program.tables}
    if read_tables:
        # a table read inside a loop adds at a cell per iteration: the loop is
        # written out, so each iteration's read is a site of its own
        roots = ir.unroll_reading(roots, lambda m: m.kind == "gather" and m.literal is not None
                                  and m.operands[0].literal[1] in read_tables)
    leaf_nodes = {n.literal[1]: n for n in ir.leaves_of(roots)}
    target_leaves = [leaf_nodes[d.name] for d in targets if d.name in leaf_nodes]
    rev = _Reverse({n.uid for n in target_leaves})
    out = Program(grid=program.grid, tables=dict(program.tables))
    _keep_guard(program, out)
    seeds = []
    for s, root in zip(program.sinks, roots):
        seed_name = name(s.name)
        seed, role = _seed(s, seed_name)
        out.decls[seed_name] = Decl(seed_name, role, seed.ttype)
        seeds.append((root, seed))
    store = rev.pullback(roots, seeds)
    keyed = next((s.group for s in program.sinks
                  if isinstance(s, SampleSum) and s.group is not None and s.policy == "ordered"), None)
    for d in program.decls.values():
        if d.role in ("per_sample", "vec_in", "mat_in", "uniform", "lookup"):
            out.decls.setdefault(d.name, d)
    for d in targets:
        grad_name = name(d.name)
        if d.name in program.tables:
            out.decls[grad_name] = Decl(grad_name, "mutable", TensorType((), "f64"))
            out.tables[grad_name] = program.tables[d.name]
            sites = [(g, cell) for table, g, cell in rev.scatters if table == d.name]
            if keyed is not None and sites and all(ir.key_only(cell, keyed) for _, cell in sites):
                # under an ordered keyed sum, each read names one cell per key:
                # the ordered fold (reference hawk/diff/ordered.py), one log
                # slot per read site, each key's lanes added in lane order
                out.sinks.append(OrderedFold(grad_name, tuple(ir.as_real(g) for g, _ in sites),
                                             tuple(cell for _, cell in sites), keyed))
                continue
            # otherwise every read's contribution is added at the cell it
            # read, in the ordered scatter's order (one stage per read site)
            for contribution, cell in sites:
                out.sinks.append(AccumWrite(grad_name, contribution, cell, "ordered"))
            continue
        lf = leaf_nodes.get(d.name)
        g = store.get(lf.uid) if lf is not None else None
        if g is None:
            g = zero_like(d.ttype)
        if g.ttype.shape != d.ttype.shape:
            g = make("splat", (g,), d.ttype.shape)
        out.decls[grad_name] = Decl(grad_name, "mutable", d.ttype)
        if d.role == "uniform":
            # a parameter's gradient: every sample's contribution, summed
            # (reference hawk/diff/transform.py:443-456, the default policy)
            out.sinks.append(SampleSum(grad_name, g, "auto"))
        else:
            out.sinks.append(Assign(grad_name, g, "mutable"))
    _drop_unused_inputs(out)
    return out


# --------------------------------------------------------------------------
# forward mode


class _Forward:
    def __init__(self, tangent_leaves: dict):
        self.deps = Deps()
        self.memo: dict = dict(tangent_leaves)   # uid -> tangent node (None: zero)

    def tangents(self, roots) -> None:
        for n in level_order(roots, self.deps):
            if n.uid in self.memo:
                continue
            self.memo[n.uid] = self._rule(n)

    def t(self, n: Node):
        return self.memo.get(n.uid)

    def _rule(self, n: Node):
        k, ops = n.kind, n.operands
        t = self.t
        if n.ttype.dtype in ("i32", "i64", "bool"):
            return None                   # an index or a mask carries no tangent
        if k == "gather" and n.literal is not None and t(ops[0]) is not None:
            # the tangent of a table read is the same clamped read of the
            # table's tangent plane (reference tests/test_diff_cross_sample.py:66-80)
            return make("gather", (t(ops[0]), *ops[1:]), n.literal)
        if k in _TERMINAL:
            return None
        if k == "add":
            return _sum((t(ops[0]), t(ops[1])))
        if k == "sub":
            ta, tb = t(ops[0]), t(ops[1])
            return _sum((ta, _o("neg", tb) if tb is not None else None))
        if k == "mul":
            a, b = ops
            ta, tb = t(a), t(b)
            return _sum((_o("mul", ta, b) if ta is not None else None,
                         _o("mul", a, tb) if tb is not None else None))
        if k == "div":
            a, b = ops
            ta, tb = t(a), t(b)
            return _sum((_o("div", ta, b) if ta is not None else None,
                         _o("neg", _o("div", _o("mul", n, tb), b)) if tb is not None else None))
        if k in _UNARY_D:
            tx = t(ops[0])
            return None if tx is None else _o("mul", tx, _UNARY_D[k](n, ops[0]))
        if k in ("dot", "mv", "mm", "outer"):
            a, b = ops
            ta, tb = t(a), t(b)
            return _sum((_o(k, ta, b) if ta is not None else None,
                         _o(k, a, tb) if tb is not None else None))
        if k == "norm":
            ta = t(ops[0])
            return None if ta is None else _o("div", _o("dot", ops[0], ta), n)
        if k in ("sum", "transpose"):
            ta = t(ops[0])
            return None if ta is None else _o(k, ta)
        if k == "splat":
            ta = t(ops[0])
            return None if ta is None else make("splat", (ta,), n.ttype.shape)
        if k == "component":
            ta = t(ops[0])
            return None if ta is None else _o("component", ta, literal=n.literal)
        if k == "vec":
            parts = [t(c) for c in ops]
            if all(p is None for p in parts):
                return None
            return _vec_like([p if p is not None else zero_like(c.ttype) for p, c in zip(parts, ops)],
                             n.ttype.shape)
        if k == "select":
            c, a, b = ops
            ta, tb = t(a), t(b)
            if ta is None and tb is None:
                return None
            return _o("select", c, ta if ta is not None else zero_like(a.ttype),
                      tb if tb is not None else zero_like(b.ttype))
        if k == "chol":
            return t(ops[0])
        if k == "cho_solve":
            f, b = ops
            da, db = t(f), t(b)
            rhs = db
            if da is not None:
                drift = _o("neg", _o("mv", _sym(da), n))
                rhs = drift if rhs is None else _o("add", rhs, drift)
            return None if rhs is None else _o("cho_solve", f, rhs)
        if k == "chol_factor":
            raise HawkError("the tangent of a Cholesky factor read as a matrix is not in this build")
        if k in _NO_DERIVATIVE:
            return None
        if k == "loop_value":
            aug = self.memo.get(("aug", ops[0].uid))
            if aug is None:
                return None
            loop, m = aug
            return ir.loop_value(loop, m + n.literal)
        if k == "loop":
            self.memo[("aug", n.uid)] = self._augment(n)
            return None
        raise HawkError(f"no forward-mode rule for the IR kind {k!r}")

    def _augment(self, loop: Node):
        info = loop.literal
        m = len(info.carries)
        free = free_inputs(loop, self.deps)
        if all(self.t(x) is None for x in loop.operands) and all(self.t(f) is None for f in free):
            return None
        uid, index, carries, mapping = fresh_placeholders(loop)
        dcs = tuple(Node("carry", (), c.ttype, (uid, m + j)) for j, c in enumerate(info.carries))
        body = ir.substitute(info.nexts, mapping)
        for c, dc in zip(carries, dcs):
            self.memo[c.uid] = dc
        self.memo[index.uid] = None
        self.tangents(body)
        dnexts = tuple(self.t(b) if self.t(b) is not None else zero_like(c.ttype)
                       for b, c in zip(body, info.carries))
        inits = tuple(loop.operands) + tuple(self.t(x) if self.t(x) is not None else zero_like(x.ttype)
                                             for x in loop.operands)
        names = tuple(info.names) + tuple(f"dot_{n}" for n in info.names)
        aug = ir.loop_node(uid, info.trip, info.start, info.step, index, carries + dcs, inits,
                           tuple(body) + dnexts, names)
        aug.literal.unroll = info.unroll
        return aug, m


def jvp(kernel, wrt=None) -> Program:
    """The forward-mode derivative: a program reading the primal inputs and a
    tangent plane ``dot_<x>`` per input of ``wrt``, and writing ``dot_<y>``
    for each per-sample sink ``y``."""
    program = _program_of(kernel)
    _refuse_prior_reads(program, "jvp")
    _refuse_extremes(program, "jvp")
    name = _namer(program, "dot")
    targets = _differentiable_inputs(program, wrt)
    roots = [s.value for s in program.sinks]
    leaf_nodes = {n.literal[1]: n for n in ir.leaves_of(roots)}
    out = Program(grid=program.grid, tables=dict(program.tables))
    for d in program.decls.values():
        if d.role in ("per_sample", "vec_in", "mat_in", "uniform", "lookup"):
            out.decls.setdefault(d.name, d)
    tangent_leaves = {}
    for d in targets:
        tname = name(d.name)
        out.decls[tname] = Decl(tname, d.role, d.ttype)
        if d.name in program.tables:
            out.tables[tname] = program.tables[d.name]
        if d.name in leaf_nodes:
            tangent_leaves[leaf_nodes[d.name].uid] = ir.leaf(d.role, tname, d.ttype)
    _keep_guard(program, out)
    fwd = _Forward(tangent_leaves)
    fwd.tangents(roots)
    for s in program.sinks:
        tname = name(s.name)
        tv = fwd.t(s.value)
        if tv is None:
            tv = zero_like(s.value.ttype)
        column = s.column if isinstance(s, SampleSum) else None
        # a vector cell's column sinks share the cell's declaration
        out.decls[tname] = Decl(tname, "mutable", s.value.ttype if column is None else program.decls[s.name].ttype)
        # the tangent sink is the primal's kind at the same lane (reference
        # hawk/diff/transform.py:1003-1022): a sum of tangents, or a keyed add of
        # tangents at the primal's key under the primal's policy
        if isinstance(s, SampleSum):
            out.sinks.append(SampleSum(tname, tv, s.policy, s.group, column=column))
        elif isinstance(s, AccumWrite):
            out.sinks.append(AccumWrite(tname, tv, s.key, s.policy))
        else:
            out.sinks.append(Assign(tname, tv, "mutable"))
    _drop_unused_inputs(out)
    return out


def _drop_unused_inputs(program: Program) -> None:
    """Keep the declarations the derived body reads or writes."""
    used = {n.literal[1] for n in ir.leaves_of(ir.sink_roots(program.sinks))}
    used |= {s.name for s in program.sinks}
    program.decls = {k: d for k, d in program.decls.items()
                     if k in used or (k == GUARD_MASK and d.role == "terminated")}

