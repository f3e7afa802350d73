"""The HIP writer of hawk's gfx950 target: IR -> one self-contained HIP
translation unit per kernel stage.

The emitted entry has the reference's device signature — one by-value mirror
per ``arg_spec`` slot, then ``long long base, count, nSamples`` (reference
``hawk/emit/cuda.py:46-54``) — and its ONE geometry prologue binds
``i = base + flat`` (reference ``:73-81``).  Each thread takes ``per_thread``
samples a workgroup-width apart, so every load and store of a wave is one
contiguous 64-lane run of a ``[component, sample]`` plane (coalesced), and the
samples of one thread are independent work for the scheduler to overlap.

The body is scalarised: a vector or matrix node is one C++ variable per
component, every operation one statement in the reference's operation order
(a ``dot``/``mv``/``mm`` adds its products left to right; the Cholesky factor
and solve follow reference ``hawk/embedded/linalg.py:233-271`` and
``:443-536``).  With ``-ffp-contract=off`` the device computes the same IEEE
operations as the host oracle built in the reference's ``native`` profile.

A rolled loop stays rolled: its loop-invariant inputs are hoisted, its carried
slots are locals, and a loop whose carries a reversed loop reads keeps a tape
(one local array per carried component) that the compiler holds in registers
when the loop is unrolled.
"""

from __future__ import annotations

import re

import math
import dataclasses
from dataclasses import dataclass, field

from . import ir
from .ir import (FINISHED_PLANE, GUARD_MASK, AccumWrite, Assign, Deps, Finish, HawkError, Node, OrderedFold,
                 Program, SampleSum, free_inputs,
                 level_order)

from .hip_target import HIP_WRITER, StageWalk, _literal  # noqa: E402  (the hip row's spellings)
from .targets import TARGETS  # noqa: E402

ABI_TAG = "aether-abi/2"
LAYOUT_SIZES = (40, 32, 32, 8, 24)

#: The by-value ABI shape of each role (reference hawk/emit/spelling.py:63-69);
#: a rank-0 ``mutable`` is a 32-byte handle, a ranked one a 40-byte mirror.
MIRROR_OF = {"out": "gref", "vec_in": "gref", "mat_in": "gref", "per_sample": "handle",
             "wide_out": "handle", "accum_out": "handle", "rows_out": "handle", "lookup": "handle",
             "uniform": "value"}



def kind_for(role: str, ttype, mode: str) -> str:
    """The ``hk_argblock`` kind name of a slot (reference hawk/runtime.py:96-110)."""
    if role == "uniform":
        return "f32" if mode == "float32" else "f64"
    shape = "gref" if role in ("out", "vec_in", "mat_in") or (role in ("mutable", "wide_out", "key_out")
                                                              and ttype.shape) else "handle"
    if shape == "handle" and ttype.dtype in ("i32", "u32"):
        return "int_handle"
    return shape


def _entries(shape: tuple) -> list:
    if len(shape) == 0:
        return [()]
    if len(shape) == 1:
        return [(i,) for i in range(shape[0])]
    return [(i, j) for i in range(shape[0]) for j in range(shape[1])]


def _flat(shape: tuple, idx) -> int:
    if isinstance(idx, int):
        idx = (idx,)
    if len(shape) == 1:
        return idx[0]
    return idx[0] * shape[1] + idx[1]


@dataclass
class Stage:
    """One per-sample stage of a kernel: the planes it binds and what it writes."""

    name: str
    arg_spec: list                  # [(role, name)]
    planes: dict                    # name -> {"role", "shape", "dtype"}
    writes: list                    # [(plane, node)]
    scratch: dict = field(default_factory=dict)   # name -> {"dtype", "per_sample": 1}
    row_sums: list = field(default_factory=list)  # [(cell, node, hi plane, comp plane)]
    key_writes: list = field(default_factory=list)  # [(plane, (node per component), group)]: one entry per key
    fused_folds: list = field(default_factory=list)  # [(out plane, scratch plane, values, cells, group)]
    block: int | None = None        # the launch block a fused fold needs (its keys never cross a block)
    guard: str | None = None        # the mask plane whose set samples the stage skips
    finish: tuple | None = None     # (mask plane, counter plane, condition node) of `terminated = cond`
    banded: bool = False            # the row sums fold double-double bands (the banded scalar mode)


class _Scope:
    def __init__(self):
        self.memo = [{}]

    def get(self, n: Node):
        for frame in reversed(self.memo):
            hit = frame.get(n.uid)
            if hit is not None:
                return hit
        return None

    def put(self, n: Node, value) -> None:
        self.memo[-1][n.uid] = value


class _Writer:
    """Scalarises nodes into C++ statements."""

    def __init__(self, stage: Stage, mode: str, nontemporal: bool = False, spell=HIP_WRITER):
        self.stage = stage
        self.mode = mode
        self.nontemporal = nontemporal
        self.spell = spell                   # the target row's writer: every piece of text
        self.lines: list = []
        self.indent = 2
        self.count = 0
        self.scope = _Scope()
        self.deps = Deps()
        self.taped = {}              # loop uid -> True when a tape_read reads it
        self.exits = {}              # loop uid -> the flag its exit set
        self.trips = {}              # loop uid -> the trips an automatic loop ran

    # -- text --------------------------------------------------------------
    def emit(self, text: str) -> None:
        self.lines.append("    " * self.indent + text)

    def fresh(self, stem: str = "v") -> str:
        self.count += 1
        return f"hk_{stem}{self.count}"

    def ctype(self, dtype: str) -> str:
        return self.spell.ctype(dtype)

    def let(self, dtype: str, expr: str, stem: str = "v") -> str:
        name = self.fresh(stem)
        self.emit(self.spell.declare(name, dtype, expr))
        return name

    # -- values ------------------------------------------------------------
    def value(self, n: Node) -> list:
        hit = self.scope.get(n)
        if hit is None:
            raise HawkError(f"internal: {n!r} used before it was emitted")
        return hit

    def scalar(self, n: Node) -> str:
        v = self.value(n)
        if len(v) != 1:
            raise HawkError(f"internal: {n!r} is not a scalar")
        return v[0]

    def run(self, roots) -> None:
        for n in level_order(roots, self.deps):
            if self.scope.get(n) is None:
                self.node(n)

    # -- nodes -------------------------------------------------------------
    def node(self, n: Node) -> None:
        k = n.kind
        handler = getattr(self, "_" + k, None)
        if handler is None:
            raise HawkError(f"the hip writer has no spelling for the IR kind {k!r}")
        out = handler(n)
        if out is not None:
            self.scope.put(n, out)

    def _leaf(self, n: Node) -> list:
        role, name = n.literal
        texts = self.spell.leaf(self, n)
        if role in ("uniform", "lookup"):
            return texts              # a value, or a table that `gather` indexes
        dt = "bool" if role == "terminated" else n.ttype.dtype
        return [self.let(dt, t, "in") for t in texts]

    def _lane_axis(self, n: Node) -> list:
        div, mod = n.literal
        if mod == 0:
            return [self.spell.sample_index_value()]          # the flat lane index
        q = "hk_i" if div == 1 else f"(hk_i / {div}LL)"
        return [self.let("i32", f"static_cast<int>({q})" if mod is None else f"static_cast<int>({q} % {mod}LL)", "ax")]

    def _floordiv(self, n: Node) -> list:
        a, b = self.scalar(n.operands[0]), self.scalar(n.operands[1])
        ct = self.ctype(n.ttype.dtype)
        q = self.let(n.ttype.dtype, f"static_cast<{ct}>({a}) / static_cast<{ct}>({b})", "q")
        # toward minus infinity, as Python's //
        return [self.let(n.ttype.dtype, f"({q} * static_cast<{ct}>({b}) != static_cast<{ct}>({a}) && "
                                        f"((static_cast<{ct}>({a}) < 0) != (static_cast<{ct}>({b}) < 0))) ? {q} - 1 : {q}", "q")]

    def _mod(self, n: Node) -> list:
        a, b = self.scalar(n.operands[0]), self.scalar(n.operands[1])
        ct = self.ctype(n.ttype.dtype)
        r = self.let(n.ttype.dtype, f"static_cast<{ct}>({a}) % static_cast<{ct}>({b})", "r")
        # the sign of the divisor, as Python's %
        return [self.let(n.ttype.dtype, f"({r} != 0 && (({r} < 0) != (static_cast<{ct}>({b}) < 0))) ? {r} + "
                                        f"static_cast<{ct}>({b}) : {r}", "r")]

    def _clamped_flat(self, n: Node) -> str:
        """The row-major flat cell of a clamped table read: each index clamped
        into [0, extent) of its axis (the first axis's extent from the bound
        cells when it is a runtime one)."""
        table, *keys = n.operands
        p = self.value(table)[0]
        extents = n.literal[1]
        rest = 1
        for e in extents[1:]:
            rest *= e
        flat = None
        for j, (k, e) in enumerate(zip(keys, extents)):
            extent = f"({self.spell.plane_extent_value(p)} / {rest}LL)" if e is None else f"{e}LL"
            idx = self.let("i64", f"static_cast<long long>({self.scalar(k)})", "k")
            c = self.let("i64", f"{idx} < 0 ? 0LL : ({idx} >= {extent} ? {extent} - 1 : {idx})", "k")
            stride = 1
            for e2 in extents[j + 1:]:
                stride *= e2
            term = c if stride == 1 else f"{c} * {stride}LL"
            flat = term if flat is None else f"{flat} + {term}"
        return self.let("i64", flat, "cell")

    def _table_index(self, n: Node) -> list:
        return [self.let("i32", f"static_cast<int>({self._clamped_flat(n)})", "cell")]

    def _gather(self, n: Node) -> list:
        # one read of the table (kept in cache: many samples share a cell)
        table = n.operands[0]
        p = self.value(table)[0]
        if n.literal is not None:                      # a Table read: clamped, never out of the plane
            return [self.let(n.ttype.dtype, self.spell.at(self, p, self._clamped_flat(n)), "g")]
        # a scatter target's adjoint: a key outside [0, cells), the skip key -1 included, reads 0
        k = self.scalar(n.operands[1])
        return [self.let(n.ttype.dtype, self.spell.at(self, p, k, guard_cells=True), "g")]

    def load(self, ref: str) -> str:
        return self.spell.load(self, ref)

    def store(self, ref: str, value: str) -> str:
        return self.spell.store(self, None, ref, value)

    def _const(self, n: Node) -> list:
        return [self.spell.const(n)]

    _iconst = _const

    def _sample_count(self, n: Node) -> list:
        return [self.let("f64", "static_cast<Real>(nSamples)", "ns")]

    def _real(self, n: Node) -> list:
        return [self.spell.op(self, n, [x]) for x in self.value(n.operands[0])]

    def _neg(self, n: Node) -> list:
        return [self.let(n.ttype.dtype, self.spell.op(self, n, [x])) for x in self.value(n.operands[0])]

    def _unary(self, n: Node) -> list:
        return [self.let(n.ttype.dtype, self.spell.op(self, n, [x])) for x in self.value(n.operands[0])]

    _exp = _sin = _cos = _tanh = _sqrt = _log = _abs = _unary

    def _bcast(self, n: Node, k: int) -> list:
        v = self.value(n.operands[k])
        size = n.ttype.size if n.ttype.shape else 1
        return v * size if len(v) == 1 and size > 1 else v

    def _binary(self, n: Node) -> list:
        a, b = self._bcast(n, 0), self._bcast(n, 1)
        return [self.let(n.ttype.dtype, self.spell.op(self, n, [x, y])) for x, y in zip(a, b)]

    _add = _sub = _mul = _div = _binary

    def _compare(self, n: Node) -> list:
        a, b = self.scalar(n.operands[0]), self.scalar(n.operands[1])
        return [self.let("bool", self.spell.op(self, n, [a, b]), "c")]

    _lt = _le = _gt = _ge = _eq = _ne = _compare

    def _select(self, n: Node) -> list:
        c = self.scalar(n.operands[0])
        a, b = self.value(n.operands[1]), self.value(n.operands[2])
        return [self.let(n.ttype.dtype, self.spell.select(self, n, c, x, y)) for x, y in zip(a, b)]

    def _fold(self, terms: list, dtype: str) -> str:
        acc = terms[0]
        for t in terms[1:]:
            acc = self.let(dtype, self.spell.op(self, "add", [acc, t]))
        return acc

    def _mul_text(self, x: str, y: str) -> str:
        return self.spell.op(self, "mul", [x, y])

    def _dot(self, n: Node) -> list:
        a, b = self.value(n.operands[0]), self.value(n.operands[1])
        prods = [self.let(n.ttype.dtype, self._mul_text(x, y)) for x, y in zip(a, b)]
        return [self._fold(prods, n.ttype.dtype)]

    def _norm(self, n: Node) -> list:
        a = self.value(n.operands[0])
        prods = [self.let(n.ttype.dtype, self._mul_text(x, x)) for x in a]
        return [self.let(n.ttype.dtype, f"sqrt({self._fold(prods, n.ttype.dtype)})")]

    def _sum(self, n: Node) -> list:
        return [self._fold(self.value(n.operands[0]), n.ttype.dtype)]

    def _splat(self, n: Node) -> list:
        return self.value(n.operands[0]) * n.ttype.size

    def _component(self, n: Node) -> list:
        src = n.operands[0]
        return [self.value(src)[_flat(src.ttype.shape, n.literal)]]

    def _vec(self, n: Node) -> list:
        return [self.scalar(c) for c in n.operands]

    def _transpose(self, n: Node) -> list:
        r, c = n.operands[0].ttype.shape
        v = self.value(n.operands[0])
        return [v[i * c + j] for j in range(c) for i in range(r)]

    def _mv(self, n: Node) -> list:
        m, v = self.value(n.operands[0]), self.value(n.operands[1])
        r, c = n.operands[0].ttype.shape
        dt = n.ttype.dtype
        out = []
        for i in range(r):
            prods = [self.let(dt, self._mul_text(m[i * c + j], v[j])) for j in range(c)]
            out.append(self._fold(prods, dt))
        return out

    def _mm(self, n: Node) -> list:
        a, b = self.value(n.operands[0]), self.value(n.operands[1])
        r, k = n.operands[0].ttype.shape
        c = n.operands[1].ttype.shape[1]
        dt = n.ttype.dtype
        out = []
        for i in range(r):
            for j in range(c):
                prods = [self.let(dt, self._mul_text(a[i * k + q], b[q * c + j])) for q in range(k)]
                out.append(self._fold(prods, dt))
        return out

    def _outer(self, n: Node) -> list:
        a, b = self.value(n.operands[0]), self.value(n.operands[1])
        return [self.let(n.ttype.dtype, self._mul_text(x, y)) for x in a for y in b]

    # -- Cholesky (reference hawk/embedded/linalg.py:233-271) -------------------
    def _chol(self, n: Node) -> list:
        a = self.value(n.operands[0])
        size = n.ttype.shape[0]
        stem = self.fresh("L")
        names = [f"{stem}_{i}_{j}" for i in range(size) for j in range(size)]
        info = f"{stem}_info"
        self.emit("Real " + ", ".join(f"{x} = Real(0.0)" for x in names) + ";")
        self.emit(f"int {info} = 0;")

        def el(i, j):
            return names[i * size + j]

        def sym(i, j):
            return f"(Real(0.5) * {a[i * size + j]}) + (Real(0.5) * {a[j * size + i]})"
        for j in range(size):
            self.emit(f"if ({info} == 0) {{")
            self.indent += 1
            self.emit(f"Real hk_d = {sym(j, j)};")
            for k in range(j):
                self.emit(f"hk_d = hk_d - ({el(j, k)} * {el(j, k)});")
            self.emit("if (hk_d > Real(0.0)) {")
            self.indent += 1
            self.emit("const Real hk_ljj = sqrt(hk_d);")
            self.emit(f"{el(j, j)} = hk_ljj;")
            for i in range(j + 1, size):
                self.emit(f"{{ Real hk_acc = {sym(i, j)};")
                for k in range(j):
                    self.emit(f"  hk_acc = hk_acc - ({el(i, k)} * {el(j, k)});")
                self.emit(f"  {el(i, j)} = hk_acc / hk_ljj; }}")
            self.indent -= 1
            self.emit(f"}} else {{ {info} = {j + 1}; }}")
            self.indent -= 1
            self.emit("}")
        self._chol_info_of = getattr(self, "_chol_info_of", {})
        self._chol_info_of[n.uid] = info
        return names

    def _chol_info(self, n: Node) -> list:
        f = n.operands[0]
        return [self._chol_info_of[f.uid]]

    def _chol_factor(self, n: Node) -> list:
        f = n.operands[0]
        size = f.ttype.shape[0]
        src = self.value(f)
        info = self._chol_info_of[f.uid]
        return [self.let(n.ttype.dtype, f"({info} == 0 && {j} <= {i}) ? {src[i * size + j]} : Real(0.0)")
                for i in range(size) for j in range(size)]

    def _cho_solve(self, n: Node) -> list:
        f, b = n.operands
        size = f.ttype.shape[0]
        L = self.value(f)
        info = self._chol_info_of[f.uid]
        rhs = self.value(b)
        stem = self.fresh("x")
        x = [f"{stem}_{i}" for i in range(size)]
        self.emit("Real " + ", ".join(f"{v} = Real(0.0)" for v in x) + ";")
        self.emit(f"if ({info} == 0) {{")
        self.indent += 1
        for i in range(size):                       # forward: L y = b, rows ascending
            self.emit(f"{{ Real hk_acc = {rhs[i]};")
            for j in range(i):
                self.emit(f"  hk_acc = hk_acc - ({L[i * size + j]} * {x[j]});")
            self.emit(f"  {x[i]} = hk_acc / {L[i * size + i]}; }}")
        for r in range(size):                       # backward: L^T x = y, rows descending
            i = size - 1 - r
            self.emit(f"{{ Real hk_acc = {x[i]};")
            for j in range(i + 1, size):
                self.emit(f"  hk_acc = hk_acc - ({L[j * size + i]} * {x[j]});")
            self.emit(f"  {x[i]} = hk_acc / {L[i * size + i]}; }}")
        self.indent -= 1
        self.emit("}")
        return x

    # -- loops ---------------------------------------------------------------
    def _loop(self, n: Node) -> list:
        info = n.literal
        inits = [self.value(x) for x in n.operands]
        for f in free_inputs(n, self.deps):            # hoisted: already emitted at this level
            if self.scope.get(f) is None:
                self.run([f])
        carry_vars = []
        for j, c in enumerate(info.carries):
            stem = self.fresh("c")
            names = [f"{stem}_{e}" for e in range(max(1, c.ttype.size if c.ttype.shape else 1))]
            ct = self.spell.carry_type(c.ttype)
            for name, init in zip(names, inits[j] * (len(names) if len(inits[j]) == 1 else 1)):
                self.emit(f"{ct} {name} = {init};")
            carry_vars.append(names)
        tapes = None
        if n.uid in self.taped:
            tapes = []
            for j, names in enumerate(carry_vars):
                row = [f"hk_tape{n.uid}_{j}_{e}" for e in range(len(names))]
                self.emit(self.spell.tape_decl(self.spell.carry_type(info.carries[j].ttype), row, info.trip))
                tapes.append(row)
            self.tape_of = getattr(self, "tape_of", {})
            self.tape_of[n.uid] = (tapes, info.start, info.step)
        k = f"hk_k{n.uid}"
        exited = None
        if info.exit is not None:
            exited = f"hk_exited{n.uid}"
            self.emit(f"bool {exited} = false;")
        if info.count is not None:
            # the trips run are the launch's word (reference hawk/emit/wrapper.py:973-977
            # clamps it below INT_MAX; a word below 0 runs none)
            word = self.stage.planes[info.count]["var"]
            self.emit(f"const long long hk_cnt{n.uid} = static_cast<long long>({word}[0]);")
            self.emit(self.spell.counter_decl(f"hk_trips{n.uid}"))
            self.trips[n.uid] = f"hk_trips{n.uid}"
            self.emit(self.spell.for_header(self, k, info, f"hk_cnt{n.uid}"))
        else:
            if info.unroll is True:
                self.emit("#pragma unroll")
            elif info.unroll is False:
                self.emit("#pragma unroll 1")
            self.emit(self.spell.for_header(self, k, info, None))
        self.indent += 1
        self.scope.memo.append({})
        self.scope.put(info.index, [k])
        for c, names in zip(info.carries, carry_vars):
            self.scope.put(c, names)
        if tapes is not None:
            slot = f"(({k} - {info.start}LL) / {info.step}LL)"
            for row, names in zip(tapes, carry_vars):
                for t, v in zip(row, names):
                    self.emit(self.spell.tape_write(self, t, slot, v))
        self.run(ir.body_roots(info))
        nexts = [self.value(x) for x in info.nexts]
        leave = None
        if info.exit is not None:
            leave = self.fresh("x")
            self.emit(f"const bool {leave} = {self.scalar(info.exit)};")
        temps = []
        for names, nv in zip(carry_vars, nexts):
            nv = nv * len(names) if len(nv) == 1 and len(names) > 1 else nv
            row = []
            for name, val in zip(names, nv):
                t = self.fresh("n")
                self.emit(f"const auto {t} = {val};")
                row.append(t)
            temps.append(row)
        for names, row in zip(carry_vars, temps):
            for name, t in zip(names, row):
                self.emit(f"{name} = {t};")
        if info.count is not None:
            self.emit(f"++hk_trips{n.uid};")
        if leave is not None:         # a tail break: this trip's values stand
            self.emit(self.spell.tail_break(leave, exited))
        self.scope.memo.pop()
        self.indent -= 1
        self.emit("}")
        if exited is not None:
            self.exits[n.uid] = exited
        return carry_vars

    def _loop_exit(self, n: Node) -> list:
        self.value(n.operands[0])
        return [self.exits[n.operands[0].uid]]

    def _loop_value(self, n: Node) -> list:
        return self.value(n.operands[0])[n.literal]

    def _loop_index(self, n: Node) -> list:
        raise HawkError("internal: a loop index read outside its loop")

    _carry = _loop_index

    def _tape_read(self, n: Node) -> list:
        loop, index = n.operands
        tapes, start, step = self.tape_of[loop.uid]
        k = self.scalar(index)
        slot = f"(({k} - {start}LL) / {step}LL)"
        return [f"{t}[{slot}]" for t in tapes[n.literal]]


def _stage_planes(program: Program, stage_name: str, mode: str, extra_writes: list,
                  row_sums: list = (), key_writes: list = (), fused_folds: list = ()) -> Stage:
    """The plane table and arg_spec of the per-sample stage of ``program``;
    ``row_sums`` = ``[(rows, node, red)]`` are default-policy sample
    reductions ("sum": compensated 32-sample rows; "max" / "min": one extreme
    a row) the stage writes into planes named after ``rows`` (a cell, or a
    cell's entry ``<cell>_<k>``); ``key_writes`` =
    ``[(plane, nodes, group)]`` are integer planes of one entry per key (every
    lane of the key's run of ``group`` samples stores the same value)."""
    writes = [(s.name, s.value) for s in program.sinks if isinstance(s, Assign)] + extra_writes
    finish = next((s for s in program.sinks if isinstance(s, Finish)), None)
    roots = ([node for _, node in writes] + [node for _, node, _ in row_sums]
             + [node for _, nodes, _ in key_writes for node in nodes]
             + [node for f in fused_folds for node in tuple(f[2]) + tuple(f[3])]
             + ([finish.value] if finish is not None else []))
    used_leaves = ir.leaves_of(roots)
    rows = [(cell, node, f"hk_rows_{cell}", f"hk_rows_{cell}_comp" if red == "sum" else None, red)
            for cell, node, red in row_sums]
    used = ({n.literal[1] for n in used_leaves} | {name for name, _ in writes}
            | {p for r in rows for p in r[2:4] if p} | {name for name, _, _ in key_writes}
            | {f[0] for f in fused_folds} | {f[1] for f in fused_folds})
    used |= {n.literal.count for n in ir.topo(roots) if n.kind == "loop" and n.literal.count}
    guard = GUARD_MASK if GUARD_MASK in program.decls and program.decls[GUARD_MASK].role == "terminated" else None
    if guard is not None:
        used.add(guard)
    if finish is not None:
        used.add(FINISHED_PLANE)
    decls = dict(program.decls)
    planes = {}
    for name, node in extra_writes:
        if name not in decls:
            decls[name] = ir.Decl(name, "wide_out", node.ttype)
    for name, nodes, _ in key_writes:
        decls[name] = ir.Decl(name, "key_out", ir.TensorType((len(nodes),) if len(nodes) > 1 else (), "i32"))
    for out, scratch, *_ in fused_folds:
        decls[out] = ir.Decl(out, "accum_out", ir.TensorType((), "f64"))
        decls[scratch] = ir.Decl(scratch, "fold_scratch", ir.TensorType((), "i32"))
    for _, _, hi, comp, _ in rows:
        for pname in (hi, comp) if comp else (hi,):
            decls[pname] = ir.Decl(pname, "rows_out", ir.TensorType((), "f32" if mode == "float32" else "f64"))
    prog2 = Program(decls, program.sinks, program.grid, program.tables)
    spec = ir.arg_spec(prog2, used)
    for role, name in spec:
        d = decls[name]
        planes[name] = {"role": role, "shape": list(d.ttype.shape), "dtype": d.ttype.dtype,
                        "kind": kind_for(role, d.ttype, mode), "var": f"hk_p_{name}"}
    for name, _, group in key_writes:
        planes[name]["group"] = group
    block = None
    for f in fused_folds:
        b = fold_block(f[4])
        block = b if block is None else block * b // math.gcd(block, b)
    if block is not None and block > 1024:
        raise HawkError("the fused ordered folds of this kernel need blocks of more than 1024 threads")
    return Stage(stage_name, spec, planes, writes, row_sums=rows, key_writes=list(key_writes),
                 fused_folds=list(fused_folds), block=block, guard=guard,
                 finish=(finish.name, FINISHED_PLANE, finish.value) if finish is not None else None)


#: A stage that touches at least this many component planes hands each XCD a
#: contiguous eighth of its blocks (the launcher rounds the grid up to a
#: multiple of 8; the extra workgroups find no samples): its many short runs,
#: one per plane per workgroup, then share DRAM pages within one XCD's L2.
#: Measured on MI355X: the 6x6 solve and its VJP (48 and 90 planes) gain 6 %
#: and 10 %, while plain streams (4-7 planes) lose 1-6 % and the two-body VJP
#: (18 planes, compute-bound) loses 10 %; those keep the plain order.
XCD_ORDER_PLANES = 32


def component_planes(stage: Stage) -> int:
    """How many component planes (rows of [component, sample]) the stage reads or writes."""
    total = 0
    for info in stage.planes.values():
        if info["role"] in ("uniform", "nsamples", "lookup", "rows_out", "key_out"):
            continue
        count = 1
        for e in info["shape"]:
            count *= e
        total += count
    return total


def render_stage(stage: Stage, mode: str, block: int, per_thread: int, unroll_taped: bool = True,
                 nontemporal: bool = False, xcd_order: bool | None = None, target=None) -> str:
    """The HIP source of one per-sample stage.  ``nontemporal`` marks the
    plane loads and stores as streaming (read or written once, not kept in
    cache); ``xcd_order`` (default: at least ``XCD_ORDER_PLANES`` component
    planes) hands each XCD a contiguous eighth of the blocks.  ``target`` is
    the row whose writer spells the body and whose wrapper makes the entry
    (default: the ``hip`` row)."""
    target = TARGETS["hip"] if target is None else target
    if xcd_order is None:
        xcd_order = component_planes(stage) >= XCD_ORDER_PLANES
    w = _Writer(stage, mode, nontemporal, spell=target.writer)
    roots = ([node for _, node in stage.writes] + [node for _, node, _, _, _ in stage.row_sums]
             + [node for _, nodes, _ in stage.key_writes for node in nodes]
             + [node for f in stage.fused_folds for node in tuple(f[2]) + tuple(f[3])]
             + ([stage.finish[2]] if stage.finish is not None else []))
    if stage.guard is not None and (stage.row_sums or stage.fused_folds):
        raise HawkError(f"{stage.name}: a guarded kernel (one declaring `terminated: Terminated`) commits "
                        "per-sample planes; a sum or a fold over the samples its guard skips is not in this build")
    if stage.fused_folds:
        block, per_thread = stage.block, 1
    # Which loops keep a tape: a loop that keeps or reads a tape, and every loop
    # nested in one, is unrolled, so every tape index is a constant and the tapes
    # live in registers (a checkpointed reverse keeps few enough of them live).
    for n in ir.topo(roots):
        if n.kind == "tape_read":
            w.taped[n.operands[0].uid] = True
    if unroll_taped:
        for n in ir.topo(roots):
            if n.kind != "loop":
                continue
            inner = ir.topo(n.literal.nexts)
            taped = n.uid in w.taped or any(m.kind == "tape_read" or (m.kind == "loop" and m.uid in w.taped)
                                            for m in inner)
            if taped:
                for m in [n] + [m for m in inner if m.kind == "loop"]:
                    m.literal.unroll = True
    w.run(roots)
    body = list(w.lines)
    w.lines = []
    for plane, node in stage.writes:
        info = stage.planes[plane]
        var = info["var"]
        vals = w.value(node)
        if not node.ttype.shape:
            w.emit(w.spell.component_commit(w, var, None, "=", vals[0]))
        else:
            for e in _entries(node.ttype.shape):
                c = _flat(node.ttype.shape, e)
                w.emit(w.spell.component_commit(w, var, c, "=", vals[c]))
    for plane, nodes, group in stage.key_writes:
        # every lane of a key stores the key's one value (a wave's equal
        # addresses merge into one write)
        var = stage.planes[plane]["var"]
        at = "hk_i" if group == 1 else f"hk_i / {group}LL"
        for c, node in enumerate(nodes):
            where = f"{var}[{at}]" if len(nodes) == 1 else f"{var}[{c} * {var}_cs + {at}]"
            w.emit(f"{where} = {w.value(node)[0]};")
    stores = list(w.lines)
    w.lines = []
    # the same commits with their values taken from hk_sv[hk_v][k] (the
    # two-pass full-block form): only when every written plane holds Real
    deferred = None
    targets = []                          # (plane var, component) of each deferred value
    if not stage.key_writes and all(stage.planes[p].get("dtype") in (None, "f64", "f32") for p, _ in stage.writes):
        deferred = ([], [])
        for plane, node in stage.writes:
            var = stage.planes[plane]["var"]
            vals = w.value(node)
            comps = [None] if not node.ttype.shape else [_flat(node.ttype.shape, e) for e in _entries(node.ttype.shape)]
            for c in comps:
                k = len(deferred[0])
                deferred[0].append(f"hk_sv[hk_v][{k}] = {vals[0 if c is None else c]};")
                deferred[1].append(w.spell.component_commit(w, var, c, "=", f"hk_sv[hk_v][{k}]"))
                targets.append((var, c))
        if w.lines or len(stores) != len(deferred[0]):
            deferred = None               # the stores computed a value of their own: keep one pass
        w.lines = []
    row_terms = [(w.value(node)[0], stage.planes[hi]["var"], stage.planes[comp]["var"] if comp else None, red)
                 for _, node, hi, comp, red in stage.row_sums]
    folds = [(stage.planes[out]["var"], stage.planes[scratch]["var"], [w.value(v)[0] for v in values],
              [w.value(c)[0] for c in cells], group) for out, scratch, values, cells, group in stage.fused_folds]
    body += w.lines                                   # (memoized: nothing new unless a term is a bare leaf)
    whole = _folds_whole(folds, block)
    if whole:
        body = _place_fold_stores(body, folds, block)

    real = "float" if mode == "float32" else "double"
    wrap = target.wrapper
    walk = StageWalk.of(stage, block, per_thread, xcd_order)
    out = [
        f"// hawk gfx950 stage '{stage.name}' (generated; mode {'banded' if stage.banded else mode}).",
        f"typedef {real} Real;",
        "struct GRefMirror { Real* data_; unsigned long long samples_, compStride_, sampleStride_; "
        "int deviceType_, deviceId_; };",
        "struct ScalarHandle { void* data; unsigned long long samples, stride; int deviceType, deviceId; };",
        f'extern "C" __attribute__((used)) __device__ char eagle_abi_tag[] = "{ABI_TAG}";',
        "extern \"C\" __attribute__((used)) __device__ unsigned long long eagle_layout_sizes[5] = {"
        + ", ".join(str(s) for s in LAYOUT_SIZES) + "};",
        "",
    ]
    text = "\n".join(body + stores)
    if any(c in text for c in MATH_HELPER_CALLS):
        out += MATH_DEVICE_DEFINES + _MATH_HELPERS.splitlines()
    if row_terms:
        out += _LANE_XOR_HELPERS.splitlines()
    if any(red == "sum" for *_, red in row_terms):
        out += (_BAND_ROW_SUM_HELPERS if stage.banded else _ROW_SUM_HELPERS).splitlines()
    if any(red != "sum" for *_, red in row_terms):
        out += _ROW_EXTREME_HELPERS.splitlines()
    if folds:
        out += _FOLD_HELPERS.splitlines()
    if stage.finish is not None:
        out += _FINISH_HELPER.splitlines()
    out += wrap.entry_signature(walk, stage.name).splitlines()
    out += wrap.unpack(walk).splitlines()
    auto = _auto_loop(stage)
    if stage.guard is not None:
        out += wrap.index_prologue(form="guard").splitlines()
        out += _guarded_lines(stage, w, body, stores)
    elif not row_terms and not folds:
        pair_loads = _adjacent_pairs(stage, mode, per_thread, deferred, targets, body)
        if pair_loads is not None:
            out.insert(out.index(f"typedef {real} Real;") + 1, "typedef Real hk_d2 __attribute__((ext_vector_type(2)));")
            head = wrap.index_prologue(form="full").splitlines()
            out += _pair_lines(head[0], pair_loads, deferred[0], targets, body, nontemporal)
            out += wrap.index_partial().splitlines()[3:]
        elif per_thread > 1 and deferred and deferred[0]:
            # a full block in two passes: every sample's values (and so every
            # load) first, then every store, so no load waits behind a store
            keep, commit = deferred
            head = wrap.index_prologue(form="full").splitlines()
            at = next(i for i, line in enumerate(head) if line.startswith("    if (")) + 1
            out += head[:at] + [f"    Real hk_sv[{per_thread}][{len(keep)}];"] + head[at:]
            out += body + ["        " + line for line in keep]
            out += ["    }", "#pragma unroll",
                    f"    for (int hk_v = 0; hk_v < {per_thread}; ++hk_v) {{",
                    f"        const long long hk_i = base + (static_cast<long long>(hk_blk) * {per_thread} + hk_v) * "
                    f"{block} + static_cast<long long>(threadIdx.x);"]
            out += ["        " + line for line in commit]
            out += wrap.index_partial().splitlines()
        elif per_thread > 1:
            out += wrap.index_prologue(form="full").splitlines()
            out += body + stores
            out += wrap.index_partial().splitlines()
        else:
            out += wrap.index_prologue().splitlines()
        out += body + stores
    elif row_samples(stage, per_thread) > 1:
        # Two or four samples a lane (j + 16v or j + 8v of its row), so a
        # row's first butterfly levels join in registers and 16 or 8 lanes
        # carry the rest: the same additions as the half-wave form with a half
        # or a quarter of its lane exchanges and adds a sample.  A lane past
        # `count` computes sample `base` and brings its row the identity.
        per = row_samples(stage, per_thread)
        out += wrap.index_prologue(form="rows", rows=len(row_terms), per_lane=per).splitlines()
        out += body
        opened, closed = wrap.sample_sum_frame(len(row_terms), "Real", "")
        out += opened.splitlines() + ["    " + line for line in stores] + closed.splitlines()
        out += wrap.rows_close([(term, w.spell.row_identity(red)) for term, _hi, _comp, red in row_terms]).splitlines()
        for k, (term, hi, comp, red) in enumerate(row_terms):
            if red == "sum":
                out += w.spell.sample_sum_rows(w, k, hi, comp, per, stage.banded)
            else:
                out += w.spell.sample_extreme_rows(w, red, k, hi, per)
    else:
        # Every lane of a half-wave takes part in its row's butterfly: a lane
        # past `count` computes sample `base` (always bound) and adds +0.
        out += wrap.index_prologue(form="live").splitlines()
        out += body
        opened, closed = wrap.sample_sum_frame(len(row_terms), "Real", "")
        out += opened.splitlines() + ["    " + line for line in stores] + closed.splitlines()
        for k, (term, hi, comp, red) in enumerate(row_terms):
            if red == "sum":
                out += w.spell.sample_sum(w, stage.banded, term, hi, comp)
            else:
                out += w.spell.sample_extreme(w, red, term, hi)
        out += _fused_fold_lines(folds, block, whole)
    out += wrap.index_epilogue().split("\n")
    if auto is not None:
        head = out.index(f'extern "C" __global__ void __launch_bounds__({block}) {stage.name}(')
        top = out[:head]
        if _STEPS_HELPERS.splitlines()[1] not in top:
            top += _STEPS_HELPERS.splitlines()
        out = top + out[head:]
        params, unpack = wrap.params(walk), wrap.unpack(walk).splitlines()
        out += _range_entry(stage, w, body, stores, params, unpack, block, per_thread, xcd_order, auto)
        out += _persist_entry(stage, mode, params, unpack, block, nontemporal, auto)
    return "\n".join(out)


_PLANE_INDEX = re.compile(r"(hk_p_\w+)\[")


def _adjacent_pairs(stage: Stage, mode: str, per_thread: int, deferred, targets: list, body: list):
    """The planes a light float64 stage loads, when its full blocks can run
    as pairs of adjacent samples (one 16-byte load and store a plane a pair):
    an even number of samples a thread, every written plane a scalar plane of
    Real, and every plane access in the body a scalar plane read at the lane's
    own sample.  ``None`` when the stage keeps the one-sample form."""
    if mode != "float64" or per_thread % 2 or not deferred or not deferred[0] or stage.guard is not None:
        return None
    if any(c is not None for _var, c in targets):
        return None
    text = "\n".join(body)
    if "hk_flat" in text or "threadIdx" in text:
        return None
    scalar = {info["var"] for info in stage.planes.values() if not info.get("shape") and info.get("dtype") in (None, "f64")}
    loads = []
    for m in _PLANE_INDEX.finditer(text):
        var = m.group(1)
        if not text.startswith("hk_i]", m.end()) or var not in scalar:
            return None
        if var not in loads:
            loads.append(var)
    return loads


def pair_candidate(stage: Stage, mode: str) -> bool:
    """Whether a stage can take the adjacent-pairs form at an even number of
    samples a thread, from its planes alone (the body's plane accesses are
    checked when it is rendered): float64, no reduction, fold, keyed write or
    guard, and every per-sample plane a scalar plane of Real."""
    if mode != "float64" or stage.row_sums or stage.fused_folds or stage.key_writes or stage.guard is not None:
        return False
    for info in stage.planes.values():
        if info["role"] in ("uniform", "nsamples"):
            continue
        if info["role"] not in ("per_sample", "mutable", "out") or info.get("shape") or info.get("dtype") not in (None, "f64"):
            return False
    return True


def _pair_lines(blk_line: str, loads: list, keep: list, targets: list, body: list, nontemporal: bool) -> list:
    """The full blocks of a stage as pairs of adjacent samples (see
    :func:`_adjacent_pairs`): thread t of block b takes samples 2t and 2t + 1
    of each 2 * hk_block of the block's span, the same samples the block
    covers one at a time, so a row of results is the same bits; the planes are
    read and written 16 bytes a lane.  Taken when every plane pointer and
    ``base`` keep a pair 16-byte aligned; the partial last block, and a launch
    that is not aligned, run the one-sample loop that follows."""
    ptrs = sorted(set(loads) | {var for var, _c in targets})
    aligned = " | ".join(f"reinterpret_cast<unsigned long long>({v})" for v in ptrs)
    out = [blk_line,
           f"    const bool hk_al = (({aligned}) & 15ull) == 0 && (base & 1LL) == 0;",
           "    if (hk_al && (static_cast<long long>(hk_blk) + 1) * (hk_per_thread * hk_block) <= count) {",
           "#pragma unroll",
           "    for (int hk_q = 0; hk_q < hk_per_thread / 2; ++hk_q) {",
           "        const long long hk_i0 = base + ((static_cast<long long>(hk_blk) * (hk_per_thread / 2) + hk_q)"
           " * hk_block + static_cast<long long>(threadIdx.x)) * 2;"]
    for v in loads:
        at = f"reinterpret_cast<const hk_d2*>(&{v}[hk_i0])"
        out.append(f"        const hk_d2 hk_pair_{v} = " + (f"__builtin_nontemporal_load({at});" if nontemporal else f"*{at};"))
    out += [f"        Real hk_sv[2][{len(keep)}];",
            "#pragma unroll",
            "        for (int hk_v = 0; hk_v < 2; ++hk_v) {",
            "        const long long hk_i = hk_i0 + hk_v;"]
    # each read of a loaded plane at the lane's sample (streamed or plain),
    # the plane's name not a suffix of a longer name
    reads = [(re.compile(r"__builtin_nontemporal_load\(&" + re.escape(v) + r"\[hk_i\]\)|(?<!\w)" + re.escape(v)
                         + r"\[hk_i\]"), f"hk_pair_{v}[hk_v]") for v in loads]
    for line in body:
        for pattern, pair in reads:
            line = re.sub(pattern, pair, line)
        out.append(line)
    out += ["        " + line for line in keep]
    out += ["        }"]
    for k, (var, _c) in enumerate(targets):
        at = f"reinterpret_cast<hk_d2*>(&{var}[hk_i0])"
        out += [f"        hk_d2 hk_st{k};", f"        hk_st{k}.x = hk_sv[0][{k}];", f"        hk_st{k}.y = hk_sv[1][{k}];",
                f"        __builtin_nontemporal_store(hk_st{k}, {at});" if nontemporal else f"        *{at} = hk_st{k};"]
    out += ["    }", "    return;", "    }"]
    return out


def row_samples(stage: Stage, per_thread: int) -> int:
    """Samples of a row each lane holds in a stage with row reductions: 4 at
    a multiple of four samples a thread, 2 at an even number, else 1 (a
    half-wave a row); 1 for a stage with fused folds."""
    if not stage.row_sums or stage.fused_folds:
        return 1
    return 4 if per_thread % 4 == 0 else 2 if per_thread % 2 == 0 else 1


def _auto_loop(stage: Stage):
    """The stepping loop of a ``hawk.steps(k, "auto")`` stage (its trips read
    at launch), or ``None``."""
    if stage.finish is None or stage.finish[2].kind != "loop_exit":
        return None
    loop = stage.finish[2].operands[0]
    return loop if loop.literal.count is not None else None


def _guarded_lines(stage: Stage, w: _Writer, body: list, stores: list, fast: bool = False) -> list:
    """The per-sample scope of a guarded stage.  The stage skips the samples
    its mask has finished.  Every lane of a wave reaches the finish count
    together (no lane leaves early), and a lane past `count` takes no sample.
    ``fast``: the ``_range`` entry's scope, which also counts a sample finished
    on entry and keeps each lane's trips in ``hk_ran``."""
    mask = stage.planes[stage.guard]["var"]
    out = ["        const bool hk_in = hk_flat < count;",
           "        const long long hk_i = base + (hk_in ? hk_flat : 0LL);"]
    if stage.finish is not None:
        out += ["        bool hk_new = false;"]
    out += [f"        if ({w.spell.guard([mask])}) {{"]
    out += ["    " + line for line in body + stores]
    if stage.finish is not None:
        cond = w.value(stage.finish[2])[0]
        out += [w.spell.finish(w, mask, cond)]
    if fast:
        loop = _auto_loop(stage)
        out += [f"            hk_ran = hk_ran > static_cast<unsigned>({w.trips[loop.uid]}) ? hk_ran"
                f" : static_cast<unsigned>({w.trips[loop.uid]});",
                f"            hk_ransum += static_cast<unsigned long long>({w.trips[loop.uid]});",
                "        } else if (hk_in) {",
                "            hk_new = true;               // finished on entry: counted by the fast entries"]
    out += ["        }"]
    if stage.finish is not None:
        out += [f"        hk_finish_count({stage.planes[stage.finish[1]]['var']}, hk_new);"]
    return out


#: The step reports of the fast entries (reference ``hawk/emit/cuda.py:277-370``):
#: a wave's largest and total trip counts, each added by one atomic a wave.
_STEPS_HELPERS = r"""
__device__ __forceinline__ void hk_steps_report(unsigned int* steps_max, unsigned long long* steps_sum,
                                                unsigned int most, unsigned long long total) {
    for (int o = 32; o > 0; o >>= 1) {
        const unsigned int m = __shfl_xor(most, o);
        most = m > most ? m : most;
        total += __shfl_xor(total, o);
    }
    if ((threadIdx.x & 63u) == 0u) {
        if (steps_max != nullptr && most != 0u) atomicMax(steps_max, most);
        if (steps_sum != nullptr && total != 0ull) atomicAdd(steps_sum, total);
    }
}
__device__ __forceinline__ void hk_count_report(unsigned int* counter, unsigned int n) {
    for (int o = 32; o > 0; o >>= 1) n += __shfl_xor(n, o);
    if ((threadIdx.x & 63u) == 0u && n != 0u) atomicAdd(counter, n);
}
"""

#: Samples a wave of the persistent entry claims with one atomic add (four a
#: lane): one counter serves the whole grid, and a claim per needy lane set
#: made it the bottleneck (measured on MI355X: 13.3 ms against 0.97 ms for
#: the plain entry over 2^22 samples of 1-256 steps).
PERSIST_BATCH = 256

#: The extra slots of the fast entries, after the kernel's own (each a
#: handle or a value in the argument block, before the partition triple).
RANGE_SLOTS = ("int_handle", "handle")                      # steps max (u32), steps sum (u64)
PERSIST_SLOTS = ("int_handle", "int_handle", "handle", "int")   # claim counter, steps max, steps sum, chunk


def _range_entry(stage, w, body, stores, params, unpack, block, per_thread, xcd_order, loop) -> list:
    """``<name>_range``: the stage over ``[base, base+count)``, one lane a
    sample, that also reports the steps taken (the largest and the total, into
    ``hk_steps`` / ``hk_stepsum`` when not null) and counts a sample finished
    on entry (reference ``hawk/emit/cuda.py:692-784``)."""
    out = [f'extern "C" __global__ void __launch_bounds__({block}) {stage.name}_range(',
           "        " + ",\n        ".join(params[:-3] + ["ScalarHandle hk_steps_m", "ScalarHandle hk_stepsum_m"]
                                         + params[-3:]) + ") {",
           "    (void)nSamples;"]
    out += unpack                       # indented, as the wrapper spells it
    out += ["    unsigned int* hk_steps = reinterpret_cast<unsigned int*>(hk_steps_m.data);",
            "    unsigned long long* hk_stepsum = reinterpret_cast<unsigned long long*>(hk_stepsum_m.data);",
            "    unsigned int hk_ran = 0u;",
            "    unsigned long long hk_ransum = 0ull;"]
    out += ["    const unsigned hk_blk = (gridDim.x & 7u) ? blockIdx.x"
            " : (blockIdx.x & 7u) * (gridDim.x >> 3) + (blockIdx.x >> 3);"] if xcd_order else \
        ["    const unsigned hk_blk = blockIdx.x;"]
    out += ["#pragma unroll",
            f"    for (int hk_v = 0; hk_v < {per_thread}; ++hk_v) {{",
            f"        const long long hk_flat = (static_cast<long long>(hk_blk) * {per_thread} + hk_v) * {block}"
            " + static_cast<long long>(threadIdx.x);"]
    out += _guarded_lines(stage, w, body, stores, fast=True)
    out += ["    }", "    hk_steps_report(hk_steps, hk_stepsum, hk_ran, hk_ransum);", "}", ""]
    return out


def _persist_entry(stage, mode, params, unpack, block, nontemporal, loop) -> list:
    """``<name>_persist``: a persistent grid whose waves claim samples
    (reference ``hawk/emit/cuda.py:465-689``).  A lane without a sample takes
    the next one at a claim: one ballot, one atomic add of the wave's needy
    lanes to ``hk_next`` by the wave's first needy lane, each lane taking the
    base plus its rank.  A claimed sample not finished on entry loads its
    carried values and the step's inputs into registers; the wave then runs up
    to ``hk_chunk`` trips of the step, each lane on its own sample; a lane
    whose sample leaves (its exit, or the launch's trips) writes it back and
    finishes it, and claims again at the next claim.  A wave leaves once
    every lane's claim fell past ``count`` and none holds a sample.  Each
    sample runs exactly the trips one launch of the stage runs, so the bits
    are the stage's; which lane runs it, and when, moves.  The finish count
    (samples finished in the launch or on entry) and the steps taken are
    added once a wave, at the end."""
    info = loop.literal
    mask = stage.planes[stage.guard]["var"]
    counter = stage.planes[stage.finish[1]]["var"]
    word = stage.planes[info.count]["var"]
    deps = Deps()
    free = free_inputs(loop, deps)
    # the claim: every free input of the step and the carried values' launch-start values
    wc = _Writer(stage, mode, nontemporal)
    wc.indent = 5
    wc.deps = deps
    wc.run(list(loop.operands) + free)
    live, live_set, claim = [], [], list(wc.lines)
    for m, f in enumerate(free):
        vals = wc.value(f)
        names = [f"hk_pl{m}_{e}" for e in range(len(vals))]
        live.append((f, names))
        ct = wc.ctype(f.ttype.dtype)
        live_set += [f"{ct} {nm}{{}};" for nm in names]
        claim += ["    " * 5 + f"{nm} = {v};" for nm, v in zip(names, vals)]
    carries = []
    for j, (c, x) in enumerate(zip(info.carries, loop.operands)):
        vals = wc.value(x)
        size = max(1, c.ttype.size if c.ttype.shape else 1)
        vals = vals * size if len(vals) == 1 and size > 1 else vals
        names = [f"hk_pc{j}_{e}" for e in range(size)]
        carries.append((c, names))
        live_set += [f"{wc.ctype(c.ttype.dtype)} {nm}{{}};" for nm in names]
        claim += ["    " * 5 + f"{nm} = {v};" for nm, v in zip(names, vals)]
    # one trip of the step, over the registers
    ws = _Writer(stage, mode, nontemporal)
    ws.indent = 4
    ws.deps = deps
    for f, names in live:
        ws.scope.put(f, names)
    for c, names in carries:
        ws.scope.put(c, names)
    ws.scope.put(info.index, ["hk_trip"])
    ws.run(ir.body_roots(info))
    nexts = [ws.value(x) for x in info.nexts]
    leave = ws.scalar(info.exit)
    step = list(ws.lines)
    temps, assign = [], []
    for (c, names), nv in zip(carries, nexts):
        nv = nv * len(names) if len(nv) == 1 and len(names) > 1 else nv
        for nm, val in zip(names, nv):
            t = f"hk_t_{nm[3:]}"
            temps.append("    " * 4 + f"const auto {t} = {val};")
            assign.append("    " * 4 + f"{nm} = {t};")
    # the write-back: each commit is a carried value (its loop_value)
    commit = []
    for plane, node in stage.writes:
        j = node.literal
        names = carries[j][1]
        var = stage.planes[plane]["var"]
        st = ws.store if nontemporal else (lambda ref, val: f"{ref} = {val};")
        if not node.ttype.shape:
            commit.append("    " * 4 + st(f"{var}[hk_i]", names[0]))
        else:
            for e in _entries(node.ttype.shape):
                cidx = _flat(node.ttype.shape, e)
                commit.append("    " * 4 + st(f"{var}[{cidx} * {var}_cs + hk_i]", names[cidx]))
    out = [f'extern "C" __global__ void __launch_bounds__({block}) {stage.name}_persist(',
           "        " + ",\n        ".join(params[:-3] + ["ScalarHandle hk_next_m", "ScalarHandle hk_steps_m",
                                                      "ScalarHandle hk_stepsum_m", "long long hk_chunk"]
                                         + params[-3:]) + ") {",
           "    (void)nSamples;"]
    out += unpack                       # indented, as the wrapper spells it
    out += ["    unsigned int* hk_next = reinterpret_cast<unsigned int*>(hk_next_m.data);",
            "    unsigned int* hk_steps = reinterpret_cast<unsigned int*>(hk_steps_m.data);",
            "    unsigned long long* hk_stepsum = reinterpret_cast<unsigned long long*>(hk_stepsum_m.data);",
            f"    const long long hk_budget = static_cast<long long>({word}[0]);",
            "    const long long hk_span = hk_chunk < 1 ? 1 : hk_chunk;     // every chunk runs a trip",
            "    const unsigned hk_lane = threadIdx.x & 63u;",
            "    const unsigned long long hk_below = (1ull << hk_lane) - 1ull;"]
    out += ["    " + d for d in live_set]
    out += ["    bool hk_has = false, hk_out = false;",
            "    long long hk_i = base, hk_trip = 0;",
            "    unsigned int hk_most = 0u, hk_fin = 0u;",
            "    unsigned long long hk_total = 0ull;",
            "    long long hk_qn = 0, hk_qe = 0;        // the wave's batch of sample offsets (the same in every lane)",
            "    while (true) {",
            "        // the claim: the wave's lanes without a sample take the next ones of the",
            "        // wave's batch, in lane order; a spent batch is refilled by one atomic add",
            "        const bool hk_needy = !hk_has && !hk_out;",
            "        const unsigned long long hk_need = __ballot(hk_needy);",
            "        if (hk_need != 0ull) {",
            "            if (hk_qn >= hk_qe) {",
            "                const int hk_lead = __ffsll(static_cast<long long>(hk_need)) - 1;",
            "                unsigned int hk_b = 0u;",
            "                if (hk_lane == static_cast<unsigned>(hk_lead))",
            f"                    hk_b = atomicAdd(hk_next, {PERSIST_BATCH}u);",
            "                hk_b = __shfl(hk_b, hk_lead);",
            "                hk_qn = static_cast<long long>(hk_b);",
            f"                hk_qe = hk_qn + {PERSIST_BATCH}LL < count ? hk_qn + {PERSIST_BATCH}LL : count;",
            "            }",
            "            if (hk_qn >= count) {",
            "                hk_out = true;                       // every sample is taken",
            "            } else {",
            "                const long long hk_avail = hk_qe - hk_qn;",
            "                const long long hk_r = static_cast<long long>(__popcll(hk_need & hk_below));",
            "                if (hk_needy && hk_r < hk_avail) {",
            "                    hk_i = base + hk_qn + hk_r;",
            f"                    if ({mask}[hk_i] == 0) {{"]
    out += claim
    out += ["                        hk_has = true;",
            "                        hk_trip = 0;",
            "                    } else {",
            "                        ++hk_fin;                // finished on entry",
            "                    }",
            "                }",
            "                const long long hk_took = static_cast<long long>(__popcll(hk_need));",
            "                hk_qn += hk_took < hk_avail ? hk_took : hk_avail;",
            "            }",
            "        }",
            "        if (__ballot(hk_has) == 0ull) {",
            "            if (__ballot(!hk_out) == 0ull) break;",
            "            continue;",
            "        }",
            "        if (hk_has) {",
            "            bool hk_exit = false;",
            "            for (long long hk_c = 0; hk_c < hk_span && hk_trip < hk_budget; ++hk_c) {"]
    out += step + temps + assign
    out += ["                ++hk_trip;",
            f"                if ({leave}) {{ hk_exit = true; break; }}",
            "            }",
            "            if (hk_exit || hk_trip >= hk_budget) {"]
    out += commit
    out += [f"                if (hk_exit) {{ {mask}[hk_i] = 1; ++hk_fin; }}",
            "                const unsigned int hk_ran = hk_trip > 0 ? static_cast<unsigned int>(hk_trip) : 0u;",
            "                hk_most = hk_ran > hk_most ? hk_ran : hk_most;",
            "                hk_total += hk_ran;",
            "                hk_has = false;",
            "            }",
            "        }",
            "    }",
            f"    hk_count_report({counter}, hk_fin);",
            "    hk_steps_report(hk_steps, hk_stepsum, hk_most, hk_total);",
            "}", ""]
    return out


#: The finish count (reference ``hawk/emit/wrapper.py:522-537``): one atomic
#: add a wave, of how many of its lanes finished their sample this launch.
_FINISH_HELPER = r"""
__device__ __forceinline__ void hk_finish_count(unsigned int* counter, bool newly) {
    const unsigned long long m = __ballot(newly);
    if ((threadIdx.x & 63u) == 0u && m != 0ull) atomicAdd(counter, static_cast<unsigned int>(__popcll(m)));
}
"""


#: LDS a fused fold stages a chunk of its slots in, per block, when the
#: block's contributions to every slot do not fit :data:`FOLD_LDS_WHOLE`.
FOLD_LDS_BYTES = 16384
#: LDS, per block, that may hold every fused fold's contributions to every
#: slot at once; each lane then stores each contribution as soon as it is
#: computed, so none stays in a register until the fold.
FOLD_LDS_WHOLE = 60 * 1024


def _folds_whole(folds: list, block: int) -> bool:
    """Whether every fused fold's contributions fit :data:`FOLD_LDS_WHOLE` at once."""
    total = sum(len(v) * (block // g) * ((g + 1) * 8 + 4) for _, _, v, _, g in folds)
    return bool(folds) and total <= FOLD_LDS_WHOLE


def _place_fold_stores(body: list, folds: list, block: int) -> list:
    """``body`` with each fused fold's LDS buffer declared first and each
    contribution's LDS store placed right after the line that computes it."""
    decl = []
    after: dict = {}
    for i, (_, _, values, _, g) in enumerate(folds):
        keys = block // g
        stride = keys * (g + 1)
        decl += [f"        __shared__ Real hk_fv{i}[{len(values) * stride}];",
                 f"        __shared__ int hk_fc{i}[{len(values) * keys}];",
                 f"        const int hk_fk{i} = static_cast<int>(threadIdx.x) / {g};",
                 f"        const int hk_fr{i} = static_cast<int>(threadIdx.x) - hk_fk{i} * {g};"]
        for e, var in enumerate(values):
            after.setdefault(var, []).append(f"hk_fv{i}[{e * stride} + hk_fk{i} * {g + 1} + hk_fr{i}] = {var};")
    out = list(decl)
    defined = re.compile(r"^(\s*)const [\w:<> ]+ (\w+) = ")
    for line in body:
        out.append(line)
        m = defined.match(line)
        if m and m.group(2) in after:
            out += [m.group(1) + text for text in after.pop(m.group(2))]
    for texts in after.values():                  # a contribution the body does not compute (a literal)
        out += ["        " + text for text in texts]
    return out


def fold_block(group: int) -> int | None:
    """The launch block of a stage that folds keys of ``group`` lanes in LDS:
    a multiple of 64 (a whole wave) and of ``group`` (no key crosses a block),
    at least 256 threads where that fits; ``None`` past 1024 threads."""
    b = group * 64 // math.gcd(group, 64)
    if b > 1024:
        return None
    return b * max(1, 256 // b)


def _fold_chunk(group: int, block: int, width: int) -> int:
    """Slots a fused fold stages at once: within :data:`FOLD_LDS_BYTES`, and no
    more pairs than the block has threads."""
    keys = block // group
    per_slot = keys * (group + 1) * 8 + keys * 4
    return max(1, min(width, group, FOLD_LDS_BYTES // per_slot))


def _fused_fold_lines(folds: list, block: int, whole: bool = False) -> list:
    """The ordered fold of each fused fold after the stage's values (the
    reference's log and fold, hawk/emit/team.py:281-312, without the log): the
    block's lanes put each slot's contribution into LDS, key k's run at
    k * (group + 1) (the pad keeps a pair's reads on other banks than its
    neighbours'), and key k's first lane its cell; then one thread per (key,
    slot) adds the key's run in lane order from +0 and stores the sum at the
    cell, counting the cell's claims (a second claim is reported, as the
    unfused fold does).  Every thread reaches every barrier: a lane past
    `count` computed sample `base` and its key is skipped.  With ``whole``,
    the body already stored every contribution in each fold's own buffer
    (:func:`_place_fold_stores`) and each fold is one chunk."""
    if not folds:
        return []
    if whole:
        return _whole_fold_lines(folds, block)
    lds_v = max(_fold_chunk(g, block, len(v)) * (block // g) * (g + 1) for _, _, v, _, g in folds)
    lds_c = max(_fold_chunk(g, block, len(v)) * (block // g) for _, _, v, _, g in folds)
    lines = [f"        __shared__ Real hk_fv[{lds_v}];",
             f"        __shared__ int hk_fc[{lds_c}];"]
    for out, scratch, values, cells, g in folds:
        keys = block // g
        chunk = _fold_chunk(g, block, len(values))
        stride = keys * (g + 1)
        lines += [f"        {{  // ordered fold into {out[5:]}: {len(values)} slots, {g} lanes a key, "
                  f"{keys} keys a block, {chunk} slots at a time",
                  f"            const int hk_fk = static_cast<int>(threadIdx.x) / {g};",
                  f"            const int hk_fr = static_cast<int>(threadIdx.x) - hk_fk * {g};"]
        for c0 in range(0, len(values), chunk):
            part = list(range(c0, min(len(values), c0 + chunk)))
            for j, e in enumerate(part):
                lines.append(f"            hk_fv[{j * stride} + hk_fk * {g + 1} + hk_fr] = {values[e]};")
            lines.append("            if (hk_fr == 0) {")
            for j, e in enumerate(part):
                lines.append(f"                hk_fc[{j * keys} + hk_fk] = {cells[e]};")
            lines += ["            }",
                      "            __syncthreads();",
                      f"            if (threadIdx.x < {keys * len(part)}) {{",
                      f"                const int hk_fs = static_cast<int>(threadIdx.x) / {keys};",
                      f"                const int hk_fq = static_cast<int>(threadIdx.x) - hk_fs * {keys};",
                      f"                if (static_cast<long long>(hk_blk) * {block} + hk_fq * {g} < count) {{",
                      f"                    const Real* hk_fp = hk_fv + hk_fs * {stride} + hk_fq * {g + 1};",
                      "                    Real hk_fsum = Real(0);",
                      "                    #pragma unroll 8",
                      f"                    for (int hk_fj = 0; hk_fj < {g}; ++hk_fj) hk_fsum = hk_fsum + hk_fp[hk_fj];",
                      f"                    hk_fold_store(hk_fsum, hk_fc[hk_fs * {keys} + hk_fq], {out}_n, {out}, "
                      f"{scratch} + 64, {scratch});",
                      "                }",
                      "            }",
                      "            __syncthreads();"]
        lines.append("        }")
    return lines


#: fp64 exp, sin and cos of this target (``HK_MATH_QUAL`` is the qualifier:
#: ``__device__ __forceinline__`` on the device; a host compiler builds the
#: same text to test it).  Method: Cody–Waite reduction with the constant's
#: head cut to trailing zeros, so the first step is exact, then a polynomial
#: on the reduced interval whose coefficients are Chebyshev fits computed at
#: 60 digits (mpmath ``chebyfit``) and rounded to double, evaluated by Horner
#: with fused multiply-adds.
#:
#: * exp: x = k ln2 + r, ln2 as a 42-bit head and a tail, |r| <= ln2/2;
#:   exp r = 1 + r + r^2 P(r), P of degree 10 fitting (e^r - 1 - r)/r^2
#:   (fit error 0.002 ulp of the result); 2^k by ldexp, which rounds once into
#:   the subnormal range.  The input is clamped to [-1200, 1200], where exp
#:   is 0 or inf anyway; NaN returns NaN.
#: * sin, cos: x = q pi/2 + r, pi/2 as two 33-bit heads and a tail (q * head
#:   exact for |x| < 2^17), |r| <= pi/4; sin r = r + r^3 S(r^2) with S of
#:   degree 6, cos r = 1 - r^2/2 + r^4 C(r^2) with C of degree 5 (1 - r^2/2
#:   kept with its rounding error); the quadrant q mod 4 picks and signs one
#:   of them.  |x| >= 2^17, infinities and NaN go to the library's sin/cos
#:   (its long reduction); sin returns x itself below 2^-26 (sin x rounds to
#:   x there, and -0 stays -0).  (A reduction by pi and one polynomial over
#:   |r| <= pi/2 was measured and dropped: it takes the sine without a
#:   select, but its mean error against glibc is 0.19 ulp against 0.12.)
_MATH_HELPERS = """
// hk_c(c): the constant c held in a scalar register pair, which the
// multiply-adds read directly; a literal the compiler can see would be
// rebuilt by two vector moves per sample.
HK_MATH_QUAL double hk_c(double c) {
    HK_MATH_PIN(c);
    return c;
}

// P(r) with exp r = 1 + r + r^2 P(r), |r| <= ln2/2.
HK_MATH_QUAL double hk_exp_poly(double r) {
    double p = hk_c(0x1.1f72fc848c527p-29);
    p = fma(p, r, hk_c(0x1.af4ddda32bea9p-26));
    p = fma(p, r, hk_c(0x1.27e4db67abc75p-22));
    p = fma(p, r, hk_c(0x1.71de0237479e4p-19));
    p = fma(p, r, hk_c(0x1.a01a01a6d7833p-16));
    p = fma(p, r, hk_c(0x1.a01a01abe6327p-13));
    p = fma(p, r, hk_c(0x1.6c16c16c162d6p-10));
    p = fma(p, r, hk_c(0x1.11111111100dfp-7));
    p = fma(p, r, hk_c(0x1.5555555555556p-5));
    p = fma(p, r, hk_c(0x1.5555555555557p-3));
    return fma(p, r, 0.5);
}

// x = k ln2 + r, |r| <= ln2/2; k returned through *k.
HK_MATH_QUAL double hk_exp_reduce(double x, double* k) {
    *k = rint(x * hk_c(0x1.71547652b82fep+0));
    const double r = fma(-*k, hk_c(0x1.62e42fefa3800p-1), x);
    return fma(-*k, hk_c(0x1.ef35793c76730p-45), r);
}

HK_MATH_QUAL double hk_exp(double x) {
    double k;
    const double r = hk_exp_reduce(fmin(fmax(x, -1200.0), 1200.0), &k);
    const double e = ldexp(1.0 + fma(r * r, hk_exp_poly(r), r), static_cast<int>(k));
    return x != x ? x + x : e;
}

// exp a - 1 for 0 <= a <= 64 (the tanh's argument), t = 2^k:
// (t - 1 + t r) + t r^2 P(r).  t r is exact and t - 1 >= t |r| for k >= 1
// (k = 0 makes t - 1 zero), so the head's sum and its rounding error are
// exact (Fast2Sum); the tail joins the error term before the last rounding,
// which keeps the cancellation just above a = ln2/2 from costing an ulp.
HK_MATH_QUAL double hk_expm1_pos(double a) {
    double k;
    const double r = hk_exp_reduce(a, &k);
    const double t = ldexp(1.0, static_cast<int>(k));
    const double tr = t * r;
    const double head = (t - 1.0) + tr;
    const double err = tr - (head - (t - 1.0));
    return head + fma(tr * r, hk_exp_poly(r), err);
}

HK_MATH_QUAL double hk_quadrant(double r, int n) {
    const double w = r * r;
    double s = hk_c(-0x1.ab17d393166dcp-41);
    s = fma(s, w, hk_c(0x1.61217f0abf087p-33));
    s = fma(s, w, hk_c(-0x1.ae645412c46d3p-26));
    s = fma(s, w, hk_c(0x1.71de3a5460952p-19));
    s = fma(s, w, hk_c(-0x1.a01a01a019938p-13));
    s = fma(s, w, hk_c(0x1.1111111111110p-7));
    s = fma(s, w, hk_c(-0x1.5555555555555p-3));
    const double sr = fma(r * w, s, r);
    double c = hk_c(-0x1.907da3000171dp-37);
    c = fma(c, w, hk_c(0x1.1eeb68e8ab8d4p-29));
    c = fma(c, w, hk_c(-0x1.27e4fa17d97fdp-22));
    c = fma(c, w, hk_c(0x1.a01a019f4eafap-16));
    c = fma(c, w, hk_c(-0x1.6c16c16c16967p-10));
    c = fma(c, w, hk_c(0x1.5555555555555p-5));
    const double hz = 0.5 * w;
    const double t = 1.0 - hz;
    const double cr = t + (((1.0 - t) - hz) + (w * w) * c);
    const double v = (n & 1) ? cr : sr;
    return (n & 2) ? -v : v;
}

HK_MATH_QUAL double hk_reduce(double x, int* n) {
    const double q = rint(x * hk_c(0x1.45f306dc9c883p-1));
    double r = fma(-q, hk_c(0x1.921fb54400000p+0), x);
    r = fma(-q, hk_c(0x1.0b4611a600000p-34), r);
    r = fma(-q, hk_c(0x1.3198a2e037073p-69), r);
    *n = static_cast<int>(q);
    return r;
}

HK_MATH_QUAL double hk_sin(double x) {
    if (!(fabs(x) < 0x1p17)) return sin(x);
    int n;
    const double r = hk_reduce(x, &n);
    const double y = hk_quadrant(r, n);
    return fabs(x) < 0x1p-26 ? x : y;
}

// sin x for x >= +0 or NaN: hk_sin's bits without its test for tiny
// arguments (below 2^-26 the reduction leaves r = x and the quadrant's
// r + r^3 S rounds to x; only -0 needed the test).
HK_MATH_QUAL double hk_sin_nonneg(double x) {
    if (!(x < 0x1p17)) return sin(x);
    int n;
    const double r = hk_reduce(x, &n);
    return hk_quadrant(r, n);
}

HK_MATH_QUAL double hk_cos(double x) {
    if (!(fabs(x) < 0x1p17)) return cos(x);
    int n;
    const double r = hk_reduce(x, &n);
    return hk_quadrant(r, n + 1);
}

// exp x for x <= 0 or NaN: hk_exp's bits without its upper clamp.
HK_MATH_QUAL double hk_exp_nonpos(double x) {
    double k;
    const double r = hk_exp_reduce(fmax(x, -1200.0), &k);
    const double e = ldexp(1.0 + fma(r * r, hk_exp_poly(r), r), static_cast<int>(k));
    return x != x ? x + x : e;
}

// sqrt x for x in [2^-700, DBL_MAX] or NaN.  y ~ 1/sqrt(x) from the
// hardware's reciprocal square root, then the coupled Newton-Raphson
// iteration on g ~ sqrt(x) and h ~ 1/(2 sqrt(x)) and two residual
// corrections d = x - g^2, each an exact fused multiply-add.  This is the
// device compiler's own sequence for sqrt, so the bits are sqrt's, less the
// rescaling of operands below 2^-767 and the test for 0 and infinity.
HK_MATH_QUAL double hk_sqrt_normal(double x) {
    const double y = HK_RSQ(x);
    double g = x * y;
    double h = y * 0.5;
    const double e = fma(-h, g, 0.5);
    g = fma(g, e, g);
    double d = fma(-g, g, x);
    h = fma(h, e, h);
    g = fma(d, h, g);
    d = fma(-g, g, x);
    return fma(d, h, g);
}

// a / b for a in [0, 2^100] and b in [2, 2^100] (or NaN): the device's own
// division sequence (a reciprocal refined by two Newton-Raphson steps, the
// quotient, its exact residual and one correction) without the operand
// scaling and the special-case fixup, which such operands never need; so the
// bits are the correctly rounded a / b.  (Below a = 2^-52, b rounds to 2 and
// every step is exact.)
HK_MATH_QUAL double hk_div_mid(double a, double b) {
    double y = HK_RCP(b);
    double e = fma(-b, y, 1.0);
    y = fma(y, e, y);
    e = fma(-b, y, 1.0);
    y = fma(y, e, y);
    const double q = a * y;
    return fma(fma(-b, q, a), y, q);
}

// tanh x = sign(x) e / (e + 2), e = expm1(2|x|) >= 0; +-1 from |x| = 22 on.
HK_MATH_QUAL double hk_tanh(double x) {
    const double a = fabs(x);
    const double e = hk_expm1_pos(fmin(a + a, 64.0));
    return x != x ? x + x : copysign(a >= 22.0 ? 1.0 : hk_div_mid(e, e + 2.0), x);
}

// tanh x for |x| <= 20 or NaN: hk_tanh's bits without its clamp, its
// saturation test and its NaN select (NaN passes through expm1 and the
// quotient).
HK_MATH_QUAL double hk_tanh_mid(double x) {
    const double a = fabs(x);
    const double e = hk_expm1_pos(a + a);
    return copysign(hk_div_mid(e, e + 2.0), x);
}
"""

#: The fp64 math calls this target spells with its own helpers, and the
#: qualifiers the device build gives them.
MATH_HELPER_CALLS = ("hk_exp(", "hk_sin(", "hk_cos(", "hk_tanh(", "hk_exp_nonpos(", "hk_sqrt_normal(",
                     "hk_tanh_mid(", "hk_sin_nonneg(")
MATH_DEVICE_DEFINES = ["#define HK_MATH_QUAL __device__ __forceinline__",
                       "#define HK_MATH_PIN(c) asm(\"\" : \"+s\"(c))",
                       "#define HK_RSQ(x) __builtin_amdgcn_rsq(x)",
                       "#define HK_RCP(x) __builtin_amdgcn_rcp(x)"]


def _whole_fold_lines(folds: list, block: int) -> list:
    """The fold phase of fused folds whose contributions are all in LDS."""
    lines = []
    for i, (out, scratch, values, cells, g) in enumerate(folds):
        keys = block // g
        lines.append(f"        if (hk_fr{i} == 0) {{")
        lines += [f"            hk_fc{i}[{e * keys} + hk_fk{i}] = {c};" for e, c in enumerate(cells)]
        lines.append("        }")
    lines.append("        __syncthreads();")
    for i, (out, scratch, values, cells, g) in enumerate(folds):
        keys = block // g
        stride = keys * (g + 1)
        pairs = keys * len(values)
        lines += [f"        // ordered fold into {out[5:]}: {len(values)} slots, {g} lanes a key, {keys} keys a block",
                  f"        for (int hk_ft = static_cast<int>(threadIdx.x); hk_ft < {pairs}; hk_ft += {block}) {{",
                  f"            const int hk_fs = hk_ft / {keys};",
                  f"            const int hk_fq = hk_ft - hk_fs * {keys};",
                  f"            if (static_cast<long long>(hk_blk) * {block} + hk_fq * {g} < count) {{",
                  f"                const Real* hk_fp = hk_fv{i} + hk_fs * {stride} + hk_fq * {g + 1};",
                  "                Real hk_fsum = Real(0);",
                  "                #pragma unroll 8",
                  f"                for (int hk_fj = 0; hk_fj < {g}; ++hk_fj) hk_fsum = hk_fsum + hk_fp[hk_fj];",
                  f"                hk_fold_store(hk_fsum, hk_fc{i}[hk_fs * {keys} + hk_fq], {out}_n, {out}, "
                  f"{scratch} + 64, {scratch});",
                  "            }",
                  "        }"]
    return lines


#: The store of a fused fold's sum: a cell outside the gradient plane sets
#: status bit 0; a cell claimed twice sets bit 1 and lowers status[1] to it.
_FOLD_HELPERS = """
__device__ __forceinline__ void hk_fold_store(Real s, int c, unsigned long long cells, Real* out, int* claims,
                                              int* status) {
    if (c < 0 || static_cast<unsigned long long>(c) >= cells) { atomicOr(status, 1); return; }
    if (atomicAdd(claims + c, 1) != 0) { atomicOr(status, 2); atomicMin(status + 1, c); }
    out[c] = s;
}
"""


#: The row sum of a default-policy ``hawk.sum`` (reference
#: ``hawk/emit/wrapper.py:542-665``): the 32 samples of a row (one half of a
#: wave64) combine as compensated (hi, comp) pairs over the pairs (l, l ^ 16),
#: (l, l ^ 8), ..., (l, l ^ 1) — the pairs of the reference's warp butterfly
#: and of its host row walk.  The combine is symmetric, so both lanes of a
#: pair hold its bits and every lane of the half ends with the row's partial.
_LANE_XOR_HELPERS = """
// The value of lane l ^ off (off = 1, 2, 4, 8, 16: a lane of the same half
// wave): DPP quad permutations for 1 and 2 and the bit mode of ds_swizzle (and
// mask 0x1f, xor mask off) for the others, with no lane address to compute
// and no LDS memory touched, where __shfl_xor issues a ds_bpermute on a
// computed address (the rows of a default-policy sum: 0.39-0.44 ms against
// 0.30-0.35 ms for two sums over 2^26 samples, the same bits).
__device__ __forceinline__ int hk_lane_xor_b32(int v, int off) {
    if (off == 1) return __builtin_amdgcn_mov_dpp(v, 0xB1, 0xF, 0xF, false);
    if (off == 2) return __builtin_amdgcn_mov_dpp(v, 0x4E, 0xF, 0xF, false);
    if (off == 4) return __builtin_amdgcn_ds_swizzle(v, 0x101F);
    if (off == 8) return __builtin_amdgcn_ds_swizzle(v, 0x201F);
    return __builtin_amdgcn_ds_swizzle(v, 0x401F);
}
__device__ __forceinline__ double hk_lane_xor(double v, int off) {
    return __hiloint2double(hk_lane_xor_b32(__double2hiint(v), off), hk_lane_xor_b32(__double2loint(v), off));
}
__device__ __forceinline__ float hk_lane_xor(float v, int off) {
    return __int_as_float(hk_lane_xor_b32(__float_as_int(v), off));
}
"""

_ROW_SUM_HELPERS = """
__device__ __forceinline__ bool hk_finite(Real x) { return (x - x) == Real(0); }
// The rounding error of s = a + b, +0 for an exact sum: Knuth's TwoSum,
// exact for any finite a and b, so the same value as the reference's Fast2Sum
// on the operands ordered by magnitude (aether::accum::twoSumErr), without the
// ordering's compare and selects.  Its callers drop it when s is not finite.
__device__ __forceinline__ Real hk_two_sum_err(Real a, Real b, Real s) {
    const Real bb = s - a;
    return ((a - (s - bb)) + (b - bb)) + Real(0);
}
__device__ __forceinline__ void hk_row_sum(Real& h, Real& c) {
#pragma unroll
    for (int off = 16; off > 0; off >>= 1) {
        const Real h2 = hk_lane_xor(h, off);
        const Real c2 = hk_lane_xor(c, off);
        const Real t = h + h2;
        c = hk_finite(t) ? (c + c2) + hk_two_sum_err(h, h2, t) : Real(0);
        h = t;
    }
}
// Two compensated pairs joined, as at each level of hk_row_sum.
__device__ __forceinline__ void hk_row_join(Real& h, Real& c, Real h2, Real c2) {
    const Real t = h + h2;
    c = hk_finite(t) ? (c + c2) + hk_two_sum_err(h, h2, t) : Real(0);
    h = t;
}
// A row held two or four samples a lane (lane j of a 16- or 8-lane group:
// samples j + 16v, or j + 8v): the pairs whose lanes share a register file
// join in registers, the first level's (+0 + +0) + err being err, and the
// lanes then take the remaining pairs (l, l ^ off) as in hk_row_sum: the same
// additions on a half or a quarter of the lanes.
__device__ __forceinline__ void hk_row_sum2(const Real (&s)[2], Real& h, Real& c) {
    h = s[0] + s[1];
    c = hk_finite(h) ? hk_two_sum_err(s[0], s[1], h) : Real(0);
#pragma unroll
    for (int off = 8; off > 0; off >>= 1) hk_row_join(h, c, hk_lane_xor(h, off), hk_lane_xor(c, off));
}
__device__ __forceinline__ void hk_row_sum4(const Real (&s)[4], Real& h, Real& c) {
    h = s[0] + s[2];                                            // pair (j, j + 16)
    c = hk_finite(h) ? hk_two_sum_err(s[0], s[2], h) : Real(0);
    Real h8 = s[1] + s[3];                                      // pair (j + 8, j + 24)
    const Real c8 = hk_finite(h8) ? hk_two_sum_err(s[1], s[3], h8) : Real(0);
    hk_row_join(h, c, h8, c8);                                  // pair (j, j + 8)
#pragma unroll
    for (int off = 4; off > 0; off >>= 1) hk_row_join(h, c, hk_lane_xor(h, off), hk_lane_xor(c, off));
}
"""


#: The row extremes of ``hawk.max`` / ``hawk.min`` (reference
#: ``hawk/emit/wrapper.py:543-600``: ``ssExtreme_``, ``ssIdentity_``,
#: ``sampleSumRow_``'s pairs): a row's 32 lanes combine by the pairs
#: (l, l ^ 16), ..., (l, l ^ 1), each pair as the extreme of (the lower
#: lane's value, the upper lane's) that ignores a NaN operand, so every lane of
#: the half ends with the row's extreme; a lane past ``count`` holds -inf (max)
#: or +inf (min).  The operand order is the reference's row walk's, slot l
#: with slot l + off: it decides the sign of an extreme of +0 and -0.
_ROW_EXTREME_HELPERS = """
__device__ __forceinline__ Real hk_extreme(int op, Real a, Real b) {
    if (a != a) return b;
    if (b != b) return a;
    return op == 1 ? (b > a ? b : a) : (b < a ? b : a);
}
__device__ __forceinline__ void hk_row_extreme(int op, Real& h) {
#pragma unroll
    for (int off = 16; off > 0; off >>= 1) {
        const Real h2 = hk_lane_xor(h, off);
        const bool low = (threadIdx.x & off) == 0;
        h = low ? hk_extreme(op, h, h2) : hk_extreme(op, h2, h);
    }
}
// Two or four samples a lane (j + 16v or j + 8v of the row): the pairs in
// the lane's registers first, the lower slot the left operand, then the pairs
// (l, l ^ off) across the lanes.
__device__ __forceinline__ Real hk_row_extreme_lanes(int op, Real h, int top) {
#pragma unroll
    for (int off = 16; off > 0; off >>= 1) {
        if (off > top) continue;
        const Real h2 = hk_lane_xor(h, off);
        const bool low = (threadIdx.x & off) == 0;
        h = low ? hk_extreme(op, h, h2) : hk_extreme(op, h2, h);
    }
    return h;
}
__device__ __forceinline__ Real hk_row_extreme2(int op, const Real (&s)[2]) {
    return hk_row_extreme_lanes(op, hk_extreme(op, s[0], s[1]), 8);
}
__device__ __forceinline__ Real hk_row_extreme4(int op, const Real (&s)[4]) {
    return hk_row_extreme_lanes(op, hk_extreme(op, hk_extreme(op, s[0], s[2]), hk_extreme(op, s[1], s[3])), 4);
}
"""


#: The row sum of the banded mode: each lane's term is the double-double
#: band (term, +0), and the 32 lanes of a row combine by the pairs of the
#: default sum's row with the band add of Hida, Li and Bailey's QD library
#: (TwoSum of the leading parts, TwoSum of the low parts, two quick
#: renormalisations); a non-finite leading sum drops the low part.  Knuth's
#: TwoSum is exact in either operand order, so the add is symmetric and every
#: lane of the half ends with the row's band.  The row stores (hi, lo).
_BAND_ROW_SUM_HELPERS = """
__device__ __forceinline__ bool hk_finite(double x) { return (x - x) == 0.0; }
__device__ __forceinline__ void hk_band_add(double& h, double& l, double h2, double l2) {
    double s = h + h2;
    const double sb = s - h;
    double e = (h - (s - sb)) + (h2 - sb);
    if (!hk_finite(s)) { h = s; l = 0.0; return; }
    const double t = l + l2;
    const double tb = t - l;
    const double f = (l - (t - tb)) + (l2 - tb);
    e = e + t;
    double q = s + e;
    e = e - (q - s);
    s = q;
    e = e + f;
    q = s + e;
    l = e - (q - s);
    h = q;
}
__device__ __forceinline__ void hk_band_row_sum(double& h, double& l) {
#pragma unroll
    for (int off = 16; off > 0; off >>= 1) {
        const double h2 = hk_lane_xor(h, off);
        const double l2 = hk_lane_xor(l, off);
        hk_band_add(h, l, h2, l2);
    }
}
// Two or four samples of a row a lane (j + 16v or j + 8v): the pairs whose
// lanes share a register file join in registers, each sample the band
// (term, +0), then the lanes take the remaining pairs (l, l ^ off).
__device__ __forceinline__ void hk_band_row_sum2(const double (&s)[2], double& h, double& l) {
    h = s[0];
    l = 0.0;
    hk_band_add(h, l, s[1], 0.0);
#pragma unroll
    for (int off = 8; off > 0; off >>= 1) hk_band_add(h, l, hk_lane_xor(h, off), hk_lane_xor(l, off));
}
__device__ __forceinline__ void hk_band_row_sum4(const double (&s)[4], double& h, double& l) {
    h = s[0];
    l = 0.0;
    hk_band_add(h, l, s[2], 0.0);                 // pair (j, j + 16)
    double h8 = s[1], l8 = 0.0;
    hk_band_add(h8, l8, s[3], 0.0);               // pair (j + 8, j + 24)
    hk_band_add(h, l, h8, l8);                    // pair (j, j + 8)
#pragma unroll
    for (int off = 4; off > 0; off >>= 1) hk_band_add(h, l, hk_lane_xor(h, off), hk_lane_xor(l, off));
}
"""


_FP_CALL = re.compile(r"\b(?:hk_)?(?:exp|sin|cos|tanh|sqrt|log|fabs)(?:_nonpos|_normal|_mid|_nonneg)?\(")
_FP_BINARY = re.compile(r"(?<=[\w\)\]]) [-+*/] (?=[\w\(])")
_PLANE_ACCESS = re.compile(r"hk_p_\w+(?:\[|_m\.|_cs\b)")
_SAMPLE_LOOP = re.compile(r"^\s*for \(long long \w+ = (-?\d+)LL; \w+ != (-?\d+)LL; \w+ \+= (-?\d+)LL\) \{")


def fp_ops_per_sample(source: str) -> int:
    """The floating-point operations one sample executes in a rendered
    per-sample stage: every binary + - * / and every exp/sin/cos/tanh/sqrt/
    log/fabs call in the value statements (plane loads, stores and index
    arithmetic excluded), each loop body counted trip times.  A division, a
    square root and a transcendental each count as one operation."""
    total = 0
    mult = [1]
    opens = []               # brace depth at which each sample loop was opened
    depth = 0
    body = source[source.index("const long long hk_i = base"):]
    for line in body.splitlines():
        m = _SAMPLE_LOOP.match(line)
        if m:
            start, stop, step = (int(x) for x in m.groups())
            mult.append(mult[-1] * max(0, (stop - start) // step))
            opens.append(depth)
        elif not _PLANE_ACCESS.search(line) and "hk_flat" not in line:
            total += mult[-1] * (len(_FP_BINARY.findall(line)) + len(_FP_CALL.findall(line)))
        depth += line.count("{") - line.count("}")
        while opens and depth <= opens[-1]:
            opens.pop()
            mult.pop()
    return total


@dataclass
class Plan:
    """How one kernel runs on the hip target: its per-sample stage (if any)
    and the team stages after it."""

    stage: Stage | None
    source: str | None
    team: list                      # [{"op": ..., planes...}]
    planes: dict                    # every plane a caller binds: name -> {"role", "shape", "dtype"}
    algorithmic_ops: int = 0        # FP ops per sample of the program as traced (before carried reuse)
    block: int | None = None        # a launch block the stage needs (a fused fold's), else the build's choice


def _mm16_products(program: Program):
    """``(inputs, products)`` when every sink of ``program`` assigns a 16x16
    product of two input planes, each possibly transposed (a forward ``C = A @ B``
    or its VJP): the kernel then runs as one MFMA team stage.  ``None`` otherwise."""
    sinks = program.sinks
    if not sinks or len(sinks) > 2 or not all(isinstance(s, Assign) for s in sinks):
        return None
    ins, prods = [], []

    def operand(n):
        transposed = n.kind == "transpose"
        if transposed:
            n = n.operands[0]
        if n.kind != "leaf" or n.ttype.shape != (16, 16) or n.literal[0] != "mat_in":
            return None
        pname = n.literal[1]
        if pname not in ins:
            ins.append(pname)
        return ins.index(pname), transposed

    for s in sinks:
        v = s.value
        if v.kind != "mm" or v.ttype.shape != (16, 16) or program.decls[s.name].ttype.shape != (16, 16):
            return None
        lhs, rhs = operand(v.operands[0]), operand(v.operands[1])
        if lhs is None or rhs is None:
            return None
        prods.append([lhs[0], rhs[0], lhs[1], rhs[1]])
    if len(ins) > 3 or len(prods) > len(ins):
        return None
    return ins, prods


def _carry_repeats(program: Program) -> Program:
    """``program`` with :func:`ir.carry_repeats` applied to its sinks' values
    (one pass over all of them, so values the sinks share stay shared)."""
    roots = ir.sink_roots(program.sinks)
    new = ir.carry_repeats(roots)
    if all(a is b for a, b in zip(new, roots)):
        return program
    it = iter(new)
    sinks = []
    for s in program.sinks:
        if isinstance(s, OrderedFold):
            values = tuple(next(it) for _ in s.values)
            sinks.append(dataclasses.replace(s, values=values, cells=tuple(next(it) for _ in s.cells)))
        elif isinstance(s, AccumWrite):
            value = next(it)
            sinks.append(dataclasses.replace(s, value=value, key=next(it)))
        else:
            sinks.append(dataclasses.replace(s, value=next(it)))
    return Program(program.decls, sinks, program.grid, program.tables)


def _refuse_unbanded(program: Program, name: str) -> None:
    """The banded mode builds the sample sums (the default policy and
    ``policy="ordered"``) with band accumulators; a reduction it has no band
    stage for is refused by name, as the reference refuses the reductions its
    banded build cannot certify (``hawk/emit/wrapper.py:158-196``)."""
    for s in program.sinks:
        what = None
        if isinstance(s, SampleSum) and s.group is not None:
            what = f"hawk.sum({s.name}, over=...)"
        elif isinstance(s, AccumWrite):
            what = f"hawk.scatter({s.name})"
        elif isinstance(s, OrderedFold):
            what = f"the ordered gradient fold into {s.name}"
        if what is not None:
            raise HawkError(f"{name}: {what} has no banded stage on the hip target; build this kernel in float64 "
                            "(the banded mode folds hawk.sum over the samples, default or ordered policy)")


def plan_kernel(program: Program, name: str, mode: str = "float64", block: int = 256,
                per_thread: int = 1, nontemporal: bool = False, reuse_carries: bool = True,
                fuse_folds: bool = True, target=None) -> Plan:
    """Split ``program`` into its per-sample stage and team stages, and render
    the per-sample stage.  With ``reuse_carries``, a loop's value that its next
    iteration would compute again is carried instead (:func:`ir.carry_repeats`);
    ``Plan.algorithmic_ops`` still counts the program as traced.  With
    ``fuse_folds``, an ordered fold whose keys fit a block (:func:`fold_block`)
    is done by the stage in LDS; otherwise the stage logs and a team stage folds."""
    target = TARGETS["hip"] if target is None else target
    if mode not in target.modes:
        said = [repr(m) for m in target.modes]
        said = said[0] if len(said) == 1 else ", ".join(said[:-1]) + " or " + said[-1]
        raise HawkError(f"mode={mode!r}: the {target.id} target builds {said}")
    banded = mode == "banded"
    if banded:
        _refuse_unbanded(program, name)
    if reuse_carries:
        reused = _carry_repeats(program)
        if reused is not program:
            traced = plan_kernel(program, name, mode, block, per_thread, nontemporal, reuse_carries=False,
                                 fuse_folds=fuse_folds, target=target)
            plan = plan_kernel(reused, name, mode, block, per_thread, nontemporal, reuse_carries=False,
                               fuse_folds=fuse_folds, target=target)
            plan.algorithmic_ops = traced.algorithmic_ops
            return plan
    if banded:
        mode = "float64"            # the banded mode's values are float64; its reductions fold bands
    products = _mm16_products(program)
    if products is not None:
        ins, prods = products
        outs = [s.name for s in program.sinks]
        dtype = "f32" if mode == "float32" else "f64"
        planes = {pname: {"role": program.decls[pname].role, "shape": [16, 16], "dtype": dtype}
                  for pname in ins + outs}
        return Plan(None, None, [{"op": "mm16", "in": ins, "out": outs, "products": prods, "dtype": dtype}],
                    planes)
    assigned = {id(s.value): s.name for s in program.sinks if isinstance(s, Assign)}
    extra, team, row_sums, key_writes, fused = [], [], [], [], []
    for s in program.sinks:
        if isinstance(s, OrderedFold):
            if fuse_folds and fold_block(s.group) is not None:
                # the stage folds in LDS: its claims and status are cleared before it runs
                scratch = f"hk_fold_{s.name}"
                fused.append((s.name, scratch, s.values, s.cells, s.group))
                team.append({"op": "fused_fold", "out": s.name, "scratch": scratch, "group": s.group,
                             "width": len(s.values), "before": True})
                continue
            # the stage logs each lane's contributions (one component plane per
            # read site) and each key's cells; the fold adds them per key
            values, cells = f"hk_logv_{s.name}", f"hk_logc_{s.name}"
            width = len(s.values)
            extra.append((values, ir.make("vec", s.values) if width > 1 else s.values[0]))
            key_writes.append((cells, s.cells, s.group))
            team.append({"op": "ordered_fold", "v": values, "c": cells, "out": s.name, "group": s.group,
                         "width": width})
            continue
        if isinstance(s, SampleSum) and s.group is None and (s.policy != "ordered" or s.op != "sum"):
            # the default policy, and max / min whatever the policy (exact either
            # way): rows of 32 samples in the stage, the canonical finish after
            rows = s.name if s.column is None else f"{s.name}_{s.column}"
            row_sums.append((rows, s.value, s.op))
            if s.op == "sum":
                t = {"op": "band_rows" if banded else "row_sum", "hi": f"hk_rows_{rows}",
                     "comp": f"hk_rows_{rows}_comp", "out": s.name}
            else:
                t = {"op": "row_extreme", "red": s.op, "hi": f"hk_rows_{rows}", "out": s.name}
            if s.column is not None:
                t["column"] = s.column            # the entry of a vector cell this stage stores
            team.append(t)
        elif isinstance(s, SampleSum):
            src = assigned.get(id(s.value))
            if src is None and s.value.kind == "leaf" and s.value.literal[0] == "per_sample":
                src = s.value.literal[1]
            if src is None:
                src = f"hk_sum_{s.name}" if s.column is None else f"hk_sum_{s.name}_{s.column}"
                extra.append((src, s.value))
            if s.group is None:
                team.append({"op": "band_ordered_sum" if banded else "ordered_sum", "u": src, "out": s.name,
                             **({} if s.column is None else {"column": s.column})})
            elif s.policy == "ordered":
                team.append({"op": "keyed_sum", "u": src, "out": s.name, "group": s.group})
            else:                                   # the default policy over some axes
                team.append({"op": "keyed_comp", "u": src, "out": s.name, "group": s.group})
        elif isinstance(s, AccumWrite):
            src = assigned.get(id(s.value))
            if src is None and s.value.kind == "leaf" and s.value.literal[0] == "per_sample":
                src = s.value.literal[1]
            if src is None:
                src = f"hk_scatter_{s.name}_{len(team)}"
                extra.append((src, s.value))
            if s.key.kind == "leaf" and s.key.literal[0] == "per_sample":
                key = s.key.literal[1]
            else:                                   # a computed key (a table read's cell): stored by the stage
                key = f"hk_key_{s.name}_{len(team)}"
                extra.append((key, s.key))
            team.append({"op": "ordered_scatter", "key": key, "v": src, "target": s.name})
    has_stage = any(isinstance(s, (Assign, Finish)) for s in program.sinks) or extra or row_sums or fused
    if has_stage and team and GUARD_MASK in program.decls and program.decls[GUARD_MASK].role == "terminated":
        raise HawkError(f"{name}: a guarded kernel (one declaring `terminated: Terminated`) commits per-sample "
                        "planes; a sum or a scatter over the samples its guard skips is not in this build")
    stage = source = None
    if has_stage:
        stage = _stage_planes(program, name, mode, extra, row_sums, key_writes, fused)
        stage.banded = banded
        source = render_stage(stage, mode, block, per_thread, nontemporal=nontemporal, target=target)
    planes = {}
    if stage is not None:
        for pname, info in stage.planes.items():
            planes[pname] = {k: info[k] for k in ("role", "shape", "dtype")}
            if info["role"] == "rows_out":
                planes[pname]["rows"] = 32                 # one value per 32 samples
            if info["role"] == "key_out":
                planes[pname]["group"] = info["group"]     # one value per `group` samples
            if info["role"] == "fold_scratch":
                planes[pname]["cells_of"] = pname[len("hk_fold_"):]   # 64 status words + a claim per cell
    for t in team:
        for key in ("u", "key", "v"):
            pname = t.get(key)
            if pname and pname not in planes:
                d = program.decls[pname]
                planes[pname] = {"role": d.role, "shape": list(d.ttype.shape), "dtype": d.ttype.dtype}
        for key in ("out", "target"):
            pname = t.get(key)
            if pname and isinstance(pname, str):
                # a vector cell (one entry a column) keeps its declared shape
                shape = list(program.decls[pname].ttype.shape) if t.get("column") is not None else []
                planes[pname] = {"role": "cell" if t["op"] in ("ordered_sum", "row_sum", "keyed_sum", "keyed_comp",
                                                              "band_rows", "band_ordered_sum", "row_extreme")
                                 else "accum_out",
                                 "shape": shape, "dtype": "f32" if mode == "float32" else "f64"}
                if t["op"] in ("keyed_sum", "keyed_comp"):
                    planes[pname]["group"] = t["group"]       # one cell per `group` samples
    for pname, info in planes.items():
        if pname.startswith("hk_"):
            info["scratch"] = True
        if mode == "float32" and info["dtype"] == "f64":
            info["dtype"] = "f32"                # a float32 build's real planes hold float32
    return Plan(stage, source, team, planes, fp_ops_per_sample(source) if source else 0,
                block=stage.block if stage is not None else None)
