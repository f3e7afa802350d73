"""The ``hip`` row's writer and wrapper: every piece of gfx950 HIP text the
per-sample renderer (:class:`hawk_amd.emit_hip._Writer`, the traversal) emits.

The reference splits its emitter the same way (``hawk/emit/writer.py``: a
writer spells each construct, ``WRITER_MEMBERS``; ``hawk/emit/wrapper.py:225-284``:
a wrapper wraps a body for one execution model), and a target row pairs one
of each (``hawk/targets/__init__.py:37-71``).  These two objects are that
pair for MI355X: :data:`HIP_WRITER` answers every member of the reference's
writer seam and :data:`HIP_WRAPPER` every member of its wrapper seam, over
this repository's IR.  A construct this build has no form for (the
reference's multi-branch dispatch, a scattered store from the per-sample
stage: scatters here are team stages) is refused by name.

Members take already-rendered operand text and return text; ``r`` is the
renderer, whose ``let`` / ``emit`` / ``stage`` the writer uses as the
reference's writers use their renderer's ``_emit`` and walk.
"""

from __future__ import annotations

import math
from dataclasses import dataclass
from types import MappingProxyType
from typing import Mapping

from .ir import HawkError, Node

_INF = math.inf
_WHOLE = (-_INF, _INF)


def _widen(lo: float, hi: float) -> tuple:
    """An interval grown outward by a relative 2^-50 at each end, so that a
    bound computed in Python's doubles still holds for the device's rounded
    result of the same operation."""
    if lo != lo or hi != hi:
        return _WHOLE
    return lo - abs(lo) * 2.0 ** -50, hi + abs(hi) * 2.0 ** -50


def _range_memo(r) -> dict:
    memo = getattr(r, "_value_ranges", None)
    if memo is None:
        memo = {}
        try:
            r._value_ranges = memo
        except AttributeError:
            pass
    return memo


def value_range(node, memo: dict) -> tuple:
    """Bounds ``(lo, hi)`` on every non-NaN value an fp64 node can take, by
    interval arithmetic over its operands: literals, negation, ``abs``,
    ``+ - *``, the monotone ``exp`` and ``sqrt``, and ``sin``/``cos``/``tanh``
    in [-1, 1]; any other node is unbounded.  NaN is always possible and is
    not described: a helper form chosen from these bounds must carry NaN
    through by itself."""
    if not isinstance(node, Node):
        return _WHOLE
    got = memo.get(node.uid)
    if got is not None:
        return got
    k, ops = node.kind, node.operands
    out = _WHOLE
    if k == "const" and isinstance(node.literal, (int, float)) and not isinstance(node.literal, bool):
        v = float(node.literal)
        out = (v, v) if v == v else _WHOLE
    elif k in ("neg", "abs", "exp", "sqrt", "real") and ops:
        lo, hi = value_range(ops[0], memo)
        if k == "neg":
            out = (-hi, -lo)
        elif k == "abs":
            out = (lo, hi) if lo >= 0 else (-hi, -lo) if hi <= 0 else (0.0, max(-lo, hi))
        elif k == "exp":
            out = _widen(0.0 if lo < -746 else math.exp(lo), _INF if hi > 709 else math.exp(hi))
            out = (max(out[0], 0.0), out[1])
        elif k == "sqrt":
            out = _widen(math.sqrt(lo) if lo > 0 else 0.0, math.sqrt(hi) if hi >= 0 else 0.0)
            out = (max(out[0], 0.0), out[1])
        else:
            out = (lo, hi)
    elif k in ("sin", "cos", "tanh"):
        out = (-1.0, 1.0)
    elif k in ("add", "sub", "mul") and len(ops) == 2:
        (a, b), (c, d) = value_range(ops[0], memo), value_range(ops[1], memo)
        if k == "add":
            ends = (a + c, b + d)
        elif k == "sub":
            ends = (a - d, b - c)
        else:
            ends = tuple(x * y for x in (a, b) for y in (c, d))
        out = _widen(min(ends), max(ends)) if all(e == e for e in ends) else _WHOLE
    memo[node.uid] = out
    return out


#: fp64 calls with a form for a bounded operand: (helper, does it fit the
#: operand's bounds).  Each form returns the general form's bits on its
#: domain and NaN for NaN.
#: * sqrt on [2^-700, DBL_MAX]: the Newton-Raphson square root seeded by the
#:   hardware reciprocal square root, without the rescaling of tiny operands
#:   and the test for 0 and infinity that the general form needs;
#: * tanh on [-20, 20]: no clamp of the argument, no saturation test, no NaN
#:   select;
#: * exp on (-inf, 0]: no upper clamp;
#: * sin on [0, inf): no test for tiny arguments (it only keeps -0's sign).
_DOMAIN_FORMS = {
    "sqrt": ("hk_sqrt_normal", lambda lo, hi: lo >= 2.0 ** -700 and hi <= 1.7e308),
    "tanh": ("hk_tanh_mid", lambda lo, hi: lo >= -20.0 and hi <= 20.0),
    "exp": ("hk_exp_nonpos", lambda lo, hi: hi <= 0.0),
    "sin": ("hk_sin_nonneg", lambda lo, hi: lo >= 0.0),
}


#: The reference's writer seam, member for member (``hawk/emit/writer.py:29-38``).
WRITER_MEMBERS = (
    "declare", "carry_type", "tape_decl", "counter_decl", "for_header",
    "tail_break", "sample_index_value", "plane_extent_value", "hoist",
    "selector_decl", "mix_count", "predicated_rank0", "predicated_tensor",
    "switch_default_tail", "typed_zero",
    "leaf", "const", "at", "select", "op",
    "guard", "store", "scatter_store", "accum_scattered", "or_scattered", "store_compensated",
    "sample_sum", "tape_write", "finish", "exit_if",
    "component_commit", "in_place_accumulate", "zero_row",
)
#: The reference's wrapper seam (``hawk/emit/wrapper.py:225-284``).
WRAPPER_MEMBERS = ("qualifier", "entry_signature", "index_prologue", "index_epilogue", "unpack", "fold_rows",
                   "sample_sum_frame", "dispatch")

_UNARY = {"exp": "exp", "sin": "sin", "cos": "cos", "tanh": "tanh", "sqrt": "sqrt", "log": "log",
          "abs": "fabs"}
_BINARY = {"add": "+", "sub": "-", "mul": "*", "div": "/"}
_COMPARE = {"lt": "<", "le": "<=", "gt": ">", "ge": ">=", "eq": "==", "ne": "!="}
_CTYPES = {"f64": "Real", "f32": "Real", "i64": "long long", "i32": "int", "bool": "bool"}


def _literal(x: float) -> str:
    if math.isnan(x):
        return "Real(__builtin_nan(\"\"))"
    if math.isinf(x):
        return "Real(__builtin_inf())" if x > 0 else "Real(-__builtin_inf())"
    return f"Real({repr(float(x))})"


def _dtype(ttype) -> str:
    return ttype if isinstance(ttype, str) else ttype.dtype


def _refuse(what: str):
    raise HawkError(f"the hip target has no form for {what} in this build")


class HipWriter:
    """gfx950 HIP spellings (``Real`` is ``double`` or ``float`` by the
    build's mode; fp64 ``tanh``, ``exp``, ``sin`` and ``cos`` are the emitted
    ``hk_`` helpers)."""

    id = "hip"
    #: Every component of a tensor value is a named local of its own.
    names_every_tensor = True
    #: A vector is stored one component at a time.
    commits_per_component = True
    #: No library twins: every site is scalarised.
    rolled_forms = False

    # -- declarations and loops ------------------------------------------
    def ctype(self, ttype) -> str:
        return _CTYPES[_dtype(ttype)]

    def declare(self, name: str, ttype, text: str, ordered: bool = True, held: bool = False) -> str:
        return f"const {self.ctype(ttype)} {name} = {text};"

    def reads_raw(self, kind: str) -> bool:
        return False

    def carry_type(self, ttype) -> str:
        return self.ctype(ttype)

    def tape_decl(self, elem: str, name, trip: int) -> str:
        names = [name] if isinstance(name, str) else list(name)
        return f"{elem} " + ", ".join(f"{t}[{trip}]" for t in names) + ";"

    def counter_decl(self, counter: str) -> str:
        return f"long long {counter} = 0;"

    def for_header(self, r, index: str, loop, count: str | None) -> str:
        if count is not None:
            return f"for (long long {index} = 0LL; {index} < {count}; ++{index}) {{"
        return (f"for (long long {index} = {loop.start}LL; {index} != {loop.stop()}LL; "
                f"{index} += {loop.step}LL) {{")

    def tail_break(self, flag: str, exited: str | None = None) -> str:
        return f"if ({flag}) {{ {exited} = true; break; }}" if exited else f"if ({flag}) break;"

    def exit_if(self, cond: str) -> str:
        return f"if ({cond}) {{"

    def sample_index_value(self) -> str:
        return "hk_i"

    def plane_extent_value(self, var: str) -> str:
        return f"static_cast<long long>({var}_n)"

    def hoist(self, r, text: str, ttype) -> str:
        return r.let(_dtype(ttype), text)

    # -- dispatch (the reference's multi-branch kernels: not in this build) --
    def selector_decl(self, r, kname: str, kind_expr: str, k: int, *, in_range: bool = False) -> str:
        _refuse("a multi-branch dispatch selector")

    def mix_count(self, mix: str, k: int, kname: str) -> str:
        _refuse("a dispatch branch-mix count")

    def predicated_rank0(self, kname: str, texts) -> str:
        _refuse("a predicated dispatch")

    def predicated_tensor(self, r, kname: str, texts) -> str:
        _refuse("a predicated dispatch")

    def switch_default_tail(self) -> str:
        return ""

    def typed_zero(self, ttype) -> str:
        return "Real(0)" if _dtype(ttype) in ("f64", "f32") else f"static_cast<{self.ctype(ttype)}>(0)"

    # -- expressions -------------------------------------------------------
    def leaf(self, r, leaf: Node, materialised: bool = True) -> list:
        """A plane's element(s) at the lane's sample: one load per component
        (component c of a plane at ``c * compStride + i``); a mask reads its
        byte; a uniform or a table is its binding itself."""
        role, name = leaf.literal
        p = r.stage.planes[name]["var"]
        if role in ("uniform", "lookup"):
            return [p]
        if role == "terminated":
            return [f"{p}[hk_i] != 0"]
        from .emit_hip import _entries, _flat
        if not leaf.ttype.shape:
            return [self.load(r, f"{p}[hk_i]")]
        return [self.load(r, f"{p}[{_flat(leaf.ttype.shape, e)} * {p}_cs + hk_i]")
                for e in _entries(leaf.ttype.shape)]

    def load(self, r, ref: str) -> str:
        return f"__builtin_nontemporal_load(&{ref})" if r.nontemporal else ref

    def const(self, node: Node) -> str:
        if node.kind == "iconst":
            return f"{int(node.literal)}LL"
        return _literal(node.literal)

    def at(self, r, table: str, cell: str, guard_cells: bool = False) -> str:
        """A plane read at a computed index: a Table's clamped cell, or (``guard_cells``)
        a scatter target's adjoint at the key, 0 outside ``[0, cells)``."""
        if guard_cells:
            return (f"static_cast<unsigned long long>(static_cast<long long>({cell})) < {table}_n"
                    f" ? {table}[{cell}] : Real(0)")
        return f"{table}[{cell}]"

    def select(self, r, node, c: str, a: str, b: str) -> str:
        return f"{c} ? {a} : {b}"

    def op(self, r, node, args, ranks=()) -> str:
        """One scalar operation: ``+ - * /`` infix, comparisons, negation,
        the math calls (fp64 tanh, exp, sin and cos as the ``hk_`` helpers),
        ``Real(x)`` casts."""
        k = node.kind if isinstance(node, Node) else node
        if k in _BINARY:
            return f"{args[0]} {_BINARY[k]} {args[1]}"
        if k in _COMPARE:
            return f"{args[0]} {_COMPARE[k]} {args[1]}"
        if k == "neg":
            return f"-{args[0]}"
        if k == "real":
            return f"Real({args[0]})"
        if k in _UNARY:
            fn = _UNARY[k]
            # The IR's dtype is f64 in a float32 build too (there Real is
            # float): the fp64 helpers and the interval analysis, which
            # assumes double arithmetic, apply to double builds only; a
            # float32 build calls the float overloads.
            dtype = node.ttype.dtype if isinstance(node, Node) else "f64"
            if getattr(r, "mode", "float64") == "float32":
                dtype = "f32"
            if dtype == "f64" and isinstance(node, Node) and fn in _DOMAIN_FORMS:
                lo, hi = value_range(node.operands[0], _range_memo(r))
                form, fits = _DOMAIN_FORMS[fn]
                if fits(lo, hi):
                    return f"{form}({args[0]})"
            if dtype == "f64" and fn in ("tanh", "exp", "sin", "cos"):
                fn = "hk_" + fn
            return f"{fn}({args[0]})"
        _refuse(f"the operation {k!r}")

    # -- sinks and the guard -----------------------------------------------
    def guard(self, bound) -> str | None:
        """The body-wide mask condition: the lane has a sample and its mask is clear."""
        if not bound:
            return None
        return " && ".join(["hk_in"] + [f"{m}[hk_i] == 0" for m in bound])

    def store(self, r, sink, target: str, value: str) -> str:
        """An own-lane store (non-temporal when the build streams)."""
        if r.nontemporal:
            return f"__builtin_nontemporal_store({value}, &{target});"
        return f"{target} = {value};"

    def scatter_store(self, r, sink, target: str, index: str, value: str) -> None:
        _refuse("a scattered store from the per-sample stage (hawk.scatter builds as an ordered team stage)")

    def accum_scattered(self, r, sink, target: str, index: str, value: str) -> None:
        _refuse("an atomic accumulate (hawk.scatter policy 'plain'); the ordered policy is a team stage")

    def or_scattered(self, r, sink, target: str, index: str, value: str) -> None:
        _refuse("a scattered OR commit (policy 'or')")

    def store_compensated(self, r, sink, target: str, comp: str, value: str) -> None:
        _refuse("a compensated scattered commit")

    def sample_sum(self, r, banded: bool, term: str, hi: str, comp: str) -> list:
        """A default-policy ``hawk.sum``'s row: the lane's term joins its
        half-wave's row of 32 (compensated pairs, or double-double bands in
        the banded mode; a lane past ``count`` adds +0) and lane 0 of the half
        stores the row."""
        return [f"        {{ Real hk_rh = hk_live ? static_cast<Real>({term}) : Real(0), hk_rc = Real(0);",
                f"          {'hk_band_row_sum' if banded else 'hk_row_sum'}(hk_rh, hk_rc);",
                "          if ((threadIdx.x & 31) == 0 && hk_live) {",
                "              const long long hk_r = (base + hk_flat) >> 5;",
                f"              {hi}[hk_r] = hk_rh;",
                f"              {comp}[hk_r] = hk_rc;",
                "          } }"]

    def sample_sum_rows(self, r, k: int, hi: str, comp: str, per: int, banded: bool = False) -> list:
        """A default-policy ``hawk.sum``'s row with ``per`` (2 or 4) samples
        a lane: row term ``k`` of the lane's samples (``hk_rt[k]``: samples
        j + (32/per)v of its row) joins its (32/per)-lane group's row
        (compensated pairs, or bands in the banded mode), and lane 0 of the
        group stores the row when the row's first sample is live."""
        return [f"        {{ Real hk_rh, hk_rc;",
                f"          {'hk_band_row_sum' if banded else 'hk_row_sum'}{per}(hk_rt[{k}], hk_rh, hk_rc);",
                f"          if ((threadIdx.x & {32 // per - 1}) == 0 && hk_lv0) {{",
                "              const long long hk_r = (base + hk_fl0) >> 5;",
                f"              {hi}[hk_r] = hk_rh;",
                f"              {comp}[hk_r] = hk_rc;",
                "          } }"]

    def sample_extreme_rows(self, r, red: str, k: int, hi: str, per: int) -> list:
        """A ``hawk.max`` / ``hawk.min`` row with ``per`` samples a lane."""
        op = 1 if red == "max" else 2
        return [f"        {{ const Real hk_rh = hk_row_extreme{per}({op}, hk_rt[{k}]);",
                f"          if ((threadIdx.x & {32 // per - 1}) == 0 && hk_lv0) {{",
                f"              {hi}[(base + hk_fl0) >> 5] = hk_rh;",
                "          } }"]

    def row_identity(self, red: str) -> str:
        """The term a lane past ``count`` brings to its row."""
        return {"sum": "Real(0)", "max": "static_cast<Real>(-__builtin_inf())",
                "min": "static_cast<Real>(__builtin_inf())"}[red]

    def sample_extreme(self, r, red: str, term: str, hi: str) -> list:
        """A ``hawk.max`` / ``hawk.min`` row: the lane's term joins its
        half-wave's row of 32 (a lane past ``count`` holds -inf / +inf, the
        op's identity) and lane 0 of the half stores the row's extreme."""
        op, ident = (1, "-__builtin_inf()") if red == "max" else (2, "__builtin_inf()")
        return [f"        {{ Real hk_rh = hk_live ? static_cast<Real>({term}) : static_cast<Real>({ident});",
                f"          hk_row_extreme({op}, hk_rh);",
                "          if ((threadIdx.x & 31) == 0 && hk_live) {",
                f"              {hi}[(base + hk_flat) >> 5] = hk_rh;",
                "          } }"]

    def tape_write(self, r, tape: str, slot: str, value: str) -> str:
        return f"{tape}[{slot}] = {value};"

    def finish(self, r, mask: str, cond: str) -> str:
        """Mark the sample finished and count it once."""
        return f"            if ({cond}) {{ {mask}[hk_i] = 1; hk_new = true; }}"

    def component_commit(self, r, target: str, at, op: str, value: str) -> str:
        ref = f"{target}[hk_i]" if at is None else f"{target}[{at} * {target}_cs + hk_i]"
        if op == "=":
            return self.store(r, None, ref, value)
        return f"{ref} {op} {value};"

    def in_place_accumulate(self, r, target: str, k: str, value: str) -> str:
        _refuse("an accumulate into a plane row inside a lowered loop")

    def zero_row(self, r, target: str, width: int) -> str:
        _refuse("a zeroed plane row ahead of a lowered loop")


@dataclass(frozen=True)
class StageWalk:
    """A per-sample stage seen the way the reference's wrapper seam sees a
    kernel (``hawk/ir/walk.py:80-106``, the frozen ``Walk``): the slots in
    ``arg_spec`` order, ``slot_of`` / ``slot_types`` (the inverse and type
    projection of ``arg_spec``), the rows planes of the stage's reductions
    over samples (``sample_sums``), and the finish's ``(mask, counter)``.
    ``planes`` carries what the HIP spelling needs beyond the types (each
    slot's variable and mirror kind), and the launch shape the geometry seam
    binds: ``block`` threads a workgroup, ``per_thread`` samples a thread,
    ``xcd_order`` (each XCD takes a contiguous eighth of the grid)."""

    name: str
    arg_spec: tuple
    slot_of: Mapping
    slot_types: Mapping
    planes: Mapping
    sample_sums: tuple = ()
    finish: tuple | None = None
    block: int = 256
    per_thread: int = 1
    xcd_order: bool = False

    @classmethod
    def of(cls, stage, block: int, per_thread: int = 1, xcd_order: bool = False) -> "StageWalk":
        from .ir import TensorType

        spec = tuple((role, name) for role, name in stage.arg_spec)
        return cls(name=stage.name, arg_spec=spec,
                   slot_of=MappingProxyType({slot: k for k, slot in enumerate(spec)}),
                   slot_types=MappingProxyType({(role, name): TensorType(tuple(stage.planes[name]["shape"]),
                                                                         stage.planes[name]["dtype"])
                                                for role, name in spec}),
                   planes=MappingProxyType({name: dict(stage.planes[name]) for _, name in spec}),
                   sample_sums=tuple(r[2] for r in stage.row_sums),
                   finish=tuple(stage.finish[:2]) if stage.finish is not None else None,
                   block=int(block), per_thread=int(per_thread), xcd_order=bool(xcd_order))


#: The output roles: a mirror the stage writes through (not const).
_WRITTEN = ("mutable", "out", "wide_out", "key_out", "accum_out", "rows_out", "fold_scratch")


class HipWrapper:
    """How a per-sample stage is wrapped for the gfx950 launch, with the
    reference wrapper seam's members and signatures
    (``hawk/emit/wrapper.py:225-284``): ``entry_signature(walk, name)`` (one
    by-value mirror per slot in ``arg_spec`` order, then the partition triple,
    reference ``hawk/emit/cuda.py:46-54``; the body's first lines name the
    launch shape as constants), ``unpack(walk)`` (each mirror's pointer),
    ``index_prologue(segment=None, *, active=None, box=None)`` (THE one
    geometry seam, ``i = base + flat`` over those constants) and
    ``index_epilogue()``.  Each returns C++ text.  The reference's segmented,
    active-map and box prologues have no form here and are refused by name."""

    qualifier = "__device__ __forceinline__"

    def params(self, walk) -> list:
        out = []
        for role, name in walk.arg_spec:
            info = walk.planes[name]
            var = info["var"]
            if info["kind"] in ("f64", "f32"):
                out.append(f"Real {var}")
            elif info["kind"] == "gref":
                out.append(f"GRefMirror {var}_m")
            else:
                out.append(f"ScalarHandle {var}_m")
        return out + ["long long base", "long long count", "long long nSamples"]

    def entry_signature(self, walk, name: str) -> str:
        """The entry's declaration and opening: role mirrors in ``arg_spec``
        order, the int64 partition triple, and the launch shape as the
        constants ``hk_block``, ``hk_per_thread``, ``hk_xcd_order`` that the
        geometry seam reads."""
        return "\n".join([f'extern "C" __global__ void __launch_bounds__({walk.block}) {name}(',
                          "        " + ",\n        ".join(self.params(walk)) + ") {",
                          "    (void)nSamples;",
                          f"    constexpr int hk_block = {walk.block}, hk_per_thread = {walk.per_thread};",
                          f"    constexpr bool hk_xcd_order = {'true' if walk.xcd_order else 'false'};"])

    def unpack(self, walk) -> str:
        """Each mirror's pointer (and component stride, and a table's cells)."""
        out = []
        for role, name in walk.arg_spec:
            info = walk.planes[name]
            var, kind = info["var"], info["kind"]
            if kind in ("f64", "f32"):
                continue
            is_input = role not in _WRITTEN and not (walk.finish is not None and name in walk.finish)
            cq = "const " if is_input else ""
            elem = {"i32": "int", "u32": "unsigned int", "bool": "unsigned char"}.get(info["dtype"], "Real")
            if kind == "gref":
                out.append(f"{cq}{elem}* __restrict__ {var} = reinterpret_cast<{cq}{elem}*>({var}_m.data_);")
                out.append(f"const long long {var}_cs = static_cast<long long>({var}_m.compStride_);")
            else:
                out.append(f"{cq}{elem}* __restrict__ {var} = reinterpret_cast<{cq}{elem}*>({var}_m.data);")
                if role in ("lookup", "accum_out", "fold_scratch"):
                    out.append(f"const unsigned long long {var}_n = {var}_m.samples;   // cells")
        return "\n".join("    " + line for line in out)

    def index_prologue(self, segment=None, *, active=None, box=None, form: str = "plain", rows: int = 0,
                       per_lane: int = 2) -> str:
        """The launch geometry: block ``i`` of the grid (XCD x takes a
        contiguous eighth when ``hk_xcd_order``), ``hk_per_thread`` samples a
        thread, and the lane's sample ``hk_i = base + hk_flat``.  ``form``:
        "plain" (a lane past ``count`` leaves), "live" (it computes sample
        ``base`` and stores nothing: a row reduction or a fold needs every
        lane), "full" (a block wholly below ``count`` runs an unguarded copy,
        closed by :meth:`index_partial`), "guard" (the guarded stage binds
        ``hk_i`` itself), "rows" (the live form ``per_lane`` (2 or 4) samples
        of a row at a time for ``rows`` row terms: each wave takes 64 *
        per_lane consecutive samples, rows of 32, and lane j of the
        (32/per_lane)-lane group g takes samples 32g + j + (32/per_lane)v;
        ``hk_rt[k][v]`` holds row term k of sample v, closed by
        :meth:`rows_close`)."""
        if segment is not None:
            _refuse("a segmented unit's prologue (offsets-plane runs)")
        if active is not None:
            _refuse("an active-lane prologue (a device-read live count and lane map)")
        if box is not None:
            _refuse("a box prologue (a thread over several lanes of a box)")
        # Workgroup i runs on XCD i % 8: with a grid of 8k workgroups, XCD x
        # takes the contiguous blocks [x*k, (x+1)*k) (any other grid keeps the
        # plain order), so each XCD's L2 streams one contiguous eighth.
        out = ["    const unsigned hk_blk = (!hk_xcd_order || (gridDim.x & 7u)) ? blockIdx.x"
               " : (blockIdx.x & 7u) * (gridDim.x >> 3) + (blockIdx.x >> 3);"]
        if form == "rows":
            if per_lane not in (2, 4):
                _refuse(f"rows of {per_lane} samples a lane")
            g = 32 // per_lane
            gb = g.bit_length() - 1
            out += ["#pragma unroll",
                    f"    for (int hk_p = 0; hk_p < hk_per_thread / {per_lane}; ++hk_p) {{",
                    f"        Real hk_rt[{rows}][{per_lane}];",
                    "        bool hk_lv0 = false;",
                    "        long long hk_fl0 = 0;",
                    "#pragma unroll",
                    f"        for (int hk_v = 0; hk_v < {per_lane}; ++hk_v) {{",
                    f"        const long long hk_flat = (static_cast<long long>(hk_blk) * (hk_per_thread / {per_lane})"
                    f" + hk_p) * ({per_lane} * hk_block) + ((threadIdx.x >> {gb}) << 5) + (threadIdx.x & {g - 1})"
                    f" + (hk_v << {gb});",
                    "        const bool hk_live = hk_flat < count;",
                    "        const long long hk_i = base + (hk_live ? hk_flat : 0LL);"]
            return "\n".join(out)
        if form == "full":
            # a block whose samples all lie below `count` runs the unguarded
            # copy of the body: no exit between samples, so every sample's
            # loads can issue before the first store (the partial last block
            # takes the guarded copy that index_partial opens)
            out += ["    if ((static_cast<long long>(hk_blk) + 1) * (hk_per_thread * hk_block) <= count) {"]
        out += ["#pragma unroll",
                "    for (int hk_v = 0; hk_v < hk_per_thread; ++hk_v) {",
                "        const long long hk_flat = (static_cast<long long>(hk_blk) * hk_per_thread + hk_v) * hk_block"
                " + static_cast<long long>(threadIdx.x);"]
        if form == "full":
            out += ["        const long long hk_i = base + hk_flat;"]
        if form == "plain":
            out += ["        if (hk_flat >= count) break;",
                    "        const long long hk_i = base + hk_flat;"]
        elif form == "live":
            out += ["        const bool hk_live = hk_flat < count;",
                    "        const long long hk_i = base + (hk_live ? hk_flat : 0LL);"]
        return "\n".join(out)

    def index_partial(self) -> str:
        """After the full block's body (``form="full"``): close it and open the
        guarded loop of the partial last block."""
        return "\n".join(["    }", "    return;", "    }",
                          "#pragma unroll",
                          "    for (int hk_v = 0; hk_v < hk_per_thread; ++hk_v) {",
                          "        const long long hk_flat = (static_cast<long long>(hk_blk) * hk_per_thread + hk_v)"
                          " * hk_block + static_cast<long long>(threadIdx.x);",
                          "        if (hk_flat >= count) break;",
                          "        const long long hk_i = base + hk_flat;"])

    def rows_close(self, terms: list) -> str:
        """The end of one of a lane's row samples (``form="rows"``): its row terms
        (``(term, identity)``: a lane past ``count`` brings the identity) kept
        for the rows, and the first sample's liveness and index."""
        out = [f"        hk_rt[{k}][hk_v] = hk_live ? static_cast<Real>({term}) : {ident};"
               for k, (term, ident) in enumerate(terms)]
        out += ["        if (hk_v == 0) { hk_lv0 = hk_live; hk_fl0 = hk_flat; }", "        }"]
        return "\n".join(out)

    def index_epilogue(self) -> str:
        return "    }\n}\n"

    def fold_rows(self, width: int) -> int:
        """Rows of 32 samples a wave64 reduces at once: a half-wave is a row."""
        return 2

    def sample_sum_frame(self, width: int, elem: str, store: str, op: str = "sum", live: str | None = None) -> tuple:
        """(open, close) around the row reductions of a stage: every lane
        takes part (``hk_live``), the stores of a live lane only.  A sum, a
        max and a min share it; a prefix form's device-read ``live`` count
        has no form here."""
        if op not in ("sum", "max", "min"):
            _refuse(f"a sample reduction by {op!r}")
        if live is not None:
            _refuse("a sample reduction over a device-read live count")
        return ("        if (hk_live) {", "        }")

    def dispatch(self, kind_spelling: str, branch_spellings, policy: str, **kw) -> str:
        _refuse("a multi-branch dispatch")


HIP_WRITER = HipWriter()
HIP_WRAPPER = HipWrapper()
