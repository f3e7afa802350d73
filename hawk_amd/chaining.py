"""``hawk.chain``: several kernels run in sequence as one kernel.

Reference ``hawk/trace/chain.py`` (the entry) and ``hawk/ir/chain.py`` (the
binding).  Member ``j``'s read of a name binds to the value an earlier member
committed under that name; any other read is an input of the chain.  A name
no later member reads is an output; a name several members update in turn
(each reading it first) keeps its last value.  The binding is a substitution
in the IR: the composed body holds each intermediate as one value, read by
any number of members, and stores none of them, so one per-sample stage runs
the whole chain and the intermediates never reach HBM.

On gfx950 every boundary is fused, as the reference fuses every boundary
on a GPU (``hawk/ir/fusion.py:10``): a lane's registers hold the chain.  The
build estimates the fused stage's registers from the composed body
(:func:`estimate`, the reference's ``R0 + r x maxlive``,
``hawk/ir/fusion.py:33-72``), and fences the compiled kernel with it
(:func:`fence`, ``hawk/ir/fusion.py:124-126``): the sidecar records both,
and a chain that compiles past the fence is reported.  The derivative of a
chain is the derivative of its composed program.
"""

from __future__ import annotations

from . import ir
from .ir import AccumWrite, Assign, Decl, HawkError, OrderedFold, Program
from .trace import Kernel
from .types import role_of

#: The roles a member may read an intermediate as: its own lane's element.
BOUND_LEAF_ROLES = ("per_sample", "vec_in", "mat_in", "mutable")
#: The roles an intermediate may be committed as.
BOUND_SINK_ROLES = ("mutable", "out")


class Chain(Kernel):
    """A kernel composed of ``members`` in order (:func:`chain`)."""

    def __init__(self, name: str, program: Program, members: tuple, outputs: tuple):
        super().__init__(name, program)
        self.members = members
        self.outputs = outputs


def chain(*kernels, name: str) -> Chain:
    """Run ``kernels`` in sequence as ONE kernel named ``name``.

    A member's input binds to the value an earlier member committed under
    the same name; any other input is the chain's.  A name no later member
    reads is an output, and a name several members update in turn keeps its
    last value.  The values passed between members stay in the kernel: they
    are neither inputs nor outputs of the chain.  A chain of chains is the
    chain of their members.  The members must agree on their Grid (a chain
    runs as one launch)."""
    members = tuple(m for k in kernels for m in (k.members if isinstance(k, Chain) else (k,)))
    if not members:
        raise HawkError("chain: give at least one kernel")
    for k in members:
        if not isinstance(k, Kernel):
            raise HawkError(f"chain: {k!r} is not a traced kernel")
        if any(d.role == "terminated" for d in k.decls.values()):
            raise HawkError(f"chain: member {k.name!r} declares a Terminated mask (a guard, or a finish of its "
                            "own sample); a chain of guarded members is not in this build -- chain the step's "
                            "members first, then finish in one kernel")
    program, outputs = bind(members)
    return Chain(name, program, members, outputs)


def _grid_of(k: Kernel):
    g = k.program.grid
    return None if g is None else tuple(tuple(a) for a in g.axes)


def _sink_nodes(s) -> list:
    if isinstance(s, OrderedFold):
        return list(s.values) + list(s.cells)
    return [s.value, s.key] if isinstance(s, AccumWrite) else [s.value]


def _rebuilt(s, nodes: list):
    import dataclasses
    if isinstance(s, AccumWrite):
        return dataclasses.replace(s, value=nodes[0], key=nodes[1])
    if isinstance(s, OrderedFold):
        k = len(s.values)
        return dataclasses.replace(s, values=tuple(nodes[:k]), cells=tuple(nodes[k:]))
    return dataclasses.replace(s, value=nodes[0])


def bind(members, keep=()) -> tuple:
    """``(program, outputs)``: ``members`` composed in order (see the module
    text); ``keep`` names intermediates to commit as outputs too.  Refuses,
    naming both members and the name (reference ``hawk/ir/chain.py:67-127``):
    a name read with two types or two input roles; a second writer of a name
    that does not read it first; members whose Grids disagree; an
    intermediate read at another sample, or committed off its own lane (a
    sum or a scatter)."""
    first = members[0]
    for k in members[1:]:
        if _grid_of(k) != _grid_of(first):
            raise HawkError(f"chain: members {first.name!r} and {k.name!r} disagree on grid "
                            f"({_grid_of(first)!r} vs {_grid_of(k)!r}); a chain runs as one launch")
    latest: dict = {}           # name -> (member, rebuilt sink)
    inputs: dict = {}           # name -> (member, role, ttype) of an unbound read
    canon: dict = {}            # name -> the one leaf node every member's read of an input becomes
    reads: list = []            # per member: the names it reads
    for k in members:
        roots = [n for s in k.sinks for n in _sink_nodes(s)]
        order = ir.topo(roots)
        leaves = [n for n in order if n.kind == "leaf"]
        gathered = {n.operands[0].uid for n in order if n.kind == "gather"}
        reads.append({lf.literal[1] for lf in leaves})
        mapping = {}
        for lf in leaves:
            role, name = lf.literal
            if name not in latest:
                held = inputs.setdefault(name, (k.name, role, lf.ttype))
                if held[1:] != (role, lf.ttype):
                    raise HawkError(f"chain: {held[0]!r} reads {name!r} as (role={held[1]!r}, {held[2]!r}) but "
                                    f"{k.name!r} reads it as (role={role!r}, {lf.ttype!r}); rename one")
                one = canon.setdefault(name, lf)      # one input, one value (and one derivative)
                if one is not lf:
                    mapping[lf.uid] = one
                continue
            writer, sink = latest[name]
            if lf.ttype != sink.value.ttype:
                raise HawkError(f"chain: {writer!r} commits {name!r} as {sink.value.ttype!r} but {k.name!r} reads "
                                f"it as {lf.ttype!r}; one name is one value")
            if role not in BOUND_LEAF_ROLES or lf.uid in gathered or not isinstance(sink, Assign) \
                    or sink.role not in BOUND_SINK_ROLES:
                raise HawkError(f"chain: {k.name!r} reads {name!r}, which {writer!r} commits, at another sample "
                                f"(or {writer!r} commits it off its own lane); an intermediate is the lane's own "
                                "value: end the chain at that name and read the plane in a second chain")
            mapping[lf.uid] = sink.value
        for s in k.sinks:
            if s.name in latest and s.name not in reads[-1]:
                raise HawkError(f"chain: {latest[s.name][0]!r} and {k.name!r} both commit {s.name!r} and "
                                f"{k.name!r} does not read it first; the order would decide the value")
            if s.name in inputs and inputs[s.name][1] != "mutable":
                held = inputs[s.name]
                raise HawkError(f"chain: {held[0]!r} reads {s.name!r} as an input (role={held[1]!r}) but "
                                f"{k.name!r} commits it; rename one")
        new = ir.substitute(roots, mapping) if mapping else roots
        at = 0
        for s in k.sinks:
            width = len(_sink_nodes(s))
            latest[s.name] = (k.name, _rebuilt(s, new[at:at + width]))
            at += width
    writer_at = {}
    for j, k in enumerate(members):
        for s in k.sinks:
            writer_at[s.name] = j
    outputs = tuple(n for n, j in writer_at.items() if n in keep or not any(n in r for r in reads[j + 1:]))
    consumed = set(writer_at) - set(outputs) - set(inputs)
    decls: dict = {}
    tables: dict = {}
    for j, k in enumerate(members):            # an output's declaration is its last writer's
        for n, decl in k.decls.items():
            if n not in consumed and (n not in decls or writer_at.get(n) == j):
                decls[n] = decl
        for n, axes in k.program.tables.items():
            if n not in consumed:
                tables.setdefault(n, axes)
    sinks = [latest[n][1] for n in outputs]
    if not sinks:
        raise HawkError("chain: the members commit nothing a later member does not read")
    program = Program(decls, sinks, first.program.grid, tables)
    used = {n.literal[1] for n in ir.leaves_of(ir.sink_roots(sinks))} | {s.name for s in sinks}
    program.decls = {n: d for n, d in decls.items() if n in used}
    return program, outputs


#: Registers a per-sample stage holds besides its values (the lane index,
#: plane pointers and strides, loop counters), measured on gfx950 builds of
#: the example kernels.
R0 = 24
#: The fence: registers plus scratch words may pass the estimate by this
#: factor plus :data:`FENCE_SLACK` registers (the reference's constants).
FENCE_RATIO = 1.6
FENCE_SLACK = 16


def maxlive(program: Program) -> int:
    """The most elements per sample live at one point of ``program``'s body in
    its topological order: a value is live from its node (a plane read from
    the start, as the compiler hoists loads) to its last reader; a sink's
    value to the end; a literal holds no register."""
    roots = ir.sink_roots(program.sinks)
    order = ir.topo(roots)
    last = {}
    for i, node in enumerate(order):
        for o in node.operands:
            last[o.uid] = i
        if node.kind == "loop":
            for x in node.literal.nexts:
                last[x.uid] = i
    end = len(order)
    for r in roots:
        last[r.uid] = end
    delta = [0] * (end + 2)
    for i, node in enumerate(order):
        if node.kind in ("const", "iconst") or node.uid not in last or node.ttype.dtype == "tuple":
            continue
        width = 1
        for d in node.ttype.shape:
            width *= d
        delta[0 if node.kind == "leaf" else i] += width
        delta[last[node.uid] + 1] -= width
    best = live = 0
    for d in delta:
        live += d
        best = max(best, live)
    return best


def estimate(program: Program, mode: str = "float64") -> int:
    """Predicted VGPRs of the fused stage: ``R0 + r x maxlive``, r = 2 for an
    fp64 element, 1 for fp32."""
    return R0 + (2 if mode == "float64" else 1) * maxlive(program)


def fence(vgprs: int, scratch_bytes: int, est: int) -> bool:
    """Whether a compiled chain stays inside its estimate: ``vgprs + scratch / 4
    <= 1.6 x est + 16``."""
    return vgprs + scratch_bytes / 4 <= FENCE_RATIO * est + FENCE_SLACK


# --------------------------------------------------------------------------
# cuts: a chain past the register line runs as segments


#: The prefix of the plane a cut chain passes a value through from one
#: segment to the next (reference ``hawk/ir/chain.py:130``).
CROSS_PREFIX = "hwc_"
#: VGPRs a lane has before a kernel spills to scratch on gfx950: a chain is
#: cut where fusing the next member would take its estimate past this line.
REGISTER_LINE = 512


def _reads(k: Kernel) -> set:
    return {n.literal[1] for n in ir.leaves_of(ir.sink_roots(k.sinks))}


def cuts(members, mode: str = "float64", line: int = REGISTER_LINE) -> list:
    """The member boundaries to cut, greedy left to right (the shape of
    reference ``hawk/ir/fusion.py:95-121``): boundary ``b`` (before member
    ``b``) is cut when the segment from the last cut through member ``b``,
    fused, is estimated past ``line`` registers.  A matrix never crosses a cut."""
    out, a = [], 0
    for b in range(1, len(members)):
        later = set().union(*(_reads(k) for k in members[b:])) if b < len(members) else set()
        crossing = [s for k in members[a:b] for s in k.sinks if s.name in later]
        if any(len(s.value.ttype.shape) > 1 for s in crossing):
            continue
        after = set().union(*(_reads(k) for k in members[b + 1:])) if b + 1 < len(members) else set()
        program, _ = bind(members[a:b + 1], keep=tuple(after))
        if estimate(program, mode) > line:
            out.append(b)
            a = b
    return out


def segments(members, cut_at) -> list:
    """``[(program, writes, reads)]``, one per segment of ``members`` cut before
    each member index in ``cut_at`` (reference ``hawk/ir/chain.py:133-179``).
    A value one segment computes and a later one reads crosses in a plane of
    its own (``hwc_<name>``): the writer commits it there and the readers
    read their own lane's element, as any per-sample input.  ``writes`` and
    ``reads`` name those planes."""
    bounds = [0, *cut_at, len(members)]
    crossed: dict = {}                      # name -> ttype of a value an earlier segment stored
    out = []
    for a, b in zip(bounds, bounds[1:]):
        later = set().union(*(_reads(k) for k in members[b:])) if b < len(members) else set()
        program, outputs = bind(members[a:b], keep=tuple(later))
        roots = ir.sink_roots(program.sinks)
        mapping, reads = {}, []
        for lf in ir.leaves_of(roots):
            name = lf.literal[1]
            if name in crossed and lf.uid not in mapping:
                mapping[lf.uid] = ir.leaf(role_of(lf.ttype), CROSS_PREFIX + name, lf.ttype)
                reads.append(CROSS_PREFIX + name)
        sinks = list(program.sinks)
        if mapping:
            new = ir.substitute(roots, mapping)
            rebuilt, at = [], 0
            for s in sinks:
                width = len(_sink_nodes(s))
                rebuilt.append(_rebuilt(s, new[at:at + width]))
                at += width
            sinks = rebuilt
        decls = {n: d for n, d in program.decls.items() if n not in crossed}
        for name in reads:
            base = name[len(CROSS_PREFIX):]
            decls[name] = Decl(name, role_of(crossed[base]), crossed[base])
        kept, writes = [], []
        for s in sinks:
            if s.name not in later:
                kept.append(s)
                continue
            if not isinstance(s, Assign):
                raise HawkError(f"chain: {s.name!r} would cross a cut as a sum or a scatter; end the chain there")
            cross = CROSS_PREFIX + s.name
            kept.append(Assign(cross, s.value, "mutable"))
            decls[cross] = Decl(cross, "mutable", s.value.ttype)
            decls.pop(s.name, None)
            writes.append(cross)
            crossed[s.name] = s.value.ttype
        segment = Program(decls, kept, program.grid, dict(program.tables))
        used = {n.literal[1] for n in ir.leaves_of(ir.sink_roots(kept))} | {s.name for s in kept}
        segment.decls = {n: d for n, d in decls.items() if n in used}
        out.append((segment, writes, reads))
    return out
