"""``hawk.chain``: several kernels run in sequence as one kernel.

Reference ``hawk/trace/chain.py`` (the entry) and ``hawk/ir/chain.py`` (the
binding).  Member ``j``'s read of a name binds to the value an earlier member
committed under that name; any other read is an input of the chain.  A name
no later member reads is an output; a name several members update in turn
(each reading it first) keeps its last value.  Binding replaces each such
read with the committing member's node, so the composed program is one
expression graph: an intermediate is computed once in a lane's registers,
shared by every member that reads it, and never written to a plane.  One
per-sample stage then runs the whole chain, and HBM sees only the chain's
inputs and outputs.

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


def _flatten(kernels) -> tuple:
    """The members of a chain call: a chain given as a member contributes its
    own members, so chaining is associative."""
    flat = []
    for k in kernels:
        flat.extend(k.members if isinstance(k, Chain) else (k,))
    return tuple(flat)


def chain(*kernels, name: str) -> Chain:
    """ONE kernel named ``name`` that runs ``kernels`` one after another on
    each lane.

    Names connect the members: reading a name an earlier member committed
    reads that member's value, reading any other name reads an input of the
    chain.  The chain commits every name that no later member reads; a name
    several members update in turn (each reading it first) ends with the
    last update.  Values that pass from member to member never leave the
    lane.  Members that are chains contribute their own members, and all
    members must share one Grid (the chain is one launch).  Reference
    ``hawk/trace/chain.py`` (the user entry)."""
    members = _flatten(kernels)
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


class _Timeline:
    """What the members do with one name, in member order: every read (the
    member, its leaf, and whether the leaf is indexed by a computed key) and
    every commit (the member and its sink).  Within one member the reads come
    before the commits, since a member reads its planes as they were when it
    started."""

    def __init__(self, name: str):
        self.name = name
        self.events: list = []                 # ("read", j, leaf, indexed) | ("commit", j, sink)

    def commits(self) -> list:
        return [e for e in self.events if e[0] == "commit"]

    def last_commit(self) -> int | None:
        c = self.commits()
        return c[-1][1] if c else None

    def read_after(self, j: int) -> bool:
        return any(e[0] == "read" and e[1] > j for e in self.events)

    def check(self, names: list) -> None:
        """Refuse what makes the name ambiguous, in the reference's words
        (``hawk/ir/chain.py:67-127``; these texts are the interface)."""
        committed = None                       # the (member, sink) a read binds to, once a member commits
        as_input = None                        # (member, role, ttype) of the first read before any commit
        for e in self.events:
            if e[0] == "read":
                _, j, leaf, indexed = e
                role, ttype = leaf.literal[0], leaf.ttype
                if committed is None:
                    if as_input is None:
                        as_input = (names[j], role, ttype)
                    elif as_input[1:] != (role, ttype):
                        raise HawkError(f"chain: {as_input[0]!r} reads {self.name!r} as (role={as_input[1]!r}, "
                                        f"{as_input[2]!r}) but {names[j]!r} reads it as (role={role!r}, "
                                        f"{ttype!r}); rename one")
                    continue
                writer, sink = committed
                if ttype != sink.value.ttype:
                    raise HawkError(f"chain: {names[writer]!r} commits {self.name!r} as {sink.value.ttype!r} but "
                                    f"{names[j]!r} reads it as {ttype!r}; one name is one value")
                lane_local = (role in BOUND_LEAF_ROLES and not indexed and isinstance(sink, Assign)
                              and sink.role in BOUND_SINK_ROLES)
                if not lane_local:
                    raise HawkError(f"chain: {names[j]!r} reads {self.name!r}, which {names[writer]!r} commits, "
                                    f"at another sample (or {names[writer]!r} commits it off its own lane); an "
                                    "intermediate is the lane's own value: end the chain at that name and read "
                                    "the plane in a second chain")
                continue
            _, j, sink = e
            if committed is not None and not any(r[0] == "read" and r[1] == j for r in self.events):
                raise HawkError(f"chain: {names[committed[0]]!r} and {names[j]!r} both commit {self.name!r} and "
                                f"{names[j]!r} does not read it first; the order would decide the value")
            if as_input is not None and as_input[1] != "mutable" and committed is None:
                raise HawkError(f"chain: {as_input[0]!r} reads {self.name!r} as an input (role={as_input[1]!r}) "
                                f"but {names[j]!r} commits it; rename one")
            committed = (j, sink)


def _timelines(members) -> dict:
    """Every name the members touch, with its :class:`_Timeline`."""
    lines: dict = {}
    for j, k in enumerate(members):
        order = ir.topo([n for s in k.sinks for n in _sink_nodes(s)])
        indexed = {n.operands[0].uid for n in order if n.kind == "gather"}
        for leaf in (n for n in order if n.kind == "leaf"):
            name = leaf.literal[1]
            lines.setdefault(name, _Timeline(name)).events.append(("read", j, leaf, leaf.uid in indexed))
        for s in k.sinks:
            lines.setdefault(s.name, _Timeline(s.name)).events.append(("commit", j, s))
    return lines


def bind(members, keep=()) -> tuple:
    """``(program, outputs)`` of ``members`` composed in order; ``keep`` names
    values that later members read but the caller wants committed too.

    Two passes.  The first records, per name, what each member does with it
    (:class:`_Timeline`) and refuses an ambiguous name: two types or input
    roles for one name, a second commit by a member that does not read the
    name first, or a committed value read off its lane (at a computed index,
    or committed by a sum or a scatter).  The second composes: walking the
    members in order with an environment from each committed name to its
    current value, every read of a committed name becomes that value and
    every read of an input becomes one shared leaf.  Reference
    ``hawk/ir/chain.py:67-127`` (the binding rules)."""
    first = members[0]
    for k in members[1:]:
        if _grid_of(k) != _grid_of(first):
            raise HawkError(f"chain: members {first.name!r} and {k.name!r} disagree on grid "
                            f"({_grid_of(first)!r} vs {_grid_of(k)!r}); a chain runs as one launch")
    names = [k.name for k in members]
    lines = _timelines(members)
    for line in lines.values():
        line.check(names)

    env: dict = {}              # committed name -> its current sink (operands already composed)
    shared: dict = {}           # input name -> the one leaf all its reads become (one value, one derivative)
    for k in members:
        roots = [n for s in k.sinks for n in _sink_nodes(s)]
        swap = {}
        for leaf in ir.leaves_of(roots):
            name = leaf.literal[1]
            if name in env:
                swap[leaf.uid] = env[name].value
            elif shared.setdefault(name, leaf) is not leaf:
                swap[leaf.uid] = shared[name]
        composed = ir.substitute(roots, swap) if swap else roots
        pos = 0
        for s in k.sinks:
            width = len(_sink_nodes(s))
            env[s.name] = _rebuilt(s, composed[pos:pos + width])
            pos += width

    committed_in_order = list(dict.fromkeys(s.name for k in members for s in k.sinks))
    outputs = tuple(name for name in committed_in_order
                    if name in keep or not lines[name].read_after(lines[name].last_commit()))
    if not outputs:
        raise HawkError("chain: the members commit nothing a later member does not read")
    # Planes of the composed kernel: the inputs (declared by their first
    # reader) and the outputs (declared by their last committer); a value
    # passed between members has no plane.
    decls: dict = {}
    for j, k in enumerate(members):
        for name, decl in k.decls.items():
            line = lines.get(name)
            last = line.last_commit() if line is not None else None
            if name in outputs:
                if last == j:
                    decls[name] = decl
                else:
                    decls.setdefault(name, decl)
            elif name in shared:
                decls.setdefault(name, decl)
    tables = {}
    for k in members:
        for name, axes in k.program.tables.items():
            if name in decls:
                tables.setdefault(name, axes)
    sinks = [env[name] for name in outputs]
    program = Program(decls, sinks, first.program.grid, tables)
    used = {n.literal[1] for n in ir.leaves_of(ir.sink_roots(sinks))} | set(outputs)
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
