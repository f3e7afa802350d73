"""The type tier: :class:`TensorType` and the declaration vocabulary.

``Scalar``, ``Vector[n]``, ``Matrix[r, c]``, ``Index``, ``Param`` and
``Mutable[...]`` annotate the parameters of a ``@hawk.kernel`` function, as
in the reference (``hawk/types.py``, ``hawk/trace/decl.py``): a declaration
says which plane a parameter is and how it is laid out, never how it is
computed.  Planes are component-major ``[component, sample]``: element
``(c, s)`` of a ``Vector`` plane at ``c*N + s``, element ``(r, c, s)`` of a
``Matrix[R, C]`` plane at ``(r*C + c)*N + s`` (reference
``hawk/emit/wrapper.py:1029-1055``).
"""

from __future__ import annotations

from dataclasses import dataclass

class HawkError(Exception):
    """Every refusal of the authoring surface, the compiler and the runtime."""


class FinishRefusal(HawkError):
    """A refused ``terminated = cond``; the trace names the kernel in front of it."""


#: IR dtypes: reals, the 64-bit index integer of loop counters, the int32
#: plane of an ``Index`` declaration, and the bool of a comparison.
DTYPES = ("f64", "f32", "i64", "i32", "bool", "tuple")


@dataclass(frozen=True)
class TensorType:
    """A node's static type: ``shape`` (``()``, ``(w,)`` or ``(r, c)``), ``dtype``
    and an optional semantic ``tag`` (``"chol_factor"``)."""

    shape: tuple
    dtype: str
    tag: str | None = None

    @property
    def size(self) -> int:
        out = 1
        for e in self.shape:
            out *= e
        return out


Scalar = TensorType((), "f64")
Index = TensorType((), "i32")


class _VectorDecl:
    """``Vector[n]``: an ``n``-component per-sample plane."""

    def __getitem__(self, width) -> TensorType:
        if not isinstance(width, int) or width < 1:
            raise HawkError(f"Vector[...] takes a positive int width, got {width!r}")
        return TensorType((width,), "f64")

    def __repr__(self) -> str:
        return "Vector"


class _MatrixDecl:
    """``Matrix[r, c]``: an ``r x c`` per-sample plane."""

    def __getitem__(self, shape) -> TensorType:
        if (not isinstance(shape, tuple) or len(shape) != 2
                or not all(isinstance(e, int) and e >= 1 for e in shape)):
            raise HawkError(f"Matrix[...] takes two positive int extents, got {shape!r}")
        return TensorType(tuple(shape), "f64")

    def __repr__(self) -> str:
        return "Matrix"


Vector = _VectorDecl()
Matrix = _MatrixDecl()


class _ParamDecl:
    """``Param``: one value for every sample, passed by value (a uniform)."""

    def __repr__(self) -> str:
        return "Param"


Param = _ParamDecl()


class _TerminatedDecl:
    """``Terminated``: the per-sample mask of finished samples (a bool plane,
    reference ``hawk/ir/nodes.py:848-870``).  A kernel that declares it runs
    only the samples not finished yet; ``terminated = cond`` finishes a
    sample (the mask becomes ``mask | cond``) and counts each newly finished
    one in the ``finished_count`` cell."""

    def __repr__(self) -> str:
        return "Terminated"

    def __setitem__(self, key, value):
        raise FinishRefusal("assigns the Terminated declaration itself, but the kernel did not declare a "
                            "Terminated parameter: declare `terminated: Terminated` and assign `terminated = cond`")


Terminated = _TerminatedDecl()


@dataclass(frozen=True)
class MutableDecl:
    """``Mutable[T]``: a plane the kernel writes.  Assigned per sample it is an
    output plane; assigned ``hawk.sum(...)`` it is a one-cell result; the
    target of ``hawk.scatter(...)`` it is a plane of cells.  With ``axes``
    (``Mutable["key"]``) it holds one value per coordinate of those lane axes:
    the result of ``hawk.sum(x, over=...)`` over the other axes."""

    ttype: TensorType
    axes: tuple = ()


def _label(where: str, label) -> str:
    if not isinstance(label, str) or not label.isidentifier() or label.startswith("_"):
        raise HawkError(f"{where}: an axis label is a Python identifier not starting with '_', got {label!r}")
    return label


def _axes(where: str, items: tuple) -> tuple:
    """``(("label", extent or None), ...)``: a bare label (a runtime extent)
    first only, then ``"label":extent`` slices (reference
    ``hawk/trace/decl.py:135-173``)."""
    axes = []
    for pos, item in enumerate(items):
        if isinstance(item, str) and pos == 0:
            axes.append((_label(where, item), None))
        elif isinstance(item, slice) and item.step is None and isinstance(item.start, str):
            if not isinstance(item.stop, int) or isinstance(item.stop, bool) or item.stop < 1:
                raise HawkError(f"{where}: the extent of axis {item.start!r} is a positive int, got {item.stop!r}")
            axes.append((_label(where, item.start), int(item.stop)))
        elif isinstance(item, str):
            raise HawkError(f"{where}: axis {item!r} at position {pos} has no extent; only the FIRST axis may "
                            f'be bare (a runtime extent), write "{item}":<extent>')
        else:
            raise HawkError(f'{where}: an axis is "<label>" (first only) or "<label>":<extent>, got {item!r}')
    labels = [a for a, _ in axes]
    if len(set(labels)) != len(labels):
        raise HawkError(f"{where}: duplicate axis label(s) in {labels}")
    return tuple(axes)


class _MutableFactory:
    def __getitem__(self, inner) -> MutableDecl:
        if isinstance(inner, TensorType):
            return MutableDecl(inner)
        items = inner if isinstance(inner, tuple) else (inner,)
        if items and isinstance(items[0], (str, slice)):
            return MutableDecl(TensorType((), "f64"), _axes("Mutable[...]", items))
        raise HawkError(f"Mutable[...] takes Scalar, Vector[n], Matrix[r, c] or lane-axis labels "
                        f'("key", "bin":256), got {inner!r}')

    def __repr__(self) -> str:
        return "Mutable"


Mutable = _MutableFactory()


@dataclass(frozen=True)
class TableDecl:
    """``Table[Scalar]`` (a 1-D plane of cells read at a flat index) or
    ``Table["row":R, "col":C]`` (read ``t.at(row=..., col=...)`` or
    ``t[r, c]``; a bare first label is a runtime extent): a lookup plane any
    lane reads at any cell (reference ``hawk/trace/decl.py:117-132``).  Every
    index is clamped into its axis: a read outside the table reads its edge."""

    axes: tuple                  # (("label", extent or None), ...); (("cell", None),) for Table[Scalar]
    positional: bool = False


class _TableFactory:
    def __getitem__(self, key) -> TableDecl:
        if isinstance(key, TensorType):
            if key.shape or key.dtype != "f64":
                raise HawkError(f"Table[...] holds Scalar cells in this build, got {key!r}")
            return TableDecl((("cell", None),), positional=True)
        items = key if isinstance(key, tuple) else (key,)
        return TableDecl(_axes("Table[...]", items))

    def __repr__(self) -> str:
        return "Table"


Table = _TableFactory()


@dataclass(frozen=True)
class GridDecl:
    """``Grid["key", "sample":8192]``: the launch's lanes as a grid of axes, the
    last the fastest (consecutive lanes); only the first may have a runtime
    extent.  The parameter it annotates reads the lane's coordinates
    (reference ``hawk/trace/decl.py:135-173``)."""

    axes: tuple

    def static_size(self) -> int:
        """The product of the extents after the first axis (the lanes of one
        first-axis coordinate), times the first's when it is static."""
        out = 1
        for _, e in self.axes:
            out *= e if e is not None else 1
        return out


class _GridFactory:
    def __getitem__(self, key) -> GridDecl:
        items = key if isinstance(key, tuple) else (key,)
        if not items:
            raise HawkError('Grid[...] needs at least one axis, e.g. Grid["i"]')
        return GridDecl(_axes("Grid[...]", items))

    def __repr__(self) -> str:
        return "Grid"


Grid = _GridFactory()


def role_of(ttype: TensorType) -> str:
    """The read role of an input plane of type ``ttype``."""
    return {0: "per_sample", 1: "vec_in", 2: "mat_in"}[len(ttype.shape)]
