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
            raise TypeError(f"Vector[...] takes a positive int width, got {width!r}")
        return TensorType((width,), "f64")

    def __repr__(self) -> str:
        return "Vector"


class _MatrixDecl:
    """``Matrix[r, c]``: an ``r x c`` per-sample plane."""

    def __getitem__(self, shape) -> TensorType:
        if (not isinstance(shape, tuple) or len(shape) != 2
                or not all(isinstance(e, int) and e >= 1 for e in shape)):
            raise TypeError(f"Matrix[...] takes two positive int extents, got {shape!r}")
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


@dataclass(frozen=True)
class MutableDecl:
    """``Mutable[T]``: a plane the kernel writes.  Assigned per sample it is an
    output plane; assigned ``hawk.sum(...)`` it is a one-cell result; the
    target of ``hawk.scatter(...)`` it is a plane of cells."""

    ttype: TensorType


class _MutableFactory:
    def __getitem__(self, inner) -> MutableDecl:
        if isinstance(inner, TensorType):
            return MutableDecl(inner)
        raise TypeError(f"Mutable[...] takes Scalar, Vector[n] or Matrix[r, c], got {inner!r}")

    def __repr__(self) -> str:
        return "Mutable"


Mutable = _MutableFactory()


def role_of(ttype: TensorType) -> str:
    """The read role of an input plane of type ``ttype``."""
    return {0: "per_sample", 1: "vec_in", 2: "mat_in"}[len(ttype.shape)]
