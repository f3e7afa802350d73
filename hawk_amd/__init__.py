"""hawk for MI355X: the gfx950 device target of hawk's kernel language.

The authoring surface and the three doors of the reference
(``hawk/__init__.py:50-90``): ``@hawk.kernel``, the declaration vocabulary
(``Scalar``, ``Vector[n]``, ``Matrix[r, c]``, ``Index``, ``Param``,
``Mutable[...]``), ``hawk.sum`` / ``hawk.scatter``, ``hawk.math``,
``hawk.diff.vjp`` / ``jvp``, and ``hawk.build`` / ``hawk.load`` /
``hawk.run``.  ``build`` emits HIP for gfx950 and compiles it with hipRTC;
``load``/``run`` launch it through ``libhawk_core.so`` on PyTorch-ROCm
tensors.  Typical use::

    import hawk_amd as hawk
    from hawk_amd import Param, Scalar

    @hawk.kernel
    def scale(x: Scalar, a: Param, b: Param) -> Scalar:
        return a * x + b

    bundle = hawk.build([scale], "unit/")
    hawk.run(hawk.load("unit/", "scale"), x=x, a=2.0, b=1.0, out=y)   # x, y: cuda tensors
"""

from __future__ import annotations

from .ir import HawkError
from .types import Grid, Index, Matrix, Mutable, Param, Scalar, Table, TensorType, Terminated, Vector

__version__ = "0.1.0"

_LAZY = {
    "kernel": ("trace", "kernel"),
    "Kernel": ("trace", "Kernel"),
    "Value": ("trace", "Value"),
    "sum": ("trace", "sum"),
    "max": ("trace", "max"),
    "min": ("trace", "min"),
    "mean": ("trace", "mean"),
    "scatter": ("trace", "scatter"),
    "chain": ("chaining", "chain"),
    "steps": ("trace", "steps"),
    "build": ("artifact", "build_bundle"),
    "load": ("runtime", "load"),
    "run": ("runtime", "run"),
    "samples_first": ("layout", "samples_first"),
    "samples_last": ("layout", "samples_last"),
}
_SUBMODULES = ("math", "diff", "runtime", "artifact", "compile", "ir", "emit_hip", "trace", "chaining", "policy",
               "layout")

__all__ = ["Grid", "HawkError", "Index", "Matrix", "Mutable", "Param", "Scalar", "Table", "TensorType", "Terminated",
           "Vector",
           "__version__", *_LAZY, *_SUBMODULES]


def __getattr__(name: str):
    import importlib

    if name in _LAZY:
        module, attr = _LAZY[name]
        value = getattr(importlib.import_module(f".{module}", __name__), attr)
        globals()[name] = value
        return value
    if name in _SUBMODULES:
        value = importlib.import_module(f".{name}", __name__)
        globals()[name] = value
        return value
    raise AttributeError(f"module {__name__!r} has no attribute {name!r}")


def __dir__():
    return sorted(__all__)
