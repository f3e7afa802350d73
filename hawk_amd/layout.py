"""Which axis of a per-sample plane holds the samples (reference
``hawk/_plane_layout.py`` and ``hawk/runtime.py:542-566``).

The kernels of this target read a per-sample plane component-major: a
``Vector[w]`` plane is ``(w, N)``, element ``(c, s)`` at ``c * N + s``, so one
load instruction of a wave reads 64 consecutive samples of one component.
``hawk.run`` also takes a sample-major plane ``(N, w)``: ``layout=
"samples_first"`` says so for every plane of the call, ``samples_first(x)``
for one array (the marker wins; a contradiction is refused), and a plane
whose shape reads only one way needs neither.  A plane whose shape reads both
ways (``N == w``) is refused unless one of them says which.  A sample-major
plane runs through a component-major copy: its values are copied in before
the launch and, for a plane the kernel writes, copied back after it, on the
launch's stream.  ``prepare`` binds planes by address and takes
component-major planes only.
"""

from __future__ import annotations

from .ir import HawkError

LAYOUTS = ("samples_first", "samples_last")


class Marked:
    """An array marked with the axis that holds its samples."""

    __slots__ = ("array", "axis")

    def __init__(self, array, axis: str):
        if isinstance(array, Marked):
            if array.axis != axis:
                raise HawkError(f"an array marked {array.axis} is marked {axis} again")
            array = array.array
        self.array, self.axis = array, axis


def samples_first(x) -> Marked:
    """``x`` holds its samples on its first axis: ``(N, ...)``."""
    return Marked(x, "samples_first")


def samples_last(x) -> Marked:
    """``x`` holds its samples on its last axis: ``(..., N)``, this target's own layout."""
    return Marked(x, "samples_last")


def check_layout(layout) -> None:
    if layout is not None and layout not in LAYOUTS:
        raise HawkError(f"layout={layout!r} is not one of 'samples_first' (planes are (N, w)), 'samples_last' "
                        "(planes are (w, N)), or None")


def resolve(kernel, arrays: dict, layout, per_sample_roles, written_roles):
    """``(arrays, write_back)``: every marker removed and every sample-major
    plane replaced by a component-major copy; ``write_back`` lists
    ``(caller's array, copy)`` for the planes the kernel writes."""
    check_layout(layout)
    out, back, pending = {}, [], []
    for name, value in arrays.items():
        marked = value if isinstance(value, Marked) else None
        x = marked.array if marked else value
        info = kernel.planes.get(name)
        if info is None or info["role"] not in per_sample_roles or not hasattr(x, "dim"):
            if marked is not None and info is not None and info["role"] not in per_sample_roles:
                raise HawkError(f"{name!r} is not a per-sample plane: it has no sample axis to mark")
            out[name] = x
            continue
        lead = tuple(info["shape"])
        shape = tuple(x.shape)
        last = len(shape) == len(lead) + 1 and shape[:-1] == lead
        first = len(shape) == len(lead) + 1 and shape[1:] == lead
        axis = marked.axis if marked else layout  # the array's marker beats the call's layout
        if not lead:                              # a scalar plane (N,) reads the same either way
            out[name] = x
            continue
        if axis is None:
            if first and last:
                raise HawkError(f"{name!r} has shape {shape}, which reads both as (w, N) and as (N, w): pass "
                                f"layout=\"samples_first\" or layout=\"samples_last\" to the call, or mark it "
                                f"hawk.samples_first({name}) / hawk.samples_last({name})")
            axis = "samples_first" if first else "samples_last"
        if axis == "samples_last" or not first:
            if axis == "samples_first" and not first:
                said = "is marked samples_first" if marked else "is sample-major under layout='samples_first'"
                raise HawkError(f"{name!r} {said} but has shape {shape}; a {lead} plane is "
                                f"({', '.join(['N'] + [str(e) for e in lead])})")
            out[name] = x
            continue
        pending.append((name, x, info))
    for name, x, info in pending:
        copy = x.movedim(0, -1).contiguous()
        out[name] = copy
        if info["role"] in written_roles:
            back.append((x, copy))
    return out, back
