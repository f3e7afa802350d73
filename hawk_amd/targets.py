"""The targets table of this build: one row, ``hip``, for MI355X (gfx950).

A row pairs a writer (how each construct is spelled) with a wrapper (how a
per-sample body becomes a kernel entry) and carries what the build reads:
how it compiles, how the runtime enters it, its file suffixes and the
features it builds.  :func:`hawk_amd.artifact.build_bundle` and the per-sample
renderer take everything target-specific from the row; neither compares a
target's name.  The reference's table has the same shape
(``hawk/targets/__init__.py:37-71``); its ``cuda``, ``host`` and ``c`` rows
are not part of this build.
"""

from __future__ import annotations

from dataclasses import dataclass

from .hip_target import HIP_WRAPPER, HIP_WRITER, WRAPPER_MEMBERS, WRITER_MEMBERS

#: The toolchain a row compiles with (the reference's words, ``hawk/targets/__init__.py:30-31``).
GPU = "gpu"
#: How the runtime enters a built kernel: a device entry launched through the C-ABI.
ENTRY_DEVICE = "device"

#: What a kernel may use that a row may not build.  The hip row builds all of
#: them; a row listing fewer refuses the rest by name before anything renders.
FEATURES = (
    "sample_reduction",      # hawk.sum over the samples (fixed-tree, compensated or banded)
    "ordered_scatter",       # hawk.scatter / ordered gradient folds (keyed team stages)
    "active_set",            # Terminated guards and Finish masks (per-sample early exit)
    "auto_steps",            # steps="auto": the persistent and range fast entries
    "rolled_loops",          # hawk.steps loops kept rolled, with tapes for the adjoint
    "tables",                # lookup tables read with at[...]
    "chains",                # hawk.chain, fused or cut into segments
)


@dataclass(frozen=True)
class Target:
    """One row of :data:`TARGETS`.  ``writer`` answers ``WRITER_MEMBERS`` and
    ``wrapper`` ``WRAPPER_MEMBERS``; ``offload_arch`` is the code-object ISA;
    ``format`` the manifest's word for the code object; ``artifact`` and
    ``source`` the file suffixes; ``modes`` the scalar modes the row builds."""

    id: str
    about: str
    writer: object
    wrapper: object
    compile: str
    entry: str
    offload_arch: str
    format: str
    artifact: str
    source: str
    features: frozenset
    modes: tuple


TARGETS: dict[str, Target] = {t.id: t for t in (
    Target("hip", "builds gfx950 code objects for MI355X", HIP_WRITER, HIP_WRAPPER, GPU, ENTRY_DEVICE,
           "gfx950", "hsaco", ".hsaco", ".hip", frozenset(FEATURES), ("float64", "float32", "banded")),
)}

#: What ``build`` builds when ``targets`` is not given.
DEFAULT_TARGETS = ("hip",)


def row(target_id: str) -> Target:
    """The row named ``target_id``; an unknown name is refused."""
    from .ir import HawkError
    if target_id not in TARGETS:
        raise HawkError(f"targets=[{target_id!r}]: this build's target row is 'hip' (gfx950); the reference's "
                        "host and cuda rows are not part of it")
    return TARGETS[target_id]


def conforms(target: Target) -> list:
    """The seam members ``target``'s writer or wrapper lacks (empty when the
    row answers every member)."""
    def lacks(obj, m):
        if m == "qualifier":                # the wrapper's one text attribute
            return not isinstance(getattr(obj, m, None), str)
        return not callable(getattr(obj, m, None))
    missing = [f"writer.{m}" for m in WRITER_MEMBERS if lacks(target.writer, m)]
    missing += [f"wrapper.{m}" for m in WRAPPER_MEMBERS if lacks(target.wrapper, m)]
    return missing
