"""Ambient build options (reference ``hawk/emit/policy.py:66-150``).

``with hawk_amd.policy.using(launch_bounds=(128, 2)): hawk.build(...)`` gives
every build inside the block that option unless the build names its own; the
same for ``emit_form``, ``linalg_form``, ``wide_form`` and ``contraction``.
The values and their checks are the reference's.  On the hip target the forms
and ``contraction`` are recorded in each sidecar: its stages add in the order
they are written whatever the spelling, and 16x16 products always run on
MFMA, within the tolerance the reference's ``"gemm"`` route promises.
"""

from __future__ import annotations

from contextlib import contextmanager
from contextvars import ContextVar
from typing import Iterator

from .ir import HawkError

FORMS = ("auto", "static", "rolled")
LINALG_FORMS = ("auto", "team", "thread")
WIDE_FORMS = ("auto", "thread", "team")
#: ``direct`` is the kernel's own loop, ``gemm`` a matrix-multiply route.
CONTRACTION_FORMS = ("direct", "gemm")

_FORM: ContextVar[str] = ContextVar("hawk_amd_emit_form", default="auto")
_LINALG_FORM: ContextVar[str] = ContextVar("hawk_amd_linalg_form", default="auto")
_WIDE_FORM: ContextVar[str] = ContextVar("hawk_amd_wide_form", default="auto")
_CONTRACTION: ContextVar[str] = ContextVar("hawk_amd_contraction", default="direct")
_LAUNCH_BOUNDS: ContextVar = ContextVar("hawk_amd_launch_bounds", default=None)


def check_launch_bounds(launch_bounds):
    """``(threads, blocks_per_sm)`` as ints, checked as the reference checks
    them (threads a multiple of 32, threads * blocks at most 2048), or None."""
    if launch_bounds is None:
        return None
    threads, blocks = launch_bounds
    if threads < 32 or threads % 32 or blocks < 1 or threads * blocks > 2048:
        raise HawkError(f"launch_bounds=(threads, blocks) needs threads a multiple of 32 and threads*blocks "
                        f"<= 2048, got {launch_bounds!r}")
    return int(threads), int(blocks)


@contextmanager
def using(form: str = "auto", *, linalg_form: str = "auto", wide_form: str = "auto", contraction: str = "direct",
          launch_bounds=None) -> Iterator[None]:
    """Build under ``form`` (one of :data:`FORMS`), ``linalg_form``,
    ``wide_form``, ``contraction`` and ``launch_bounds`` for the duration of
    the block; an option a build passes itself wins."""
    for what, value, allowed in (("emit_form", form, FORMS), ("linalg_form", linalg_form, LINALG_FORMS),
                                 ("wide_form", wide_form, WIDE_FORMS),
                                 ("contraction", contraction, CONTRACTION_FORMS)):
        if value not in allowed:
            raise HawkError(f"{what} must be one of {allowed}, got {value!r}")
    bounds = check_launch_bounds(launch_bounds)
    tokens = (_FORM.set(form), _LINALG_FORM.set(linalg_form), _WIDE_FORM.set(wide_form),
              _CONTRACTION.set(contraction), _LAUNCH_BOUNDS.set(bounds))
    try:
        yield
    finally:
        for var, token in zip((_FORM, _LINALG_FORM, _WIDE_FORM, _CONTRACTION, _LAUNCH_BOUNDS), tokens):
            var.reset(token)


def form() -> str:
    return _FORM.get()


def linalg_form() -> str:
    return _LINALG_FORM.get()


def wide_form() -> str:
    return _WIDE_FORM.get()


def contraction() -> str:
    return _CONTRACTION.get()


def launch_bounds():
    return _LAUNCH_BOUNDS.get()
