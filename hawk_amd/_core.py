"""ctypes binding of ``libhawk_core.so`` (the C-ABI in ``include/hawk_core.h``).

This is the Python face the reference gets from its nanobind module
``hawk._core`` (reference ``src/hawk_core.cpp:518-679``): :class:`ArgBlock`
with ``bind``/``rebind``, a loaded :class:`DeviceLibrary` with ``entry``, and
:class:`DeviceEntry.run` (the one launch crossing), plus ``layout_sizes``,
``build_digest``, ``build_info`` and ``crossings``.  Loading the library runs
the same self-check the reference runs at import (reference
``hawk/__init__.py:146-212``): its stamped build digest must equal the digest
of the sources beside it, and its layout table must equal
:mod:`hawk_amd._contracts`.  A missing or stale library is refused by name —
there is no fallback path.
"""

from __future__ import annotations

import ctypes
import threading
from pathlib import Path

from . import _contracts
from .ir import HawkError

_LIB_PATH = Path(__file__).resolve().parent / "libhawk_core.so"
_lib = None
_lock = threading.Lock()

HK_OK = 0
_c_char_pp = ctypes.POINTER(ctypes.c_char_p)


def _declare(lib) -> None:
    V, I, U64, I64, SZ = ctypes.c_void_p, ctypes.c_int, ctypes.c_uint64, ctypes.c_int64, ctypes.c_size_t
    sig = {
        "hk_last_error": (ctypes.c_char_p, []),
        "hk_layout_sizes": (I, [ctypes.POINTER(U64)]),
        "hk_layout_field_name": (ctypes.c_char_p, [I]),
        "hk_build_digest": (ctypes.c_char_p, []),
        "hk_build_info": (ctypes.c_char_p, []),
        "hk_crossings": (U64, []),
        "hk_rtc_compile": (I, [ctypes.c_char_p, ctypes.c_char_p, _c_char_pp, I,
                               ctypes.POINTER(V), ctypes.POINTER(SZ), ctypes.POINTER(ctypes.c_char_p)]),
        "hk_rtc_version": (I, []),
        "hk_free": (None, [V]),
        "hk_load": (I, [V, SZ, ctypes.POINTER(V)]),
        "hk_unload": (None, [V]),
        "hk_entry_get": (I, [V, ctypes.c_char_p, ctypes.POINTER(V)]),
        "hk_argblock_new": (I, [_c_char_pp, I, ctypes.POINTER(V)]),
        "hk_argblock_free": (None, [V]),
        "hk_argblock_size": (I, [V]),
        "hk_bind": (I, [V, I, U64, U64, U64, ctypes.c_int32, ctypes.c_int32]),
        "hk_rebind": (I, [V, ctypes.POINTER(I64), ctypes.POINTER(I64), SZ]),
        "hk_launch": (I, [V, V, I64, I64, I64, ctypes.c_uint32, ctypes.c_uint32, V]),
        "hk_launch_grid": (I, [V, V, I64, I64, I64, ctypes.c_uint32, ctypes.c_uint32, V]),
        "hk_ordered_sum_scratch_bytes": (SZ, []),
        "hk_ordered_sum_f64": (I, [V, I64, V, V, V]),
        "hk_ordered_sum_f32": (I, [V, I64, V, V, V]),
        "hk_keyed_ordered_sum_f32": (I, [V, I64, I64, V, V, V]),
        "hk_ordered_scatter_f32": (I, [V, V, I64, V, I64, V, V, V]),
        "hk_ordered_fold_f64": (I, [V, V, V, V]),
        "hk_ordered_sum_noalloc_scratch_bytes": (SZ, []),
        "hk_ordered_sum_f64_noalloc": (I, [V, I64, V, V]),
        "hk_scatter_chunks": (I, [I64, I64]),
        "hk_ordered_scatter_scratch_bytes": (SZ, [I64, I64]),
        "hk_ordered_scatter_f64": (I, [V, V, I64, V, I64, V, V, V]),
        "hk_rows_finish_scratch_bytes": (SZ, [I64]),
        "hk_rows_finish_f64": (I, [V, V, I64, V, V, V]),
        "hk_rows_finish_f32": (I, [V, V, I64, V, V, V]),
        "hk_rows_extreme_f64": (I, [V, I64, ctypes.c_int32, V, V, V]),
        "hk_rows_extreme_f32": (I, [V, I64, ctypes.c_int32, V, V, V]),
        "hk_band_rows_finish_scratch_bytes": (SZ, [I64]),
        "hk_band_rows_finish_f64": (I, [V, V, I64, V, V, V]),
        "hk_band_ordered_sum_scratch_bytes": (SZ, []),
        "hk_band_ordered_sum_f64": (I, [V, I64, V, V, V]),
        "hk_keyed_ordered_sum_scratch_bytes": (SZ, [I64, I64]),
        "hk_keyed_ordered_sum_f64": (I, [V, I64, I64, V, V, V]),
        "hk_mm16_f32": (I, [ctypes.POINTER(V), I, ctypes.POINTER(V), I, ctypes.POINTER(ctypes.c_int32), I64, V]),
        "hk_mm16_f64": (I, [ctypes.POINTER(V), I, ctypes.POINTER(V), I, ctypes.POINTER(ctypes.c_int32), I64, V]),
        "hk_keyed_log_fold_scratch_bytes": (SZ, [I64]),
        "hk_keyed_sample_sum_f64": (I, [V, I64, I64, V, V]),
        "hk_keyed_sample_sum_f32": (I, [V, I64, I64, V, V]),
        "hk_keyed_log_fold_f64": (I, [V, I64, V, I64, I64, ctypes.c_int32, V, I64, V, V, V]),
        "hk_keyed_log_fold_f32": (I, [V, I64, V, I64, I64, ctypes.c_int32, V, I64, V, V, V]),
    }
    for name, (res, args) in sig.items():
        fn = getattr(lib, name)
        fn.restype = res
        fn.argtypes = args


def _self_check(lib) -> None:
    from ._build import source_digest

    stamped = lib.hk_build_digest().decode()
    recomputed = source_digest()
    if stamped != recomputed:
        raise HawkError(
            f"hawk_amd: {_LIB_PATH.name}'s build_digest is {stamped!r} but the sources beside it hash to "
            f"{recomputed!r}: this library was NOT built from these sources. Rebuild it "
            "(python -c 'import __graft_entry__ as g; g.build()' or python hawk_amd/_build.py)")
    sizes = (ctypes.c_uint64 * 5)()
    lib.hk_layout_sizes(sizes)
    for i, (field, expected) in enumerate(_contracts.LAYOUT):
        if sizes[i] != expected:
            raise HawkError(f"hawk_amd: {_LIB_PATH.name}'s layout table disagrees with hawk_amd._contracts "
                            f"in sizeof({field}): the library was built with {sizes[i]} bytes, this source "
                            f"tree declares {expected}")


def lib():
    """The loaded, self-checked library (loaded once per process)."""
    global _lib
    if _lib is not None:
        return _lib
    with _lock:
        if _lib is None:
            # PyTorch-ROCm ships its own HIP runtime (libamdhip64, libhsa-runtime64,
            # libhiprtc) under torch/lib.  Loading it first makes this library's
            # NEEDED sonames bind to that one copy; loading /opt/rocm's beside it
            # would put two HIP runtimes in one process, which faults.  Only the
            # compile worker (hawk_amd._rtc_worker), which never touches a GPU,
            # loads the system copies instead.
            import os
            if os.environ.get("HAWK_NO_TORCH_PRELOAD") != "1":
                import torch  # noqa: F401
            if not _LIB_PATH.exists():
                raise HawkError(f"hawk_amd: {_LIB_PATH} is not built; build it first "
                                "(python hawk_amd/_build.py). The hip target has no fallback path.")
            handle = ctypes.CDLL(str(_LIB_PATH), mode=ctypes.RTLD_LOCAL)
            _declare(handle)
            _self_check(handle)
            _lib = handle
    return _lib


def library_path() -> Path:
    return _LIB_PATH


def check(rc: int, exc=HawkError) -> None:
    if rc != HK_OK:
        text = lib().hk_last_error().decode(errors="replace")
        if rc == 2:
            raise IndexError(text)
        raise exc(text)


def layout_sizes() -> list:
    sizes = (ctypes.c_uint64 * 5)()
    check(lib().hk_layout_sizes(sizes))
    return list(sizes)


def layout_field_name(i: int) -> str:
    return lib().hk_layout_field_name(i).decode()


def build_digest() -> str:
    return lib().hk_build_digest().decode()


def build_info() -> dict:
    text = lib().hk_build_info().decode()
    out = {}
    for line in text.splitlines():
        if "=" in line:
            k, v = line.split("=", 1)
            out[k] = v
    return out


def crossings() -> int:
    return int(lib().hk_crossings())


def rtc_version() -> int:
    return int(lib().hk_rtc_version())


def rtc_compile(source: str, name: str, options: list) -> tuple:
    """hipRTC for gfx950: ``(code bytes, log text)``."""
    L = lib()
    opts = (ctypes.c_char_p * max(1, len(options)))(*[o.encode() for o in options])
    code = ctypes.c_void_p()
    size = ctypes.c_size_t()
    log = ctypes.c_char_p()
    rc = L.hk_rtc_compile(source.encode(), name.encode(), opts, len(options), ctypes.byref(code),
                          ctypes.byref(size), ctypes.byref(log))
    text = log.value.decode(errors="replace") if log.value else ""
    if log.value is not None:
        L.hk_free(ctypes.cast(log, ctypes.c_void_p))
    if rc != HK_OK:
        raise HawkError(L.hk_last_error().decode(errors="replace"))
    blob = ctypes.string_at(code, size.value)
    L.hk_free(code)
    return blob, text


class ArgBlock:
    """The by-value mirror block of one kernel definition (reference
    ``_core.ArgBlock``): one kind per slot in ``arg_spec`` order."""

    def __init__(self, descriptor: list):
        L = lib()
        kinds = (ctypes.c_char_p * max(1, len(descriptor)))(*[k.encode() for k in descriptor])
        handle = ctypes.c_void_p()
        check(L.hk_argblock_new(kinds, len(descriptor), ctypes.byref(handle)), ValueError)
        self._h = handle
        self.descriptor = list(descriptor)
        self._values = []

    @property
    def size(self) -> int:
        return lib().hk_argblock_size(self._h)

    def bind(self, slot: int, ptr: int, samples: int, stride: int = 1, device_type: int = 10,
             device_id: int = 0) -> None:
        check(lib().hk_bind(self._h, int(slot), int(ptr), int(samples), int(stride), int(device_type),
                            int(device_id)), ValueError)

    def bind_value(self, slot: int, value) -> None:
        """Bind a by-value slot from a Python number (copied into the block)."""
        kind = self.descriptor[slot]
        box = {"f64": ctypes.c_double, "f32": ctypes.c_float, "int": ctypes.c_longlong,
               "nsamples": ctypes.c_uint64}.get(kind)
        if box is None:
            raise ValueError(f"slot {slot} is a {kind!r} slot, not a by-value one")
        cell = box(value)
        self.bind(slot, ctypes.addressof(cell), 1)

    def rebind(self, slots, ptrs) -> None:
        n = len(slots)
        if len(ptrs) != n:
            raise ValueError("hawk_core.ArgBlock.rebind: slots and ptrs must be the same length")
        s = (ctypes.c_int64 * max(1, n))(*[int(x) for x in slots])
        p = (ctypes.c_int64 * max(1, n))(*[int(x) for x in ptrs])
        check(lib().hk_rebind(self._h, s, p, n), ValueError)

    @property
    def handle(self):
        return self._h

    def __del__(self):
        h = getattr(self, "_h", None)
        if h is not None and _lib is not None:
            _lib.hk_argblock_free(h)
            self._h = None


class DeviceEntry:
    """One resolved ``__global__`` entry; holds its library."""

    def __init__(self, library: DeviceLibrary, name: str):
        handle = ctypes.c_void_p()
        check(lib().hk_entry_get(library.handle, name.encode(), ctypes.byref(handle)))
        self._h = handle
        self.name = name
        self.library = library

    def run(self, block: ArgBlock, base: int, count: int, n_samples: int, *, threads: int = 256,
            per_thread: int = 1, stream: int = 0) -> None:
        """THE launch crossing: ``[base, base+count)`` of ``n_samples`` on ``stream``."""
        check(lib().hk_launch(self._h, block.handle, int(base), int(count), int(n_samples), int(threads),
                              int(per_thread), ctypes.c_void_p(stream or None)))

    def run_grid(self, block: ArgBlock, base: int, count: int, n_samples: int, grid: int, threads: int,
                 stream: int = 0) -> None:
        check(lib().hk_launch_grid(self._h, block.handle, int(base), int(count), int(n_samples), int(grid),
                                   int(threads), ctypes.c_void_p(stream or None)))


class DeviceLibrary:
    """One loaded gfx950 code object, ABI-checked at load (reference
    ``_core.HostLibrary``)."""

    def __init__(self, code: bytes):
        handle = ctypes.c_void_p()
        buf = ctypes.create_string_buffer(code, len(code))
        check(lib().hk_load(buf, len(code), ctypes.byref(handle)))
        self._h = handle
        self._entries = {}

    @property
    def handle(self):
        return self._h

    def entry(self, name: str) -> DeviceEntry:
        e = self._entries.get(name)
        if e is None:
            e = self._entries[name] = DeviceEntry(self, name)
        return e


def ordered_sum_scratch_bytes() -> int:
    return int(lib().hk_ordered_sum_scratch_bytes())


def ordered_sum(u: int, n: int, out: int, scratch: int, stream: int = 0) -> None:
    check(lib().hk_ordered_sum_f64(ctypes.c_void_p(u or None), int(n), ctypes.c_void_p(out),
                                   ctypes.c_void_p(scratch), ctypes.c_void_p(stream or None)))


def ordered_sum_f32(u: int, n: int, out: int, scratch: int, stream: int = 0) -> None:
    """:func:`ordered_sum` of a float32 plane into a float32 cell."""
    check(lib().hk_ordered_sum_f32(ctypes.c_void_p(u or None), int(n), ctypes.c_void_p(out),
                                   ctypes.c_void_p(scratch), ctypes.c_void_p(stream or None)))


def ordered_sum_noalloc(u: int, n: int, out: int, stream: int = 0) -> None:
    """The ordered sum on the library's static per-GPU scratch: no device
    memory is allocated (for callers that cannot allocate)."""
    check(lib().hk_ordered_sum_f64_noalloc(ctypes.c_void_p(u or None), int(n), ctypes.c_void_p(out),
                                           ctypes.c_void_p(stream or None)))


def scatter_chunks(n: int, cells: int) -> int:
    return int(lib().hk_scatter_chunks(int(n), int(cells)))


def ordered_scatter_scratch_bytes(n: int, cells: int) -> int:
    return int(lib().hk_ordered_scatter_scratch_bytes(int(n), int(cells)))


def ordered_scatter(key: int, v: int, n: int, target: int, cells: int, scratch: int, status: int,
                    stream: int = 0) -> None:
    check(lib().hk_ordered_scatter_f64(ctypes.c_void_p(key or None), ctypes.c_void_p(v or None), int(n),
                                       ctypes.c_void_p(target), int(cells), ctypes.c_void_p(scratch),
                                       ctypes.c_void_p(status), ctypes.c_void_p(stream or None)))


def ordered_scatter_f32(key: int, v: int, n: int, target: int, cells: int, scratch: int, status: int,
                        stream: int = 0) -> None:
    """:func:`ordered_scatter` of float32 values into a float32 target."""
    check(lib().hk_ordered_scatter_f32(ctypes.c_void_p(key or None), ctypes.c_void_p(v or None), int(n),
                                       ctypes.c_void_p(target), int(cells), ctypes.c_void_p(scratch),
                                       ctypes.c_void_p(status), ctypes.c_void_p(stream or None)))


def mm16(ins: list, outs: list, products: list, n: int, stream: int = 0, dtype: str = "f32") -> None:
    """Per-sample 16x16 products on MFMA: ``outs[o] = op(ins[lhs]) @ op(ins[rhs])``
    for ``products[o] = (lhs, rhs, transpose_lhs, transpose_rhs)``; planes by
    pointer, all of ``dtype`` ("f32" or "f64")."""
    if dtype not in ("f32", "f64"):
        raise ValueError(f"mm16: dtype must be 'f32' or 'f64', not {dtype!r}")
    flat = []
    for lhs, rhs, tl, tr in products:
        flat += [int(lhs), int(rhs), (1 if tl else 0) | (2 if tr else 0)]
    c_in = (ctypes.c_void_p * len(ins))(*[ctypes.c_void_p(p) for p in ins])
    c_out = (ctypes.c_void_p * len(outs))(*[ctypes.c_void_p(p) for p in outs])
    c_prod = (ctypes.c_int32 * len(flat))(*flat)
    entry = lib().hk_mm16_f64 if dtype == "f64" else lib().hk_mm16_f32
    check(entry(c_in, len(ins), c_out, len(outs), c_prod, int(n), ctypes.c_void_p(stream or None)))


def mm16_f64(ins: list, outs: list, products: list, n: int, stream: int = 0) -> None:
    """:func:`mm16` on fp64 planes."""
    mm16(ins, outs, products, n, stream, "f64")


def keyed_ordered_sum_scratch_bytes(n: int, group: int) -> int:
    return int(lib().hk_keyed_ordered_sum_scratch_bytes(int(n), int(group)))


def keyed_ordered_sum(u: int, n: int, group: int, out: int, scratch: int, stream: int = 0) -> None:
    """``out[k]`` = key k's ``group`` rows by the ordered sum's tree, k < n / group."""
    check(lib().hk_keyed_ordered_sum_f64(ctypes.c_void_p(u or None), int(n), int(group), ctypes.c_void_p(out),
                                         ctypes.c_void_p(scratch), ctypes.c_void_p(stream or None)))


def keyed_ordered_sum_f32(u: int, n: int, group: int, out: int, scratch: int, stream: int = 0) -> None:
    """:func:`keyed_ordered_sum` of a float32 plane into float32 cells."""
    check(lib().hk_keyed_ordered_sum_f32(ctypes.c_void_p(u or None), int(n), int(group), ctypes.c_void_p(out),
                                         ctypes.c_void_p(scratch), ctypes.c_void_p(stream or None)))


def keyed_sample_sum(u: int, n: int, group: int, out: int, stream: int = 0) -> None:
    """``out[k]`` = key k's ``group`` rows as a default-policy sample sum of their own."""
    check(lib().hk_keyed_sample_sum_f64(ctypes.c_void_p(u or None), int(n), int(group), ctypes.c_void_p(out or None),
                                        ctypes.c_void_p(stream or None)))


def keyed_sample_sum_f32(u: int, n: int, group: int, out: int, stream: int = 0) -> None:
    """keyed_sample_sum of a float32 plane into float32 cells."""
    check(lib().hk_keyed_sample_sum_f32(ctypes.c_void_p(u or None), int(n), int(group), ctypes.c_void_p(out or None),
                                        ctypes.c_void_p(stream or None)))


def keyed_log_fold_scratch_bytes(cells: int) -> int:
    return int(lib().hk_keyed_log_fold_scratch_bytes(int(cells)))


def keyed_log_fold(values: int, stride: int, cells_log: int, keys: int, rows: int, width: int, out: int,
                   cells: int, scratch: int, status: int, stream: int = 0) -> None:
    """``out[cells_log[e*keys + k]]`` = key k's ``rows`` contributions of slot e
    (``values[e*stride + k*rows + r]``) added in lane order from +0; status[0]
    bit 0 = a cell outside ``[0, cells)``, bit 1 = a cell named twice."""
    check(lib().hk_keyed_log_fold_f64(ctypes.c_void_p(values or None), int(stride), ctypes.c_void_p(cells_log or None),
                                      int(keys), int(rows), int(width), ctypes.c_void_p(out or None), int(cells),
                                      ctypes.c_void_p(scratch or None), ctypes.c_void_p(status or None),
                                      ctypes.c_void_p(stream or None)))


def keyed_log_fold_f32(values: int, stride: int, cells_log: int, keys: int, rows: int, width: int, out: int,
                       cells: int, scratch: int, status: int, stream: int = 0) -> None:
    """:func:`keyed_log_fold` of float32 contributions into a float32 gradient plane."""
    check(lib().hk_keyed_log_fold_f32(ctypes.c_void_p(values or None), int(stride), ctypes.c_void_p(cells_log or None),
                                      int(keys), int(rows), int(width), ctypes.c_void_p(out or None), int(cells),
                                      ctypes.c_void_p(scratch or None), ctypes.c_void_p(status or None),
                                      ctypes.c_void_p(stream or None)))


def rows_finish_scratch_bytes(rows: int) -> int:
    return int(lib().hk_rows_finish_scratch_bytes(int(rows)))


def rows_finish(hi: int, comp: int, rows: int, out: int, scratch: int, stream: int = 0) -> None:
    """Fold ``rows`` compensated row pairs into the cell ``out`` (canonical ordered tree)."""
    check(lib().hk_rows_finish_f64(ctypes.c_void_p(hi), ctypes.c_void_p(comp), int(rows), ctypes.c_void_p(out),
                                   ctypes.c_void_p(scratch), ctypes.c_void_p(stream or None)))


def rows_finish_f32(hi: int, comp: int, rows: int, out: int, scratch: int, stream: int = 0) -> None:
    """The same finish of float32 rows, in float32."""
    check(lib().hk_rows_finish_f32(ctypes.c_void_p(hi), ctypes.c_void_p(comp), int(rows), ctypes.c_void_p(out),
                                   ctypes.c_void_p(scratch), ctypes.c_void_p(stream or None)))


def rows_extreme(hi: int, rows: int, op: int, out: int, scratch: int, stream: int = 0) -> None:
    """The finish of ``hawk.max`` (op 1) / ``hawk.min`` (op 2): ``rows``
    row extremes folded in the canonical tree, the extreme stored at ``out``.
    Scratch: :func:`rows_finish_scratch_bytes` bytes."""
    check(lib().hk_rows_extreme_f64(ctypes.c_void_p(hi), int(rows), int(op), ctypes.c_void_p(out),
                                    ctypes.c_void_p(scratch), ctypes.c_void_p(stream or None)))


def rows_extreme_f32(hi: int, rows: int, op: int, out: int, scratch: int, stream: int = 0) -> None:
    """The same finish of float32 rows."""
    check(lib().hk_rows_extreme_f32(ctypes.c_void_p(hi), int(rows), int(op), ctypes.c_void_p(out),
                                    ctypes.c_void_p(scratch), ctypes.c_void_p(stream or None)))


def band_rows_finish_scratch_bytes(rows: int) -> int:
    return int(lib().hk_band_rows_finish_scratch_bytes(int(rows)))


def band_rows_finish(hi: int, lo: int, rows: int, out: int, scratch: int, stream: int = 0) -> None:
    check(lib().hk_band_rows_finish_f64(ctypes.c_void_p(hi), ctypes.c_void_p(lo), int(rows), ctypes.c_void_p(out),
                                        ctypes.c_void_p(scratch), ctypes.c_void_p(stream or None)))


def band_ordered_sum_scratch_bytes() -> int:
    return int(lib().hk_band_ordered_sum_scratch_bytes())


def band_ordered_sum(u: int, n: int, out: int, scratch: int, stream: int = 0) -> None:
    check(lib().hk_band_ordered_sum_f64(ctypes.c_void_p(u or None), int(n), ctypes.c_void_p(out),
                                        ctypes.c_void_p(scratch), ctypes.c_void_p(stream or None)))
