"""ctypes face of the CPU oracle (oracle/hawk_oracle.c) — TEST INFRASTRUCTURE.

Only tests/, the smoke check of __graft_entry__.py and bench.py's CPU
baseline use this module, and only as the checker or the baseline: the
product (hawk_amd/) never imports it.  The library is built by
``make -C oracle`` (portable profile) when it is missing.
"""

from __future__ import annotations

import ctypes
import subprocess
from pathlib import Path

import numpy as np

ROOT = Path(__file__).resolve().parent.parent
ORACLE = ROOT / "oracle"

_P = ctypes.c_void_p
_I64 = ctypes.c_int64
_D = ctypes.c_double
_libs: dict = {}


def build(profile: str = "portable") -> Path:
    out = ORACLE / {"portable": "libhawk_oracle.so", "native": "_native/libhawk_oracle.so",
                    "fast": "_fast/libhawk_oracle.so"}[profile]
    src = ORACLE / "hawk_oracle.c"
    if not out.exists() or out.stat().st_mtime < src.stat().st_mtime:
        subprocess.run(["make", "-s", "-C", str(ORACLE), f"PROFILE={profile}"], check=True)
    return out


_default_profile = ["portable"]


def use_profile(profile: str) -> None:
    """Make ``profile`` ("portable", "native" or "fast") the build the
    wrappers below call by default (the CPU baseline times "native")."""
    build(profile)
    _default_profile[0] = profile


def lib(profile: str | None = None):
    profile = profile or _default_profile[0]
    if profile in _libs:
        return _libs[profile]
    L = ctypes.CDLL(str(build(profile)))
    sigs = {
        "hko_scale": (None, [_P, _D, _D, _P, _I64, _I64]),
        "hko_energy": (None, [_P, _I64, _P, _I64, _I64]),
        "hko_energy_vjp": (None, [_P, _P, _I64, _P, _I64, _I64]),
        "hko_energy_jvp": (None, [_P, _P, _I64, _P, _I64, _I64]),
        "hko_chain": (None, [_P, _P, _I64, _I64]),
        "hko_chain_vjp": (None, [_P, _P, _P, _D, _P, _I64, _I64, _P]),
        "hko_chain_jvp": (None, [_P, _P, _I64, _P]),
        "hko_libm": (None, [ctypes.c_int, _P, _P, _I64]),
        "hko_ordered_sum": (_D, [_P, _I64]),
        "hko_ordered_sum_f32": (ctypes.c_float, [_P, _I64]),
        "hko_keyed_ordered_sum_f32": (None, [_P, _I64, _I64, _P]),
        "hko_ordered_scatter_f32": (None, [_P, _P, _I64, _P, _I64, _P, _P]),
        "hko_keyed_ordered_sum": (None, [_P, _I64, _I64, _P]),
        "hko_keyed_ordered_sum_threads": (None, [_P, _I64, _I64, _P, ctypes.c_int]),
        "hko_keyed_log_fold": (ctypes.c_int, [_P, _I64, _P, _I64, _I64, ctypes.c_int32, _P, _I64]),
        "hko_keyed_log_fold_f32": (ctypes.c_int, [_P, _I64, _P, _I64, _I64, ctypes.c_int32, _P, _I64]),
        "hko_keyed_sample_sum": (None, [_P, _I64, _I64, _P]),
        "hko_net_threads": (None, [ctypes.c_int, _P, _P, _P, _P, _P, _I64, _I64, _P, ctypes.c_int]),
        "hko_chain_members_threads": (None, [_P, _P, _P, _I64, ctypes.c_int]),
        "hko_osc_launch": (_I64, [_I64, _I64, ctypes.c_int, _D, _P, _P, _P, _P, _P, _P]),
        "hko_row_sums": (None, [_P, _I64, _P, _P]),
        "hko_rows_finish": (_D, [_P, _P, _I64]),
        "hko_sample_sum": (_D, [_P, _I64]),
        "hko_row_sums_f32": (None, [_P, _I64, _P, _P]),
        "hko_rows_finish_f32": (ctypes.c_float, [_P, _P, _I64]),
        "hko_sample_sum_f32": (ctypes.c_float, [_P, _I64]),
        "hko_band_row_sums": (None, [_P, _I64, _P, _P]),
        "hko_band_rows_finish": (_D, [_P, _P, _I64]),
        "hko_row_extremes": (None, [_P, _I64, ctypes.c_int, _P]),
        "hko_rows_extreme": (_D, [_P, _I64, ctypes.c_int]),
        "hko_sample_extreme": (_D, [_P, _I64, ctypes.c_int]),
        "hko_row_extremes_f32": (None, [_P, _I64, ctypes.c_int, _P]),
        "hko_rows_extreme_f32": (ctypes.c_float, [_P, _I64, ctypes.c_int]),
        "hko_sample_extreme_f32": (ctypes.c_float, [_P, _I64, ctypes.c_int]),
        "hko_band_sample_sum": (_D, [_P, _I64]),
        "hko_band_ordered_sum": (_D, [_P, _I64]),
        "hko_scatter_chunks": (ctypes.c_int, [_I64, _I64]),
        "hko_ordered_scatter": (None, [_P, _P, _I64, _P, _I64, _P, _P]),
        "hko_twobody": (None, [_P, _P, _D, _I64, _P, _P, _I64, _I64]),
        "hko_twobody_vjp": (None, [_P, _P, _D, _P, _P, _I64, _P, _P, _I64, _I64]),
        "hko_twobody_x": (None, [_P, _P, _D, _I64, _P, _P, _I64, _I64]),
        "hko_twobody_vjp_x": (None, [_P, _P, _D, _P, _P, _I64, _P, _P, _I64, _I64]),
        "hko_spd_solve": (None, [_P, _P, _I64, _P, _I64, _I64]),
        "hko_spd_solve_vjp": (None, [_P, _P, _P, _I64, _P, _P, _I64, _I64]),
        "hko_mm16": (None, [_P, _P, _I64, _P, _I64, _I64]),
        "hko_mm16_vjp": (None, [_P, _P, _P, _I64, _P, _P, _I64, _I64]),
        "hko_mm16_f64": (None, [_P, _P, _I64, _P, _I64, _I64]),
        "hko_mm16_vjp_f64": (None, [_P, _P, _P, _I64, _P, _P, _I64, _I64]),
        "hko_tiled": (None, [ctypes.c_int, _P, _P, _P, _P, _P, _P, _D, _D, _I64, ctypes.c_int]),
        "hko_ordered_sum_threads": (_D, [_P, _I64, ctypes.c_int]),
        "hko_ordered_scatter_threads": (None, [_P, _P, _I64, _P, _I64, _P, _P, ctypes.c_int]),
    }
    for name, (res, args) in sigs.items():
        fn = getattr(L, name)
        fn.restype, fn.argtypes = res, args
    _libs[profile] = L
    return L


def _p(a: np.ndarray):
    assert a.flags.c_contiguous
    return a.ctypes.data_as(_P)


# -- convenience wrappers (whole range) -----------------------------------------

def scale(x, a, b):
    out = np.empty_like(x)
    lib().hko_scale(_p(x), a, b, _p(out), 0, x.size)
    return out


def energy(v):
    n = v.shape[1]
    out = np.empty(n)
    lib().hko_energy(_p(v), n, _p(out), 0, n)
    return out


def energy_vjp(v, bar_out):
    n = v.shape[1]
    out = np.empty_like(v)
    lib().hko_energy_vjp(_p(v), _p(bar_out), n, _p(out), 0, n)
    return out


def energy_jvp(v, dv):
    n = v.shape[1]
    out = np.empty(n)
    lib().hko_energy_jvp(_p(v), _p(dv), n, _p(out), 0, n)
    return out


def chain(x, threads: int = 1):
    y = np.empty_like(x)
    if threads > 1:
        lib().hko_tiled(5, _p(x), None, None, None, _p(y), None, 0.0, 0.0, x.size, threads)
    else:
        lib().hko_chain(_p(x), _p(y), 0, x.size)
    return y


def chain_vjp(x, key, bar_y, bar_total, bar_bins):
    """bar_x of the chain through its three sinks (hand-derived dy/dx)."""
    x, bar_y, bar_bins = (np.ascontiguousarray(a, dtype=np.float64) for a in (x, bar_y, bar_bins))
    key = np.ascontiguousarray(key, dtype=np.int32)
    out = np.empty_like(x)
    lib().hko_chain_vjp(_p(x), _p(key), _p(bar_y), float(bar_total), _p(bar_bins), bar_bins.size, x.size, _p(out))
    return out


def chain_jvp(x, dot_x):
    x, dot_x = (np.ascontiguousarray(a, dtype=np.float64) for a in (x, dot_x))
    out = np.empty_like(x)
    lib().hko_chain_jvp(_p(x), _p(dot_x), x.size, _p(out))
    return out


def chain_dx_scale(x):
    """|d7 x| + |t7| + |d4|: the magnitudes of the three terms dy/dx of the
    chain adds (numpy), the scale a rounding error of dy/dx is measured on
    where the terms cancel."""
    t1 = np.exp(x)
    t2 = np.sin(t1)
    d3 = 1.5 * np.cos(t1) * t1
    t4 = np.tanh(1.5 * t2 + 0.25)
    d4 = (1.0 - t4 * t4) * d3
    t5 = np.sqrt(np.abs(t4) + 1.0)
    d6 = 2.0 * t5 * (0.5 / t5) * np.abs(d4) + 1.0
    t7 = np.exp(-np.abs(t5 * t5 - x))
    return np.abs(t7 * d6 * x) + t7 + np.abs(d4)


def libm(which: str, x):
    y = np.empty_like(x)
    code = {"exp": 0, "sin": 1, "tanh": 2, "sqrt": 3, "cos": 4, "log": 5}[which]
    lib().hko_libm(code, _p(x), _p(y), x.size)
    return y


def ordered_sum(u, threads: int = 1) -> float:
    if u.dtype == np.float32:                     # the float32 mode: every addition in float
        return np.float32(lib().hko_ordered_sum_f32(_p(u), u.size))
    if threads > 1:
        return lib().hko_ordered_sum_threads(_p(u), u.size, threads)
    return lib().hko_ordered_sum(_p(u), u.size)


def keyed_ordered_sum(u, group: int, threads: int = 1, profile: str = "portable"):
    """One ordered-sum cell per run of ``group`` consecutive values (float32
    cells, float32 additions, for a float32 ``u``)."""
    if getattr(u, "dtype", None) == np.float32:
        u = np.ascontiguousarray(u)
        assert u.size % group == 0
        out = np.empty(u.size // group, dtype=np.float32)
        lib(profile).hko_keyed_ordered_sum_f32(_p(u), u.size, group, _p(out))
        return out
    u = np.ascontiguousarray(u, dtype=np.float64)
    assert u.size % group == 0
    out = np.empty(u.size // group)
    if threads > 1:
        lib(profile).hko_keyed_ordered_sum_threads(_p(u), u.size, group, _p(out), threads)
    else:
        lib(profile).hko_keyed_ordered_sum(_p(u), u.size, group, _p(out))
    return out


def keyed_sample_sum(u, group: int):
    """One default-policy sample sum per run of ``group`` consecutive values
    (each a float32 sample sum, in float32, for a float32 ``u``)."""
    if getattr(u, "dtype", None) == np.float32:
        u = np.ascontiguousarray(u)
        assert u.size % group == 0
        return np.array([sample_sum_f32(u[k * group:(k + 1) * group]) for k in range(u.size // group)], np.float32)
    u = np.ascontiguousarray(u, dtype=np.float64)
    assert u.size % group == 0
    out = np.empty(u.size // group)
    lib().hko_keyed_sample_sum(_p(u), u.size, group, _p(out))
    return out


def keyed_log_fold(values, cells_log, rows: int, out):
    """The ordered gradient's fold into ``out`` (in place): ``values`` is
    ``[width, keys * rows]``, ``cells_log`` ``[width, keys]``; returns 1 when a
    cell was outside ``out``.  Float32 ``values`` and ``out`` fold in float32."""
    if getattr(values, "dtype", None) == np.float32:
        values = np.ascontiguousarray(values)
        cells_log = np.ascontiguousarray(cells_log, dtype=np.int32)
        width, keys = cells_log.shape
        assert values.shape == (width, keys * rows) and out.dtype == np.float32 and out.flags.c_contiguous
        return lib().hko_keyed_log_fold_f32(_p(values), keys * rows, _p(cells_log), keys, rows, width, _p(out),
                                            out.size)
    values = np.ascontiguousarray(values, dtype=np.float64)
    cells_log = np.ascontiguousarray(cells_log, dtype=np.int32)
    width, keys = cells_log.shape
    assert values.shape == (width, keys * rows) and out.dtype == np.float64 and out.flags.c_contiguous
    return lib().hko_keyed_log_fold(_p(values), keys * rows, _p(cells_log), keys, rows, width, _p(out), out.size)


def chain_members(x, acc, threads: int = 1, profile: str = "portable"):
    """The chain of the four example members over ``x``: ``acc`` updated in
    place, ``y`` [3, n] returned."""
    x = np.ascontiguousarray(x, dtype=np.float64)
    assert acc.dtype == np.float64 and acc.flags.c_contiguous and acc.size == x.size
    y = np.empty((3, x.size))
    lib(profile).hko_chain_members_threads(_p(x), _p(acc), _p(y), x.size, threads)
    return y


def osc_launch(K, dt, t_final, x, v, t, mask, base: int = 0, count=None, profile: str = "portable",
               trips=None) -> int:
    """One launch of the oscillator that finishes its own sample, ``K`` steps
    at most: ``x``, ``v``, ``t`` (float64) and ``mask`` (bool) updated in
    place over ``[base, base+count)``; returns how many samples it finished.
    ``trips`` (int32, optional) gets each sample's steps this launch."""
    for a in (t_final, x, v, t):
        assert a.dtype == np.float64 and a.flags.c_contiguous
    assert mask.dtype == np.bool_ and mask.flags.c_contiguous
    if trips is not None:
        assert trips.dtype == np.int32 and trips.flags.c_contiguous and trips.size == x.size
    count = x.size - base if count is None else count
    return int(lib(profile).hko_osc_launch(base, count, K, dt, _p(t_final), _p(x), _p(v), _p(t),
                                           mask.ctypes.data_as(_P), None if trips is None else _p(trips)))


def net_loss(w, mask, x, y, threads: int = 1, profile: str = "portable"):
    """Each net's loss: the ordered sum of its samples' squared residuals
    (``w[k, 24]``, ``mask[k, 8]``, ``x`` and ``y`` ``[k, s]``)."""
    w, mask, x, y = (np.ascontiguousarray(a, dtype=np.float64) for a in (w, mask, x, y))
    k, s = x.shape
    out = np.empty(k)
    lib(profile).hko_net_threads(16, _p(w), _p(mask), _p(x), _p(y), None, k, s, _p(out), threads)
    return out


def net_grad(w, mask, x, y, bar_out, threads: int = 1, profile: str = "portable"):
    """Each net's gradient wrt its weights, ``[k, 24]``: the samples'
    contributions added in lane order from +0."""
    w, mask, x, y, bar_out = (np.ascontiguousarray(a, dtype=np.float64) for a in (w, mask, x, y, bar_out))
    k, s = x.shape
    out = np.empty((k, 24))
    lib(profile).hko_net_threads(17, _p(w), _p(mask), _p(x), _p(y), _p(bar_out), k, s, _p(out), threads)
    return out


def row_sums(t):
    """The compensated (hi, comp) pair of every row of 32 terms."""
    t = np.ascontiguousarray(t, dtype=np.float64)
    rows = -(-t.size // 32)
    hi, comp = np.empty(rows), np.empty(rows)
    lib().hko_row_sums(_p(t), t.size, _p(hi), _p(comp))
    return hi, comp


def rows_finish(hi, comp) -> float:
    hi = np.ascontiguousarray(hi, dtype=np.float64)
    comp = np.ascontiguousarray(comp, dtype=np.float64)
    return lib().hko_rows_finish(_p(hi), _p(comp), hi.size)


def sample_sum(t) -> float:
    """The default-policy hawk.sum of the terms t (rows, then the canonical finish)."""
    t = np.ascontiguousarray(t, dtype=np.float64)
    return lib().hko_sample_sum(_p(t), t.size)


def row_sums_f32(t):
    """The float32 mode's rows: the compensated (hi, comp) of every 32 terms, in float32."""
    t = np.ascontiguousarray(t, dtype=np.float32)
    rows = -(-t.size // 32)
    hi, comp = np.empty(rows, dtype=np.float32), np.empty(rows, dtype=np.float32)
    lib().hko_row_sums_f32(_p(t), t.size, _p(hi), _p(comp))
    return hi, comp


def rows_finish_f32(hi, comp) -> np.float32:
    hi = np.ascontiguousarray(hi, dtype=np.float32)
    comp = np.ascontiguousarray(comp, dtype=np.float32)
    return np.float32(lib().hko_rows_finish_f32(_p(hi), _p(comp), hi.size))


def sample_sum_f32(t) -> np.float32:
    """The float32 mode's default-policy hawk.sum of the terms t (rows, then the canonical finish, in float32)."""
    t = np.ascontiguousarray(t, dtype=np.float32)
    return np.float32(lib().hko_sample_sum_f32(_p(t), t.size))


_EXTREME_OP = {"max": 1, "min": 2}


def row_extremes(t, op: str):
    """One value a row of 32 terms: the NaN-ignoring extreme ("max" or
    "min"), -inf / +inf past the last term; float32 terms give float32 rows."""
    f32 = np.asarray(t).dtype == np.float32
    t = np.ascontiguousarray(t, dtype=np.float32 if f32 else np.float64)
    hi = np.empty(-(-t.size // 32), dtype=t.dtype)
    (lib().hko_row_extremes_f32 if f32 else lib().hko_row_extremes)(_p(t), t.size, _EXTREME_OP[op], _p(hi))
    return hi


def rows_extreme(hi, op: str):
    """The canonical finish of row extremes (in the rows' dtype)."""
    f32 = np.asarray(hi).dtype == np.float32
    hi = np.ascontiguousarray(hi, dtype=np.float32 if f32 else np.float64)
    if f32:
        return np.float32(lib().hko_rows_extreme_f32(_p(hi), hi.size, _EXTREME_OP[op]))
    return lib().hko_rows_extreme(_p(hi), hi.size, _EXTREME_OP[op])


def sample_extreme(t, op: str):
    """hawk.max / hawk.min of the terms t: row extremes, then the canonical
    finish, in t's dtype (float32 terms: the float32 mode)."""
    f32 = np.asarray(t).dtype == np.float32
    t = np.ascontiguousarray(t, dtype=np.float32 if f32 else np.float64)
    if f32:
        return np.float32(lib().hko_sample_extreme_f32(_p(t), t.size, _EXTREME_OP[op]))
    return lib().hko_sample_extreme(_p(t), t.size, _EXTREME_OP[op])


def band_row_sums(t):
    """The banded rows: each row of 32 terms as a normalised double-double band (hi, lo)."""
    t = np.ascontiguousarray(t, dtype=np.float64)
    rows = -(-t.size // 32)
    hi, lo = np.empty(rows), np.empty(rows)
    lib().hko_band_row_sums(_p(t), t.size, _p(hi), _p(lo))
    return hi, lo


def band_rows_finish(hi, lo) -> float:
    hi = np.ascontiguousarray(hi, dtype=np.float64)
    lo = np.ascontiguousarray(lo, dtype=np.float64)
    return lib().hko_band_rows_finish(_p(hi), _p(lo), hi.size)


def band_sample_sum(t) -> float:
    """hawk.sum of the terms t in the banded mode (band rows, the canonical finish with band adds)."""
    t = np.ascontiguousarray(t, dtype=np.float64)
    return lib().hko_band_sample_sum(_p(t), t.size)


def band_ordered_sum(u) -> float:
    """hawk.sum(policy="ordered") in the banded mode: the fixed tree with band accumulators."""
    u = np.ascontiguousarray(u, dtype=np.float64)
    return lib().hko_band_ordered_sum(_p(u), u.size)


def scatter_chunks(n, cells) -> int:
    return lib().hko_scatter_chunks(n, cells)


def ordered_scatter(key, v, target, threads: int = 1):
    """``target`` after the ordered scatter (a copy), and the status plane."""
    out = target.copy()
    cells = out.size
    chunks = scatter_chunks(key.size, cells)
    status = np.zeros(257, dtype=np.int32)
    if out.dtype == np.float32:                   # the float32 mode: parts, cells and target in float
        assert v.dtype == np.float32
        parts = np.empty(chunks * max(cells, 1), dtype=np.float32)
        lib().hko_ordered_scatter_f32(_p(key), _p(v), key.size, _p(out), cells, _p(parts), _p(status))
        return out, status
    parts = np.empty(chunks * max(cells, 1))
    if threads > 1:
        lib().hko_ordered_scatter_threads(_p(key), _p(v), key.size, _p(out), cells, _p(parts), _p(status), threads)
    else:
        lib().hko_ordered_scatter(_p(key), _p(v), key.size, _p(out), cells, _p(parts), _p(status))
    return out, status


def twobody(r0, v0, mu, threads: int = 1):
    n = r0.shape[1]
    r, v = np.empty_like(r0), np.empty_like(v0)
    if threads > 1:
        lib().hko_tiled(9, _p(r0), _p(v0), None, None, _p(r), _p(v), mu, 0.0, n, threads)
    else:
        lib().hko_twobody(_p(r0), _p(v0), mu, n, _p(r), _p(v), 0, n)
    return r, v


def twobody_vjp(r0, v0, mu, bar_r, bar_v, threads: int = 1):
    n = r0.shape[1]
    br0, bv0 = np.empty_like(r0), np.empty_like(v0)
    if threads > 1:
        lib().hko_tiled(10, _p(r0), _p(v0), _p(bar_r), _p(bar_v), _p(br0), _p(bv0), mu, 0.0, n, threads)
    else:
        lib().hko_twobody_vjp(_p(r0), _p(v0), mu, _p(bar_r), _p(bar_v), n, _p(br0), _p(bv0), 0, n)
    return br0, bv0


def spd_solve(A, b, threads: int = 1):
    n = b.shape[1]
    x = np.empty_like(b)
    if threads > 1:
        lib().hko_tiled(11, _p(A), _p(b), None, None, _p(x), None, 0.0, 0.0, n, threads)
    else:
        lib().hko_spd_solve(_p(A), _p(b), n, _p(x), 0, n)
    return x


def spd_solve_vjp(A, b, bar_x, threads: int = 1):
    n = b.shape[1]
    bA, bb = np.empty_like(A), np.empty_like(b)
    if threads > 1:
        lib().hko_tiled(12, _p(A), _p(b), _p(bar_x), None, _p(bA), _p(bb), 0.0, 0.0, n, threads)
    else:
        lib().hko_spd_solve_vjp(_p(A), _p(b), _p(bar_x), n, _p(bA), _p(bb), 0, n)
    return bA, bb


def mm16(A, B, threads: int = 1):
    n = A.shape[-1]
    C = np.empty_like(A)
    if A.dtype == np.float64:
        assert B.dtype == np.float64
        if threads > 1:
            lib().hko_tiled(21, _p(A), _p(B), None, None, _p(C), None, 0.0, 0.0, n, threads)
        else:
            lib().hko_mm16_f64(_p(A), _p(B), n, _p(C), 0, n)
        return C
    if threads > 1:
        lib().hko_tiled(13, _p(A), _p(B), None, None, _p(C), None, 0.0, 0.0, n, threads)
    else:
        lib().hko_mm16(_p(A), _p(B), n, _p(C), 0, n)
    return C


def mm16_vjp(A, B, bar_C, threads: int = 1):
    n = A.shape[-1]
    bA, bB = np.empty_like(A), np.empty_like(B)
    if A.dtype == np.float64:
        assert B.dtype == bar_C.dtype == np.float64
        if threads > 1:
            lib().hko_tiled(22, _p(A), _p(B), _p(bar_C), None, _p(bA), _p(bB), 0.0, 0.0, n, threads)
        else:
            lib().hko_mm16_vjp_f64(_p(A), _p(B), _p(bar_C), n, _p(bA), _p(bB), 0, n)
        return bA, bB
    if threads > 1:
        lib().hko_tiled(14, _p(A), _p(B), _p(bar_C), None, _p(bA), _p(bB), 0.0, 0.0, n, threads)
    else:
        lib().hko_mm16_vjp(_p(A), _p(B), _p(bar_C), n, _p(bA), _p(bB), 0, n)
    return bA, bB
