"""The C-ABI library on the CPU: it loads (digest and layout self-check),
exports every symbol include/hawk_core.h declares, and its argument-block and
launch-argument checks refuse by name without touching a GPU."""

from __future__ import annotations

import ctypes
import re
from pathlib import Path

import pytest

from conftest import golden
from hawk_amd import _contracts, _core

HEADER = Path(__file__).resolve().parent.parent / "include" / "hawk_core.h"


def declared_symbols() -> list:
    text = HEADER.read_text()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(hk_[a-z0-9_]+)\s*\(", text)))


def test_every_declared_symbol_is_exported():
    lib = ctypes.CDLL(str(_core.library_path()))
    names = declared_symbols()
    assert len(names) >= 25
    missing = [n for n in names if not hasattr(lib, n)]
    assert not missing, missing


def test_layout_and_digest_self_check():
    assert _core.layout_sizes() == [size for _, size in _contracts.LAYOUT]
    assert [_core.layout_field_name(i) for i in range(5)] == [f for f, _ in _contracts.LAYOUT]
    from hawk_amd._build import source_digest
    assert _core.build_digest() == source_digest()
    info = _core.build_info()
    assert info["abi_tag"] == "aether-abi/2" and info["index_type_bytes"] == "8"
    assert "gfx950" in info["offload_arch"]


def test_crossings_count_every_call():
    a = _core.crossings()
    _core.layout_sizes()
    b = _core.crossings()
    assert b - a == 2          # layout_sizes and the second crossings()


def test_argblock_refuses_an_unknown_kind():
    with pytest.raises(ValueError, match="unknown slot kind 'mirror'"):
        _core.ArgBlock(["gref", "mirror"])


def test_argblock_bind_and_rebind_refusals():
    ab = _core.ArgBlock(["gref", "handle", "f64"])
    assert ab.size == 3
    ab.bind(0, 0x1000, 128)
    ab.bind(1, 0x2000, 128)
    ab.bind_value(2, 2.5)
    with pytest.raises(IndexError, match="slot 3 is outside this block's 3 slots"):
        ab.bind(3, 0x1000, 1)
    with pytest.raises(ValueError, match="by-value 'f64' slot"):
        ab.rebind([2], [0x3000])
    with pytest.raises(ValueError, match="sample stride 2"):
        ab.bind(0, 0x1000, 128, stride=2)
    with pytest.raises(ValueError, match="null pointer"):
        ab.bind(2, 0, 1)
    ab.rebind([0, 1], [0x5000, 0x6000])


@pytest.mark.parametrize("slots", [1, 2, 5, 17])
def test_a_bulk_rebind_is_one_crossing_whatever_the_slot_count(slots):
    """The rebind arm of the reference's launch-crossing card
    (tests/cards/CARD_LAUNCH_CROSSINGS.md): swapping every pointer slot costs
    ONE crossing, not one per slot; binding them one by one costs one each."""
    ab = _core.ArgBlock(["handle"] * slots)
    for s in range(slots):
        ab.bind(s, 0x1000 * (s + 1), 64)
    before = _core.crossings()
    ab.rebind(list(range(slots)), [0x9000 + 0x100 * s for s in range(slots)])
    assert _core.crossings() - before - 1 == 1          # the closing crossings() is its own crossing
    before = _core.crossings()
    for s in range(slots):
        ab.bind(s, 0x7000 + s, 64)
    assert _core.crossings() - before - 1 == slots


def test_rtc_refuses_another_architecture():
    from hawk_amd import HawkError
    with pytest.raises(HawkError, match="pinned to gfx950"):
        _core.rtc_compile('extern "C" __global__ void k() {}', "k.hip", ["--offload-arch=gfx942"])


def test_rtc_compiles_for_gfx950_without_a_gpu():
    code, _log = _core.rtc_compile('extern "C" __global__ void k(double* p) { p[threadIdx.x] = 1.0; }',
                                   "k.hip", ["-O3"])
    assert code[:4] in (b"\x7fELF", b"__CL")     # an ELF code object or a clang offload bundle


def test_rtc_reports_a_compile_error():
    from hawk_amd import HawkError
    with pytest.raises(HawkError, match="could not compile"):
        _core.rtc_compile('extern "C" __global__ void k() { undeclared(); }', "bad.hip", [])


def test_team_stage_arguments_are_checked_before_any_launch():
    L = _core.lib()
    rc = L.hk_ordered_sum_f64(None, -1, None, None, None)
    assert rc != 0 and b"n must be >= 0" in L.hk_last_error()
    rc = L.hk_ordered_scatter_f64(None, None, 10, None, 5, None, None, None)
    assert rc != 0 and b"required" in L.hk_last_error()
    assert L.hk_ordered_scatter_f64(None, None, 10, None, 0, None, None, None) == 0   # no cells: nothing
    # the keyed sum: whole groups only; no keys is nothing; scratch sizes by shape
    rc = L.hk_keyed_ordered_sum_f64(None, 10, 3, None, None, None)
    assert rc != 0 and b"whole number of groups" in L.hk_last_error()
    rc = L.hk_keyed_ordered_sum_f64(None, 10, 0, None, None, None)
    assert rc != 0 and b"group >= 1" in L.hk_last_error()
    assert L.hk_keyed_ordered_sum_f64(None, 0, 4, None, None, None) == 0
    assert L.hk_keyed_ordered_sum_scratch_bytes(12, 4) == 256                 # keys read their rows directly
    assert L.hk_keyed_ordered_sum_scratch_bytes(8, 8) == L.hk_ordered_sum_scratch_bytes()   # one key
    assert L.hk_keyed_ordered_sum_scratch_bytes(2 * 70001, 70001) == 8 * 2 * 65536 + 256
    # the ordered gradient's fold: shapes and pointers are checked before HIP
    rc = L.hk_keyed_log_fold_f64(None, 10, None, 2, 0, 1, None, 4, None, None, None)
    assert rc != 0 and b"rows and width >= 1" in L.hk_last_error()
    rc = L.hk_keyed_log_fold_f64(None, 10, None, 2, 5, 0, None, 4, None, None, None)
    assert rc != 0 and b"rows and width >= 1" in L.hk_last_error()
    rc = L.hk_keyed_log_fold_f64(None, 9, None, 2, 5, 1, None, 4, None, None, None)
    assert rc != 0 and b"shorter than keys * rows" in L.hk_last_error()
    rc = L.hk_keyed_log_fold_f64(None, 10, None, 2, 5, 1, None, 4, None, None, None)
    assert rc != 0 and b"status is required" in L.hk_last_error()
    status = (ctypes.c_int32 * 2)()
    rc = L.hk_keyed_log_fold_f64(None, 10, None, 2, 5, 1, None, 4, None, status, None)
    assert rc != 0 and b"required" in L.hk_last_error()
    assert L.hk_keyed_log_fold_scratch_bytes(1000) == 4000 and L.hk_keyed_log_fold_scratch_bytes(0) == 0
    # the default-policy keyed sum: whole groups, keys of at most 2^25 samples
    rc = L.hk_keyed_sample_sum_f64(None, 10, 3, None, None)
    assert rc != 0 and b"whole number of groups" in L.hk_last_error()
    rc = L.hk_keyed_sample_sum_f64(None, (1 << 25) + 32, (1 << 25) + 32, None, None)
    assert rc != 0 and b"policy='ordered'" in L.hk_last_error()
    assert L.hk_keyed_sample_sum_f64(None, 0, 4, None, None) == 0
    # the per-sample products: plane counts and indices are checked first
    rc = L.hk_mm16_f32(None, 0, None, 1, None, 1, None)
    assert rc != 0 and b"1..3 input planes" in L.hk_last_error()
    rc = L.hk_mm16_f64(None, 2, None, 1, None, 1, None)
    assert rc != 0 and b"hk_mm16_f64: in, out and products are required" in L.hk_last_error()
    ins = (ctypes.c_void_p * 2)(1, 2)
    outs = (ctypes.c_void_p * 1)(3)
    prods = (ctypes.c_int32 * 3)(0, 2, 0)
    rc = L.hk_mm16_f64(ins, 2, outs, 1, prods, 1, None)
    assert rc != 0 and b"outside [0, n_in)" in L.hk_last_error()
    prods = (ctypes.c_int32 * 3)(0, 1, 0)
    assert L.hk_mm16_f64(ins, 2, outs, 1, prods, 0, None) == 0     # no samples: nothing launched


def test_scatter_chunk_rule():
    """clamp(n // max(cells, 1), 1, 256), the reference's own vectors."""
    ga = golden("scatter_chunks")
    assert [_core.scatter_chunks(n, t) for n, t in ga["cases"]] == ga["chunks"]


def test_launch_arguments_are_checked_before_hip():
    ab = _core.ArgBlock(["handle"])
    L = _core.lib()
    fake = ctypes.c_void_p(1)       # never dereferenced: the checks refuse first
    rc = L.hk_launch(fake, ab.handle, 0, 10, 5, 256, 1, None)
    assert rc != 0 and b"not inside" in L.hk_last_error()
    rc = L.hk_launch(fake, ab.handle, 0, 10, 10, 100, 1, None)
    assert rc != 0 and b"multiple of 64" in L.hk_last_error()
    assert L.hk_launch(fake, ab.handle, 0, 0, 10, 256, 1, None) == 0     # empty range: nothing launched
