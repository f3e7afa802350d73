"""The targets table and its writer/wrapper seam (reference
hawk/targets/__init__.py:37-71, hawk/emit/writer.py:29-38,
hawk/emit/wrapper.py:225-284): the hip row answers every member of both
seams, the renderer and the build read the row rather than a target's name
(a row with another writer or wrapper changes the text it emits), and what
the row has no form for is refused by name."""

from __future__ import annotations

import dataclasses
import json

import pytest

import hawk_amd as hawk
from hawk_amd import examples as E
from hawk_amd.emit_hip import plan_kernel
from hawk_amd.hip_target import WRAPPER_MEMBERS, WRITER_MEMBERS, HipWrapper, HipWriter
from hawk_amd.ir import HawkError
from hawk_amd.targets import DEFAULT_TARGETS, ENTRY_DEVICE, GPU, TARGETS, conforms, row


def test_the_hip_row_answers_every_seam_member():
    hip = TARGETS["hip"]
    assert conforms(hip) == []
    assert (hip.compile, hip.entry, hip.offload_arch, hip.artifact, hip.source) == \
        (GPU, ENTRY_DEVICE, "gfx950", ".hsaco", ".hip")
    assert DEFAULT_TARGETS == ("hip",)
    assert len(WRITER_MEMBERS) == len(set(WRITER_MEMBERS)) == 33
    assert len(WRAPPER_MEMBERS) == 8


def test_conformance_names_a_missing_member():
    class Short(HipWriter):
        op = None
    bad = dataclasses.replace(TARGETS["hip"], writer=Short())
    assert conforms(bad) == ["writer.op"]


def test_the_renderer_spells_through_the_rows_writer():
    """A writer that spells fp64 exp its own way changes exactly the call
    sites (and, with no hk_ call left, the helper block drops out)."""
    from hawk_amd.emit_hip import _MATH_HELPERS, MATH_DEVICE_DEFINES

    class Renamed(HipWriter):
        def op(self, r, node, args, ranks=()):
            text = super().op(r, node, args, ranks)
            return text.replace("hk_exp(", "my_exp(", 1) if text.startswith("hk_exp(") else text
    base = plan_kernel(E.decay.program, "decay").source
    other = plan_kernel(E.decay.program, "decay",
                        target=dataclasses.replace(TARGETS["hip"], writer=Renamed())).source
    helpers = "\n".join(MATH_DEVICE_DEFINES + _MATH_HELPERS.splitlines()) + "\n"
    assert helpers in base and "= hk_exp(" in base
    assert "my_exp(" in other and "my_exp(" not in base and "HK_MATH_QUAL" not in other
    assert other.replace("my_exp(", "hk_exp(") == base.replace(helpers, "")


def test_the_renderer_wraps_through_the_rows_wrapper():
    class Ordered(HipWrapper):
        def entry_signature(self, walk, name):
            return super().entry_signature(dataclasses.replace(walk, xcd_order=True), name)
    base = plan_kernel(E.twobody.program, "twobody").source
    other = plan_kernel(E.twobody.program, "twobody",
                        target=dataclasses.replace(TARGETS["hip"], wrapper=Ordered())).source
    assert "constexpr bool hk_xcd_order = false;" in base
    assert other == base.replace("constexpr bool hk_xcd_order = false;", "constexpr bool hk_xcd_order = true;")


#: The reference's wrapper seam (hawk/emit/wrapper.py:225-284): each member's
#: parameters as (name, kind, default), ``self`` left out.
_P, _K, _V = "POSITIONAL_OR_KEYWORD", "KEYWORD_ONLY", "VAR_KEYWORD"
_NONE = object()
REFERENCE_WRAPPER = {
    "entry_signature": [("walk", _P, _NONE), ("name", _P, _NONE)],
    "index_prologue": [("segment", _P, None), ("active", _K, None), ("box", _K, None)],
    "index_epilogue": [],
    "unpack": [("walk", _P, _NONE)],
    "fold_rows": [("width", _P, _NONE)],
    "sample_sum_frame": [("width", _P, _NONE), ("elem", _P, _NONE), ("store", _P, _NONE), ("op", _P, "sum"),
                         ("live", _P, None)],
    "dispatch": [("kind_spelling", _P, _NONE), ("branch_spellings", _P, _NONE), ("policy", _P, _NONE),
                 ("kw", _V, _NONE)],
}


@pytest.mark.parametrize("member", sorted(REFERENCE_WRAPPER))
def test_the_wrapper_members_take_the_reference_parameters(member):
    """Each member accepts the reference's parameters, in its order and
    kinds, with its defaults; extra parameters only after them, keyword-only
    with a default (the hip prologue's ``form``), so a reference call binds."""
    import inspect
    params = list(inspect.signature(getattr(TARGETS["hip"].wrapper, member)).parameters.values())
    want = REFERENCE_WRAPPER[member]
    got = [(q.name, q.kind.name, _NONE if q.default is inspect.Parameter.empty else q.default)
           for q in params[:len(want)]]
    assert got == want
    for extra in params[len(want):]:
        assert extra.kind is inspect.Parameter.KEYWORD_ONLY and extra.default is not inspect.Parameter.empty


def test_the_wrapper_answers_the_reference_calls():
    """The calls the reference's renderer makes (hawk/emit/render.py), over a
    walk of a planned stage: the text of each member is the stage's own."""
    import re

    from hawk_amd.hip_target import StageWalk
    plan = plan_kernel(E.twobody.program, "twobody", block=128)
    per_thread = int(re.search(r"hk_per_thread = (\d+);", plan.source).group(1))
    walk = StageWalk.of(plan.stage, 128, per_thread)
    wrap = TARGETS["hip"].wrapper
    assert walk.arg_spec == tuple(tuple(x) for x in plan.stage.arg_spec)
    assert [walk.slot_of[slot] for slot in walk.arg_spec] == list(range(len(walk.arg_spec)))
    assert walk.slot_types[("uniform", "mu")].dtype == "f64"
    assert walk.slot_types[("vec_in", "r0")].shape == (3,)
    sig = wrap.entry_signature(walk, "twobody")
    unpack = wrap.unpack(walk)
    prologue = wrap.index_prologue()
    epilogue = wrap.index_epilogue()
    for text in (sig, unpack, prologue, epilogue):
        assert isinstance(text, str) and text in plan.source
    assert sig.startswith('extern "C" __global__ void __launch_bounds__(128) twobody(')
    assert "GRefMirror hk_p_r0_m" in sig and sig.index("hk_p_r0_m") < sig.index("long long base")
    assert "const Real* __restrict__ hk_p_r0" in unpack and "Real* __restrict__ hk_p_r =" in unpack
    assert "const long long hk_i = base + hk_flat;" in prologue
    for kw, words in (({"segment": object()}, "segmented unit"), ({"active": object()}, "active-lane"),
                      ({"box": object()}, "box prologue")):
        with pytest.raises(HawkError, match=words):
            wrap.index_prologue(**kw)


def test_a_row_builds_only_its_modes():
    narrow = dataclasses.replace(TARGETS["hip"], modes=("float64",))
    with pytest.raises(HawkError, match=r"mode='float32': the hip target builds 'float64'"):
        plan_kernel(E.scale.program, "scale", mode="float32", target=narrow)


@pytest.mark.parametrize("member, args, words", [
    ("scatter_store", (None, None, "t", "k", "v"), "scattered store"),
    ("accum_scattered", (None, None, "t", "k", "v"), "atomic accumulate"),
    ("or_scattered", (None, None, "t", "k", "v"), "scattered OR"),
    ("store_compensated", (None, None, "t", "c", "v"), "compensated scattered"),
    ("in_place_accumulate", (None, "t", "k", "v"), "accumulate into a plane row"),
    ("zero_row", (None, "t", 3), "zeroed plane row"),
])
def test_writer_members_without_a_form_are_refused_by_name(member, args, words):
    with pytest.raises(HawkError, match=f"the hip target has no form for .*{words}"):
        getattr(TARGETS["hip"].writer, member)(*args)


def test_wrapper_members_without_a_form_are_refused_by_name():
    with pytest.raises(HawkError, match="multi-branch dispatch"):
        TARGETS["hip"].wrapper.dispatch("k", ["a", "b"], "select")
    with pytest.raises(HawkError, match="sample reduction by 'prod'"):
        TARGETS["hip"].wrapper.sample_sum_frame(1, "double", "", op="prod")
    with pytest.raises(HawkError, match="device-read live count"):
        TARGETS["hip"].wrapper.sample_sum_frame(1, "double", "", live="hawk_live")


def test_an_unknown_row_is_refused():
    with pytest.raises(HawkError, match=r"targets=\['cuda'\]: this build's target row is 'hip'"):
        row("cuda")


def test_the_build_records_what_the_row_says(tmp_path):
    bundle = hawk.build([E.scale], tmp_path)
    side = json.loads((tmp_path / "scale.json").read_text())
    manifest = json.loads((tmp_path / "manifest.json").read_text())
    hip = TARGETS["hip"]
    assert (side["target"], side["offload_arch"], side["format"], side["entry_kind"]) == \
        (hip.id, hip.offload_arch, hip.format, hip.entry)
    assert side["source"] == "scale" + hip.source and side["code_object"] == "scale" + hip.artifact
    assert (tmp_path / side["code_object"]).is_file() and (tmp_path / side["source"]).is_file()
    assert (manifest["target"], manifest["offload_arch"]) == (hip.id, hip.offload_arch)
    assert bundle.digest == manifest["digest"]


def test_the_benchs_latency_probe_builds_for_gfx950(tmp_path):
    """bench.py --latency's probe kernel compiles through the build's hipRTC
    path and carries the ABI tag every loaded code object is checked for; it
    is a measurement mode of the bench, not part of the package."""
    import importlib

    import bench
    from hawk_amd.compile import compile_source
    code, _key, hit = compile_source(bench.LATENCY_SOURCE, "hawk_latency", cache_dir=tmp_path)
    assert not hit and code[:4] == b"\x7fELF" and b"aether-abi/2" in code
    assert sorted(bench.LATENCY_PROBES) == list(range(len(bench.LATENCY_PROBES)))
    assert importlib.util.find_spec("hawk_amd.latency") is None
