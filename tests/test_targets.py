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
        def index_prologue(self, block, per_thread, xcd_order, form="plain"):
            return super().index_prologue(block, per_thread, True, form)
    base = plan_kernel(E.twobody.program, "twobody").source
    other = plan_kernel(E.twobody.program, "twobody",
                        target=dataclasses.replace(TARGETS["hip"], wrapper=Ordered())).source
    assert "const unsigned hk_blk = blockIdx.x;" in base and "(gridDim.x & 7u)" not in base
    assert "(gridDim.x & 7u)" in other and "const unsigned hk_blk = blockIdx.x;" not in other


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
    with pytest.raises(HawkError, match="sample reduction by 'max'"):
        TARGETS["hip"].wrapper.sample_sum_frame(1, "double", "", op="max")


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
