"""Which axis of a per-sample plane holds the samples (reference
hawk/_plane_layout.py, hawk/runtime.py:542-566): the resolution on CPU
tensors, without a GPU."""

import pytest
import torch

import hawk_amd as hawk
from hawk_amd import layout as L
from hawk_amd.runtime import _PER_SAMPLE, _WRITTEN


class _K:
    planes = {"v": {"role": "vec_in", "shape": [3]}, "out": {"role": "mutable", "shape": []},
              "m": {"role": "mutable", "shape": [2, 2]}, "a": {"role": "uniform", "shape": []}}


def _resolve(arrays, layout=None):
    return L.resolve(_K, arrays, layout, _PER_SAMPLE, _WRITTEN)


def test_component_major_planes_pass_through_untouched():
    v, out = torch.randn(3, 10), torch.zeros(10)
    got, back = _resolve({"v": v, "out": out, "a": 2.0})
    assert got["v"] is v and got["out"] is out and got["a"] == 2.0 and back == []


def test_a_sample_major_plane_runs_through_a_component_major_copy():
    v = torch.randn(10, 3)
    m = torch.randn(10, 2, 2)
    got, back = _resolve({"v": v, "m": m})
    assert got["v"].shape == (3, 10) and got["v"].is_contiguous() and torch.equal(got["v"], v.t())
    assert got["m"].shape == (2, 2, 10) and torch.equal(got["m"][1, 0], m[:, 1, 0])
    assert [d is m for d, _ in back] == [True]          # m is written, v is read only


def test_a_plane_that_reads_both_ways_needs_a_word():
    v = torch.randn(3, 3)
    with pytest.raises(hawk.HawkError, match="reads both as"):
        _resolve({"v": v})
    got, _ = _resolve({"v": v}, layout="samples_first")
    assert torch.equal(got["v"], v.t())
    got, _ = _resolve({"v": hawk.samples_last(v)}, layout="samples_first")     # the marker wins
    assert got["v"] is v
    got, _ = _resolve({"v": hawk.samples_first(v)})
    assert torch.equal(got["v"], v.t())


def test_layout_refusals_name_the_problem():
    with pytest.raises(hawk.HawkError, match="is not one of"):
        _resolve({}, layout="rows")
    with pytest.raises(hawk.HawkError, match="marked samples_first but has shape"):
        _resolve({"v": hawk.samples_first(torch.randn(3, 10))})
    with pytest.raises(hawk.HawkError, match="no sample axis"):
        _resolve({"a": hawk.samples_first(torch.randn(3))})
    with pytest.raises(hawk.HawkError, match="marked samples_first is marked samples_last"):
        hawk.samples_last(hawk.samples_first(torch.randn(3)))


def test_a_cut_chain_resolves_the_callers_planes_once(tmp_path):
    """A chain cut into segments (a register line of 32) with its Vector[3]
    output given sample-major: the caller's planes are resolved once, at the
    chain, so every segment binds component-major planes (the crossing plane
    hwc_a is (3, N)), the sample count is N, and the output's copy is written
    back after the last segment."""
    import json

    import chain_members as C
    from hawk_amd import runtime as R

    class _Segment:                       # a segment's sidecar without its code object (no device here)
        def __init__(self, directory, name):
            self.name = name
            self.planes = json.loads((directory / f"{name}.json").read_text())["planes"]

        def caller_planes(self):
            return [n for n, p in self.planes.items() if not p.get("scratch")]

    chained = hawk.chain(*C.MEMBERS, name="fixture")
    hawk.build([chained], tmp_path, register_line=32)
    side = json.loads((tmp_path / "fixture.json").read_text())
    saved = R.load
    R.load = _Segment
    try:
        cut = R.ChainedKernel(tmp_path, side)
    finally:
        R.load = saved
    n = 10
    x, acc, y = torch.rand(n, dtype=torch.float64), torch.rand(n, dtype=torch.float64), torch.zeros(n, 3,
                                                                                                    dtype=torch.float64)
    for how in ({"layout": "samples_first"}, {}):
        bindings, back = cut.resolve_call({"x": x, "acc": acc, "y": y}, **how)
        assert [seg.name for seg, _ in bindings] == [f"fixture__s{i}" for i in range(4)]
        for seg, planes in bindings:
            for name, t in planes.items():
                lead = tuple((cut.planes.get(name) or cut.crossing[name])["shape"])
                assert tuple(t.shape) == lead + (n,), (seg.name, name, tuple(t.shape))
        assert [d is y for d, _ in back] == [True] and back[0][1].shape == (3, n)
    with pytest.raises(hawk.HawkError, match="sample-major under layout='samples_first'"):
        cut.resolve_call({"x": x, "acc": acc, "y": torch.zeros(3, n, dtype=torch.float64)}, "samples_first")
    with pytest.raises(hawk.HawkError, match="no plane is a tensor"):
        cut._bindings({"x": 1.0, "acc": 2.0, "y": 3.0}, n_samples=5)
