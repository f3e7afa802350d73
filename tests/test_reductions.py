"""Reductions over the samples: ``hawk.sum / max / min / mean(x)`` stored to a
``Mutable`` cell, the ``where=`` mask, and a vector cell (one entry a
column), as the reference's tests/test_reduce_samples.py and
tests/test_sample_sum.py lay them out.

* CPU: the team stages and planes a build plans, the derivative refusals, and
  the IR's value of each cell (tests/ir_eval.py) against numpy;
* GPU (marked ``gpu``): every cell bit for bit the CPU oracle's (row
  extremes and the canonical finish for max / min, compensated rows for sum
  and mean), float64 and float32, at sizes 1, 31, 32, 33, 1000, 100003,
  300007; max and min equal numpy's exactly; a vector cell's entries are each
  column's own sum; repeated launches give the same bits.
"""

from __future__ import annotations

import numpy as np
import pytest

import oracle_lib as O
from conftest import rng

import hawk_amd as hawk
from hawk_amd import HawkError, Mutable, Scalar, Vector, kernel
from hawk_amd.diff import jvp, vjp
from ir_eval import evaluate

SIZES = (1, 31, 32, 33, 1000, 100_003, 300_007)
OPS = ("sum", "mean", "max", "min")


@kernel
def cell_sum(x: Scalar, t: Mutable[Scalar]):
    t = hawk.sum(x * x)


@kernel
def cell_mean(x: Scalar, t: Mutable[Scalar]):
    t = hawk.mean(x * x)


@kernel
def cell_max(x: Scalar, t: Mutable[Scalar]):
    t = hawk.max(x * 1.5)


@kernel
def cell_min(x: Scalar, t: Mutable[Scalar]):
    t = hawk.min(x * 1.5)


@kernel
def fold_max(x: Scalar, hi: Mutable[Scalar]):
    hi = hawk.max(x, where=x > 0.0)


@kernel
def fold_min(x: Scalar, lo: Mutable[Scalar]):
    lo = hawk.min(x, where=x < 0.0)


@kernel
def masked_sum(x: Scalar, t: Mutable[Scalar], c: Mutable[Scalar]):
    t = hawk.sum(x, where=x > 0.25)
    c = hawk.sum(x > 0.25)


@kernel
def fold_vec(v: Vector[3], t: Mutable[Vector[3]]):
    t = hawk.sum(v * 2.0)


@kernel
def vec_max(v: Vector[3], t: Mutable[Vector[3]]):
    t = hawk.max(v)


@kernel
def two_cells(x: Scalar, y: Mutable[Scalar], hi: Mutable[Scalar], s: Mutable[Scalar]):
    y = x + 1.0
    hi = hawk.max(x)
    s = hawk.sum(x)


CELLS = {"sum": cell_sum, "mean": cell_mean, "max": cell_max, "min": cell_min}
KERNELS = [*CELLS.values(), fold_max, fold_min, masked_sum, fold_vec, vec_max, two_cells]


# -- CPU: plans, refusals, the IR's value ------------------------------------------

def test_a_max_is_a_row_extreme_team_stage(tmp_path):
    b = hawk.build([cell_max, cell_min, cell_mean], tmp_path)
    assert b.sidecar("cell_max")["team"] == [{"op": "row_extreme", "red": "max", "hi": "hk_rows_t", "out": "t"}]
    assert b.sidecar("cell_min")["team"][0]["red"] == "min"
    sc = b.sidecar("cell_max")
    assert sc["planes"]["hk_rows_t"]["rows"] == 32 and "hk_rows_t_comp" not in sc["planes"]
    assert sc["planes"]["t"]["role"] == "cell" and sc["planes"]["t"]["shape"] == []
    assert b.sidecar("cell_mean")["team"][0]["op"] == "row_sum"
    src = (tmp_path / "cell_max.hip").read_text()
    # four samples of a row a lane (its launch shape takes four samples a
    # thread); a lane past the run brings -inf
    assert "hk_row_extreme4(1, hk_rt[0])" in src and "-__builtin_inf()" in src
    for pt, form in ((1, "hk_row_extreme(1, hk_rh)"), (2, "hk_row_extreme2(1, hk_rt[0])"),
                     (6, "hk_row_extreme2(1, hk_rt[0])"), (8, "hk_row_extreme4(1, hk_rt[0])")):
        hawk.build([cell_max], tmp_path / f"pt{pt}", per_thread=pt)
        body = (tmp_path / f"pt{pt}" / "cell_max.hip").read_text().split('extern "C" __global__')[-1]
        assert form in body, (pt, form)


def test_a_vector_cell_is_one_row_stage_per_column(tmp_path):
    b = hawk.build([fold_vec], tmp_path)
    team = b.sidecar("fold_vec")["team"]
    assert [(t["op"], t["hi"], t["out"], t["column"]) for t in team] == [
        ("row_sum", f"hk_rows_t_{k}", "t", k) for k in range(3)]
    assert b.sidecar("fold_vec")["planes"]["t"]["shape"] == [3]


def test_an_ordered_vector_sum_is_one_ordered_stage_per_column(tmp_path):
    @kernel
    def ordered_vec(v: Vector[2], t: Mutable[Vector[2]]):
        t = hawk.sum(v, policy="ordered")

    b = hawk.build([ordered_vec], tmp_path)
    team = b.sidecar("ordered_vec")["team"]
    assert [(t["op"], t["out"], t["column"]) for t in team] == [("ordered_sum", "t", 0), ("ordered_sum", "t", 1)]


@pytest.mark.parametrize("op", ("max", "min"))
def test_max_and_min_over_samples_refuse_to_differentiate(op):
    with pytest.raises(HawkError, match="ambiguous at a tie"):
        vjp(CELLS[op], wrt=("x",))
    with pytest.raises(HawkError, match="ambiguous at a tie"):
        jvp(CELLS[op], wrt=("x",))


def test_refusals_name_the_rewrite():
    with pytest.raises(HawkError, match=r"hawk.sum\(x, where=mask\) / hawk.sum\(mask\)"):
        @kernel
        def bad_mean(x: Scalar, t: Mutable[Scalar]):
            t = hawk.mean(x, where=x > 0.0)
    with pytest.raises(HawkError, match="where= is this lane's bool mask"):
        @kernel
        def bad_mask(x: Scalar, t: Mutable[Scalar]):
            t = hawk.max(x, where=x)
    with pytest.raises(HawkError, match="policy="):
        @kernel
        def bad_policy(x: Scalar, t: Mutable[Scalar]):
            t = hawk.min(x, policy="fast")


def test_the_sum_of_a_mean_has_a_broadcast_adjoint():
    """d mean(x*x) / dx_i = 2 x_i / n: the reverse of the cell is a broadcast
    of its adjoint, the sample count a constant (reference
    tests/test_reduce_samples.py, test_a_sum_over_samples_has_a_broadcast_adjoint)."""
    d = vjp(cell_mean, wrt=("x",))
    x = np.array([1.5, -2.0, 0.25, 3.0])
    got = evaluate(d, {"x": x, "bar_t": 2.0}, x.size)
    np.testing.assert_allclose(got["bar_x"], 2.0 * 2 * x / x.size, rtol=1e-15)
    fwd = evaluate(cell_mean.program, {"x": x}, x.size)["t"]          # the per-sample terms
    np.testing.assert_allclose(fwd.sum(), np.mean(x * x), rtol=1e-15)


def test_vector_and_masked_terms_in_the_ir():
    """Each column sink reads its own entry; a masked lane is the identity."""
    got = [s for s in fold_vec.program.sinks]
    assert [(s.name, s.column, s.op) for s in got] == [("t", k, "sum") for k in range(3)]
    from ir_eval import Evaluator
    v = rng(4).normal(size=(3, 50))
    ev = Evaluator({"v": v}, 50)
    for k, s in enumerate(got):
        np.testing.assert_array_equal(ev.value(s.value), 2.0 * v[k])
    x = rng(5).uniform(-2, 2, 50)
    ev = evaluate(fold_max.program, {"x": x}, 50)
    np.testing.assert_array_equal(ev["hi"], np.where(x > 0, x, -np.inf))
    ev = evaluate(masked_sum.program, {"x": x}, 50)
    np.testing.assert_array_equal(ev["c"], (x > 0.25).astype(float))


# -- GPU: every cell the oracle's bits ---------------------------------------------

@pytest.fixture(scope="module", params=["float64", "float32"])
def built(request, tmp_path_factory):
    root = tmp_path_factory.mktemp(f"reduce_{request.param}")
    hawk.build(KERNELS, root, mode=request.param)
    return root, request.param


def _x(n, mode):
    g = rng(n)
    return (g.normal(size=n) * np.exp(g.normal(size=n))).astype(mode)


def dev(a, gpu):
    import torch
    return torch.from_numpy(np.ascontiguousarray(a)).to(gpu)


def host(t):
    return t.detach().cpu().numpy()


def _want(op, x, mode):
    """The oracle's cell: the term computed in the build's precision, then the
    rows and the canonical finish in it."""
    dt = np.dtype(mode).type
    if op == "sum":
        t = x * x
    elif op == "mean":
        t = (x * x) / dt(x.size)
    else:
        t = x * dt(1.5)
    if op in ("max", "min"):
        return O.sample_extreme(t, op)
    return O.sample_sum_f32(t) if mode == "float32" else O.sample_sum(t)


@pytest.mark.gpu
@pytest.mark.parametrize("n", SIZES)
@pytest.mark.parametrize("op", OPS)
def test_cells_are_the_oracles_bits(built, gpu, op, n):
    root, mode = built
    x = _x(n, mode)
    print(f"reduction {op} {mode} n={n}", flush=True)
    k = hawk.load(root, f"cell_{op}")
    want = np.asarray(_want(op, x, mode), dtype=mode)
    out = dev(np.full(1, np.nan, dtype=mode), gpu)
    hawk.run(k, x=dev(x, gpu), t=out)
    got = host(out)[0]
    assert got.tobytes() == want.tobytes(), (got, want)
    if op in ("max", "min"):
        t = x * np.dtype(mode).type(1.5)
        assert got.tobytes() == (t.max() if op == "max" else t.min()).tobytes()


@pytest.mark.gpu
@pytest.mark.parametrize("op", OPS)
def test_cells_are_bitwise_across_launches(built, gpu, op):
    root, mode = built
    n = 65536 + 17
    x = dev(_x(n, mode), gpu)
    k = hawk.load(root, f"cell_{op}")
    first = None
    for _ in range(4):
        out = dev(np.full(1, np.nan, dtype=mode), gpu)
        hawk.run(k, x=x, t=out)
        got = host(out).tobytes()
        first = first or got
        assert got == first


@pytest.mark.gpu
@pytest.mark.parametrize("n", (1, 33, 1000, 100_003))
def test_masked_cells(built, gpu, n):
    """where=: a masked lane is the identity (-inf for max, +inf for min, 0
    for a sum); the sum of a mask counts its true lanes.  A mask with no true
    lane leaves the identity."""
    root, mode = built
    x = rng(n + 1).uniform(-2, 2, n).astype(mode)
    print(f"masked reductions {mode} n={n}", flush=True)
    hi, lo = dev(np.full(1, np.nan, mode), gpu), dev(np.full(1, np.nan, mode), gpu)
    hawk.run(hawk.load(root, "fold_max"), x=dev(x, gpu), hi=hi)
    hawk.run(hawk.load(root, "fold_min"), x=dev(x, gpu), lo=lo)
    inf = np.dtype(mode).type(np.inf)
    want_hi = O.sample_extreme(np.where(x > 0, x, -inf).astype(mode), "max")
    want_lo = O.sample_extreme(np.where(x < 0, x, inf).astype(mode), "min")
    assert host(hi)[0].tobytes() == np.asarray(want_hi, mode).tobytes()
    assert host(lo)[0].tobytes() == np.asarray(want_lo, mode).tobytes()
    pos = x[x > 0]
    assert host(hi)[0] == (pos.max() if pos.size else -np.inf)
    t, c = dev(np.full(1, np.nan, mode), gpu), dev(np.full(1, np.nan, mode), gpu)
    hawk.run(hawk.load(root, "masked_sum"), x=dev(x, gpu), t=t, c=c)
    zero = np.dtype(mode).type(0)
    sum_of = O.sample_sum_f32 if mode == "float32" else O.sample_sum
    assert host(t)[0].tobytes() == np.asarray(sum_of(np.where(x > 0.25, x, zero).astype(mode)), mode).tobytes()
    assert host(c)[0] == np.count_nonzero(x > 0.25)


@pytest.mark.gpu
@pytest.mark.parametrize("n", (1, 31, 1000, 100_003))
def test_vector_cells_are_each_columns_reduction(built, gpu, n):
    root, mode = built
    v = rng(n + 2).normal(size=(3, n)).astype(mode)
    print(f"vector cells {mode} n={n}", flush=True)
    t = dev(np.full(3, np.nan, mode), gpu)
    hawk.run(hawk.load(root, "fold_vec"), v=dev(v, gpu), t=t)
    sum_of = O.sample_sum_f32 if mode == "float32" else O.sample_sum
    want = np.array([sum_of(v[k] * np.dtype(mode).type(2.0)) for k in range(3)], mode)
    assert host(t).tobytes() == want.tobytes()
    m = dev(np.full(3, np.nan, mode), gpu)
    hawk.run(hawk.load(root, "vec_max"), v=dev(v, gpu), t=m)
    assert host(m).tobytes() == v.max(axis=1).tobytes()


@pytest.mark.gpu
@pytest.mark.parametrize("n", (1, 17, 33, 4096 * 3 + 81, 100_003))
def test_both_row_layouts_are_the_oracles_bits(gpu, tmp_path, n):
    """The rows four samples a lane (samples j + 8v of a row in lane j of an
    8-lane group, at a multiple of four samples a thread: the default for
    these kernels), two (j + 16v, at an even number) and one
    (``per_thread=1``: a half-wave a row) give the oracle's bits for a sum, a
    max and a min, in both scalar modes, and for a sum of bands in the banded
    mode."""
    for mode in ("float64", "float32"):
        x = _x(n, mode)
        for pt, form in ((1, "hk_row_sum(hk_rh"), (2, "hk_row_sum2("), (4, "hk_row_sum4("), (6, "hk_row_sum2(")):
            root = tmp_path / f"{mode}_{pt}"
            hawk.build([cell_sum, cell_max, cell_min], root, mode=mode, per_thread=pt)
            body = (root / "cell_sum.hip").read_text().split('extern "C" __global__')[-1]
            assert form in body, (pt, form)
            for op in ("sum", "max", "min"):
                print(f"row layout {mode} per_thread={pt} {op} n={n}", flush=True)
                out = dev(np.full(1, np.nan, dtype=mode), gpu)
                hawk.run(hawk.load(root, f"cell_{op}"), x=dev(x, gpu), t=out)
                want = np.asarray(_want(op, x, mode), dtype=mode)
                assert host(out)[0].tobytes() == want.tobytes(), (mode, pt, op, host(out)[0], want)
    # the banded mode's rows (bands) in the same three layouts
    x = _x(n, "float64")
    for pt, form in ((1, "hk_band_row_sum(hk_rh"), (2, "hk_band_row_sum2("), (4, "hk_band_row_sum4(")):
        root = tmp_path / f"banded_{pt}"
        hawk.build([cell_sum], root, mode="banded", per_thread=pt)
        assert form in (root / "cell_sum.hip").read_text().split('extern "C" __global__')[-1], (pt, form)
        print(f"row layout banded per_thread={pt} n={n}", flush=True)
        out = dev(np.full(1, np.nan), gpu)
        hawk.run(hawk.load(root, "cell_sum"), x=dev(x, gpu), t=out)
        assert host(out)[0] == O.band_sample_sum(x * x), (pt, host(out)[0])


@pytest.mark.gpu
def test_a_stage_with_a_plane_and_two_kinds_of_cell(built, gpu):
    root, mode = built
    n = 4096 * 32 + 5
    x = _x(n, mode)
    y, hi, s = (dev(np.full(k, np.nan, mode), gpu) for k in (n, 1, 1))
    hawk.run(hawk.load(root, "two_cells"), x=dev(x, gpu), y=y, hi=hi, s=s)
    assert host(y).tobytes() == (x + np.dtype(mode).type(1.0)).tobytes()
    assert host(hi)[0] == x.max()
    sum_of = O.sample_sum_f32 if mode == "float32" else O.sample_sum
    assert host(s)[0].tobytes() == np.asarray(sum_of(x), mode).tobytes()


@pytest.mark.gpu
def test_nan_rows_follow_the_reference_operators(built, gpu):
    """A row ignores a NaN unless all its lanes are NaN; the finish keeps the
    right operand when the left is NaN (the oracle's pins, on the device)."""
    root, mode = built
    k = hawk.load(root, "cell_max")
    for x in (np.concatenate([np.full(32, np.nan), np.ones(32)]), np.concatenate([np.ones(32), np.full(32, np.nan)]),
              np.full(40, np.nan), np.array([0.0, -0.0]), np.array([-0.0, 0.0])):
        x = x.astype(mode)
        out = dev(np.full(1, 7.0, mode), gpu)
        hawk.run(k, x=dev(x, gpu), t=out)
        want = np.asarray(O.sample_extreme(x * np.dtype(mode).type(1.5), "max"), mode)
        assert host(out)[0].tobytes() == want.tobytes(), x


@pytest.fixture(scope="module")
def built_banded(tmp_path_factory):
    root = tmp_path_factory.mktemp("reduce_banded")
    hawk.build([cell_max, cell_min, cell_mean, fold_vec], root, mode="banded")
    return root


@pytest.mark.gpu
@pytest.mark.parametrize("n", (1, 33, 100_003))
def test_banded_cells(built_banded, gpu, n):
    """The banded mode: max / min take the same exact rows and finish; a mean
    and a vector cell's entries are band sums (the oracle's band rows and
    finish), bit for bit."""
    x = _x(n, "float64")
    print(f"banded reductions n={n}", flush=True)
    for op in ("max", "min"):
        out = dev(np.full(1, np.nan), gpu)
        hawk.run(hawk.load(built_banded, f"cell_{op}"), x=dev(x, gpu), t=out)
        want = (x * 1.5).max() if op == "max" else (x * 1.5).min()
        assert host(out)[0] == want
    out = dev(np.full(1, np.nan), gpu)
    hawk.run(hawk.load(built_banded, "cell_mean"), x=dev(x, gpu), t=out)
    assert host(out)[0] == O.band_sample_sum((x * x) / float(n))
    v = rng(n + 9).normal(size=(3, n))
    t = dev(np.full(3, np.nan), gpu)
    hawk.run(hawk.load(built_banded, "fold_vec"), v=dev(v, gpu), t=t)
    assert host(t).tolist() == [O.band_sample_sum(v[k] * 2.0) for k in range(3)]
