"""The authoring surface, the IR and the derivative transforms, on the CPU:
tracing and arg_spec order, refusals by name, the rolled loop, and the
vjp/jvp of every benchmark kernel against central differences (through the
numpy IR interpreter) and against the oracle's operation order."""

from __future__ import annotations

import numpy as np
import pytest

import hawk_amd as hawk
import oracle_lib as O
from hawk_amd import HawkError, Index, Matrix, Mutable, Param, Scalar, Vector, ir
from hawk_amd import examples as E
from hawk_amd.diff import jvp, vjp
from hawk_amd.math import dot, exp, sqrt
from ir_eval import evaluate
from net_axis import net_problem


def test_declarations_give_roles_and_the_canonical_arg_spec():
    from hawk_amd.emit_hip import plan_kernel
    p = plan_kernel(E.energy_vjp.program, "energy_vjp")
    # ROLE_ORDER: mutable, out, ..., vec_in, ..., per_sample, ..., uniform
    assert p.stage.arg_spec == [("mutable", "bar_v"), ("vec_in", "v"), ("per_sample", "bar_out")]
    p = plan_kernel(E.scale.program, "scale")
    assert p.stage.arg_spec == [("out", "out"), ("per_sample", "x"), ("uniform", "a"), ("uniform", "b")]
    assert [p.stage.planes[n]["kind"] for _, n in p.stage.arg_spec] == ["gref", "handle", "f64", "f64"]


def test_a_returned_value_commits_into_out():
    assert [(type(s).__name__, s.name) for s in E.scale.sinks] == [("Assign", "out")]
    assert E.scale.decls["out"].role == "out"


def test_sum_and_scatter_become_team_stages():
    from hawk_amd.emit_hip import plan_kernel
    p = plan_kernel(E.chain.program, "chain")
    ops = sorted(t["op"] for t in p.team)
    assert ops == ["ordered_scatter", "ordered_sum"]
    assert {t.get("u") or t.get("v") for t in p.team} == {"y"}     # both read the stored y, no extra plane
    assert p.planes["total"]["role"] == "cell" and p.planes["bins"]["role"] == "accum_out"


def test_refuses_a_branch_on_a_traced_value():
    with pytest.raises(HawkError, match="where"):
        @hawk.kernel
        def k(x: Scalar, y: Mutable[Scalar]):
            if x > 0.0:
                y = x
            else:
                y = -x


def test_refuses_an_undeclared_parameter():
    with pytest.raises(HawkError, match="no declaration"):
        @hawk.kernel
        def k(x, y: Mutable[Scalar]):
            y = x


def test_refuses_a_non_literal_trip_count():
    with pytest.raises(HawkError, match="literal int"):
        @hawk.kernel
        def k(x: Scalar, n: Param, y: Mutable[Scalar]):
            acc = x
            for i in range(n):
                acc = acc * x
            y = acc


def test_vjp_refuses_a_prior_read():
    @hawk.kernel
    def running(x: Scalar, m: Mutable[Scalar]):
        m = m + x
    with pytest.raises(HawkError, match="before it writes it"):
        vjp(running)


def test_sum_read_back_is_refused():
    with pytest.raises(HawkError, match="stage boundary"):
        @hawk.kernel
        def k(x: Scalar, y: Mutable[Scalar]):
            y = x / hawk.sum(x, policy="ordered")


def test_the_loop_is_rolled_with_its_carries():
    loops = [n for n in ir.topo([s.value for s in E.twobody.sinks]) if n.kind == "loop"]
    assert len(loops) == 1
    info = loops[0].literal
    assert info.trip == E.SUBSTEPS and info.names == ("rr", "vv")


def test_energy_vjp_is_the_reference_rule():
    """bar_v = (bar_out * 0.5) * v + (bar_out * 0.5) * v: the oracle's expression, bit for bit."""
    g = np.random.default_rng(7)
    n = 1000
    v = g.normal(size=(3, n))
    bar_out = g.normal(size=n)
    got = evaluate(E.energy_vjp.program, {"v": v, "bar_out": bar_out}, n)["bar_v"]
    assert got.tobytes() == O.energy_vjp(v, bar_out).tobytes()
    dv = g.normal(size=(3, n))
    got = evaluate(E.energy_jvp.program, {"v": v, "dot_v": dv}, n)["dot_out"]
    assert got.tobytes() == O.energy_jvp(v, dv).tobytes()


def _central(fn, x, h):
    return (fn(x + h) - fn(x - h)) / (2 * h)


def test_twobody_vjp_ir_matches_the_oracle_and_finite_differences():
    n = 64
    g = np.random.default_rng(3)
    d = g.normal(size=(3, n))
    d /= np.linalg.norm(d, axis=0)
    r0 = d * g.uniform(0.5, 2.0, n)
    v0 = g.normal(0.0, 0.3, size=(3, n))
    bar_r, bar_v = g.normal(size=(3, n)), g.normal(size=(3, n))
    env = {"r0": r0, "v0": v0, "mu": 1.0, "bar_r": bar_r, "bar_v": bar_v}
    got = evaluate(E.twobody_vjp.program, env, n)
    want_r0, want_v0 = O.twobody_vjp(r0, v0, 1.0, bar_r, bar_v)
    np.testing.assert_allclose(got["bar_r0"], want_r0, rtol=1e-13, atol=1e-15)
    np.testing.assert_allclose(got["bar_v0"], want_v0, rtol=1e-13, atol=1e-15)
    fwd = evaluate(E.twobody.program, {"r0": r0, "v0": v0, "mu": 1.0}, n)
    wr, wv = O.twobody(r0, v0, 1.0)
    assert fwd["r"].tobytes() == wr.tobytes() and fwd["v"].tobytes() == wv.tobytes()
    # <bar, J e_c> by central differences for each input component
    h = 1e-6
    for name, grad in (("r0", got["bar_r0"]), ("v0", got["bar_v0"])):
        for c in range(3):
            e = np.zeros((3, n))
            e[c] = h

            def loss(delta):
                args = {"r0": r0, "v0": v0}
                args[name] = args[name] + delta
                r, v = O.twobody(np.ascontiguousarray(args["r0"]), np.ascontiguousarray(args["v0"]), 1.0)
                return (bar_r * r).sum(axis=0) + (bar_v * v).sum(axis=0)
            fd = (loss(e) - loss(-e)) / (2 * h)
            np.testing.assert_allclose(grad[c], fd, rtol=1e-6, atol=1e-8)


def test_spd_vjp_ir_matches_the_oracle_and_finite_differences():
    n = 32
    g = np.random.default_rng(4)
    B = g.normal(size=(n, 6, 6))
    A = np.ascontiguousarray((np.matmul(B, B.transpose(0, 2, 1)) + 6.0 * np.eye(6)).transpose(1, 2, 0))
    b = np.ascontiguousarray(g.normal(size=(n, 6)).T)
    bar_x = g.normal(size=(6, n))
    x = evaluate(E.spd_solve.program, {"A": A, "b": b}, n)["x"]
    assert x.tobytes() == O.spd_solve(A, b).tobytes()
    got = evaluate(E.spd_solve_vjp.program, {"A": A, "b": b, "bar_x": bar_x}, n)
    wA, wb = O.spd_solve_vjp(A, b, bar_x)
    assert got["bar_A"].tobytes() == wA.tobytes() and got["bar_b"].tobytes() == wb.tobytes()
    h = 1e-6
    for (i, j) in ((0, 0), (2, 5), (5, 1)):
        e = np.zeros_like(A)
        e[i, j] = h
        fd = ((bar_x * O.spd_solve(A + e, b)).sum(0) - (bar_x * O.spd_solve(A - e, b)).sum(0)) / (2 * h)
        # a symmetric-part derivative: the unsymmetric perturbation reads 0.5(e + e^T)
        np.testing.assert_allclose(got["bar_A"][i, j], fd, rtol=1e-6, atol=1e-9)


def test_jvp_and_vjp_are_adjoint_on_a_loop():
    """<bar, J t> == <J^T bar, t> for the rolled two-body loop (forward mode through
    the augmented loop, reverse mode through the taped reverse loop)."""
    n = 16
    g = np.random.default_rng(9)
    d = g.normal(size=(3, n))
    d /= np.linalg.norm(d, axis=0)
    r0 = d * g.uniform(0.5, 2.0, n)
    v0 = g.normal(0.0, 0.3, size=(3, n))
    tr, tv = g.normal(size=(3, n)), g.normal(size=(3, n))
    br, bv = g.normal(size=(3, n)), g.normal(size=(3, n))
    tangent = evaluate(jvp(E.twobody, wrt=("r0", "v0")),
                       {"r0": r0, "v0": v0, "mu": 1.0, "dot_r0": tr, "dot_v0": tv}, n)
    adjoint = evaluate(E.twobody_vjp.program, {"r0": r0, "v0": v0, "mu": 1.0, "bar_r": br, "bar_v": bv}, n)
    lhs = (br * tangent["dot_r"]).sum(0) + (bv * tangent["dot_v"]).sum(0)
    rhs = (adjoint["bar_r0"] * tr).sum(0) + (adjoint["bar_v0"] * tv).sum(0)
    np.testing.assert_allclose(lhs, rhs, rtol=1e-11)


def test_chain_forward_is_the_oracle_expression():
    """The chain's IR computes the oracle's operations (transcendentals aside):
    evaluated with numpy's libm the two agree to a few ulp."""
    x = np.random.default_rng(5).normal(size=4096)
    prog = E.chain.program
    y = evaluate(prog, {"x": x, "key": np.zeros(4096, np.int32)}, 4096)["y"]
    np.testing.assert_allclose(y, O.chain(x), rtol=1e-12, atol=1e-14)


def test_emitted_source_has_one_geometry_prologue():
    from hawk_amd.emit_hip import plan_kernel
    src = plan_kernel(E.energy.program, "energy").source
    geometry = [line for line in src.splitlines() if "blockIdx.x" in line]
    assert len(geometry) == 1 and "const unsigned hk_blk =" in geometry[0]
    assert src.count("hk_i = base + hk_flat") == 1
    assert 'eagle_abi_tag[] = "aether-abi/2"' in src
    assert "eagle_layout_sizes[5] = {40, 32, 32, 8, 24}" in src


def test_build_writes_the_unit(tmp_path):
    b = hawk.build([E.scale, E.chain], tmp_path)
    names = sorted(p.name for p in tmp_path.iterdir())
    assert names == ["chain.hip", "chain.hsaco", "chain.json", "manifest.json", "scale.hip", "scale.hsaco",
                     "scale.json"]
    side = b.sidecar("chain")
    assert side["target"] == "hip" and side["offload_arch"] == "gfx950"
    assert side["descriptor"] == ["handle", "handle"]    # y (mutable, rank 0) and x (per_sample)
    assert hawk.compile.cache_stats()["hits"] + hawk.compile.cache_stats()["misses"] >= 2


def test_build_refuses_another_target(tmp_path):
    with pytest.raises(HawkError, match="'hip'"):
        hawk.build([E.scale], tmp_path, targets=("cuda",))


def test_a_kernel_defined_in_a_function_reads_its_local_names():
    from hawk_amd import Scalar as LocalScalar

    @hawk.kernel
    def k(x: LocalScalar) -> LocalScalar:
        return x + 1.0
    assert k.decls["x"].role == "per_sample"


def test_resources_are_recorded_and_the_vjp_tape_fits_in_registers(tmp_path):
    """The sidecar carries each entry's register/scratch figures from the code
    object's own metadata; the checkpointed two-body VJP keeps its tapes in
    registers (no scratch)."""
    b = hawk.build([E.energy, E.twobody_vjp], tmp_path)
    r = b.sidecar("twobody_vjp")["resources"]
    assert r["private_segment_fixed_size"] == 0 and r["vgpr_spill_count"] == 0
    assert r["waves_per_simd"] >= 1
    assert b.sidecar("energy")["resources"]["waves_per_simd"] == 8


def test_checkpointed_reverse_keeps_the_bits():
    """Strip-mining the 32-step recurrence before reversal replays the same
    operations: the VJP is bit-identical to the oracle's single-tape reverse."""
    n = 48
    g = np.random.default_rng(12)
    d = g.normal(size=(3, n))
    d /= np.linalg.norm(d, axis=0)
    r0 = d * g.uniform(0.5, 2.0, n)
    v0 = g.normal(0.0, 0.3, size=(3, n))
    br, bv = g.normal(size=(3, n)), g.normal(size=(3, n))
    got = evaluate(E.twobody_vjp.program, {"r0": r0, "v0": v0, "mu": 1.0, "bar_r": br, "bar_v": bv}, n)
    w0, w1 = O.twobody_vjp(r0, v0, 1.0, br, bv)
    assert got["bar_r0"].tobytes() == w0.tobytes() and got["bar_v0"].tobytes() == w1.tobytes()
    loops = [m for m in ir.topo([s.value for s in E.twobody_vjp.sinks]) if m.kind == "loop"]
    assert sorted(m.literal.trip for m in loops) == [4, 4, 4, 8, 8]


def test_fp_op_count_of_the_emitted_stages():
    """The sidecar's per-sample operation count is read off the code emitted
    for the program as traced: scale is a*x+b (2), energy
    0.5*((v0*v0+v1*v1)+v2*v2) (6), the chain's eight stages 14 (exp, sin, 2,
    tanh, 3, 2, exp+fabs, 2), and the two-body loop body (two force
    evaluations, 40 ops) counts 32 times."""
    from hawk_amd import emit_hip

    def count(k):
        return emit_hip.plan_kernel(k.program, k.name, "float64", 256, 1, True).algorithmic_ops
    assert count(E.scale) == 2
    assert count(E.energy) == 6
    assert count(E.chain) == 14
    assert count(E.twobody) == 40 * 32


@pytest.mark.parametrize("mode,dtype", [("float32", "f32"), ("float64", "f64")])
def test_mm16_and_its_vjp_are_one_mfma_team_stage(tmp_path, mode, dtype):
    """In either scalar mode a kernel whose sinks are 16x16 products of input
    planes runs as one mm16 team stage of that mode's planes: the forward one
    product, the VJP two with the transposes of bar_A = bar_C B^T and
    bar_B = A^T bar_C."""
    b = hawk.build([E.mm16, E.mm16_vjp], tmp_path, mode=mode)
    fwd, rev = b.sidecar("mm16"), b.sidecar("mm16_vjp")
    assert fwd["entry"] is None and fwd["team"] == [{"op": "mm16", "in": ["A", "B"], "out": ["C"],
                                                     "products": [[0, 1, False, False]], "dtype": dtype}]
    assert {p["dtype"] for p in fwd["planes"].values()} == {dtype}
    (t,) = rev["team"]
    assert t["out"] == ["bar_A", "bar_B"] and t["dtype"] == dtype
    named = [(t["in"][l], t["in"][r], tl, tr) for l, r, tl, tr in t["products"]]
    assert named == [("bar_C", "B", False, True), ("A", "bar_C", True, False)]


def test_default_sum_is_a_row_sum_team_stage(tmp_path):
    """hawk.sum(x) with the default policy: the stage writes compensated
    32-sample rows into runtime-owned planes, a row_sum team stage finishes the
    cell; the rows are not planes the caller binds."""
    b = hawk.build([E.sample_total], tmp_path)
    sc = b.sidecar("sample_total")
    assert sc["team"] == [{"op": "row_sum", "hi": "hk_rows_total", "comp": "hk_rows_total_comp", "out": "total"}]
    assert sc["planes"]["hk_rows_total"]["rows"] == 32 and sc["planes"]["hk_rows_total"]["scratch"]
    assert sc["planes"]["total"]["role"] == "cell"
    assert [n for r, n in sc["arg_spec"] if r == "rows_out"] == ["hk_rows_total", "hk_rows_total_comp"]


def test_param_gradient_is_a_summed_cell_matching_finite_differences():
    """vjp(param_planes(twobody), wrt=(r0, v0, mu)): bar_r0 / bar_v0 are the
    plain VJP's planes, bar_mu is a default-policy hawk.sum of each sample's
    contribution, and that sum is d/dmu of sum_s <bar, (r, v)(mu)> by central
    differences of the oracle's forward."""
    import math
    n = 200
    g = np.random.default_rng(11)
    d = g.normal(size=(3, n))
    d /= np.linalg.norm(d, axis=0)
    r0 = d * g.uniform(0.5, 2.0, n)
    v0 = g.normal(0.0, 0.3, size=(3, n))
    bar_r, bar_v = g.normal(size=(3, n)), g.normal(size=(3, n))
    env = {"r0": r0, "v0": v0, "mu": 1.3, "bar_r": bar_r, "bar_v": bar_v}
    prog = E.twobody_vjp_mu.program
    assert [type(s).__name__ for s in prog.sinks] == ["Assign", "Assign", "SampleSum"]
    got = evaluate(prog, env, n)
    plain = evaluate(E.twobody_vjp.program, env, n)
    assert got["bar_r0"].tobytes() == plain["bar_r0"].tobytes()
    assert got["bar_v0"].tobytes() == plain["bar_v0"].tobytes()

    def loss(mu):
        r, v = O.twobody(r0, v0, mu)
        return math.fsum(((bar_r * r).sum(axis=0) + (bar_v * v).sum(axis=0)).tolist())
    h = 1e-6
    fd = (loss(1.3 + h) - loss(1.3 - h)) / (2 * h)
    total = O.sample_sum(got["bar_mu"])
    assert abs(total - fd) <= 1e-6 * abs(fd) + 1e-8


def _ref_case(n, cells, seed):
    """The reference's scatter case (tests/test_scatter_ordered.py:81-87)."""
    g = np.random.default_rng(seed)
    key = g.integers(0, cells, n).astype(np.int32)
    x = g.normal(size=n) * np.exp(g.normal(size=n))
    return key, x


def test_scatter_vjp_is_a_gather_matching_finite_differences():
    """vjp(add_sq, wrt=x) of scatter(acc)[key] += x*x reads bar_acc at the key:
    bar_x == 2 x bar_acc[key] (to the reference's rtol 1e-12; here bit for bit),
    and central differences of g . acc(x) agree at 6 samples (eps 1e-6, rtol
    1e-5, atol 1e-7), as reference tests/test_scatter_ordered.py:124-157."""
    n, cells = 3000, 11
    key, x = _ref_case(n, cells, seed=5)
    g = np.random.default_rng(9).normal(size=cells)
    prog = E.add_sq_grad.program
    assert prog.decls["bar_acc"].role == "lookup"
    bar = evaluate(prog, {"key": key, "x": x, "bar_acc": g}, n)["bar_x"]
    assert bar.tobytes() == (2 * x * g[key]).tobytes()

    def loss(v):
        acc, status = O.ordered_scatter(key, v * v, np.zeros(cells))
        assert not status[1:].any()
        return float(g @ acc)
    eps = 1e-6
    for i in np.random.default_rng(2).choice(n, 6, replace=False):
        hi, lo = x.copy(), x.copy()
        hi[i] += eps
        lo[i] -= eps
        np.testing.assert_allclose((loss(hi) - loss(lo)) / (2 * eps), bar[i], rtol=1e-5, atol=1e-7)


def test_gather_of_a_skip_or_outside_key_reads_zero():
    n, cells = 500, 7
    g = np.random.default_rng(3)
    key = g.integers(-3, cells + 3, n).astype(np.int32)
    x = g.normal(size=n)
    table = g.normal(size=cells)
    bar = evaluate(E.add_sq_grad.program, {"key": key, "x": x, "bar_acc": table}, n)["bar_x"]
    inside = (key >= 0) & (key < cells)
    assert np.all(bar[~inside] == 0.0) and (~inside).sum() > 50
    assert bar[inside].tobytes() == (2 * x[inside] * table[key[inside]]).tobytes()
    with pytest.raises(HawkError, match="lookup"):
        ir.make("gather", (ir.leaf("per_sample", "t", ir.TensorType((), "f64")), ir.leaf("per_sample", "k", ir.TensorType((), "i32"))))


def _chain_case(n, cells, seed):
    g = np.random.default_rng(seed)
    x = g.normal(size=n)
    key = g.integers(-1, cells, n).astype(np.int32)          # -1: the scatter's skip key
    return g, x, key


def test_chain_vjp_through_all_three_sinks():
    """vjp(chain, wrt=x): the seeds are a plane (bar_y), a broadcast cell
    (bar_total, the reverse of a sum over samples) and a gather (bar_bins[key],
    the transpose of a keyed add).  Within 4 ulp / 1e-13 of the oracle's
    hand-derived bar_x, and central differences of the whole loss
    bar_y.y + bar_total*sum(y) + bar_bins.bins(y) agree."""
    import math
    n, cells = 2000, 13
    g, x, key = _chain_case(n, cells, 31)
    bar_y, bar_bins, bar_total = g.normal(size=n), g.normal(size=cells), 0.625
    prog = E.chain_vjp.program
    roles = {name: d.role for name, d in prog.decls.items()}
    assert roles["bar_y"] == "per_sample" and roles["bar_total"] == "uniform" and roles["bar_bins"] == "lookup"
    env = {"x": x, "key": key, "bar_y": bar_y, "bar_total": bar_total, "bar_bins": bar_bins}
    got = evaluate(prog, env, n)["bar_x"]
    want = O.chain_vjp(x, key, bar_y, bar_total, bar_bins)
    scale = O.chain_dx_scale(x) * (np.abs(bar_y) + abs(bar_total) + np.abs(bar_bins).max())
    assert np.all(np.abs(got - want) <= 1e-13 * scale + 1e-300)

    def loss(v):
        y = O.chain(v)
        bins, _ = O.ordered_scatter(key, y, np.zeros(cells))
        return math.fsum((bar_y * y).tolist()) + bar_total * math.fsum(y.tolist()) + math.fsum((bar_bins * bins).tolist())
    eps = 1e-6
    for i in np.random.default_rng(4).choice(n, 8, replace=False):
        hi, lo = x.copy(), x.copy()
        hi[i] += eps
        lo[i] -= eps
        np.testing.assert_allclose((loss(hi) - loss(lo)) / (2 * eps), got[i], rtol=1e-5, atol=1e-7)


def test_chain_jvp_keeps_the_sinks_kinds_and_policies():
    """jvp(chain, wrt=x): dot_y per sample, dot_total an ordered sum of dot_y and
    dot_bins an ordered keyed add of dot_y at the primal's key (reference
    hawk/diff/transform.py:1003-1022), planned as the same two team stages
    reading the stored dot_y."""
    from hawk_amd.emit_hip import plan_kernel
    prog = E.chain_jvp.program
    kinds = {s.name: (type(s).__name__, getattr(s, "policy", None)) for s in prog.sinks}
    assert kinds == {"dot_y": ("Assign", None), "dot_total": ("SampleSum", "ordered"),
                     "dot_bins": ("AccumWrite", "ordered")}
    p = plan_kernel(prog, "chain_jvp")
    assert sorted((t["op"], t.get("u") or t.get("v")) for t in p.team) == [("ordered_scatter", "dot_y"),
                                                                         ("ordered_sum", "dot_y")]
    n = 3000
    g, x, key = _chain_case(n, 5, 32)
    dx = g.normal(size=n)
    got = evaluate(prog, {"x": x, "key": key, "dot_x": dx}, n)
    want = O.chain_jvp(x, dx)
    scale = O.chain_dx_scale(x) * np.abs(dx)
    assert np.all(np.abs(got["dot_y"] - want) <= 1e-13 * scale + 1e-300)
    assert got["dot_total"].tobytes() == got["dot_y"].tobytes()     # the same per-sample terms
    h = 1e-6
    fd = (O.chain(x + h * dx) - O.chain(x - h * dx)) / (2 * h)
    ok = np.abs(got["dot_y"] - fd) <= 1e-5 * np.abs(fd) + 1e-7
    assert ok.mean() > 0.995                                          # central differences straddle a kink


def test_vjp_of_a_default_sum_seeds_a_broadcast():
    """vjp(sample_total): y = 2x and total = sum(x*x) give bar_x = 2 bar_y + 2x bar_total."""
    prog = vjp(E.sample_total, wrt=("x",))
    assert prog.decls["bar_total"].role == "uniform"
    n = 400
    g = np.random.default_rng(8)
    x, bar_y = g.normal(size=n), g.normal(size=n)
    got = evaluate(prog, {"x": x, "bar_y": bar_y, "bar_total": -1.25}, n)["bar_x"]
    np.testing.assert_allclose(got, 2 * bar_y + 2 * x * -1.25, rtol=1e-15, atol=1e-15)


def test_carried_reuse_keeps_the_bits_and_halves_the_leapfrog_force_evaluations():
    """The leapfrog's closing half-kick evaluates a(r') and the next substep's
    opening half-kick a(r') again; the emitter carries the first instead
    (ir.carry_repeats).  The program computes the same bits (the numpy
    interpreter, bit for bit), the loop body holds one sqrt and one division
    instead of two, and the sidecar's algorithmic count is still the traced
    program's."""
    from hawk_amd.emit_hip import _carry_repeats, fp_ops_per_sample, plan_kernel
    n = 300
    g = np.random.default_rng(12)
    d = g.normal(size=(3, n))
    d /= np.linalg.norm(d, axis=0)
    env = {"r0": d * g.uniform(0.5, 2.0, n), "v0": g.normal(0.0, 0.3, size=(3, n)), "mu": 1.1,
           "bar_r": g.normal(size=(3, n)), "bar_v": g.normal(size=(3, n))}
    for k in (E.twobody, E.twobody_vjp):
        reused = _carry_repeats(k.program)
        assert reused is not k.program
        a, b = evaluate(k.program, env, n), evaluate(reused, env, n)
        assert all(a[x].tobytes() == b[x].tobytes() for x in a), k.name
    p = plan_kernel(E.twobody.program, "twobody")
    body = p.source[p.source.index("for (long long hk_k"):]
    assert body.count("sqrt(") == 1 and body.count(" / ") == 1
    assert p.algorithmic_ops == 1280 and fp_ops_per_sample(p.source) < 900
    plain = plan_kernel(E.twobody.program, "twobody", reuse_carries=False)
    assert plain.algorithmic_ops == 1280 and plain.source.count("sqrt(") == 2


def test_carried_reuse_leaves_a_value_that_reads_the_index_alone():
    """x_{k+1} = x_k + sqrt(x_k + k): sqrt(x + k) of the next iteration reads a
    different index, so nothing is carried."""
    from hawk_amd.emit_hip import _carry_repeats

    @hawk.kernel
    def walk(x: Scalar, y: Mutable[Scalar]):
        acc = x
        for k in range(8):
            acc = acc + sqrt(acc + k)
        y = acc
    assert _carry_repeats(walk.program) is walk.program


# -- lane axes: Grid[...] and hawk.sum(x, over=...) ------------------------------------------

@hawk.kernel
def keyed_rows(lane: hawk.Grid["a", "b":8], x: Scalar, y: Mutable["a"]):
    y = hawk.sum(x, over="b", policy="ordered")


@hawk.kernel
def lane_coords(lane: hawk.Grid["a", "b":4, "c":8], y: Mutable[Scalar]):
    y = lane.a * 100.0 + lane.b * 10.0 + lane[-1] + 0.0 * lane.flat


def test_grid_axes_and_refusals_follow_the_reference():
    """Grid labels in numpy order, only the first bare; a sum over some axes
    sums the TRAILING ones only (reference tests/test_ordered_trailing_axes.py:20-38,
    same messages), under either policy."""
    assert hawk.Grid["key", "sample":8].axes == (("key", None), ("sample", 8))
    with pytest.raises(HawkError, match="only the FIRST axis may"):
        hawk.Grid["a", "b"]
    with pytest.raises(HawkError, match="duplicate"):
        hawk.Grid["a", "a":3]
    with pytest.raises(HawkError, match=r"policy='ordered' sums over the trailing lane axes only"):
        @hawk.kernel
        def leading(lane: hawk.Grid["a":4, "b":8], x: Scalar, y: Mutable["b":8]):
            y = hawk.sum(x, over="a", policy="ordered")
    with pytest.raises(HawkError, match=r"over=\('b'\)|over='b'"):
        @hawk.kernel
        def middle(lane: hawk.Grid["a", "b":4, "c":8], x: Scalar, y: Mutable["a"]):
            y = hawk.sum(x, over="b", policy="ordered")

    @hawk.kernel
    def last_two(lane: hawk.Grid["a", "b":4, "c":8], x: Scalar, y: Mutable["a"]):
        y = hawk.sum(x, over=("b", "c"), policy="ordered")
    assert [(s.name, s.group) for s in last_two.sinks] == [("y", 32)]
    # the default policy over some axes: each key's run is a default sample sum of its own
    @hawk.kernel
    def compensated(lane: hawk.Grid["a", "b":8], x: Scalar, y: Mutable["a"]):
        y = hawk.sum(x, over="b")
    assert [(s.name, s.policy, s.group) for s in compensated.sinks] == [("y", "auto", 8)]
    from hawk_amd.emit_hip import plan_kernel
    assert plan_kernel(compensated.program, "c").team == [{"op": "keyed_comp", "u": "x", "out": "y", "group": 8}]
    with pytest.raises(HawkError, match=r"policy='auto' sums over the trailing lane axes only"):
        @hawk.kernel
        def leading_default(lane: hawk.Grid["a":4, "b":8], x: Scalar, y: Mutable["b":8]):
            y = hawk.sum(x, over="a")
    with pytest.raises(HawkError, match="Grid parameter"):
        @hawk.kernel
        def no_grid(x: Scalar, y: Mutable["a"]):
            y = hawk.sum(x, over="b", policy="ordered")
    with pytest.raises(HawkError, match=r"Mutable\['a'\]"):
        @hawk.kernel
        def plain_cell(lane: hawk.Grid["a", "b":8], x: Scalar, y: Mutable[Scalar]):
            y = hawk.sum(x, over="b", policy="ordered")


def test_lane_coordinates_are_the_numpy_order_of_the_grid():
    n = 3 * 32
    got = evaluate(lane_coords.program, {}, n)["y"]
    i = np.arange(n)
    assert np.array_equal(got, (i // 32) * 100.0 + ((i // 8) % 4) * 10.0 + i % 8)


def test_keyed_sum_plans_a_keyed_team_stage_and_its_derivatives(tmp_path):
    """The keyed sum is one team stage reading x in place; its VJP gathers the
    key's adjoint (bar_y is a lookup plane of keys, key = lane // 8); its JVP
    is the keyed sum of the tangents."""
    b = hawk.build([keyed_rows], tmp_path)
    sc = b.sidecar("keyed_rows")
    assert sc["team"] == [{"op": "keyed_sum", "u": "x", "out": "y", "group": 8}]
    assert sc["planes"]["y"]["group"] == 8 and sc["grid"] == [["a", None], ["b", 8]]
    back = vjp(keyed_rows, wrt=("x",))
    assert back.decls["bar_y"].role == "lookup"
    n = 5 * 8
    bar = np.random.default_rng(1).normal(size=5)
    got = evaluate(back, {"x": np.zeros(n), "bar_y": bar}, n)["bar_x"]
    assert got.tobytes() == np.repeat(bar, 8).tobytes()
    fwd = jvp(keyed_rows, wrt=("x",))
    assert [(type(s).__name__, s.name, s.group) for s in fwd.sinks] == [("SampleSum", "dot_y", 8)]


# -- Table reads and their derivatives ------------------------------------------------------

@hawk.kernel
def table_pick(table: hawk.Table[Scalar], where: hawk.Index, x: Scalar, y: Mutable[Scalar]):
    y = table.at(where) * x + table.at(where - 1000) + table[where + 3] * table[where // 2]


@hawk.kernel
def table_grid(lane: hawk.Grid["e", "a":4], t: hawk.Table["e":8, "a":4], x: Scalar) -> Scalar:
    return t.at(e=lane.e, a=lane.a) * x + t[lane.a, lane.e] + t[lane.flat % 5]


def _scatter_eval(program, env, n, target):
    """The table gradient ``target`` of a derived program: every read site's
    per-sample contribution added at its cell (numpy's add.at)."""
    from ir_eval import Evaluator
    ev = Evaluator(env, n)
    out = np.zeros(np.asarray(env[target[4:]]).size)
    for s in program.sinks:
        if s.name == target:
            np.add.at(out, ev.value(s.key), ev.value(s.value))
    return out


def test_table_reads_clamp_every_index_into_the_table():
    """A read outside the table reads its edge (reference
    tests/test_table_clamp.py:1-8); t[i] is the flat read, t[r, c] / t.at(r=, c=)
    one index per axis in declared order; // and % on indices are Python's."""
    n = 400
    g = np.random.default_rng(5)
    table = g.normal(size=37)
    where = g.integers(-50, 90, n).astype(np.int32)
    x = g.normal(size=n)
    got = evaluate(table_pick.program, {"table": table, "where": where, "x": x}, n)["y"]
    c = lambda i: table[np.clip(i, 0, 36)]
    want = c(where) * x + c(where - 1000) + c(where + 3) * c(where // 2)
    assert got.tobytes() == want.tobytes()
    t = g.normal(size=(8, 4))
    m = 8 * 4 * 3                       # lanes past the table's first extent read its last row
    xg = g.normal(size=m)
    got = evaluate(table_grid.program, {"t": t, "x": xg}, m)["out"]
    i = np.arange(m)
    e, a = i // 4, i % 4
    want = t[np.clip(e, 0, 7), a] * xg + t[np.clip(a, 0, 7), np.clip(e, 0, 3)] + t.reshape(-1)[i % 5]
    assert got.tobytes() == want.tobytes()
    with pytest.raises(HawkError, match=r"takes one index per declared axis \['e', 'a'\], got 3"):
        @hawk.kernel
        def wrong(lane: hawk.Grid["e", "a":4], t: hawk.Table["e":8, "a":4]) -> Scalar:
            return t[lane.e, lane.a, 0]


def test_table_read_vjp_scatters_to_the_cells_read_and_matches_finite_differences():
    """vjp wrt a table: each read site adds its contribution at the cell it
    read, as an ordered scatter into bar_<table> (reference
    tests/test_diff_cross_sample.py:40-63); central differences on table
    entries agree, and wrt=x stays a per-sample gradient."""
    from hawk_amd.emit_hip import plan_kernel
    n = 300
    g = np.random.default_rng(6)
    table = g.normal(size=37)
    where = g.integers(-5, 45, n).astype(np.int32)
    x, bar_y = g.normal(size=n), g.normal(size=n)
    back = vjp(table_pick, wrt=("table", "x"))
    kinds = sorted((type(s).__name__, s.name) for s in back.sinks)
    assert kinds.count(("AccumWrite", "bar_table")) == 4 and ("Assign", "bar_x") in kinds
    env = {"table": table, "where": where, "x": x, "bar_y": bar_y}
    bar_table = _scatter_eval(back, env, n, "bar_table")

    def loss(tab):
        return float(bar_y @ evaluate(table_pick.program, {"table": tab, "where": where, "x": x}, n)["y"])
    h = 1e-6
    for cell in (0, 3, 17, 36):
        up, dn = table.copy(), table.copy()
        up[cell] += h
        dn[cell] -= h
        np.testing.assert_allclose((loss(up) - loss(dn)) / (2 * h), bar_table[cell], rtol=1e-6, atol=1e-8)
    p = plan_kernel(back, "pick_vjp")
    scatters = [t for t in p.team if t["op"] == "ordered_scatter"]
    assert len(scatters) == 4 and all(t["key"].startswith("hk_key_bar_table") for t in scatters)
    assert p.planes[scatters[0]["key"]]["dtype"] == "i32"


def test_table_read_jvp_reads_the_tangent_table():
    fwd = jvp(table_pick, wrt=("table",))
    assert fwd.decls["dot_table"].role == "lookup" and fwd.tables["dot_table"] == (("cell", None),)
    n = 200
    g = np.random.default_rng(7)
    table, dt = g.normal(size=37), g.normal(size=37)
    where = g.integers(-5, 45, n).astype(np.int32)
    x = g.normal(size=n)
    got = evaluate(fwd, {"table": table, "dot_table": dt, "where": where, "x": x}, n)["dot_y"]
    h = 1e-6
    f = lambda tab: evaluate(table_pick.program, {"table": tab, "where": where, "x": x}, n)["y"]
    np.testing.assert_allclose(got, (f(table + h * dt) - f(table - h * dt)) / (2 * h), rtol=1e-6, atol=1e-8)


def _fold_of(program, env, n, name):
    """A fold sink's gradient plane: its IR contributions and cells, folded by the oracle."""
    values, cells = evaluate(program, env, n)[name]
    group = next(s.group for s in program.sinks if s.name == name)
    for c in cells:                                 # one cell per key and slot
        assert (c.reshape(-1, group) == c.reshape(-1, group)[:, :1]).all()
    out = np.zeros(env["W"].size)
    assert O.keyed_log_fold(np.stack(values), np.stack([c[::group] for c in cells]), group, out) == 0
    return out


def test_an_ordered_keyed_sums_table_gradient_is_the_log_fold():
    """vjp of a kernel holding hawk.sum(over=..., policy="ordered") wrt a
    Table read by the kept axis (the reference's net axis,
    tests/test_net_axis.py): each read site, each iteration of the loop
    around it included, is a slot of the ordered fold (reference
    hawk/diff/ordered.py); the gradient equals the numpy loop over the nets
    (the reference's tolerance, 1e-10) and central differences of the loss."""
    from hawk_amd.emit_hip import plan_kernel
    s, k = 40, 5
    net = E.net_loss_for(s)
    back = vjp(net, wrt=("W",))
    assert [type(x).__name__ for x in back.sinks] == ["OrderedFold"]
    p = plan_kernel(back, "net_grad", fuse_folds=False)
    assert p.team == [{"op": "ordered_fold", "v": "hk_logv_bar_W", "c": "hk_logc_bar_W", "out": "bar_W",
                       "group": s, "width": E.NET_WEIGHTS}]
    assert p.planes["hk_logc_bar_W"] == {"role": "key_out", "shape": [24], "dtype": "i32", "group": s,
                                         "scratch": True}
    assert p.planes["bar_W"]["role"] == "accum_out" and p.block is None
    # 40 lanes a key fit blocks of 320 threads (8 keys): the stage folds in LDS, no log
    p = plan_kernel(back, "net_grad")
    assert p.team == [{"op": "fused_fold", "out": "bar_W", "scratch": "hk_fold_bar_W", "group": s,
                       "width": E.NET_WEIGHTS, "before": True}]
    assert p.block == 320 and not any(n.startswith("hk_log") for n in p.planes)
    assert ("accum_out", "bar_W") in p.stage.arg_spec and "__syncthreads" in p.source
    w, x, y, mask, loss, grad = net_problem(k, s, 3)
    env = {"W": w.ravel(), "mask": mask.ravel(), "x": x.ravel(), "y": y.ravel()}
    got = _fold_of(back, {**env, "bar_out": np.ones(k)}, k * s, "bar_W").reshape(k, -1)
    np.testing.assert_allclose(got, grad, rtol=1e-10, atol=1e-10)
    assert (got[np.repeat(mask == 0.0, 3, axis=1)] == 0.0).all()

    def total(wv):
        terms = evaluate(net.program, {**env, "W": wv.ravel()}, k * s)["out"]
        return O.keyed_ordered_sum(terms, s)
    np.testing.assert_allclose(total(w), loss, rtol=1e-12)
    h = 1e-6
    for net_i, col in ((0, 0), (2, 4), (4, 17), (1, 23)):
        up, dn = w.copy(), w.copy()
        up[net_i, col] += h
        dn[net_i, col] -= h
        slope = (total(up)[net_i] - total(dn)[net_i]) / (2 * h)
        assert abs(got[net_i, col] - slope) <= 1e-6 * max(1.0, abs(slope))
    # the JVP: the keyed ordered sum of the tangents
    fwd = jvp(net, wrt=("W",))
    dw = np.random.default_rng(4).normal(size=w.shape)
    dterms = evaluate(fwd, {**env, "dot_W": dw.ravel()}, k * s)["dot_out"]
    np.testing.assert_allclose(O.keyed_ordered_sum(dterms, s), (total(w + h * dw) - total(w - h * dw)) / (2 * h),
                               rtol=1e-6, atol=1e-8)


@hawk.kernel
def _by_sample(lane: hawk.Grid["key", "sample":4], t: hawk.Table[Scalar], x: Scalar) -> Scalar:
    return hawk.sum(t.at(lane.sample) * x, over="sample", policy="ordered")


@hawk.kernel
def _in_a_loop(t: hawk.Table[Scalar], where: Index, x: Scalar, y: Mutable[Scalar]):
    acc = 0.0 * x
    for j in range(3):
        acc = acc + t.at(where + j) * x
    y = acc


def test_a_table_gradient_the_fold_cannot_take_is_the_ordered_scatter():
    """A read whose cell changes within a key (here by the summed axis) is not
    one cell per key, so its gradient stays the ordered scatter (the reference
    folds it into one cell per key, hawk/diff/ordered.py:61-67, which adds
    other cells' contributions into it); so are reads in a loop of a kernel
    with no keyed sum, one scatter per read and iteration."""
    from hawk_amd.emit_hip import plan_kernel
    back = vjp(_by_sample, wrt=("t",))
    assert [type(s).__name__ for s in back.sinks] == ["AccumWrite"]
    assert [t["op"] for t in plan_kernel(back, "by_sample_vjp").team] == ["ordered_scatter"]
    back = vjp(_in_a_loop, wrt=("t",))
    assert [type(s).__name__ for s in back.sinks] == ["AccumWrite"] * 3
    n = 50
    g = np.random.default_rng(9)
    table, where, x, bar_y = g.normal(size=11), g.integers(-2, 12, n).astype(np.int32), g.normal(size=n), \
        g.normal(size=n)
    want = np.zeros(11)
    for j in range(3):
        np.add.at(want, np.clip(where + j, 0, 10), bar_y * x)
    from ir_eval import Evaluator
    ev = Evaluator({"t": table, "where": where, "x": x, "bar_y": bar_y}, n)
    got = np.zeros(11)
    for s in back.sinks:
        np.add.at(got, ev.value(s.key), ev.value(s.value))
    np.testing.assert_allclose(got, want, rtol=1e-12)


def test_a_long_loop_reading_a_differentiated_table_is_refused():
    @hawk.kernel
    def long_loop(t: hawk.Table[Scalar], x: Scalar, y: Mutable[Scalar]):
        acc = 0.0 * x
        for j in range(ir.UNROLL_MAX + 1):
            acc = acc + t.at(j) * x
        y = acc
    with pytest.raises(HawkError, match="written out for at most"):
        vjp(long_loop, wrt=("t",))
    vjp(long_loop, wrt=("x",))                  # a per-sample gradient keeps the loop rolled


def _long_double_chain(x):
    """acc and y of the chain members in long double (the oracle of the chain tests)."""
    ld = np.longdouble
    x = x.astype(ld)
    a = np.stack([np.sin(x), np.cos(x), x * ld("0.5")])
    b = np.exp(-(a * a).sum(axis=0)) + x
    return a, b


def test_chain_binds_members_by_name_and_stores_no_intermediate():
    """hawk.chain (reference tests/test_chain.py:180-194): the composed kernel
    binds x and acc and commits acc and y; a and b stay in the kernel; a chain
    of chains is the chain of its members; the composed values are the
    members' run one after another, bit for bit (same operations)."""
    import chain_members as C
    from hawk_amd.emit_hip import plan_kernel
    chained = hawk.chain(*C.MEMBERS, name="fixture")
    assert {n for _, n in chained.arg_spec} == {"x", "acc", "y"}
    assert chained.outputs == ("acc", "y") and chained.members == C.MEMBERS
    nested = hawk.chain(hawk.chain(C.unit_circle, C.decay, name="front"), C.accumulate, C.scale_vec, name="fixture")
    assert nested.members == C.MEMBERS
    assert plan_kernel(nested.program, "k").source == plan_kernel(chained.program, "k").source
    assert [t for t in plan_kernel(chained.program, "k").planes] and \
        set(plan_kernel(chained.program, "k").planes) == {"x", "acc", "y"}
    n = 257
    g = np.random.default_rng(5)
    x, acc = g.uniform(0.1, 2.0, n), g.uniform(0.0, 1.0, n)
    got = evaluate(chained.program, {"x": x, "acc": acc}, n)
    a = evaluate(C.unit_circle.program, {"x": x}, n)["a"]
    b = evaluate(C.decay.program, {"a": a, "x": x}, n)["b"]
    want_acc = evaluate(C.accumulate.program, {"b": b, "acc": acc}, n)["acc"]
    want_y = evaluate(C.scale_vec.program, {"a": a, "b": b}, n)["y"]
    assert got["acc"].tobytes() == want_acc.tobytes() and got["y"].tobytes() == want_y.tobytes()
    la, lb = _long_double_chain(x)
    np.testing.assert_allclose(got["y"], (la * lb).astype(np.float64), rtol=1e-14)


def test_a_chain_build_records_its_members_estimate_and_fence(tmp_path):
    """The build fuses every boundary (the reference does on a GPU,
    hawk/ir/fusion.py:10) and records the register estimate R0 + 2 maxlive
    and the fence 1.6 est + 16 against the compiled kernel's VGPRs."""
    import json

    import chain_members as C
    from hawk_amd.chaining import R0, estimate, fence, maxlive
    chained = hawk.chain(*C.MEMBERS, name="fixture")
    assert maxlive(chained.program) == 8            # x, acc, the three of a and y's three at the end
    assert estimate(chained.program) == R0 + 16
    hawk.build([chained], tmp_path)
    side = json.loads((tmp_path / "fixture.json").read_text())
    assert side["chain"]["members"] == ["unit_circle", "decay", "accumulate", "scale_vec"]
    assert side["chain"]["outputs"] == ["acc", "y"] and side["chain"]["estimate_vgprs"] == R0 + 16
    vgprs = side["resources"]["vgpr_count"]
    assert side["chain"]["within_fence"] is fence(vgprs, 0, R0 + 16) is True
    assert not fence(200, 0, 40) and fence(80, 0, 40)


def test_chain_refusals_name_both_members_and_the_name():
    """The reference's refusals, by text (tests/test_chain.py:196-242)."""
    import chain_members as C
    with pytest.raises(HawkError, match=r"'unit_circle' commits 'a' .* but 'flat_a' reads it"):
        hawk.chain(C.unit_circle, C.flat_a, name="c")
    with pytest.raises(HawkError, match=r"'decay' and 'blind_b' both commit 'b'"):
        hawk.chain(C.unit_circle, C.decay, C.blind_b, name="c")
    with pytest.raises(HawkError, match=r"members 'unit_circle' and 'on_grid' disagree on grid"):
        hawk.chain(C.unit_circle, C.on_grid, name="c")
    with pytest.raises(HawkError, match=r"'pick' reads 'table', which 'fill' commits, at another sample"):
        hawk.chain(C.fill, C.pick, name="c")
    with pytest.raises(HawkError, match=r"'reads_total' reads 't', which 'total_of' commits, at another sample"):
        hawk.chain(C.total_of, C.reads_total, name="c")
    with pytest.raises(HawkError, match="give at least one kernel"):
        hawk.chain(name="c")


@pytest.mark.parametrize("direction", ["jvp", "vjp"])
def test_chain_derivatives_are_the_composed_programs(direction):
    """The derivative of a chain (reference tests/test_chain.py:497-511) is
    the derivative of its composed program: against the long-double chain
    rule and central differences of the chain's value."""
    import chain_members as C
    members = (C.unit_circle, C.decay, C.scale_vec)
    chained = hawk.chain(*members, name="dchain")
    n = 300
    g = np.random.default_rng(11)
    x = g.uniform(0.2, 1.5, n)
    seed = g.uniform(0.5, 1.5, (3, n))
    ld = np.longdouble
    la, lb = _long_double_chain(x)
    da = np.stack([np.cos(x.astype(ld)), -np.sin(x.astype(ld)), np.full(n, ld("0.5"))])
    db = np.exp(-(la * la).sum(axis=0)) * (-2 * (la * da).sum(axis=0)) + 1
    tangent = da * lb + la * db                  # dy/dx, (3, n)
    if direction == "jvp":
        got = evaluate(jvp(chained, wrt=("x",)), {"x": x, "dot_x": np.ones(n)}, n)["dot_y"]
        ref = tangent
    else:
        got = evaluate(vjp(chained, wrt=("x",)), {"x": x, "bar_y": seed}, n)["bar_x"]
        ref = (seed.astype(ld) * tangent).sum(axis=0)
    np.testing.assert_allclose(got, ref.astype(np.float64), rtol=1e-13, atol=1e-15)
    h = 1e-6
    yv = lambda xv: evaluate(chained.program, {"x": xv}, n)["y"]
    fd = (yv(x + h) - yv(x - h)) / (2 * h)
    fd = fd if direction == "jvp" else (seed * fd).sum(axis=0)
    assert np.max(np.abs(got - fd)) / np.max(np.abs(fd)) < 1e-8
    # every member's read of x is one input, so the derivative reaches all of them
    assert len({id(n) for n in ir.leaves_of(ir.sink_roots(chained.sinks)) if n.literal[1] == "x"}) == 1


def test_a_chain_past_the_register_line_is_cut_into_segments(tmp_path):
    """The cut rule (reference hawk/ir/fusion.py:95-121): at the spill line
    the example chain fuses whole; with a line of 32 registers every boundary
    is cut, each segment a kernel of its own, the values passing through
    hwc_ planes; the segments composed give the fused chain's values, bit for
    bit (the same operations)."""
    import json

    import chain_members as C
    from hawk_amd import chaining as CH
    chained = hawk.chain(*C.MEMBERS, name="fixture")
    assert CH.cuts(C.MEMBERS) == [] and CH.cuts(C.MEMBERS, line=32) == [1, 2, 3]
    segs = CH.segments(C.MEMBERS, [1, 2, 3])
    assert [(w, r) for _, w, r in segs] == [(["hwc_a"], []), (["hwc_b"], ["hwc_a"]), ([], ["hwc_b"]),
                                            ([], ["hwc_a", "hwc_b"])]
    n = 101
    g = np.random.default_rng(2)
    x, acc0 = g.uniform(0.1, 2.0, n), g.uniform(0.0, 1.0, n)
    env = {"x": x, "acc": acc0}
    for prog, _, _ in segs:                     # each segment reads the planes the earlier ones wrote
        env = {**env, **evaluate(prog, env, n)}
    fused = evaluate(chained.program, {"x": x, "acc": acc0}, n)
    assert env["y"].tobytes() == fused["y"].tobytes() and env["acc"].tobytes() == fused["acc"].tobytes()
    hawk.build([chained], tmp_path, register_line=32)
    side = json.loads((tmp_path / "fixture.json").read_text())
    assert side["segments"] == ["fixture__s0", "fixture__s1", "fixture__s2", "fixture__s3"]
    assert side["crossing"] == {"hwc_a": {"shape": [3], "dtype": "f64"}, "hwc_b": {"shape": [], "dtype": "f64"}}
    assert set(side["planes"]) == {"x", "acc", "y"} and side["cuts"] == [1, 2, 3]


def test_a_chain_passes_params_tables_and_grids_through(tmp_path):
    """Members on one Grid, reading a Param and a Table, chain like any
    others: the Param and the Table stay inputs of the chain, the keyed sum
    of the last member reads the first member's per-lane value, and the
    composed values are the members' run in turn."""
    from hawk_amd import Grid, Param, Table

    @hawk.kernel
    def weigh(lane: Grid["key", "s":4], w: Table["key", "j":2], x: Scalar, scale: Param, u: Mutable[Scalar]):
        u = w.at(key=lane.key, j=0) * x * scale + w.at(key=lane.key, j=1)

    @hawk.kernel
    def total(lane: Grid["key", "s":4], u: Scalar) -> Scalar:
        return hawk.sum(u * u, over="s", policy="ordered")

    chained = hawk.chain(weigh, total, name="wt")
    assert {n for _, n in chained.arg_spec} == {"w", "x", "scale", "out"}
    assert chained.program.tables == {"w": (("key", None), ("j", 2))}
    n = 40
    g = np.random.default_rng(4)
    w, x = g.normal(size=20), g.normal(size=n)
    got = evaluate(chained.program, {"w": w, "x": x, "scale": 1.5}, n)["out"]
    u = evaluate(weigh.program, {"w": w, "x": x, "scale": 1.5}, n)["u"]
    assert got.tobytes() == (u * u).tobytes()
    back = vjp(chained, wrt=("w",))                 # the keyed sum is ordered: the table's gradient folds
    assert [type(s).__name__ for s in back.sinks] == ["OrderedFold"]


def test_the_banded_mode_plans_band_stages_and_refuses_what_it_cannot_fold():
    """mode="banded": the default-policy sums' rows fold double-double bands in
    the stage (hk_band_row_sum) and in the finish (band_rows), the ordered sum
    is the banded fixed tree (band_ordered_sum); a keyed sum or a scatter is
    refused by name (the reference refuses the reductions its banded build
    cannot certify, hawk/emit/wrapper.py:158-196)."""
    from hawk_amd.emit_hip import plan_kernel
    p = plan_kernel(E.band_total.program, "band_total", mode="banded")
    assert [(t["op"], t["out"]) for t in p.team] == [("band_rows", "s"), ("band_rows", "s_sq"),
                                                     ("band_ordered_sum", "s_ord")]
    assert "hk_band_row_sum(hk_rh, hk_rc);" in p.source and "hk_row_sum(" not in p.source
    assert "typedef double Real;" in p.source
    f64 = plan_kernel(E.band_total.program, "band_total", mode="float64")
    assert [t["op"] for t in f64.team] == ["row_sum", "row_sum", "ordered_sum"] and "hk_band" not in f64.source
    with pytest.raises(HawkError, match="hawk.scatter\\(acc\\) has no banded stage"):
        plan_kernel(E.ordered_add.program, "ordered_add", mode="banded")
    with pytest.raises(HawkError, match="'float64', 'float32' or 'banded'"):
        plan_kernel(E.band_total.program, "band_total", mode="float16")


def test_a_banded_build_records_its_mode_and_binds_float64_cells(tmp_path):
    b = hawk.build([E.band_total], tmp_path, mode="banded")
    side = b.sidecar("band_total")
    assert side["mode"] == "banded" and {t["op"] for t in side["team"]} == {"band_rows", "band_ordered_sum"}
    assert all(side["planes"][c] == {"role": "cell", "shape": [], "dtype": "f64"} for c in ("s", "s_sq", "s_ord"))


# -- the build cache (reference hawk/compile/cache.py:347-459, hawk/artifact/bundle.py:1497-1575) ------

def _unit_bytes(directory):
    return {p.name: p.read_bytes() for p in sorted(directory.iterdir()) if p.suffix in (".hsaco", ".json", ".hip")}


def test_a_second_build_is_all_hits_and_publishes_the_same_bytes(tmp_path):
    from hawk_amd import compile as C
    cache = tmp_path / "cache"
    kernels = [E.scale, E.energy, E.energy_vjp, E.chain]
    before = C.cache_stats()
    hawk.build(kernels, tmp_path / "a", cache_dir=cache)
    mid = C.cache_stats()
    assert mid["misses"] - before["misses"] == 4 and mid["hits"] == before["hits"]
    hawk.build(kernels, tmp_path / "b", cache_dir=cache)
    after = C.cache_stats()
    assert after["hits"] - mid["hits"] == 4 and after["misses"] == mid["misses"]
    a, b = _unit_bytes(tmp_path / "a"), _unit_bytes(tmp_path / "b")
    assert sorted(a) == sorted(b) and "manifest.json" in a
    assert all(a[name] == b[name] for name in a)          # code objects, sidecars and manifest, byte for byte


def test_a_changed_option_or_toolchain_misses(tmp_path, monkeypatch):
    from hawk_amd import compile as C
    from hawk_amd.emit_hip import plan_kernel
    cache = tmp_path / "cache"
    src = plan_kernel(E.scale.program, "scale").source
    _, key, hit = C.compile_source(src, "scale", cache_dir=cache)
    assert not hit
    assert C.compile_source(src, "scale", cache_dir=cache)[2]                       # the same: a hit
    _, key2, hit2 = C.compile_source(src, "scale", options=C.RTC_OPTIONS + ("-DHAWK_PROBE=1",), cache_dir=cache)
    assert not hit2 and key2 != key
    real = C.toolchain()
    monkeypatch.setattr(C, "toolchain", lambda: real + ";another-comgr")
    _, key3, hit3 = C.compile_source(src, "scale", cache_dir=cache)
    assert not hit3 and key3 not in (key, key2)


@pytest.mark.parametrize("damage", ["truncate", "flip", "no_record"])
def test_a_damaged_cache_entry_is_rebuilt_not_loaded(tmp_path, damage):
    from hawk_amd import compile as C
    from hawk_amd.emit_hip import plan_kernel
    cache = tmp_path / "cache"
    src = plan_kernel(E.energy.program, "energy").source
    code, key, _ = C.compile_source(src, "energy", cache_dir=cache)
    obj, record = cache / f"{key}.hsaco", cache / f"{key}.json"
    if damage == "truncate":
        obj.write_bytes(code[: len(code) // 2])
    elif damage == "flip":
        obj.write_bytes(code[:100] + bytes([code[100] ^ 1]) + code[101:])
    else:
        record.unlink()
    again, key2, hit = C.compile_source(src, "energy", cache_dir=cache)
    assert not hit and key2 == key and again == code       # rebuilt, the same code object
    assert obj.read_bytes() == code and C.compile_source(src, "energy", cache_dir=cache)[2]


def test_the_references_build_options_are_taken(tmp_path):
    """hawk.build accepts the reference's options (reference
    hawk/artifact/bundle.py:1349-1420): launch_bounds fixes the block,
    opt_level and defines reach hipRTC, the forms and the rest are recorded,
    name goes into the manifest and derivative names a kernel's primal."""
    import json
    b = hawk.build([E.scale, E.energy], tmp_path, emit_form="static", linalg_form="team", wide_form="thread",
                   launch_bounds=(128, 2), opt_level="O2", defines=("HAWK_PROBE=1",), name="unit",
                   derivative={"energy": "scale"}, host_profile="native", literal_table=True)
    sc = b.sidecar("scale")
    assert sc["launch"]["block"] == 128
    # blocks=2 of 128 threads: 4 waves a CU, one per SIMD, the default; 8 of 256 ask for 8 waves a SIMD
    assert "waves_per_eu" not in sc["launch"] and "__launch_bounds__(128)" in (tmp_path / "scale.hip").read_text()
    dense = hawk.build([E.scale], tmp_path / "dense", launch_bounds=(256, 8)).sidecar("scale")
    assert dense["launch"]["waves_per_eu"] == 8
    assert "__launch_bounds__(256, 8)" in (tmp_path / "dense" / "scale.hip").read_text()
    assert "-O2" in sc["compile_options"] and "-O3" not in sc["compile_options"]
    assert "-DHAWK_PROBE=1" in sc["compile_options"]
    assert sc["build_options"] == {"emit_form": "static", "linalg_form": "team", "wide_form": "thread",
                                   "launch_bounds": [128, 2], "host_profile": "native", "opt_level": "O2",
                                   "literal_table": True, "defines": ["HAWK_PROBE=1"]}
    assert b.sidecar("energy")["primal"] == "scale" and "primal" not in sc
    assert json.loads((tmp_path / "manifest.json").read_text())["name"] == "unit"
    plain = hawk.build([E.scale], tmp_path / "plain")
    assert "build_options" not in plain.sidecar("scale") and "-O3" in plain.sidecar("scale")["compile_options"]


@pytest.mark.parametrize("kw, says", [
    ({"kind": object()}, "execution kind"),
    ({"layout_sizes_override": [40, 32, 32, 8, 24]}, "test-only door"),
    ({"embedded_profile": object()}, "MISRA C"),
    ({"device_arch": "sm_90"}, "builds gfx950"),
    ({"emit_form": "unrolled"}, "emit_form must be one of"),
    ({"linalg_form": "warp"}, "linalg_form must be one of"),
    ({"wide_form": "lane"}, "wide_form must be one of"),
    ({"opt_level": "O4"}, "opt_level must be one of"),
    ({"host_profile": "fast"}, "host_profile must be one of"),
    ({"launch_bounds": (96, 2)}, "multiple of 64"),
    ({"launch_bounds": (1024, 4)}, "threads*blocks <= 2048"),
    ({"defines": ("-O0",)}, "NAME or NAME=VALUE"),
])
def test_the_references_build_options_are_refused_by_name(tmp_path, kw, says):
    import re
    with pytest.raises(hawk.HawkError, match=re.escape(says)):
        hawk.build([E.scale], tmp_path, **kw)


def test_ambient_options_reach_the_build_and_an_explicit_one_wins(tmp_path):
    """reference tests/test_ambient_policy.py:26-32: launch_bounds from
    policy.using reaches a build inside the block, an explicit argument wins,
    and a build outside the block has none; contraction is recorded."""
    from hawk_amd import policy
    with policy.using(launch_bounds=(128, 2), contraction="gemm", form="rolled"):
        amb = hawk.build([E.scale], tmp_path / "a").sidecar("scale")
        exp = hawk.build([E.scale], tmp_path / "b", launch_bounds=(64, 4)).sidecar("scale")
    plain = hawk.build([E.scale], tmp_path / "c").sidecar("scale")
    assert amb["launch"]["block"] == 128 and amb["build_options"]["launch_bounds"] == [128, 2]
    assert amb["build_options"]["contraction"] == "gemm" and amb["build_options"]["emit_form"] == "rolled"
    assert exp["launch"]["block"] == 64 and exp["build_options"]["launch_bounds"] == [64, 4]
    assert "build_options" not in plain and (plain["launch"]["block"], plain["launch"]["per_thread"]) == (64, 2)
    # (scale's own shape: pairs of adjacent samples)
    with pytest.raises(hawk.HawkError, match="contraction must be one of"):
        with policy.using(contraction="blas"):
            pass


def test_light_scalar_streams_run_in_pairs_of_adjacent_samples(tmp_path):
    """A light stream whose planes are all scalar float64 planes (``scale``)
    builds 64 threads of a pair of adjacent samples, each plane read and
    written 16 bytes a lane behind an alignment test, with the one-sample
    loop after it; at an even number of samples a thread the pair form is
    taken whatever the block; the float32 mode, an odd number of samples a
    thread and a stage with a vector plane keep one sample a lane."""
    sc = hawk.build([E.scale], tmp_path / "a").sidecar("scale")
    assert (sc["launch"]["block"], sc["launch"]["per_thread"]) == (64, 2)
    src = (tmp_path / "a" / "scale.hip").read_text().split('extern "C" __global__')[-1]
    assert "const hk_d2 hk_pair_hk_p_x = __builtin_nontemporal_load(reinterpret_cast<const hk_d2*>(&hk_p_x[hk_i0]))" in src
    assert "__builtin_nontemporal_store(hk_st0, reinterpret_cast<hk_d2*>(&hk_p_out[hk_i0]))" in src
    assert "& 15ull) == 0 && (base & 1LL) == 0" in src
    assert "if (hk_flat >= count) break;" in src                   # the one-sample loop after the pairs
    hawk.build([E.scale], tmp_path / "b", block=256, per_thread=4)
    assert "hk_pair_" in (tmp_path / "b" / "scale.hip").read_text()
    for d, kw in (("c", {"mode": "float32"}), ("d", {"per_thread": 3})):
        sc = hawk.build([E.scale], tmp_path / d, **kw).sidecar("scale")
        assert "hk_pair_" not in (tmp_path / d / "scale.hip").read_text(), kw
    assert sc["launch"]["per_thread"] == 3
    hawk.build([E.energy], tmp_path / "e", block=64, per_thread=2)
    assert "hk_pair_" not in (tmp_path / "e" / "energy.hip").read_text()   # a Vector[3] plane
