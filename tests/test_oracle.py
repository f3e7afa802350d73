"""Pins the CPU oracle (oracle/hawk_oracle.c) before it is trusted as the
parity checker: the reference's golden vectors, closed forms, brute force,
numpy/LAPACK, finite differences and invariants — each chosen so a plausible
mistake (a dropped term, a wrong sign, a transposed operand, a wrong index,
a changed order) fails one of them."""

from __future__ import annotations

import numpy as np
import pytest

import oracle_lib as O
from conftest import golden, within_contract


def tree_sum(x: np.ndarray) -> float:
    """The fixed tree in NumPy (reference tests/test_ordered_fixed_tree.py:25-40)."""
    V, W, G = 65536, 1024, 64
    part = np.zeros(V, x.dtype)
    for r in range(0, len(x), V):
        row = x[r:r + V]
        part[:len(row)] += row

    def tree(s):
        s = s.copy()
        w = len(s) // 2
        while w:
            s[:w] += s[w:2 * w]
            w //= 2
        return s[0]
    return tree(np.array([tree(part[g * W:(g + 1) * W]) for g in range(G)], x.dtype))


def test_energy_readme_golden_vectors():
    ga = golden("energy_readme")
    v = np.array(ga["v"])
    assert O.energy(v).tolist() == ga["energy"]
    assert O.energy_vjp(v, np.array(ga["bar_out"])).tolist() == ga["bar_v"]


def test_energy_closed_forms():
    g = np.random.default_rng(0)
    v, dv, bo = g.normal(size=(3, 999)), g.normal(size=(3, 999)), g.normal(size=999)
    assert O.energy(v).tobytes() == (0.5 * (((v[0] * v[0]) + (v[1] * v[1])) + (v[2] * v[2]))).tobytes()
    assert O.energy_vjp(v, bo).tobytes() == (bo * v).tobytes()          # 2*((0.5 b) v) == b v exactly
    d = ((dv[0] * v[0]) + (dv[1] * v[1])) + (dv[2] * v[2])
    assert O.energy_jvp(v, dv).tobytes() == d.tobytes()                   # 0.5*(d + d) == d exactly


def test_scale_is_one_mul_and_one_add():
    x = np.random.default_rng(1).uniform(-1, 1, 1000)
    assert O.scale(x, 2.0, 1.0).tobytes() == ((2.0 * x) + 1.0).tobytes()


@pytest.mark.parametrize("n", golden("ordered_sum_sizes")["sizes"])
def test_ordered_sum_is_the_numpy_tree(n):
    g = np.random.default_rng(n)
    x = g.normal(size=n) * np.exp(g.normal(size=n))
    assert O.ordered_sum(x) == tree_sum(x)
    assert O.ordered_sum(x, threads=6) == tree_sum(x)


def test_ordered_sum_small_cases():
    assert O.ordered_sum(np.zeros(0)) == 0.0
    assert O.ordered_sum(np.array([3.5])) == 3.5
    x = np.arange(1.0, 70001.0)
    assert O.ordered_sum(x) == 70000 * 70001 / 2


def test_scatter_chunk_rule():
    ga = golden("scatter_chunks")
    assert [O.scatter_chunks(n, t) for n, t in ga["cases"]] == ga["chunks"]


@pytest.mark.parametrize("n, cells, heavy", golden("ordered_scatter_cases")["cases"])
def test_ordered_scatter_equals_add_at_and_replays(n, cells, heavy):
    ga = golden("ordered_scatter_cases")
    g = np.random.default_rng(n)
    key = g.integers(0, cells, n).astype(np.int32)
    if heavy:
        key[g.random(n) < 0.9] = cells // 2
    empty = ga["empty_cell"]
    if cells == empty["cells"]:
        key[key == empty["moved_from"]] = empty["moved_to"]
    x = g.normal(size=n) * np.exp(g.normal(size=n))
    want = np.zeros(cells)
    np.add.at(want, key, x)
    a, sa = O.ordered_scatter(key, x, np.zeros(cells))
    b, _ = O.ordered_scatter(key, x, np.zeros(cells), threads=4)
    assert a.tobytes() == b.tobytes()
    assert not sa[1:].any() and sa[0] == cells
    np.testing.assert_allclose(a, want, rtol=ga["rtol"], atol=ga["rtol"] * np.abs(want).max())
    if cells == empty["cells"]:
        assert a[empty["moved_from"]] == 0.0
    base = np.linspace(1.0, 2.0, cells)             # the sum adds onto what the plane held
    more, _ = O.ordered_scatter(key, x, base)
    np.testing.assert_allclose(more - base, a, rtol=1e-9, atol=1e-9 * np.abs(a).max())


def test_ordered_scatter_is_the_serial_chunk_walk():
    """Brute force in Python over a small case: per-(key, chunk) sums in lane order
    from 0, then per cell in chunk order from 0, added onto the target."""
    g = np.random.default_rng(3)
    n, cells = 2000, 9
    key = g.integers(-1, cells + 2, n).astype(np.int32)
    x = g.normal(size=n)
    base = g.normal(size=cells)
    chunks = O.scatter_chunks(n, cells)
    span = -(-n // chunks)
    parts = [[0.0] * chunks for _ in range(cells)]
    bad = [0] * chunks
    for r in range(n):
        b, k = r // span, int(key[r])
        if k == -1:
            continue
        if 0 <= k < cells:
            parts[k][b] = parts[k][b] + float(x[r])
        else:
            bad[b] = 1
    want = base.copy()
    for c in range(cells):
        s = 0.0
        for b in range(chunks):
            s = s + parts[c][b]
        want[c] = want[c] + s
    got, status = O.ordered_scatter(key, x, base)
    assert got.tobytes() == want.tobytes()
    assert list(status[1:1 + chunks]) == bad


@pytest.mark.parametrize("which, lo, hi", [("exp", -30, 30), ("sin", 0.01, 200), ("tanh", -3, 3), ("sqrt", 0, 9)])
def test_libm_is_close_to_numpy(which, lo, hi):
    x = np.random.default_rng(2).uniform(lo, hi, 10000)
    want = {"exp": np.exp, "sin": np.sin, "tanh": np.tanh, "sqrt": np.sqrt}[which](x)
    ulps = np.abs(O.libm(which, x) - want) / np.spacing(np.abs(want))
    assert ulps.max() <= 2.0      # two libms, each within an ulp of the true value


def _twobody_inputs(n, seed):
    g = np.random.default_rng(seed)
    d = g.normal(size=(3, n))
    d /= np.linalg.norm(d, axis=0)
    return d * g.uniform(0.5, 2.0, n), g.normal(0.0, 0.3, size=(3, n))


def test_twobody_conserves_energy_and_angular_momentum():
    r0, v0 = _twobody_inputs(200, 3)
    r, v = O.twobody(r0, v0, 1.0)

    def energy(r, v):
        return 0.5 * (v * v).sum(0) - 1.0 / np.linalg.norm(r, axis=0)
    drift = np.abs(energy(r, v) - energy(r0, v0)) / np.abs(energy(r0, v0))
    assert drift.max() < 1e-5
    L0, L1 = np.cross(r0.T, v0.T), np.cross(r.T, v.T)
    np.testing.assert_allclose(L1, L0, rtol=1e-12, atol=1e-13)


def test_twobody_matches_a_numpy_leapfrog():
    """The same KDK step in numpy (vectorised): a transposed or dropped term fails."""
    r0, v0 = _twobody_inputs(100, 4)
    r, v = r0.copy(), v0.copy()
    dt = 1e-3
    for _ in range(32):
        r2 = ((r[0] * r[0]) + (r[1] * r[1])) + (r[2] * r[2])
        a = (-1.0 / (r2 * np.sqrt(r2))) * r
        vh = v + (0.5 * dt) * a
        r = r + dt * vh
        r2 = ((r[0] * r[0]) + (r[1] * r[1])) + (r[2] * r[2])
        a = (-1.0 / (r2 * np.sqrt(r2))) * r
        v = vh + (0.5 * dt) * a
    wr, wv = O.twobody(r0, v0, 1.0)
    assert wr.tobytes() == r.tobytes() and wv.tobytes() == v.tobytes()


def test_twobody_vjp_is_the_transposed_jacobian():
    n = 20
    r0, v0 = _twobody_inputs(n, 5)
    g = np.random.default_rng(6)
    br, bv = g.normal(size=(3, n)), g.normal(size=(3, n))
    gr0, gv0 = O.twobody_vjp(r0, v0, 1.0, br, bv)
    h = 1e-6
    for name in ("r0", "v0"):
        for c in range(3):
            e = np.zeros((3, n))
            e[c] = h

            def loss(sign):
                a = r0 + sign * e if name == "r0" else r0
                b = v0 + sign * e if name == "v0" else v0
                r, v = O.twobody(np.ascontiguousarray(a), np.ascontiguousarray(b), 1.0)
                return (br * r).sum(0) + (bv * v).sum(0)
            fd = (loss(1) - loss(-1)) / (2 * h)
            got = (gr0 if name == "r0" else gv0)[c]
            np.testing.assert_allclose(got, fd, rtol=1e-6, atol=1e-8)


def _spd(n, seed):
    g = np.random.default_rng(seed)
    B = g.normal(size=(n, 6, 6))
    A = np.matmul(B, B.transpose(0, 2, 1)) + 6.0 * np.eye(6)
    b = g.normal(size=(n, 6))
    return A, b, np.ascontiguousarray(A.transpose(1, 2, 0)), np.ascontiguousarray(b.T)


def test_spd_solve_matches_lapack():
    A, b, Ap, bp = _spd(500, 1)
    x = O.spd_solve(Ap, bp)
    want = np.linalg.solve(A, b[..., None])[..., 0].T
    np.testing.assert_allclose(x, want, rtol=1e-12, atol=1e-13)
    resid = np.matmul(A, x.T[..., None])[..., 0] - b
    assert np.abs(resid).max() < 1e-12


def test_spd_solve_refuses_an_indefinite_matrix_with_zeros():
    A = np.eye(6)[..., None].repeat(2, axis=2).copy()
    A[3, 3, 1] = -1.0
    b = np.ones((6, 2))
    x = O.spd_solve(np.ascontiguousarray(A), b)
    assert np.all(x[:, 0] == 1.0) and np.all(x[:, 1] == 0.0)


def test_spd_vjp_closed_form_and_finite_differences():
    A, b, Ap, bp = _spd(40, 2)
    bar_x = np.random.default_rng(3).normal(size=(6, 40))
    bA, bb = O.spd_solve_vjp(Ap, bp, bar_x)
    lam = np.linalg.solve(A.transpose(0, 2, 1), bar_x.T[..., None])[..., 0]     # A^T lam = g (A symmetric)
    np.testing.assert_allclose(bb, lam.T, rtol=1e-11, atol=1e-13)
    x = np.linalg.solve(A, b[..., None])[..., 0]
    outer = lam[:, :, None] * x[:, None, :]
    want = -0.5 * (outer + outer.transpose(0, 2, 1))
    np.testing.assert_allclose(bA, want.transpose(1, 2, 0), rtol=1e-10, atol=1e-13)
    h = 1e-6
    for i, j in ((0, 0), (1, 4), (5, 2)):
        e = np.zeros_like(Ap)
        e[i, j] = h
        e[j, i] = h if i != j else h
        fd = ((bar_x * O.spd_solve(Ap + e, bp)).sum(0) - (bar_x * O.spd_solve(Ap - e, bp)).sum(0)) / (2 * h)
        got = bA[i, j] + (bA[j, i] if i != j else 0.0)
        np.testing.assert_allclose(got, fd, rtol=1e-6, atol=1e-9)


def test_mm16_brute_force_and_vjp():
    g = np.random.default_rng(8)
    n = 50
    A = g.normal(0, 0.25, size=(16, 16, n)).astype(np.float32)
    B = g.normal(0, 0.25, size=(16, 16, n)).astype(np.float32)
    G = g.normal(0, 0.25, size=(16, 16, n)).astype(np.float32)
    C = O.mm16(A, B)
    want = np.einsum("ikn,kjn->ijn", A.astype(np.float64), B.astype(np.float64))
    scale = np.einsum("ikn,kjn->ijn", np.abs(A).astype(np.float64), np.abs(B).astype(np.float64))
    assert np.all(np.abs(C - want) <= 1e-6 * scale + 1e-30)
    # the rolled order: k ascending, from the first product
    acc = A[0, 0] * B[0, 0]
    for k in range(1, 16):
        acc = acc + A[0, k] * B[k, 0]
    assert C[0, 0].tobytes() == acc.tobytes()
    bA, bB = O.mm16_vjp(A, B, G)
    wA = np.einsum("ikn,jkn->ijn", G.astype(np.float64), B.astype(np.float64))
    wB = np.einsum("kin,kjn->ijn", A.astype(np.float64), G.astype(np.float64))
    np.testing.assert_allclose(bA, wA, rtol=1e-4, atol=1e-5)
    np.testing.assert_allclose(bB, wB, rtol=1e-4, atol=1e-5)


def test_mm16_f64_is_exact_on_integers_and_within_the_dot_bound():
    """The float64 products: on small integers every product and partial sum
    is exact, so C, bar_A and bar_B must equal the integer products bit for
    bit (a dropped term, a swapped index or a missing transpose changes them);
    on normal inputs each element lies within gamma_15 * sum |a||b| of the
    product in long double (the textbook bound of a 16-term dot product)."""
    g = np.random.default_rng(18)
    n = 40
    Ai, Bi, Gi = (g.integers(-8, 9, size=(16, 16, n)) for _ in range(3))
    A, B, G = (x.astype(np.float64) for x in (Ai, Bi, Gi))
    assert (O.mm16(A, B) == np.einsum("ikn,kjn->ijn", Ai, Bi)).all()
    bA, bB = O.mm16_vjp(A, B, G)
    assert (bA == np.einsum("ikn,jkn->ijn", Gi, Bi)).all()
    assert (bB == np.einsum("kin,kjn->ijn", Ai, Gi)).all()
    A, B, G = (g.normal(0, 0.25, size=(16, 16, n)) for _ in range(3))
    gamma = 15 * 2.0 ** -53 / (1 - 15 * 2.0 ** -53)
    L = np.longdouble
    want = np.einsum("ikn,kjn->ijn", A.astype(L), B.astype(L))
    scale = np.einsum("ikn,kjn->ijn", np.abs(A), np.abs(B))
    assert (np.abs(O.mm16(A, B).astype(L) - want) <= gamma * scale).all()
    bA, bB = O.mm16_vjp(A, B, G)
    assert (np.abs(bA.astype(L) - np.einsum("ikn,jkn->ijn", G.astype(L), B.astype(L)))
            <= gamma * np.einsum("ikn,jkn->ijn", np.abs(G), np.abs(B))).all()
    assert (np.abs(bB.astype(L) - np.einsum("kin,kjn->ijn", A.astype(L), G.astype(L)))
            <= gamma * np.einsum("kin,kjn->ijn", np.abs(A), np.abs(G))).all()


def test_threaded_tiles_are_the_serial_bits():
    x = np.random.default_rng(9).normal(size=100_003)
    assert O.chain(x, threads=7).tobytes() == O.chain(x).tobytes()
    r0, v0 = _twobody_inputs(1001, 7)
    a = O.twobody(r0, v0, 1.0)
    b = O.twobody(r0, v0, 1.0, threads=5)
    assert a[0].tobytes() == b[0].tobytes() and a[1].tobytes() == b[1].tobytes()


# -- the default-policy sample sum (compensated rows, canonical finish) ------

def _ulp(x):
    return np.spacing(np.abs(np.float64(x)))


@pytest.mark.parametrize("n", [1, 31, 32, 33, 1000, 65536])
def test_row_sums_equal_the_float64_reference(n):
    """Each row's hi + comp equals the float64 sum of its 32 terms within
    1e-14 of the run's sum of |term| (the reference's own row check,
    tests/test_sample_sum.py:36-38, :98-112), and is the correctly rounded
    sum to one ulp (math.fsum)."""
    import math
    t = np.random.default_rng(n).normal(size=n) * np.exp(np.random.default_rng(n + 1).normal(size=n))
    hi, comp = O.row_sums(t)
    pad = np.zeros(hi.size * 32)
    pad[:n] = t
    rows = pad.reshape(-1, 32)
    got = hi + comp
    assert np.all(np.abs(got - rows.sum(1)) <= 1e-14 * np.abs(rows).sum(1) + 1e-300)
    exact = np.array([math.fsum(r) for r in rows])
    assert np.all(np.abs(got - exact) <= _ulp(exact))


def test_row_sums_compensate_cancellation():
    """Rows whose terms cancel to 1e-8 of their magnitude: the compensated
    pair gives the correctly rounded sum, which the plain pairwise tree of the
    same rows misses by many ulps — a dropped or sign-flipped compensation
    term fails here."""
    import math
    g = np.random.default_rng(7)
    base = g.normal(size=(64, 16)) * 1e8
    t = np.concatenate([base, -base + g.normal(size=(64, 16))], axis=1)
    t = np.take_along_axis(t, np.argsort(g.random(t.shape), axis=1), axis=1).reshape(-1)
    hi, comp = O.row_sums(t)
    exact = np.array([math.fsum(r) for r in t.reshape(-1, 32)])
    assert np.all(np.abs(hi + comp - exact) <= _ulp(exact))
    plain = t.reshape(-1, 32).copy()
    w = 16
    while w:
        plain[:, :w] += plain[:, w:2 * w]
        w //= 2
    assert np.max(np.abs(plain[:, 0] - exact) / _ulp(exact)) > 100


# -- the float32 mode's default-policy sum: the same algorithm in float32 -----

@pytest.mark.parametrize("n", [1, 31, 32, 33, 1000, 65536])
def test_float32_rows_are_compensated_sums(n):
    """Each float32 row's hi + comp (read exactly in float64) is the row's
    exact sum to within 2^-44 of its sum of |term|: the compensation keeps
    about twice float32's precision, which the plain float32 pairwise tree of
    the same rows misses by orders of magnitude (a dropped or sign-flipped
    compensation fails)."""
    import math
    g = np.random.default_rng(n)
    t = (g.normal(size=n) * np.exp(g.normal(size=n))).astype(np.float32)
    hi, comp = O.row_sums_f32(t)
    assert hi.dtype == np.float32 and comp.dtype == np.float32
    pad = np.zeros(hi.size * 32, dtype=np.float32)
    pad[:n] = t
    rows = pad.reshape(-1, 32).astype(np.float64)
    exact = np.array([math.fsum(r) for r in rows])
    got = hi.astype(np.float64) + comp.astype(np.float64)
    assert np.all(np.abs(got - exact) <= 2.0 ** -44 * np.abs(rows).sum(1) + 1e-300)
    plain = pad.reshape(-1, 32).copy()
    w = 16
    while w:
        plain[:, :w] += plain[:, w:2 * w]
        w //= 2
    if n >= 1000:
        assert np.max(np.abs(plain[:, 0].astype(np.float64) - exact) / (np.abs(rows).sum(1) + 1e-300)) > 2.0 ** -30


@pytest.mark.parametrize("rows", [1, 257, 4097, 3 * 4096 + 17])
def test_float32_finish_is_within_an_ulp_of_the_exact_sum(rows):
    """The float32 finish across leaf boundaries equals the exact sum of every
    hi and comp to within one float32 ulp (the last rounding of hi + comp is
    half of it), and an exactly representable total comes out exactly."""
    import math
    g = np.random.default_rng(rows)
    hi = (g.normal(size=rows) * np.exp(g.normal(size=rows))).astype(np.float32)
    comp = (hi * g.normal(size=rows) * np.float32(2.0 ** -26)).astype(np.float32)
    exact = math.fsum(np.concatenate([hi, comp]).astype(np.float64))
    got = O.rows_finish_f32(hi, comp)
    assert isinstance(got, np.float32)
    assert abs(float(got) - exact) <= float(np.spacing(np.float32(abs(exact))))
    ints = g.integers(-1000, 1000, rows).astype(np.float32)
    assert float(O.rows_finish_f32(ints, np.zeros_like(ints))) == float(ints.astype(np.int64).sum())


def test_float32_sum_is_float32_arithmetic():
    """The float32 sum is not the float64 sum rounded at the end: terms whose
    float32 partials round differ from the float64 oracle's, and both agree
    with the exact sum to their own precision."""
    import math
    t = (np.arange(1, 5001, dtype=np.float64) / 7.0).astype(np.float32)
    s32 = O.sample_sum_f32(t)
    exact = math.fsum(t.astype(np.float64))
    assert abs(float(s32) - exact) <= float(np.spacing(np.float32(exact)))
    assert abs(O.sample_sum(t.astype(np.float64)) - exact) <= np.spacing(exact)
    assert float(O.sample_sum_f32(np.float32([1e8, 1.0, -1e8]))) == 1.0


@pytest.mark.parametrize("rows", [1, 255, 256, 257, 4095, 4096, 4097, 3 * 4096 + 17, 70000])
def test_rows_finish_is_the_correctly_rounded_sum(rows):
    """The finish across leaf boundaries (4096 rows a leaf) equals fsum of
    every hi and comp to one ulp.  The bits of the leaf structure beyond that
    are pinned only by the fsum property (the reference pins them against
    eagle's ordered finish by import, tests/test_run_cells.py:83-99)."""
    import math
    g = np.random.default_rng(rows)
    hi = g.normal(size=rows) * np.exp(g.normal(size=rows))
    comp = hi * g.normal(size=rows) * 1e-17
    exact = math.fsum(np.concatenate([hi, comp]))
    assert abs(O.rows_finish(hi, comp) - exact) <= _ulp(exact)


def test_sample_sum_special_values():
    assert O.sample_sum(np.zeros(100)) == 0.0 and not np.signbit(O.sample_sum(np.zeros(100)))
    assert O.sample_sum(np.zeros(0)) == 0.0
    x = np.ones(5000)
    x[1234] = np.inf
    assert O.sample_sum(x) == np.inf
    x[999] = -np.inf
    assert np.isnan(O.sample_sum(x))
    x = np.ones(5000)
    x[17] = np.nan
    assert np.isnan(O.sample_sum(x))
    assert O.sample_sum(np.arange(1.0, 100001.0)) == 100000 * 100001 / 2


EXTREME_SIZES = [1, 31, 32, 33, 1000, 100_003, 300_007]


@pytest.mark.parametrize("dtype", [np.float64, np.float32])
@pytest.mark.parametrize("n", EXTREME_SIZES)
def test_sample_extremes_are_numpys_max_and_min(n, dtype):
    """hawk.max / hawk.min on NaN-free data are exact: the oracle's rows and
    finish give numpy's max and min bit for bit (a dropped row, a wrong
    identity or a swapped op fails), in either dtype."""
    g = np.random.default_rng(n)
    x = (g.normal(size=n) * np.exp(3 * g.normal(size=n))).astype(dtype)
    got_max, got_min = O.sample_extreme(x, "max"), O.sample_extreme(x, "min")
    assert got_max.dtype == dtype if hasattr(got_max, "dtype") else dtype == np.float64
    assert np.asarray(got_max, dtype).tobytes() == np.max(x).tobytes()
    assert np.asarray(got_min, dtype).tobytes() == np.min(x).tobytes()


@pytest.mark.parametrize("n", [1, 31, 33, 1000, 65536 + 17])
def test_row_extremes_are_the_padded_rows_max_and_min(n):
    """The rows, as the reference's own test checks them
    (tests/test_sample_sum.py:303-306): a masked lane's identity (-inf for
    max, +inf for min) fills the mask and the ragged row's tail."""
    x = np.random.default_rng(n).uniform(-2, 2, n)
    rows = -(-n // 32)

    def per_row(t, fill):
        return np.pad(t, (0, rows * 32 - n), constant_values=fill).reshape(rows, 32)
    hi = O.row_extremes(np.where(x > 0, x, -np.inf), "max")
    lo = O.row_extremes(np.where(x < 0, x, np.inf), "min")
    assert np.array_equal(hi, per_row(np.where(x > 0, x, -np.inf), -np.inf).max(1))
    assert np.array_equal(lo, per_row(np.where(x < 0, x, np.inf), np.inf).min(1))


def test_extreme_nans_zeros_and_the_empty_run():
    """What the reference's operators fix beyond numpy: a row ignores a NaN
    (ssExtreme_, hawk/emit/wrapper.py:543-550) unless every lane is NaN; the
    finish's np.where(a > b, a, b) (hawk/_cells.py:66-71) lets a NaN partial
    on the left give way and one on the right win; +0 against -0 keeps the
    row's lower slot and the finish's right operand; no samples give the
    identity.  A transposed operand in either combine fails one of these."""
    row = np.full(32, np.nan)
    row[5], row[20] = 3.0, -1.0
    assert O.sample_extreme(row, "max") == 3.0 and O.sample_extreme(row, "min") == -1.0
    assert np.isnan(O.sample_extreme(np.full(32, np.nan), "max"))
    # 40 NaNs: row 0 is NaN, row 1 ignores its 8 NaNs (-inf), the finish keeps the right
    assert O.sample_extreme(np.full(40, np.nan), "max") == -np.inf
    # rows [NaN, 1]: NaN > 1 is false, so the finish keeps 1; rows [1, NaN]: NaN
    nan_then_one = np.concatenate([np.full(32, np.nan), np.ones(32)])
    assert O.rows_extreme(np.array([np.nan, 1.0]), "max") == 1.0
    assert O.sample_extreme(nan_then_one, "max") == 1.0
    assert np.isnan(O.rows_extreme(np.array([1.0, np.nan]), "max"))
    assert np.isnan(O.sample_extreme(nan_then_one[::-1].copy(), "min"))
    # signed zeros: the row keeps slot l against slot l + off, the finish b on a tie
    assert not np.signbit(O.sample_extreme(np.array([0.0, -0.0]), "max"))
    assert np.signbit(O.sample_extreme(np.array([-0.0, 0.0]), "max"))
    assert np.signbit(O.rows_extreme(np.array([0.0, -0.0]), "max"))
    assert not np.signbit(O.rows_extreme(np.array([-0.0, 0.0]), "min"))
    assert O.sample_extreme(np.zeros(0), "max") == -np.inf
    assert O.sample_extreme(np.zeros(0, np.float32), "min") == np.float32(np.inf)
    # a NaN that is a row's only finite-breaking value among infinities
    x = np.full(64, -np.inf)
    x[40] = np.nan
    assert O.sample_extreme(x, "max") == -np.inf


def _chain_kinks(x):
    """|t4| and |t6| of the chain: where either is near 0 the chain has a kink."""
    t4 = np.tanh(1.5 * np.sin(np.exp(x)) + 0.25)
    t6 = (np.sqrt(np.abs(t4) + 1.0) ** 2) - x
    return np.minimum(np.abs(t4), np.abs(t6))


def test_chain_derivative_matches_central_differences():
    """The oracle's hand-derived dy/dx (chain_jvp with dot_x = 1) against central
    differences of the oracle's forward, on both sides of both kinks."""
    g = np.random.default_rng(21)
    x = np.concatenate([g.normal(size=4000), g.uniform(-4.0, 3.0, 4000)])
    x = x[_chain_kinks(x) > 1e-3]
    h = 1e-6
    fd = (O.chain(x + h) - O.chain(x - h)) / (2 * h)
    d = O.chain_jvp(x, np.ones_like(x))
    assert np.all(np.abs(d - fd) <= 1e-5 * np.abs(fd) + 1e-7)
    # both signs of t6 (the exp(-|t6|) kink) are present in the sample
    t4 = np.tanh(1.5 * np.sin(np.exp(x)) + 0.25)
    t6 = (np.sqrt(np.abs(t4) + 1.0) ** 2) - x
    assert (t6 > 0).any() and (t6 < 0).any() and (t4 > 0).any() and (t4 < 0).any()


def test_chain_oracle_is_the_composition_of_its_operations():
    """hko_chain is glibc's exp/sin/tanh and the IEEE operations in the order
    the per-element bound differentiates (tests/chain_bound.py), bit for bit."""
    import chain_bound as CB
    g = np.random.default_rng(22)
    x = np.concatenate([g.normal(size=20000), g.uniform(-6.0, 6.0, 5000), [0.0, -0.0, 1e-300, 700.0, -700.0]])
    assert CB.parts(x)["y"].tobytes() == O.chain(x).tobytes()


def _nudge(ulps):
    """A planted mistake: move every value by ``ulps`` units in its last place."""
    return lambda v: v + ulps * np.spacing(np.abs(v))


def test_chain_bound_admits_the_allowances_and_catches_larger_mistakes():
    """The per-element bound of the chain, pinned by mistakes planted in the
    oracle's own composition (on the CPU): each transcendental moved by its
    4-ulp allowance, all four at once, is inside the bound at every element;
    a transcendental off by 64 ulps, a dropped term and a swapped operand are
    caught.  (64 ulps are 16 allowances, caught only where one operation
    dominates: the bound adds every operation's allowance, twice.)"""
    import chain_bound as CB
    g = np.random.default_rng(23)
    x = np.concatenate([g.normal(size=200_000), g.uniform(-4.0, 3.0, 50_000)])
    base = CB.parts(x)
    bound = CB.element_bound(x, base)
    assert np.all(bound > 0)
    for name in ("t1", "t2", "t4", "t7"):
        for u in (4, -4):
            moved = CB.parts(x, {name: _nudge(u)})["y"]
            assert CB.within(moved, base["y"], bound).all(), (name, u)
    together = CB.parts(x, {n: _nudge(4) for n in ("t1", "t2", "t4", "t7")})["y"]
    assert CB.within(together, base["y"], bound).all()
    # mistakes the bound must see: 64 ulps in any one transcendental on at least 2 % of the samples
    # (those where it dominates y's sensitivity), 1024 ulps on at least 90 %
    for name in ("t1", "t2", "t4", "t7"):
        for u, share in ((64, 0.02), (1024, 0.9)):
            wrong = CB.parts(x, {name: _nudge(u)})["y"]
            assert (~CB.within(wrong, base["y"], bound)).mean() > share, (name, u)
    dropped = CB.parts(x, {"y": lambda v: v - base["t4"]})["y"]          # y = t7 x: the t4 term lost
    assert (~CB.within(dropped, base["y"], bound)).mean() > 0.9
    swapped = CB.parts(x, {"t7": lambda v: O.libm("exp", -base["t6"])})["y"]     # exp(-t6) for exp(-|t6|)
    flagged = ~CB.within(swapped, base["y"], bound)
    assert flagged[base["t6"] < -1e-3].all() and (base["t6"] < -1e-3).sum() > 10_000
    # a plain 4-ulp bar on y would reject legitimate 4-ulp transcendentals where y cancels
    assert (~within_contract(together, base["y"], rel=0.0)).any()


def test_chain_vjp_gathers_the_bins_adjoint_at_the_key():
    """bar_x = dy/dx * (bar_y + bar_total + bar_bins[key]); a key outside
    [0, cells), the skip key -1 among them, gathers 0."""
    g = np.random.default_rng(22)
    n, cells = 3000, 11
    x = g.normal(size=n)
    key = g.integers(-1, cells + 2, n).astype(np.int32)
    bar_y, bar_bins = g.normal(size=n), g.normal(size=cells)
    got = O.chain_vjp(x, key, bar_y, 0.75, bar_bins)
    d = O.chain_jvp(x, np.ones(n))
    inside = (key >= 0) & (key < cells)
    gathered = np.where(inside, bar_bins[np.where(inside, key, 0)], 0.0)
    assert np.array_equal(got, d * ((bar_y + 0.75) + gathered))
    assert (~inside).sum() > 100


def _np_tree(s):
    s = s.copy()
    w = len(s) // 2
    while w:
        s[:w] += s[w:2 * w]
        w //= 2
    return s[0]


def _np_ordered_sum(x):
    """The fixed grouping in NumPy (reference tests/test_ordered_fixed_tree.py:25-40)."""
    V, G, W = 65536, 64, 1024
    part = np.zeros(V, x.dtype)
    for r in range(0, len(x), V):
        row = x[r:r + V]
        part[:len(row)] += row
    return _np_tree(np.array([_np_tree(part[g * W:(g + 1) * W]) for g in range(G)], x.dtype))


@pytest.mark.parametrize("keys, group", [(1, 1), (4, 8), (7, 1), (3, 1000), (2, 65536), (2, 70001), (300, 17)])
def test_keyed_ordered_sum_is_the_numpy_tree_per_key(keys, group):
    """hawk.sum(x, over=<trailing axes>, policy="ordered"): each key's run of
    `group` values takes the reference's fixed tree, bit for bit against its
    NumPy emulation run on that key's values alone."""
    g = np.random.default_rng(keys * 1000 + group)
    x = g.normal(size=keys * group) * np.exp(g.normal(size=keys * group))
    got = O.keyed_ordered_sum(x, group)
    want = np.array([_np_ordered_sum(x[k * group:(k + 1) * group]) for k in range(keys)])
    assert got.tobytes() == want.tobytes()
    assert O.keyed_ordered_sum(x, group, threads=3).tobytes() == got.tobytes()


@pytest.mark.parametrize("keys,rows,width", [(1, 1, 1), (3, 40, 24), (5, 7, 3), (2, 64, 2), (4, 65, 5),
                                             (2, 300, 1)])
def test_keyed_log_fold_is_the_serial_loop(keys, rows, width):
    """The ordered gradient's fold (reference hawk/emit/team.py:281-312): per
    key and slot, the key's rows added one after another from +0 in plain
    Python floats (IEEE doubles, the same single roundings), stored at the
    slot's cell; cells no pair names keep their values; a cell outside the
    plane is reported and not stored."""
    g = np.random.default_rng(keys * 100 + rows + width)
    v = g.normal(size=(width, keys * rows)) * np.exp(3 * g.normal(size=(width, keys * rows)))
    cells = keys * width + 7
    c = g.permutation(cells)[:keys * width].reshape(width, keys).astype(np.int32)
    out = np.full(cells, -3.5)
    assert O.keyed_log_fold(v, c, rows, out) == 0
    want = np.full(cells, -3.5)
    for e in range(width):
        for k in range(keys):
            s = 0.0
            for r in range(rows):
                s = s + float(v[e, k * rows + r])
            want[c[e, k]] = s
    assert out.tobytes() == want.tobytes()
    if keys * width > 1:
        c2 = c.copy()
        c2[0, 0] = cells
        out2 = np.full(cells, -3.5)
        assert O.keyed_log_fold(v, c2, rows, out2) == 1
        assert out2[c[0, 0]] == -3.5


def test_net_axis_oracle_is_the_loop_over_nets_and_its_slope():
    """The net-axis restatement (reference tests/test_net_axis.py): each net's
    loss and gradient equal the numpy loop over the nets (the reference's
    tolerances, 1e-12 and 1e-10), the gradient is the loss's central
    difference slope, masked units have exactly zero gradient, and the
    threaded run gives the same bits."""
    from net_axis import net_problem
    k, s = 7, 40
    w, x, y, mask, loss, grad = net_problem(k, s, 5)
    got_loss = O.net_loss(w, mask, x, y)
    got = O.net_grad(w, mask, x, y, np.ones(k))
    np.testing.assert_allclose(got_loss, loss, rtol=1e-12)
    np.testing.assert_allclose(got, grad, rtol=1e-10, atol=1e-10)
    dead = np.repeat(mask == 0.0, 3, axis=1)
    assert (got[dead] == 0.0).all() and (got[~dead] != 0.0).all()
    h = 1e-6
    for net, col in ((0, 0), (3, 10), (6, 23), (5, 5)):
        up, dn = w.copy(), w.copy()
        up[net, col] += h
        dn[net, col] -= h
        slope = (O.net_loss(up, mask, x, y)[net] - O.net_loss(dn, mask, x, y)[net]) / (2 * h)
        assert abs(got[net, col] - slope) <= 1e-6 * max(1.0, abs(slope))
    bar = np.random.default_rng(1).normal(size=k)
    scaled = O.net_grad(w, mask, x, y, bar)
    np.testing.assert_allclose(scaled, got * bar[:, None], rtol=1e-12, atol=1e-300)
    assert O.net_loss(w, mask, x, y, threads=3).tobytes() == got_loss.tobytes()
    assert O.net_grad(w, mask, x, y, bar, threads=3).tobytes() == scaled.tobytes()


def test_chain_members_oracle_is_the_long_double_chain():
    """The chain of the four example members in C (glibc sin/cos/exp) within
    a few ulp of the same formulas in long double, acc updated in place;
    threaded == serial."""
    g = np.random.default_rng(5)
    n = 10_001
    x, acc = g.uniform(0.1, 2.0, n), g.uniform(0.0, 1.0, n)
    got_acc = acc.copy()
    y = O.chain_members(x, got_acc)
    ld = np.longdouble
    xl = x.astype(ld)
    a = np.stack([np.sin(xl), np.cos(xl), xl * ld("0.5")])
    b = np.exp(-(a * a).sum(axis=0)) + xl
    np.testing.assert_allclose(y, (a * b).astype(np.float64), rtol=4e-16 * 8)
    np.testing.assert_allclose(got_acc, (acc.astype(ld) + b * b).astype(np.float64), rtol=4e-16 * 8)
    acc2 = acc.copy()
    assert O.chain_members(x, acc2, threads=3).tobytes() == y.tobytes() and acc2.tobytes() == got_acc.tobytes()


@pytest.mark.parametrize("keys,group", [(1, 1000), (7, 32), (5, 40), (3, 33), (4, 1), (2, 4096 * 32 + 5)])
def test_keyed_sample_sum_is_each_keys_default_sum(keys, group):
    """The default policy over some axes: each key's run is a default-policy
    sample sum of its own, so one key is the whole run's sum bit for bit, and
    each key is within a few ulp of math.fsum of its values (compensated rows,
    the reference's row bound of tests/test_sample_sum.py:36-38)."""
    import math
    g = np.random.default_rng(keys * 7 + group)
    x = g.normal(size=keys * group) * np.exp(g.normal(size=keys * group))
    got = O.keyed_sample_sum(x, group)
    for k in range(keys):
        run = x[k * group:(k + 1) * group]
        assert got[k] == O.sample_sum(run)
        exact = math.fsum(run)
        assert abs(got[k] - exact) <= 4 * np.spacing(abs(exact)) + 1e-14 * np.abs(run).sum()


# -- banded reductions ------------------------------------------------------------

def _exact_integers(n, seed, bits=40):
    """Terms k * 2^-20 with |k| < 2^bits: every partial sum of up to 2^20 of
    them fits a double-double exactly, so a band sum is the exact sum rounded
    once.  Returns the terms and the exact sum (a Fraction)."""
    from fractions import Fraction
    k = np.random.default_rng(seed).integers(-(1 << bits), 1 << bits, n, dtype=np.int64)
    return k.astype(np.float64) * 2.0 ** -20, Fraction(int(k.sum()), 1 << 20)


@pytest.mark.parametrize("n", [1, 31, 32, 33, 1000, 65537, 3 * 65536 + 777, (1 << 20) + 5])
def test_band_sums_round_the_exact_sum_once_where_double_double_holds_it(n):
    """Where every partial fits a double-double the banded sums (default and
    ordered) are the exact sum correctly rounded, bit for bit."""
    x, exact = _exact_integers(n, n)
    want = float(exact)
    assert O.band_sample_sum(x) == want
    assert O.band_ordered_sum(x) == want


def test_band_sums_where_the_plain_ordered_tree_loses_terms():
    """Lane l of the ordered tree adds rows l, l + 65536, ...: with rows 2^60,
    1, -2^60, 1 each plain lane loses its first 1; the banded lanes keep it."""
    V = 65536
    x = np.concatenate([np.full(V, 2.0 ** 60), np.ones(V), np.full(V, -(2.0 ** 60)), np.ones(V)])
    assert O.band_ordered_sum(x) == 2.0 * V
    assert O.ordered_sum(x) == 1.0 * V                      # the plain fixed tree
    assert O.band_sample_sum(x) == 2.0 * V


#: Seven terms whose exact sum is the second (the rest cancel in pairs), and
#: which a double-double keeps only when they join one band in this order: as
#: the bands of seven lanes folded by the 64-group tree the sum comes out 0.
BAND_LANE_TERMS = [9.4039548065783e-37, -1.1419282818997418e-54, 8.077935669463161e-28, -9.4039548065783e-37,
                   -8.077935669463161e-28, -1.75, 1.75]


@pytest.mark.parametrize("lane", [0, 5, 127, 128, 8191])
def test_band_ordered_sum_adds_one_virtual_lanes_rows_as_one_band(lane):
    """The reference's banded geometry (hawk/emit/team.py:26-30, :225-245):
    128 lanes a group, 8192 virtual lanes, lane l adding rows l, l + 8192, ...
    as terms of one band.  With the seven terms above on rows lane + 8192 j
    and zeros elsewhere, the sum is exactly the second term; the 65536-lane
    geometry would fold them as seven lanes' bands and give 0."""
    from fractions import Fraction
    n = 7 * 8192 + 3
    x = np.zeros(n)
    x[lane + 8192 * np.arange(7)] = BAND_LANE_TERMS
    assert sum(Fraction(v) for v in BAND_LANE_TERMS) == Fraction(BAND_LANE_TERMS[1])
    assert O.band_ordered_sum(x) == BAND_LANE_TERMS[1]


def _ulp53(got: float, exact) -> float:
    from fractions import Fraction
    if exact == 0:
        return 0.0 if got == 0.0 else float("inf")
    return float(abs(Fraction(got) - exact) / Fraction(float(np.spacing(abs(float(exact))))))


@pytest.mark.parametrize("n", [1000, 3 * 65536 + 777])
def test_band_sums_within_a_hundredth_of_an_ulp_on_the_reference_cancelling_series(n):
    """The reference's banded bound (tests/test_banded_sum.py, tests/test_banded_ordered.py):
    rows of 2^30, 1, -2^30, 1, float32-exact, within 0.01 ULP53 of the exact
    rational row sums and total; and within half an ulp on uniform float32 data."""
    from fractions import Fraction
    x = np.tile([2.0 ** 30, 1.0, -(2.0 ** 30), 1.0], n // 4 + 1)[:n].astype(np.float32).astype(np.float64)
    hi, lo = O.band_row_sums(x)
    for r in range(min(hi.size, 64)):
        exact = sum(Fraction(float(v)) for v in x[r * 32:(r + 1) * 32])
        assert _ulp53(hi[r], exact) <= 0.01
        assert Fraction(float(hi[r])) + Fraction(float(lo[r])) == exact      # the band holds the row exactly
    total = sum(Fraction(float(v)) for v in x)
    assert _ulp53(O.band_sample_sum(x), total) <= 0.01
    assert _ulp53(O.band_ordered_sum(x), total) <= 0.01
    u = np.random.default_rng(n).uniform(-2.0, 2.0, n).astype(np.float32).astype(np.float64)
    total = sum(Fraction(float(v)) for v in u)
    assert _ulp53(O.band_sample_sum(u), total) <= 0.5 and _ulp53(O.band_ordered_sum(u), total) <= 0.5


def test_band_rows_are_normalised_and_special_values_follow_ieee():
    g = np.random.default_rng(9)
    x = g.normal(size=5000) * np.exp(g.normal(size=5000) * 10)
    hi, lo = O.band_row_sums(x)
    assert np.all(np.abs(lo) <= np.spacing(np.abs(hi)) / 2)
    assert O.band_sample_sum(np.zeros(0)) == 0.0 and O.band_ordered_sum(np.zeros(0)) == 0.0
    z = O.band_sample_sum(np.full(100, -0.0))
    assert z == 0.0 and not np.signbit(z)
    for f in (O.band_sample_sum, O.band_ordered_sum):
        y = np.ones(70000)
        y[12345] = np.inf
        assert f(y) == np.inf
        y[23456] = -np.inf
        assert np.isnan(f(y))
        y = np.ones(70000)
        y[5] = np.nan
        assert np.isnan(f(y))


@pytest.mark.parametrize("n", [8, 1000, 1003, 4099])
def test_the_interchanged_twobody_loops_are_the_serial_bits(n):
    """The CPU baseline's config-3 loops with the host target's interchange
    (a tile of 8 samples steps together; reference hawk/emit/host.py:1061):
    bit for bit the sample-by-sample loops, a ragged tail included, in the
    exact and the native profiles and through the threaded tiles."""
    r0, v0 = _twobody_inputs(n, 17)
    g = np.random.default_rng(18)
    br, bv = g.normal(size=(3, n)), g.normal(size=(3, n))
    for profile in ("portable", "native"):
        L = O.lib(profile)
        r, v, rx, vx = (np.empty((3, n)) for _ in range(4))
        L.hko_twobody(O._p(r0), O._p(v0), 1.0, n, O._p(r), O._p(v), 0, n)
        L.hko_twobody_x(O._p(r0), O._p(v0), 1.0, n, O._p(rx), O._p(vx), 0, n)
        assert r.tobytes() == rx.tobytes() and v.tobytes() == vx.tobytes()
        a, b, ax, bx = (np.empty((3, n)) for _ in range(4))
        L.hko_twobody_vjp(O._p(r0), O._p(v0), 1.0, O._p(br), O._p(bv), n, O._p(a), O._p(b), 0, n)
        L.hko_twobody_vjp_x(O._p(r0), O._p(v0), 1.0, O._p(br), O._p(bv), n, O._p(ax), O._p(bx), 0, n)
        assert a.tobytes() == ax.tobytes() and b.tobytes() == bx.tobytes()
    tr, tv = O.twobody(r0, v0, 1.0, threads=3)
    assert tr.tobytes() == r.tobytes() and tv.tobytes() == v.tobytes()
    ta, tb = O.twobody_vjp(r0, v0, 1.0, br, bv, threads=3)
    assert ta.tobytes() == a.tobytes() and tb.tobytes() == b.tobytes()


# -- the float32 mode's ordered reductions ----------------------------------

@pytest.mark.parametrize("n", golden("ordered_sum_sizes")["sizes"])
def test_float32_ordered_sum_is_the_numpy_float32_tree(n):
    """The reference's team stages add `Real`s: in float32 every lane sum and
    tree level is a float addition.  NumPy's tree over float32 arrays is the
    closed form (reference tests/test_ordered_fixed_tree.py:25-40)."""
    g = np.random.default_rng(n + 32)
    x = (g.normal(size=n) * np.exp(g.normal(size=n))).astype(np.float32)
    got = O.ordered_sum(x)
    assert isinstance(got, np.float32) and got.tobytes() == np.float32(tree_sum(x)).tobytes()


def test_float32_ordered_sum_is_float32_arithmetic():
    """Small integers are exact in float32: their sums are the integer sums;
    on normal values the float32 tree rounds where the float64 one does not."""
    x = np.arange(1, 70001, dtype=np.float32)
    assert O.ordered_sum(x) == np.float32(70000 * 70001 / 2)
    y = np.random.default_rng(34).normal(size=1 << 20).astype(np.float32)
    assert O.ordered_sum(y) != np.float32(O.ordered_sum(y.astype(np.float64)))
    assert O.ordered_sum(y) == np.float32(tree_sum(y))


def test_float32_keyed_ordered_sum_is_each_keys_tree():
    g = np.random.default_rng(40)
    for group in (1, 7, 64, 4096, 70001):
        u = g.normal(size=3 * group).astype(np.float32)
        got = O.keyed_ordered_sum(u, group)
        assert got.dtype == np.float32
        want = [np.float32(tree_sum(u[k * group:(k + 1) * group])) for k in range(3)]
        assert got.tobytes() == np.array(want, np.float32).tobytes()


def test_float32_ordered_scatter_is_the_serial_chunk_walk():
    """Brute force with numpy float32 scalars over a small case (per (key,
    chunk) in lane order from 0, per cell in chunk order from 0, onto the
    target), and integer values against np.add.at exactly."""
    g = np.random.default_rng(33)
    n, cells = 3000, 11
    key = g.integers(-1, cells + 2, n).astype(np.int32)
    x = g.normal(size=n).astype(np.float32)
    base = g.normal(size=cells).astype(np.float32)
    chunks = O.scatter_chunks(n, cells)
    span = -(-n // chunks)
    parts = np.zeros((cells, chunks), np.float32)
    bad = [0] * chunks
    for r in range(n):
        b, k = r // span, int(key[r])
        if k == -1:
            continue
        if 0 <= k < cells:
            parts[k, b] = np.float32(parts[k, b] + x[r])
        else:
            bad[b] = 1
    want = base.copy()
    for c in range(cells):
        s = np.float32(0.0)
        for b in range(chunks):
            s = np.float32(s + parts[c, b])
        want[c] = np.float32(want[c] + s)
    got, status = O.ordered_scatter(key, x, base)
    assert got.dtype == np.float32 and got.tobytes() == want.tobytes()
    assert list(status[1:1 + chunks]) == bad
    ki = g.integers(0, 300, 200_000).astype(np.int32)
    xi = g.integers(-50, 51, 200_000).astype(np.float32)
    exact = np.zeros(300, np.float64)
    np.add.at(exact, ki, xi.astype(np.float64))
    got, _ = O.ordered_scatter(ki, xi, np.zeros(300, np.float32))
    assert (got.astype(np.float64) == exact).all()


def test_float32_keyed_log_fold_is_each_runs_float32_walk():
    """The float32 fold: each (slot, key) run added in np.float32 from 0 in
    lane order and stored at its cell; a cell outside the plane is reported
    and not stored."""
    g = np.random.default_rng(44)
    keys, rows, width = 30, 17, 3
    v = g.normal(size=(width, keys * rows)).astype(np.float32)
    cells = keys * width + 5
    c = g.permutation(cells)[:keys * width].reshape(width, keys).astype(np.int32)
    out = np.full(cells, 7.0, np.float32)
    assert O.keyed_log_fold(v, c, rows, out) == 0
    want = np.full(cells, 7.0, np.float32)
    for e in range(width):
        for k in range(keys):
            s = np.float32(0.0)
            for r in range(rows):
                s = np.float32(s + v[e, k * rows + r])
            want[c[e, k]] = s
    assert out.tobytes() == want.tobytes()
    c[1, 4] = cells + 3
    assert O.keyed_log_fold(v, c, rows, np.zeros(cells, np.float32)) == 1
