"""Parity of the hip target with the CPU oracle, at sizes the oracle runs in
seconds.  Every case builds inputs from a seeded generator, runs the kernel on
the MI355X through hawk.build/load/run (the C-ABI), and compares with the
oracle's host-target restatement on the same inputs:

* bit-exact for the ordered sum, the ordered scatter, and the kernels built
  from IEEE operations only (configs 1, 2, 4a and the two-body forward);
* within 4 ulp or 1e-13 relative (the north star's fp64 bar) otherwise.
"""

from __future__ import annotations

import numpy as np
import pytest

import oracle_lib as O
from conftest import golden, rng, ulp_diff, within_contract

pytestmark = pytest.mark.gpu


def dev(a, gpu):
    import torch
    return torch.from_numpy(np.ascontiguousarray(a)).to(gpu)


def host(t):
    return t.detach().cpu().numpy()


def _load(unit, name):
    import hawk_amd as hawk
    return hawk.load(unit, name)


def tree_sum(x: np.ndarray) -> float:
    """The fixed grouping in NumPy: 65536 virtual lanes adding rows in order,
    the halving tree over each group of 1024, then over the 64 groups."""
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


# -- config 1 -------------------------------------------------------------------

@pytest.mark.parametrize("n", [1, 255, 1000, 65537, (1 << 20) + 3])
def test_scale_is_the_oracle_bitwise(unit, gpu, n):
    import hawk_amd as hawk
    x = rng(1).uniform(-1.0, 1.0, n)
    out = dev(np.zeros(n), gpu)
    hawk.run(_load(unit, "scale"), x=dev(x, gpu), a=2.0, b=1.0, out=out)
    want = O.scale(x, 2.0, 1.0)
    assert host(out).tobytes() == want.tobytes()


def test_a_partition_writes_its_range_only(unit, gpu):
    """A run over [base, base+count) with the true n_samples writes exactly that
    range (reference tests/test_serial_oracle.py:7-35): a prime N, an uneven cut,
    and a sentinel elsewhere."""
    import hawk_amd as hawk
    n, base, count = 100_003, 31_337, 40_009
    x = rng(11).uniform(-1.0, 1.0, n)
    out = dev(np.full(n, -12345.0), gpu)
    hawk.run(_load(unit, "scale"), x=dev(x, gpu), a=2.0, b=1.0, out=out, base=base, count=count)
    got = host(out)
    want = O.scale(x, 2.0, 1.0)
    assert np.all(got[:base] == -12345.0) and np.all(got[base + count:] == -12345.0)
    assert got[base:base + count].tobytes() == want[base:base + count].tobytes()


def test_scale_in_pairs_of_adjacent_samples(unit, gpu):
    """``scale`` runs its full blocks as pairs of adjacent samples, 16 bytes a
    lane, when the planes and ``base`` keep a pair 16-byte aligned, and the
    one-sample loop otherwise: both give the oracle's bits, over a partition
    with an even base (pairs, then a partial block), an odd base, planes that
    start one element into their buffers, and in place."""
    import hawk_amd as hawk
    k = _load(unit, "scale")
    assert (k.launch_shape["block"], k.launch_shape["per_thread"]) == (64, 2)
    n = 100_003
    x = rng(12).uniform(-1.0, 1.0, n + 1)
    want = O.scale(x, 2.0, 1.0)
    for base, count in ((4096, 50_001), (31_337, 40_009), (0, n)):
        print(f"scale pairs: base={base} count={count}", flush=True)
        out = dev(np.full(n, -12345.0), gpu)
        hawk.run(k, x=dev(x[:n], gpu), a=2.0, b=1.0, out=out, base=base, count=count)
        got = host(out)
        assert np.all(got[:base] == -12345.0) and np.all(got[base + count:] == -12345.0)
        assert got[base:base + count].tobytes() == want[base:base + count].tobytes()
    print("scale pairs: planes one element into their buffers", flush=True)
    X, OUT = dev(x, gpu), dev(np.zeros(n + 1), gpu)
    hawk.run(k, x=X[1:], a=2.0, b=1.0, out=OUT[1:])
    assert host(OUT)[1:].tobytes() == want[1:].tobytes()
    print("scale pairs: in place", flush=True)
    Y = dev(x[:n].copy(), gpu)
    hawk.run(k, x=Y, a=2.0, b=1.0, out=Y)
    assert host(Y).tobytes() == want[:n].tobytes()


def test_empty_run_touches_nothing(unit, gpu):
    import hawk_amd as hawk
    x = dev(np.zeros(16), gpu)
    out = dev(np.full(16, 7.0), gpu)
    hawk.run(_load(unit, "scale"), x=x, a=2.0, b=1.0, out=out, base=3, count=0)
    assert np.all(host(out) == 7.0)


# -- config 2 -------------------------------------------------------------------

def test_energy_readme_vectors(unit, gpu):
    """The reference's own golden vectors."""
    import hawk_amd as hawk
    ga = golden("energy_readme")
    v = np.array(ga["v"])
    e = dev(np.zeros(4), gpu)
    hawk.run(_load(unit, "energy"), v=dev(v, gpu), out=e)
    assert host(e).tolist() == ga["energy"]
    bar_v = dev(np.zeros((3, 4)), gpu)
    hawk.run(_load(unit, "energy_vjp"), v=dev(v, gpu), bar_out=dev(np.array(ga["bar_out"]), gpu), bar_v=bar_v)
    assert host(bar_v).tolist() == ga["bar_v"]


@pytest.mark.parametrize("n", [7, 4097, 300_001])
def test_energy_fwd_vjp_jvp_are_the_oracle_bitwise(unit, gpu, n):
    import hawk_amd as hawk
    g = rng(2)
    v = g.normal(size=(3, n))
    bar_out = g.normal(size=n)
    dv = g.normal(size=(3, n))
    out = dev(np.zeros(n), gpu)
    hawk.run(_load(unit, "energy"), v=dev(v, gpu), out=out)
    assert host(out).tobytes() == O.energy(v).tobytes()
    bar_v = dev(np.zeros((3, n)), gpu)
    hawk.run(_load(unit, "energy_vjp"), v=dev(v, gpu), bar_out=dev(bar_out, gpu), bar_v=bar_v)
    assert host(bar_v).tobytes() == O.energy_vjp(v, bar_out).tobytes()
    dot_out = dev(np.zeros(n), gpu)
    hawk.run(_load(unit, "energy_jvp"), v=dev(v, gpu), dot_v=dev(dv, gpu), dot_out=dot_out)
    assert host(dot_out).tobytes() == O.energy_jvp(v, dv).tobytes()


# -- config 3 -------------------------------------------------------------------

def _twobody_inputs(n, seed=3):
    g = rng(seed)
    d = g.normal(size=(3, n))
    d /= np.linalg.norm(d, axis=0)
    r0 = d * g.uniform(0.5, 2.0, n)
    v0 = g.normal(0.0, 0.3, size=(3, n))
    return r0, v0


@pytest.mark.parametrize("n", [5, 20_011])
def test_twobody_forward_and_vjp(unit, gpu, n):
    import hawk_amd as hawk
    r0, v0 = _twobody_inputs(n)
    r = dev(np.zeros((3, n)), gpu)
    v = dev(np.zeros((3, n)), gpu)
    hawk.run(_load(unit, "twobody"), r0=dev(r0, gpu), v0=dev(v0, gpu), mu=1.0, r=r, v=v)
    wr, wv = O.twobody(r0, v0, 1.0)
    assert within_contract(host(r), wr).all() and within_contract(host(v), wv).all()
    assert host(r).tobytes() == wr.tobytes() and host(v).tobytes() == wv.tobytes()
    g = rng(103)
    bar_r, bar_v = g.normal(size=(3, n)), g.normal(size=(3, n))
    br0 = dev(np.zeros((3, n)), gpu)
    bv0 = dev(np.zeros((3, n)), gpu)
    hawk.run(_load(unit, "twobody_vjp"), r0=dev(r0, gpu), v0=dev(v0, gpu), mu=1.0, bar_r=dev(bar_r, gpu),
             bar_v=dev(bar_v, gpu), bar_r0=br0, bar_v0=bv0)
    wbr0, wbv0 = O.twobody_vjp(r0, v0, 1.0, bar_r, bar_v)
    assert within_contract(host(br0), wbr0).all()
    assert within_contract(host(bv0), wbv0).all()
    # the checkpointed rolled reverse replays the oracle's operations: the same bits
    assert host(br0).tobytes() == wbr0.tobytes() and host(bv0).tobytes() == wbv0.tobytes()


# -- config 4a ------------------------------------------------------------------

def _spd_inputs(n, seed=4):
    g = rng(seed)
    B = g.normal(size=(n, 6, 6))
    A = np.einsum("nij,nkj->nik", B, B) + 6.0 * np.eye(6)
    b = g.normal(size=(n, 6))
    return np.ascontiguousarray(A.transpose(1, 2, 0)), np.ascontiguousarray(b.T)


@pytest.mark.parametrize("n", [3, 10_007])
def test_spd_solve_and_vjp_are_the_oracle(unit, gpu, n):
    import hawk_amd as hawk
    A, b = _spd_inputs(n)
    x = dev(np.zeros((6, n)), gpu)
    hawk.run(_load(unit, "spd_solve"), A=dev(A, gpu), b=dev(b, gpu), x=x)
    want = O.spd_solve(A, b)
    assert host(x).tobytes() == want.tobytes()
    bar_x = rng(104).normal(size=(6, n))
    bA = dev(np.zeros((6, 6, n)), gpu)
    bb = dev(np.zeros((6, n)), gpu)
    hawk.run(_load(unit, "spd_solve_vjp"), A=dev(A, gpu), b=dev(b, gpu), bar_x=dev(bar_x, gpu), bar_A=bA,
             bar_b=bb)
    wA, wb = O.spd_solve_vjp(A, b, bar_x)
    assert within_contract(host(bA), wA).all() and within_contract(host(bb), wb).all()
    assert host(bA).tobytes() == wA.tobytes() and host(bb).tobytes() == wb.tobytes()


# -- config 5 -------------------------------------------------------------------

@pytest.mark.parametrize("n", golden("ordered_sum_sizes")["sizes"])
def test_ordered_sum_is_the_numpy_tree_bitwise_and_replays(unit, gpu, n):
    import hawk_amd as hawk
    g = rng(n)
    x = g.normal(size=n) * np.exp(g.normal(size=n))
    k = _load(unit, "ordered_total")
    runs = []
    for _ in range(3):
        total = dev(np.zeros(1), gpu)
        hawk.run(k, x=dev(x, gpu), total=total)
        runs.append(host(total))
    assert runs[0].tobytes() == runs[1].tobytes() == runs[2].tobytes()
    assert runs[0][0] == tree_sum(x)
    assert runs[0][0] == O.ordered_sum(x)


# The split walk's window is 12288 keys and each tail range 6144 more:
# 12288 has no tail, 12289 a one-key range, 18433 a second range of one key,
# 61440 eight full ranges, 3 cells over 1000 lanes leaves empty chunks; 65536
# is config 5's cell count (eight full ranges and one of 4096 keys).
@pytest.mark.parametrize("cells, n, heavy", [(7, 30_000, False), (1000, 30_000, False), (1500, 30_000, False),
                                             (7, 20_000, True), (1, 3000, False), (200, 50, False),
                                             (1000, 1000, False), (3, 1000, False), (65536, 400_000, False),
                                             (12288, 300_001, False), (12289, 300_001, False),
                                             (18433, 500_000, False), (61440, 700_000, False),
                                             (40_000, 2_000_003, True),
                                             (65536, 3_000_017, False),
                                             (70_000, 300_000, False), (600_000, 1_300_000, False)])
def test_ordered_scatter_is_the_serial_walk_bitwise(unit, gpu, cells, n, heavy):
    import hawk_amd as hawk
    g = rng(cells + n)
    key = g.integers(0, cells, n).astype(np.int32)
    if heavy:
        key[g.random(n) < 0.9] = cells // 2
    key[::7] = -1
    print(f"scatter cells={cells} n={n} heavy={heavy}", flush=True)
    x = g.normal(size=n) * np.exp(g.normal(size=n))
    acc0 = np.linspace(1.0, 2.0, cells)
    k = _load(unit, "ordered_add")
    outs = []
    for _ in range(2):
        acc = dev(acc0, gpu)
        hawk.run(k, key=dev(key, gpu), x=dev(x, gpu), acc=acc)
        outs.append(host(acc))
    want, status = O.ordered_scatter(key, x, acc0)
    assert not status[1:].any()
    assert outs[0].tobytes() == outs[1].tobytes()
    assert outs[0].tobytes() == want.tobytes()
    assert k.scatter_chunks == O.scatter_chunks(n, cells)


@pytest.mark.parametrize("n, cells, heavy", golden("ordered_scatter_cases")["cases"])
def test_ordered_scatter_reference_cases(unit, gpu, n, cells, heavy):
    """The reference's scatter cases: add.at within 1e-12, an empty cell stays
    zero, replays are bitwise, a second run adds onto what the plane held —
    and every result is the oracle's bits."""
    import hawk_amd as hawk
    ga = golden("ordered_scatter_cases")
    g = rng(n)
    key = g.integers(0, cells, n).astype(np.int32)
    if heavy:
        key[g.random(n) < 0.9] = cells // 2
    empty = ga["empty_cell"]
    if cells == empty["cells"]:
        key[key == empty["moved_from"]] = empty["moved_to"]
    x = g.normal(size=n) * np.exp(g.normal(size=n))
    k = _load(unit, "ordered_add")
    seen = []
    for base in (np.zeros(cells), np.zeros(cells), np.linspace(1.0, 2.0, cells)):
        acc = dev(base, gpu)
        hawk.run(k, key=dev(key, gpu), x=dev(x, gpu), acc=acc)
        seen.append(host(acc))
        assert seen[-1].tobytes() == O.ordered_scatter(key, x, base)[0].tobytes()
    assert seen[0].tobytes() == seen[1].tobytes()
    want = np.zeros(cells)
    np.add.at(want, key, x)
    np.testing.assert_allclose(seen[0], want, rtol=ga["rtol"], atol=ga["rtol"] * np.abs(want).max())
    if cells == empty["cells"]:
        assert seen[0][empty["moved_from"]] == 0.0


@pytest.mark.parametrize("n", [1 << 20, 1 << 22])
def test_ordered_scatter_zipf_keys_into_65536_cells(unit, gpu, n):
    """Config 5's key shape, Zipf(1.1) folded into 65536 cells (a head key
    with a tenth of the lanes, a uniform floor over every cell), with skip
    keys: the oracle's bits, the same on a replay."""
    import hawk_amd as hawk
    cells = 1 << 16
    g = rng(n + 11)
    key = ((g.zipf(1.1, n) - 1) % cells).astype(np.int32)
    key[g.random(n) < 0.01] = -1
    x = g.normal(size=n)
    acc0 = g.normal(size=cells)
    k = _load(unit, "ordered_add")
    print(f"scatter zipf n={n}", flush=True)
    outs = []
    for _ in range(2):
        acc = dev(acc0, gpu)
        hawk.run(k, key=dev(key, gpu), x=dev(x, gpu), acc=acc)
        outs.append(host(acc))
    want, status = O.ordered_scatter(key, x, acc0)
    assert not status[1:].any()
    assert outs[0].tobytes() == outs[1].tobytes() == want.tobytes()


@pytest.mark.parametrize("cells", [5, 30_000])
def test_ordered_scatter_special_values(unit, gpu, cells):
    """-0.0, infinities, NaN and subnormals through every bucket kind (window
    keys 0..31, classes, tail ranges): the oracle's bits, NaN as NaN.  A key
    whose only values are -0.0 sums to +0.0 (the walk starts at +0.0)."""
    import hawk_amd as hawk
    n = 50_000
    g = rng(cells)
    key = g.integers(0, cells, n).astype(np.int32)
    x = g.normal(size=n)
    special = np.array([-0.0, np.inf, -np.inf, np.nan, 5e-324, -5e-324, 1e-310])
    hit = g.random(n) < 0.02
    x[hit] = special[g.integers(0, len(special), hit.sum())]
    lone = [1, cells - 1]
    for c in lone:
        key[key == c] = 0
    key[[10, 20, 30]] = lone[0]
    x[[10, 20, 30]] = -0.0
    key[40] = lone[1]
    x[40] = -0.0
    acc0 = np.zeros(cells)
    acc = dev(acc0, gpu)
    print(f"scatter specials cells={cells}", flush=True)
    hawk.run(_load(unit, "ordered_add"), key=dev(key, gpu), x=dev(x, gpu), acc=acc)
    got = host(acc)
    want, status = O.ordered_scatter(key, x, acc0)
    nan = np.isnan(want)
    assert (np.isnan(got) == nan).all()
    assert got[~nan].tobytes() == want[~nan].tobytes()
    assert np.signbit(got[lone]).tolist() == [False, False]


def test_ordered_scatter_reports_a_bad_key(unit, gpu):
    import hawk_amd as hawk
    from hawk_amd import HawkError
    key = np.arange(100, dtype=np.int32) % 10
    key[57] = 12
    key[58] = -3
    x = np.ones(100)
    acc = dev(np.zeros(10), gpu)
    with pytest.raises(HawkError, match="outside \\[0, 10\\)"):
        hawk.run(_load(unit, "ordered_add"), key=dev(key, gpu), x=dev(x, gpu), acc=acc)
    want, status = O.ordered_scatter(key, x, np.zeros(10))
    assert status[1:].any()
    assert host(acc).tobytes() == want.tobytes()


def test_domain_forms_give_the_general_forms_bits_on_the_device(gpu):
    """Where interval arithmetic bounds an operand, the emitter spells sqrt,
    tanh and exp in their bounded forms; on the device each gives the bits of
    the general form on the same operand: sqrt is numpy's (correctly rounded)
    over [e^-480, e^480], tanh on 1.5 sin x + 0.25 is the general tanh of
    the device's own argument, exp(-|x|) is the general exp of -|x|, sin of
    exp(x) is the general sin of the device's own exp(x), NaN and infinities
    included."""
    import tempfile
    import hawk_amd as hawk
    from hawk_amd import Scalar, kernel
    from hawk_amd import math as m

    @kernel
    def sq_arg(x: Scalar) -> Scalar:
        return m.exp(m.tanh(x) * 480.0)

    @kernel
    def sq(x: Scalar) -> Scalar:
        return m.sqrt(m.exp(m.tanh(x) * 480.0))

    @kernel
    def th_arg(x: Scalar) -> Scalar:
        return m.sin(x) * 1.5 + 0.25

    @kernel
    def th_mid(x: Scalar) -> Scalar:
        return m.tanh(m.sin(x) * 1.5 + 0.25)

    @kernel
    def th_any(x: Scalar) -> Scalar:
        return m.tanh(x)

    @kernel
    def ex_neg(x: Scalar) -> Scalar:
        return m.exp(-m.abs(x))

    @kernel
    def ex_any(x: Scalar) -> Scalar:
        return m.exp(x)

    @kernel
    def sn_pos(x: Scalar) -> Scalar:
        return m.sin(m.exp(x))

    @kernel
    def sn_any(x: Scalar) -> Scalar:
        return m.sin(x)

    from hawk_amd.emit_hip import plan_kernel
    assert "= hk_sqrt_normal(" in plan_kernel(sq.program, "sq").source
    assert "= hk_tanh_mid(" in plan_kernel(th_mid.program, "th_mid").source
    assert "= hk_exp_nonpos(" in plan_kernel(ex_neg.program, "ex_neg").source
    assert "= hk_sin_nonneg(" in plan_kernel(sn_pos.program, "sn_pos").source
    d = tempfile.mkdtemp()
    hawk.build([sq_arg, sq, th_arg, th_mid, th_any, ex_neg, ex_any, sn_pos, sn_any], d)
    g = rng(17)
    x = np.concatenate([g.normal(size=150_000) * 3, g.uniform(-0.02, 0.02, 50_000), g.uniform(-800, 800, 50_000),
                        [0.0, -0.0, np.inf, -np.inf, np.nan, 5e-324, 1e-300]])

    def run(name, arg):
        out = dev(np.zeros_like(arg), gpu)
        hawk.run(hawk.load(d, name), x=dev(arg, gpu), out=out)
        return host(out)

    def same(a, b):
        nan = np.isnan(a)
        assert np.array_equal(nan, np.isnan(b))
        assert a[~nan].tobytes() == b[~nan].tobytes()

    same(run("sq", x), np.sqrt(run("sq_arg", x)))
    same(run("th_mid", x), run("th_any", run("th_arg", x)))
    same(run("ex_neg", x), run("ex_any", -np.abs(x)))
    same(run("sn_pos", x), run("sn_any", run("ex_any", x)))


@pytest.mark.parametrize("which", ["exp", "sin", "cos", "tanh"])
def test_device_helpers_are_the_host_builds_bits(gpu, which, tmp_path):
    """exp, sin and cos (below 2^17, where they run their own reduction) and
    tanh on the device are the host build of the same text bit for bit: the
    operations are IEEE's on both sides.  For tanh this pins the quotient
    e / (e + 2) taken without the division's scaling and fixup: seeded by
    the hardware's reciprocal estimate on the device and by the correctly
    rounded 1/b on the host, both give the correctly rounded quotient."""
    import tempfile
    import hawk_amd as hawk
    import math_host
    from hawk_amd import Scalar, kernel
    from hawk_amd import math as m

    fn = {"exp": m.exp, "sin": m.sin, "cos": m.cos, "tanh": m.tanh}[which]

    @kernel
    def one(x: Scalar) -> Scalar:
        return fn(x)

    d = tempfile.mkdtemp()
    hawk.build([one], d)
    g = rng(23)
    if which == "exp":
        x = np.concatenate([g.normal(size=400_000) * 5, g.uniform(-745.2, 709.8, 400_000),
                            [0.0, -0.0, np.inf, -np.inf, np.nan, 5e-324, -1e-310, 709.8, -745.2, 1e300]])
    elif which == "tanh":
        x = np.concatenate([g.uniform(-2, 2, 400_000), g.uniform(-30, 30, 200_000),
                            np.exp(g.uniform(-745, 3, 100_000)) * np.sign(g.normal(size=100_000)),
                            [0.0, -0.0, np.inf, -np.inf, np.nan, 5e-324, 22.0, -21.999]])
    else:
        x = np.concatenate([np.exp(g.normal(size=400_000)), g.uniform(-200, 200, 200_000),
                            g.uniform(-1.3e5, 1.3e5, 200_000), np.pi / 2 * np.arange(-3000, 3000),
                            g.uniform(-1e-7, 1e-7, 20_000), [0.0, -0.0, 5e-324, -1e-310, 131071.99]])
    out = dev(np.zeros_like(x), gpu)
    hawk.run(hawk.load(d, "one"), x=dev(x, gpu), out=out)
    got = host(out)
    want = math_host.build(tmp_path)(which, x)
    nan = np.isnan(want)
    assert np.array_equal(np.isnan(got), nan)
    assert got[~nan].tobytes() == want[~nan].tobytes()


@pytest.mark.parametrize("which", ["exp", "sin", "cos", "tanh", "sqrt"])
def test_transcendentals_are_within_4_ulp_of_glibc(unit, gpu, which):
    """The device's fp64 exp/sin/tanh/sqrt on the chain's argument ranges, in ULP of
    glibc (reference tests/test_math_parity.py: device within ULP of host)."""
    import hawk_amd as hawk
    from hawk_amd import Scalar, kernel
    from hawk_amd import math as m

    fn = {"exp": m.exp, "sin": m.sin, "cos": m.cos, "tanh": m.tanh, "sqrt": m.sqrt}[which]

    @kernel
    def one(x: Scalar) -> Scalar:
        return fn(x)

    import tempfile
    d = tempfile.mkdtemp()
    hawk.build([one], d)
    g = rng(6)
    if which == "exp":
        x = np.concatenate([g.normal(size=100_000) * 5, -np.abs(g.normal(size=20_000)) * 20])
    elif which in ("sin", "cos"):
        x = np.concatenate([np.exp(g.normal(size=100_000)), g.uniform(-200, 200, 20_000),
                            g.uniform(-1.4e5, 1.4e5, 20_000), np.pi / 2 * np.arange(-300, 300)])
    elif which == "tanh":
        x = np.concatenate([g.uniform(-2, 2, 100_000), g.normal(size=20_000) * 1e-3, g.uniform(-30, 30, 20_000),
                            np.exp(g.uniform(-700, 3, 20_000)) * np.sign(g.normal(size=20_000)),
                            [0.0, 5e-324, -5e-324, 1e-300, 19.06, 21.99, 22.0, 22.01, 710.0, -710.0]])
    else:
        x = np.abs(g.normal(size=120_000)) + 1.0
    out = dev(np.zeros_like(x), gpu)
    hawk.run(hawk.load(d, "one"), x=dev(x, gpu), out=out)
    u = ulp_diff(host(out), O.libm(which, x))
    assert u.max() <= 4.0, f"{which}: max {u.max()} ulp"
    if which == "tanh":
        # tanh is sign(x) e / (e + 2), e = expm1(2|x|): odd, so -0 stays -0, +-1 far out, NaN through
        special = np.array([-0.0, np.inf, -np.inf, np.nan, -30.0])
        out = dev(np.zeros_like(special), gpu)
        hawk.run(hawk.load(d, "one"), x=dev(special, gpu), out=out)
        got = host(out)
        assert np.signbit(got[0]) and got[0] == 0.0 and got[1] == 1.0 and got[2] == -1.0
        assert np.isnan(got[3]) and got[4] == -1.0


@pytest.mark.parametrize("n", [1000, 262_147])
def test_chain_kernel_total_and_bins(unit, gpu, n):
    """The fused chain's y, every element within the chain's per-element bound
    of the oracle (tests/chain_bound.py: each operation's allowance carried to
    y to first order); the ordered total and the bins bit-exact against the
    oracle's walk of the same y."""
    import chain_bound as CB
    import hawk_amd as hawk
    g = rng(5)
    x = g.normal(size=n)
    cells = 1 << 16
    key = ((g.zipf(1.1, n) - 1) % cells).astype(np.int32)
    y = dev(np.zeros(n), gpu)
    total = dev(np.zeros(1), gpu)
    bins = dev(np.zeros(cells), gpu)
    print(f"chain n={n}", flush=True)
    hawk.run(_load(unit, "chain"), x=dev(x, gpu), key=dev(key, gpu), y=y, total=total, bins=bins)
    gy = host(y)
    wy = O.chain(x)
    ok = CB.within(gy, wy, CB.element_bound(x))
    assert ok.all(), f"{(~ok).sum()} of {n} outside the per-element bound"
    assert host(total)[0] == O.ordered_sum(gy)
    want_bins, status = O.ordered_scatter(key, gy, np.zeros(cells))
    assert not status[1:].any()
    assert host(bins).tobytes() == want_bins.tobytes()


def test_chain_each_operation_on_its_own_inputs(unit, gpu):
    """The chain's per-sample stage decomposed, element by element: the stage
    that also stores its four transcendentals' results gives the fused
    chain's y bit for bit; each transcendental is within 4 ulp of glibc at the
    device's own argument; every IEEE operation between them is the oracle's
    correctly rounded operation on the device's values, bit for bit."""
    import hawk_amd as hawk
    n = 262_147
    g = rng(55)
    x = np.concatenate([g.normal(size=n - 7), [0.0, -0.0, 5.5, -5.5, 1e-300, 3.0, -3.0]])
    X = dev(x, gpu)
    outs = {k: dev(np.full(n, np.nan), gpu) for k in ("e1", "s2", "h4", "e7", "y")}
    print("chain_steps", flush=True)
    hawk.run(_load(unit, "chain_steps"), x=X, **outs)
    t1, t2, t4, t7, y = (host(outs[k]) for k in ("e1", "s2", "h4", "e7", "y"))
    fused = dev(np.zeros(n), gpu)
    hawk.run(_load(unit, "chain"), x=X, key=dev(np.zeros(n, np.int32), gpu), y=fused,
             total=dev(np.zeros(1), gpu), bins=dev(np.zeros(1), gpu))
    assert host(fused).tobytes() == y.tobytes()
    assert ulp_diff(t1, O.libm("exp", x)).max() <= 4.0
    assert ulp_diff(t2, O.libm("sin", t1)).max() <= 4.0
    t3 = (1.5 * t2) + 0.25
    assert ulp_diff(t4, O.libm("tanh", t3)).max() <= 4.0
    t6 = (np.sqrt(np.abs(t4) + 1.0) * np.sqrt(np.abs(t4) + 1.0)) - x
    assert ulp_diff(t7, O.libm("exp", -np.abs(t6))).max() <= 4.0
    assert y.tobytes() == ((t7 * x) + t4).tobytes()


def _config5_inputs(n):
    """Config 5's inputs as the benchmark draws them: x ~ N(0,1), then Zipf(1.1)
    keys folded into 65536 cells, from one generator seeded 5."""
    g = rng(5)
    x = g.normal(size=n)
    key = ((g.zipf(1.1, n) - 1) % (1 << 16)).astype(np.int32)
    return x, key


def test_config5_at_the_benchmarks_own_shape(unit, gpu):
    """The timed workload itself, N = 2^26 with the benchmark's inputs: one
    launch of the fused chain + ordered sum + ordered scatter (256 chunks of
    64 tiles into 65536 cells).  Every y within the per-element bound; the
    total the fixed tree of the device's y, bit for bit; every bin the serial
    walk over the device's y, bit for bit; a second launch the same bits.  The
    worst error and the count outside the plain 4 ulp / 1e-13 bar are printed
    (the figures the design notes record)."""
    import chain_bound as CB
    import hawk_amd as hawk
    n = 1 << 26
    cells = 1 << 16
    x, key = _config5_inputs(n)
    print("config 5 at 2^26: launch", flush=True)
    k = _load(unit, "chain")
    X, KEY = dev(x, gpu), dev(key, gpu)
    y = dev(np.zeros(n), gpu)
    runs = []
    for _ in range(2):
        total, bins = dev(np.zeros(1), gpu), dev(np.zeros(cells), gpu)
        hawk.run(k, x=X, key=KEY, y=y, total=total, bins=bins)
        runs.append((host(y), host(total), host(bins)))
    del X, KEY, y
    assert k.scatter_chunks == 256
    got = runs[0][0]
    assert all(r[0].tobytes() == got.tobytes() and r[1].tobytes() == runs[0][1].tobytes()
               and r[2].tobytes() == runs[0][2].tobytes() for r in runs[1:])
    print("config 5 at 2^26: total and bins against the oracle", flush=True)
    assert runs[0][1][0] == O.ordered_sum(got, threads=16)
    want_bins, status = O.ordered_scatter(key, got, np.zeros(cells), threads=16)
    assert not status[1:].any()
    assert runs[0][2].tobytes() == want_bins.tobytes()
    print("config 5 at 2^26: y against the per-element bound", flush=True)
    p = CB.parts(x)
    want = p["y"]
    assert want.tobytes() == O.chain(x, threads=16).tobytes()
    bound = CB.element_bound(x, p)
    err = np.abs(got - want)
    ok = CB.within(got, want, bound)
    plain = within_contract(got, want)
    u = ulp_diff(got, want)
    print(f"chain 2^26: outside the bound {(~ok).sum()}; outside 4 ulp / 1e-13: {(~plain).sum()}; "
          f"worst {u.max():.1f} ulp ({(err / np.abs(want)).max():.3g} relative, {err.max():.3g} absolute); "
          f"worst error / bound {(err / bound).max():.3f}; bit-identical {(got == want).mean():.4f}", flush=True)
    assert ok.all()


def test_ordered_scatter_past_one_tail_group(unit, gpu):
    """N = 2^27 + 12295 Zipf keys into 65536 cells: 256 chunks of 524336
    lanes, 129 tiles a chunk, so each tail range streams its bins in two
    groups of slots (128, then one).  The serial walk's bits."""
    import hawk_amd as hawk
    n = (1 << 27) + 12295
    cells = 1 << 16
    g = rng(n)
    key = ((g.zipf(1.1, n) - 1) % cells).astype(np.int32)
    x = g.normal(size=n)
    span = -(-n // 256)
    assert -(-span // 4096) == 129
    k = _load(unit, "ordered_add")
    print(f"scatter zipf n={n} (two tail groups)", flush=True)
    acc = dev(np.zeros(cells), gpu)
    hawk.run(k, key=dev(key, gpu), x=dev(x, gpu), acc=acc)
    got = host(acc)
    want, status = O.ordered_scatter(key, x, np.zeros(cells), threads=16)
    assert not status[1:].any()
    assert got.tobytes() == want.tobytes()


def test_ordered_scatter_past_one_tail_batch(unit, gpu):
    """N = 2^26 + 12345 Zipf keys into 65536 cells: 256 chunks of 262193 lanes,
    65 tiles a chunk (one slot past the benchmark's 64), each tail range read
    from its bins in batches of 2048 entries.  Skip keys on 1 % of the lanes.
    The serial walk's bits, and the same bits on a replay."""
    import hawk_amd as hawk
    n = (1 << 26) + 12345
    cells = 1 << 16
    g = rng(n)
    key = ((g.zipf(1.1, n) - 1) % cells).astype(np.int32)
    key[g.random(n) < 0.01] = -1
    x = g.normal(size=n)
    acc0 = g.normal(size=cells)
    k = _load(unit, "ordered_add")
    print(f"scatter zipf n={n} (two tail batches)", flush=True)
    K, X = dev(key, gpu), dev(x, gpu)
    outs = []
    for _ in range(2):
        acc = dev(acc0, gpu)
        hawk.run(k, key=K, x=X, acc=acc)
        outs.append(host(acc))
    assert k.scatter_chunks == 256
    span = -(-n // 256)
    assert -(-span // 4096) == 65
    want, status = O.ordered_scatter(key, x, acc0, threads=16)
    assert not status[1:].any()
    assert outs[0].tobytes() == outs[1].tobytes() == want.tobytes()


# -- config 4b --------------------------------------------------------------------

def _mm_bound(X, Y):
    """Per element of X @ Y (planes [16, 16, n]): 1e-6 * sum_k |x_ik| |y_kj|,
    the north star's fp32 bar written as a bound on the products' magnitudes."""
    return 1e-6 * np.einsum("ikn,kjn->ijn", np.abs(X).astype(np.float64), np.abs(Y).astype(np.float64))


def _mm_exact(X, Y):
    return np.einsum("ikn,kjn->ijn", X.astype(np.float64), Y.astype(np.float64))


@pytest.mark.parametrize("n", [1, 31, 32, 33, 1000, 65_537])
def test_mm16_forward_and_vjp_on_mfma(unit32, gpu, n):
    """C = A @ B and its VJP (bar_A = bar_C B^T, bar_B = A^T bar_C) per sample,
    fp32 on MFMA: every element within 1e-6 * sum |a||b| of the exact product,
    and of the oracle's fp32 loop."""
    import hawk_amd as hawk
    g = rng(4)
    A = g.normal(0.0, 0.25, size=(16, 16, n)).astype(np.float32)
    B = g.normal(0.0, 0.25, size=(16, 16, n)).astype(np.float32)
    bar_C = rng(104).normal(0.0, 0.25, size=(16, 16, n)).astype(np.float32)
    C = dev(np.zeros((16, 16, n), np.float32), gpu)
    hawk.run(_load(unit32, "mm16"), A=dev(A, gpu), B=dev(B, gpu), C=C)
    got = host(C)
    bound = _mm_bound(A, B)
    assert (np.abs(got - _mm_exact(A, B)) <= bound).all()
    assert (np.abs(got - O.mm16(A, B)) <= 2 * bound).all()
    bA = dev(np.zeros((16, 16, n), np.float32), gpu)
    bB = dev(np.zeros((16, 16, n), np.float32), gpu)
    hawk.run(_load(unit32, "mm16_vjp"), A=dev(A, gpu), B=dev(B, gpu), bar_C=dev(bar_C, gpu), bar_A=bA, bar_B=bB)
    Bt, At = B.transpose(1, 0, 2), A.transpose(1, 0, 2)
    wA, wB = O.mm16_vjp(A, B, bar_C)
    assert (np.abs(host(bA) - _mm_exact(bar_C, Bt)) <= _mm_bound(bar_C, Bt)).all()
    assert (np.abs(host(bB) - _mm_exact(At, bar_C)) <= _mm_bound(At, bar_C)).all()
    assert (np.abs(host(bA) - wA) <= 2 * _mm_bound(bar_C, Bt)).all()
    assert (np.abs(host(bB) - wB) <= 2 * _mm_bound(At, bar_C)).all()


#: gamma_16 = 16u / (1 - 16u), u = 2^-53: a 16-term fp64 dot product summed in
#: any order, with any mix of rounded and fused steps, lies within
#: gamma_16 * sum_k |x_ik| |y_kj| of the exact value (about 1.8e-15 of the
#: magnitudes, inside the north star's 1e-13 relative bar for fp64).
_GAMMA16 = 16 * 2.0 ** -53 / (1 - 16 * 2.0 ** -53)


def _mm_exact_ld(X, Y):
    L = np.longdouble
    return np.einsum("ikn,kjn->ijn", X.astype(L), Y.astype(L))


@pytest.mark.parametrize("n", [1, 15, 16, 17, 33, 1000, 65_537])
def test_mm16_f64_forward_and_vjp_on_mfma(unit, gpu, n):
    """The float64 mode's C = A @ B and its VJP on v_mfma_f64_16x16x4f64: on
    integer inputs (every partial sum exact) the bits of the oracle's loop;
    on normal inputs every element within gamma_16 * sum |a||b| of the
    product in long double, and within twice that of the oracle."""
    import hawk_amd as hawk
    g = rng(5)
    ints = [g.integers(-8, 9, size=(16, 16, n)).astype(np.float64) for _ in range(3)]
    normals = [g.normal(0.0, 0.25, size=(16, 16, n)) for _ in range(3)]
    for exact, (A, B, bar_C) in ((True, ints), (False, normals)):
        # n = 16 makes (16, 16, n) read both ways: the call says the samples are last
        C = dev(np.zeros((16, 16, n)), gpu)
        hawk.run(_load(unit, "mm16"), A=dev(A, gpu), B=dev(B, gpu), C=C, layout="samples_last")
        bA, bB = dev(np.zeros((16, 16, n)), gpu), dev(np.zeros((16, 16, n)), gpu)
        hawk.run(_load(unit, "mm16_vjp"), A=dev(A, gpu), B=dev(B, gpu), bar_C=dev(bar_C, gpu), bar_A=bA, bar_B=bB,
                 layout="samples_last")
        got = [host(C), host(bA), host(bB)]
        Bt, At = B.transpose(1, 0, 2), A.transpose(1, 0, 2)
        pairs = [(A, B), (bar_C, Bt), (At, bar_C)]
        want = [O.mm16(A, B), *O.mm16_vjp(A, B, bar_C)]
        for x, w, (X, Y) in zip(got, want, pairs):
            if exact:
                assert x.tobytes() == w.tobytes()
                continue
            bound = _GAMMA16 * np.einsum("ikn,kjn->ijn", np.abs(X), np.abs(Y))
            assert (np.abs(x.astype(np.longdouble) - _mm_exact_ld(X, Y)) <= bound).all()
            assert (np.abs(x - w) <= 2 * bound).all()



# -- the default-policy sample sum (a7') ----------------------------------------

@pytest.mark.parametrize("n", [1, 31, 32, 33, 1000, 65_536, 4096 * 32 + 5, 300_001])
def test_default_sum_is_the_oracle_bitwise(unit, gpu, n):
    """hawk.sum(x * x) with the default policy: 32-sample compensated rows on
    the device (half-wave butterflies) and the canonical finish, the oracle's
    bits on every replay; the stage's per-sample output is untouched by it."""
    import hawk_amd as hawk
    g = rng(n)
    x = g.normal(size=n) * np.exp(g.normal(size=n))
    k = _load(unit, "sample_total")
    want = O.sample_sum(x * x)
    for _ in range(3):
        y = dev(np.zeros(n), gpu)
        total = dev(np.zeros(1), gpu)
        hawk.run(k, x=dev(x, gpu), y=y, total=total)
        assert host(total)[0] == want
        assert host(y).tobytes() == (2.0 * x).tobytes()


@pytest.mark.parametrize("n", [1, 33, 1000, 4096 * 32 + 5, 300_001])
def test_float32_default_sum_is_the_oracle_bitwise(unit32, gpu, n):
    """The float32 mode's hawk.sum(x * x): float32 rows on the device (the
    stage's half-wave butterflies in float32) and the float32 finish, the
    float32 oracle's bits on every replay; y = 2 x in float32."""
    import hawk_amd as hawk
    g = rng(n)
    x = (g.normal(size=n) * np.exp(g.normal(size=n))).astype(np.float32)
    k = _load(unit32, "sample_total")
    want = O.sample_sum_f32(x * x)
    print(f"float32 default sum n={n}", flush=True)
    for _ in range(3):
        y = dev(np.zeros(n, dtype=np.float32), gpu)
        total = dev(np.zeros(1, dtype=np.float32), gpu)
        hawk.run(k, x=dev(x, gpu), y=y, total=total)
        assert host(total)[0].tobytes() == want.tobytes()
        assert host(y).tobytes() == (np.float32(2.0) * x).tobytes()


def test_float32_default_sum_special_values(unit32, gpu):
    import hawk_amd as hawk
    k = _load(unit32, "plain_total")

    def total_of(x):
        t = dev(np.full(1, 7.0, dtype=np.float32), gpu)
        hawk.run(k, x=dev(np.asarray(x, dtype=np.float32), gpu), total=t)
        return host(t)[0]
    z = total_of(np.zeros(1000))
    assert z == 0.0 and not np.signbit(z)
    x = np.ones(5000, dtype=np.float32)
    x[1234] = np.inf
    assert total_of(x) == np.inf
    x[999] = -np.inf
    assert np.isnan(total_of(x))
    assert total_of(np.float32([1e8, 1.0, -1e8])) == 1.0
    x = (np.arange(1, 200_001) % 97).astype(np.float32)
    assert total_of(x) == O.sample_sum_f32(x)


def test_float32_transcendentals_on_the_device(gpu, tmp_path):
    """A float32 build of sqrt(|sin x| + 1e-50) + exp(-|x|) + tanh(2 sin x):
    the float overloads on float operands, within the north star's 1e-6
    relative of the float64 value (measured on the sum of the terms'
    magnitudes); at x = 0 the square root is 0, not NaN (1e-50 rounds to
    0.0f, so a bounded double form seeded by rsq would give NaN there)."""
    import hawk_amd as hawk
    from hawk_amd import Scalar, kernel
    from hawk_amd import math as m

    @kernel
    def tiny(x: Scalar) -> Scalar:
        return m.sqrt(m.abs(m.sin(x)) + 1e-50) + m.exp(-m.abs(x)) + m.tanh(m.sin(x) * 2.0)

    hawk.build([tiny], tmp_path, mode="float32")
    x = np.concatenate([[0.0, -0.0, 1e-30, np.pi], rng(77).normal(size=100_000) * 3]).astype(np.float32)
    y = dev(np.full(x.size, np.nan, np.float32), gpu)
    hawk.run(hawk.load(tmp_path, "tiny"), x=dev(x, gpu), out=y)
    got = host(y).astype(np.float64)
    xd = x.astype(np.float64)
    s = np.sin(xd)
    want = np.sqrt(np.abs(s)) + np.exp(-np.abs(xd)) + np.tanh(2.0 * s)
    scale = np.sqrt(np.abs(s)) + np.exp(-np.abs(xd)) + np.abs(np.tanh(2.0 * s))
    assert not np.isnan(got).any()
    assert got[0] == 1.0 and got[1] == 1.0
    assert (np.abs(got - want) <= 1e-6 * scale + 4 * np.spacing(np.float32(scale)).astype(np.float64)).all()


def test_default_sum_special_values(unit, gpu):
    import hawk_amd as hawk
    k = _load(unit, "plain_total")

    def total_of(x):
        t = dev(np.full(1, 7.0), gpu)
        hawk.run(k, x=dev(x, gpu), total=t)
        return host(t)[0]
    z = total_of(np.zeros(1000))
    assert z == 0.0 and not np.signbit(z)
    x = np.ones(5000)
    x[1234] = np.inf
    assert total_of(x) == np.inf
    x[999] = -np.inf
    assert np.isnan(total_of(x))
    assert total_of(np.arange(1.0, 100_001.0)) == 100_000 * 100_001 / 2


@pytest.mark.parametrize("n", [1, 1000, 65_537])
def test_param_gradient_cell_on_the_device(unit, gpu, n):
    """The two-body VJP with mu's gradient: bar_r0 / bar_v0 are the oracle's
    bits, bar_mu is the default-policy sum of the per-sample contributions the
    IR gives (tests/ir_eval.py), bit for bit."""
    import hawk_amd as hawk
    from hawk_amd import examples as E
    from ir_eval import evaluate
    g = rng(3 + n)
    d = g.normal(size=(3, n))
    d /= np.linalg.norm(d, axis=0)
    r0 = d * g.uniform(0.5, 2.0, n)
    v0 = g.normal(0.0, 0.3, size=(3, n))
    bar_r, bar_v = g.normal(size=(3, n)), g.normal(size=(3, n))
    bR0, bV0 = dev(np.zeros((3, n)), gpu), dev(np.zeros((3, n)), gpu)
    bmu = dev(np.zeros(1), gpu)
    hawk.run(_load(unit, "twobody_vjp_mu"), r0=dev(r0, gpu), v0=dev(v0, gpu), mu=1.3, bar_r=dev(bar_r, gpu),
             bar_v=dev(bar_v, gpu), bar_r0=bR0, bar_v0=bV0, bar_mu=bmu)
    want_r0, want_v0 = O.twobody_vjp(r0, v0, 1.3, bar_r, bar_v)
    assert host(bR0).tobytes() == want_r0.tobytes() and host(bV0).tobytes() == want_v0.tobytes()
    terms = evaluate(E.twobody_vjp_mu.program, {"r0": r0, "v0": v0, "mu": 1.3, "bar_r": bar_r, "bar_v": bar_v},
                     n)["bar_mu"]
    assert host(bmu)[0] == O.sample_sum(terms)


# -- partitions and special values ------------------------------------------------

@pytest.mark.parametrize("name", ["energy", "energy_vjp", "energy_jvp", "twobody", "twobody_vjp", "spd_solve",
                                  "spd_solve_vjp"])
def test_every_per_sample_kernel_runs_a_partition(unit, gpu, name):
    """A run over [base, base+count) with the true n_samples writes exactly
    that range, with the oracle's bits (one GPU's share of a sharded run,
    reference tests/test_serial_oracle.py:203); a sentinel stays elsewhere."""
    import hawk_amd as hawk
    n, base, count = 20_011, 7_001, 9_973
    g = rng(21)
    d = g.normal(size=(3, n))
    d /= np.linalg.norm(d, axis=0)
    r0 = d * g.uniform(0.5, 2.0, n)
    v3, t3, w3 = g.normal(size=(3, n)), g.normal(size=(3, n)), g.normal(size=(3, n))
    Bm = g.normal(size=(n, 6, 6))
    A = np.ascontiguousarray((np.matmul(Bm, Bm.transpose(0, 2, 1)) + 6.0 * np.eye(6)).transpose(1, 2, 0))
    b6, bx = g.normal(size=(6, n)), g.normal(size=(6, n))
    s1 = g.normal(size=n)
    cases = {
        "energy": ({"v": v3}, {"out": (n,)}, lambda: {"out": O.energy(v3)}),
        "energy_vjp": ({"v": v3, "bar_out": s1}, {"bar_v": (3, n)}, lambda: {"bar_v": O.energy_vjp(v3, s1)}),
        "energy_jvp": ({"v": v3, "dot_v": t3}, {"dot_out": (n,)}, lambda: {"dot_out": O.energy_jvp(v3, t3)}),
        "twobody": ({"r0": r0, "v0": 0.3 * v3, "mu": 1.0}, {"r": (3, n), "v": (3, n)},
                    lambda: dict(zip(("r", "v"), O.twobody(r0, 0.3 * v3, 1.0)))),
        "twobody_vjp": ({"r0": r0, "v0": 0.3 * v3, "mu": 1.0, "bar_r": t3, "bar_v": w3},
                        {"bar_r0": (3, n), "bar_v0": (3, n)},
                        lambda: dict(zip(("bar_r0", "bar_v0"), O.twobody_vjp(r0, 0.3 * v3, 1.0, t3, w3)))),
        "spd_solve": ({"A": A, "b": b6}, {"x": (6, n)}, lambda: {"x": O.spd_solve(A, b6)}),
        "spd_solve_vjp": ({"A": A, "b": b6, "bar_x": bx}, {"bar_A": (6, 6, n), "bar_b": (6, n)},
                          lambda: dict(zip(("bar_A", "bar_b"), O.spd_solve_vjp(A, b6, bx)))),
    }
    ins, outs, want = cases[name]
    planes = {k: (dev(v, gpu) if isinstance(v, np.ndarray) else v) for k, v in ins.items()}
    for k, shape in outs.items():
        planes[k] = dev(np.full(shape, -12345.0), gpu)
    hawk.run(_load(unit, name), base=base, count=count, **planes)
    for k, w in want().items():
        got = host(planes[k])
        assert np.all(got[..., :base] == -12345.0) and np.all(got[..., base + count:] == -12345.0), k
        assert got[..., base:base + count].tobytes() == np.ascontiguousarray(w[..., base:base + count]).tobytes(), k


SPECIALS = np.array([0.0, -0.0, np.inf, -np.inf, np.nan, 5e-324, -5e-324, 2.2250738585072014e-308, 1e-310,
                     -1e-310, 1.0, -1.0, 709.782712893384, 709.79, -745.13321910194122, -745.2, 710.0, -1000.0,
                     1e300, -1e300, 3.141592653589793, 1.5707963267948966, 1e-8, 19.0615, 20.0, -20.0, 1e15,
                     6.283185307179586e10, 0.5, 2.0, 4.0, 1e-300])


@pytest.mark.parametrize("which", ["exp", "sin", "cos", "tanh", "sqrt"])
def test_transcendentals_on_special_values(unit, gpu, which):
    """The special-value corpus of reference tests/test_math_parity.py (signed
    zeros, infinities, NaN, subnormals, overflow and underflow edges, large
    arguments): NaN where glibc gives NaN, a zero of glibc's sign, an infinity
    exactly, and every finite value within 4 ulp of glibc."""
    import tempfile

    import hawk_amd as hawk
    from hawk_amd import Scalar, kernel
    from hawk_amd import math as m

    fn = {"exp": m.exp, "sin": m.sin, "cos": m.cos, "tanh": m.tanh, "sqrt": m.sqrt}[which]

    @kernel
    def special(x: Scalar) -> Scalar:
        return fn(x)

    d = tempfile.mkdtemp()
    hawk.build([special], d)
    x = np.ascontiguousarray(SPECIALS)
    out = dev(np.zeros_like(x), gpu)
    hawk.run(hawk.load(d, "special"), x=dev(x, gpu), out=out)
    got, want = host(out), O.libm(which, x)
    for xi, g_, w_ in zip(x, got, want):
        if np.isnan(w_):
            assert np.isnan(g_), (which, xi, g_)
        elif w_ == 0.0:
            assert g_ == 0.0 and np.signbit(g_) == np.signbit(w_), (which, xi, g_, w_)
        elif np.isinf(w_):
            assert g_ == w_, (which, xi, g_)
        else:
            assert ulp_diff(np.array([g_]), np.array([w_]))[0] <= 4.0, (which, xi, g_, w_)


# -- derivatives through the team sinks --------------------------------------------

@pytest.mark.parametrize("n, cells, outside", [(3000, 11, False), ((1 << 22) + 5, 4096, True)])
def test_scatter_vjp_is_a_gather_on_the_device(unit, gpu, n, cells, outside):
    """add_sq_grad, the VJP of scatter(acc)[key] += x*x: bar_x == 2 x bar_acc[key]
    bit for bit (the reference's bar is rtol 1e-12), a key outside [0, cells) or
    the skip key -1 gathering 0; the prepared launcher gives the same bits; and
    on the reference's case central differences of g . acc(x), with acc from the
    device's ordered scatter, agree at 6 samples (reference
    tests/test_scatter_ordered.py:124-157: eps 1e-6, rtol 1e-5, atol 1e-7)."""
    import hawk_amd as hawk
    g = rng(5)
    key = g.integers(-2 if outside else 0, cells + (2 if outside else 0), n).astype(np.int32)
    x = g.normal(size=n) * np.exp(g.normal(size=n))
    table = rng(9).normal(size=cells)
    print(f"add_sq_grad n={n} cells={cells}", flush=True)
    kern = _load(unit, "add_sq_grad")
    bar = dev(np.full(n, np.nan), gpu)
    dkey, dx, dtab = dev(key, gpu), dev(x, gpu), dev(table, gpu)
    hawk.run(kern, key=dkey, x=dx, bar_acc=dtab, bar_x=bar)
    inside = (key >= 0) & (key < cells)
    gathered = np.where(inside, table[np.where(inside, key, 0)], 0.0)
    want = 2 * x * gathered                 # a gathered 0 keeps x's sign: (+-0) + (+-0)
    got = host(bar)
    assert got.tobytes() == want.tobytes()
    if outside:
        assert (~inside).sum() > 1000
    bar2 = dev(np.full(n, np.nan), gpu)
    kern.prepare(key=dkey, x=dx, bar_acc=dtab, bar_x=bar2)()
    assert host(bar2).tobytes() == want.tobytes()
    if outside:
        return
    fwd = _load(unit, "add_sq")

    def loss(v):
        acc = dev(np.zeros(cells), gpu)
        hawk.run(fwd, key=dkey, x=dev(v, gpu), acc=acc)
        return float(table @ host(acc))
    eps = 1e-6
    for i in np.random.default_rng(2).choice(n, 6, replace=False):
        hi, lo = x.copy(), x.copy()
        hi[i] += eps
        lo[i] -= eps
        np.testing.assert_allclose((loss(hi) - loss(lo)) / (2 * eps), got[i], rtol=1e-5, atol=1e-7)


def _chain_bound(got, want, scale):
    """The fp64 bar where dy/dx cancels: within 4 ulp / 1e-13 relative of the
    oracle, or 1e-13 of the magnitudes of the terms that cancel."""
    return within_contract(got, want) | (np.abs(got - want) <= 1e-13 * scale)


@pytest.mark.parametrize("n", [1000, 262_147])
def test_chain_vjp_on_the_device(unit, gpu, n):
    """vjp(chain, wrt=x) on the device: bar_x within the bar of the oracle's
    hand-derived dy/dx * (bar_y + bar_total + bar_bins[key]); keys include the
    skip key -1 (its gather reads 0)."""
    import hawk_amd as hawk
    g = rng(40)
    cells = 1 << 12
    x = g.normal(size=n)
    key = g.integers(-1, cells, n).astype(np.int32)
    bar_y, bar_bins, bar_total = g.normal(size=n), g.normal(size=cells), 0.625
    out = dev(np.full(n, np.nan), gpu)
    print(f"chain_vjp n={n}", flush=True)
    hawk.run(_load(unit, "chain_vjp"), x=dev(x, gpu), key=dev(key, gpu), bar_y=dev(bar_y, gpu),
             bar_total=bar_total, bar_bins=dev(bar_bins, gpu), bar_x=out)
    want = O.chain_vjp(x, key, bar_y, bar_total, bar_bins)
    scale = O.chain_dx_scale(x) * (np.abs(bar_y) + abs(bar_total) + np.abs(bar_bins).max())
    ok = _chain_bound(host(out), want, scale)
    assert ok.all(), f"{(~ok).sum()} of {n} outside the bar"


@pytest.mark.parametrize("n", [1000, 262_147])
def test_chain_jvp_on_the_device(unit, gpu, n):
    """jvp(chain, wrt=x): dot_y within the bar of the oracle's dy/dx * dot_x;
    dot_total and dot_bins (keys with the skip key -1) bit for bit the oracle's
    ordered sum and ordered scatter of the device's dot_y."""
    import hawk_amd as hawk
    g = rng(41)
    cells = 1 << 12
    x, dx = g.normal(size=n), g.normal(size=n)
    key = g.integers(-1, cells, n).astype(np.int32)
    dot_y, dot_total, dot_bins = dev(np.zeros(n), gpu), dev(np.zeros(1), gpu), dev(np.zeros(cells), gpu)
    print(f"chain_jvp n={n}", flush=True)
    hawk.run(_load(unit, "chain_jvp"), x=dev(x, gpu), dot_x=dev(dx, gpu), key=dev(key, gpu), dot_y=dot_y,
             dot_total=dot_total, dot_bins=dot_bins)
    gy = host(dot_y)
    ok = _chain_bound(gy, O.chain_jvp(x, dx), O.chain_dx_scale(x) * np.abs(dx))
    assert ok.all(), f"{(~ok).sum()} of {n} outside the bar"
    assert host(dot_total)[0] == O.ordered_sum(gy)
    want_bins, status = O.ordered_scatter(key, gy, np.zeros(cells))
    assert not status[1:].any()
    assert host(dot_bins).tobytes() == want_bins.tobytes()


# -- keyed ordered sums over trailing lane axes ------------------------------------------------

def _keyed_kernels(group):
    import hawk_amd as hawk
    from hawk_amd import Grid, Mutable, Scalar

    @hawk.kernel
    def ksum(lane: Grid["key", "sample":group], x: Scalar) -> Scalar:
        return hawk.sum(x, over="sample", policy="ordered")
    return ksum


@pytest.mark.parametrize("n", [1, 1000, 65536, 3 * 65536 + 777, 200003])
def test_keyed_ordered_sum_reference_cases(gpu, tmp_path, n):
    """Reference tests/test_ordered_fixed_tree.py:43-79: the one-key kernel
    total(lane: Grid["key", "sample":n], x) = hawk.sum(x, over="sample",
    policy="ordered") gives the fixed tree's bits (the oracle, pinned to the
    reference's NumPy emulation) on three replays."""
    import hawk_amd as hawk
    k = _keyed_kernels(n)
    hawk.build([k], tmp_path)
    kern = hawk.load(tmp_path, "ksum")
    x = rng(n).normal(size=n) * np.exp(rng(n + 1).normal(size=n))
    X = dev(x, gpu)
    runs = []
    for _ in range(3):
        out = dev(np.zeros(1), gpu)
        hawk.run(kern, x=X, out=out)
        runs.append(host(out).tobytes())
    assert runs[0] == runs[1] == runs[2]
    assert np.frombuffer(runs[0])[0] == O.ordered_sum(x)


@pytest.mark.parametrize("keys, group", [(4, 8), (1000, 5000), (3, 200003), (70000, 7), (2, 65536), (17, 1025),
                                         (5, 1), (65536, 64), (16384, 40), (1001, 33), (3000, 2), (12345, 63),
                                         (999, 65)])
def test_keyed_ordered_sum_many_keys(gpu, tmp_path, keys, group):
    """One cell per key, each key's run by the fixed tree, bit for bit the
    oracle's (and, for the reference's A=4, B=8 case, numpy's row sums within
    rtol 1e-13, tests/test_ordered_trailing_axes.py:66-76); two launches give
    the same bits."""
    import hawk_amd as hawk
    kern_def = _keyed_kernels(group)
    hawk.build([kern_def], tmp_path)
    kern = hawk.load(tmp_path, "ksum")
    n = keys * group
    x = rng(7 + group).uniform(-2.0, 2.0, n) * np.exp(rng(8).normal(size=n))
    X = dev(x, gpu)
    print(f"keyed sum keys={keys} group={group}", flush=True)
    out = dev(np.full(keys, np.nan), gpu)
    hawk.run(kern, x=X, out=out)
    got = host(out)
    assert got.tobytes() == O.keyed_ordered_sum(x, group).tobytes()
    out2 = dev(np.full(keys, np.nan), gpu)
    kern.prepare(x=X, out=out2)()
    assert host(out2).tobytes() == got.tobytes()
    if (keys, group) == (4, 8):
        np.testing.assert_allclose(got, x.reshape(keys, group).sum(axis=1), rtol=1e-13, atol=1e-13)


def test_keyed_sum_derivatives_and_lane_coordinates_on_the_device(gpu, tmp_path):
    """The VJP of y = hawk.sum(f(x), over="b", policy="ordered") reads each
    lane's key adjoint (bar_x = f'(x) * bar_y[lane // 8]); the JVP's tangent
    cells are the keyed sums of the tangents (the oracle's bits); lane
    coordinates are the numpy order of the Grid; the Grid's runtime extent can
    be given by label."""
    import hawk_amd as hawk
    from hawk_amd import Grid, Mutable, Scalar
    from hawk_amd.diff import jvp, vjp
    from hawk_amd.trace import Kernel

    @hawk.kernel
    def rows(lane: Grid["a", "b":8], x: Scalar, y: Mutable["a"]):
        y = hawk.sum(x * x, over="b", policy="ordered")

    @hawk.kernel
    def coords(lane: Grid["a", "b":4, "c":8], y: Mutable[Scalar]):
        y = lane.a * 100.0 + lane.b * 10.0 + lane[-1]

    @hawk.kernel
    def iota(lane: Grid["key", "sample":16], y: Mutable["key"]):
        y = hawk.sum(lane.sample * 1.0, over="sample", policy="ordered")

    back = Kernel("rows_vjp", vjp(rows, wrt=("x",)))
    fwd = Kernel("rows_jvp", jvp(rows, wrt=("x",)))
    hawk.build([rows, back, fwd, coords, iota], tmp_path)
    keys = 50_000
    n = keys * 8
    g = rng(21)
    x, bar, dx = g.normal(size=n), g.normal(size=keys), g.normal(size=n)
    X = dev(x, gpu)
    bx = dev(np.full(n, np.nan), gpu)
    hawk.run(hawk.load(tmp_path, "rows_vjp"), x=X, bar_y=dev(bar, gpu), bar_x=bx)
    assert host(bx).tobytes() == (2.0 * x * np.repeat(bar, 8)).tobytes() or \
        host(bx).tobytes() == ((x * np.repeat(bar, 8)) + (x * np.repeat(bar, 8))).tobytes()
    dy = dev(np.full(keys, np.nan), gpu)
    hawk.run(hawk.load(tmp_path, "rows_jvp"), x=X, dot_x=dev(dx, gpu), dot_y=dy)
    from ir_eval import evaluate
    terms = evaluate(fwd.program, {"x": x, "dot_x": dx}, n)["dot_y"]
    assert host(dy).tobytes() == O.keyed_ordered_sum(terms, 8).tobytes()
    yc = dev(np.zeros(3 * 32), gpu)
    hawk.run(hawk.load(tmp_path, "coords"), y=yc)
    i = np.arange(3 * 32)
    assert host(yc).tobytes() == ((i // 32) * 100.0 + ((i // 8) % 4) * 10.0 + i % 8).tobytes()
    yi = dev(np.zeros(1000), gpu)
    hawk.run(hawk.load(tmp_path, "iota"), key=1000, y=yi)
    assert np.all(host(yi) == 120.0)


# -- Table reads and their derivatives -------------------------------------------------------

def _table_kernels():
    import hawk_amd as hawk
    from hawk_amd import Grid, Index, Mutable, Scalar, Table

    @hawk.kernel
    def tpick(table: Table[Scalar], where: Index, x: Scalar, y: Mutable[Scalar]):
        y = table.at(where) * x + table.at(where - 1000) + table[where + 3] * table[where // 2]

    @hawk.kernel
    def tgrid(lane: Grid["e", "a":4], t: Table["e":8, "a":4], x: Scalar) -> Scalar:
        return t.at(e=lane.e, a=lane.a) * x + t[lane.a, lane.e] + t[lane.flat % 5]
    return tpick, tgrid


def test_table_reads_and_derivatives_on_the_device(gpu, tmp_path):
    """Clamped Table reads (reference tests/test_table_clamp.py) bit for bit
    against numpy; the VJP wrt the table is the ordered scatter of each read
    site's contribution at the cell it read (the oracle's walk of the IR's
    contributions, bit for bit), bar_x and the JVP the IR's bits; an empty
    table is refused."""
    import hawk_amd as hawk
    from hawk_amd import HawkError
    from hawk_amd.diff import jvp, vjp
    from hawk_amd.trace import Kernel
    from ir_eval import Evaluator, evaluate
    tpick, tgrid = _table_kernels()
    back = Kernel("tpick_vjp", vjp(tpick, wrt=("table", "x")))
    fwd = Kernel("tpick_jvp", jvp(tpick, wrt=("table",)))
    hawk.build([tpick, tgrid, back, fwd], tmp_path)
    n, cells = 200_003, 4099
    g = rng(31)
    table, dt = g.normal(size=cells), g.normal(size=cells)
    where = g.integers(-100, cells + 100, n).astype(np.int32)
    x, bar_y = g.normal(size=n), g.normal(size=n)
    env = {"table": table, "where": where, "x": x}
    T, W, X = dev(table, gpu), dev(where, gpu), dev(x, gpu)
    y = dev(np.full(n, np.nan), gpu)
    hawk.run(hawk.load(tmp_path, "tpick"), table=T, where=W, x=X, y=y)
    c = lambda i: table[np.clip(i, 0, cells - 1)]
    assert host(y).tobytes() == (c(where) * x + c(where - 1000) + c(where + 3) * c(where // 2)).tobytes()

    bt = dev(np.zeros(cells), gpu)
    bx = dev(np.full(n, np.nan), gpu)
    print("table vjp", flush=True)
    hawk.run(hawk.load(tmp_path, "tpick_vjp"), table=T, where=W, x=X, bar_y=dev(bar_y, gpu), bar_table=bt,
             bar_x=bx)
    genv = {**env, "bar_y": bar_y}
    ev = Evaluator(genv, n)
    want = np.zeros(cells)
    for s in back.program.sinks:
        if s.name == "bar_table":
            want, status = O.ordered_scatter(ev.value(s.key).astype(np.int32), ev.value(s.value), want)
            assert not status[1:].any()
    assert host(bt).tobytes() == want.tobytes()
    assert host(bx).tobytes() == evaluate(back.program, genv, n)["bar_x"].tobytes()

    dy = dev(np.full(n, np.nan), gpu)
    hawk.run(hawk.load(tmp_path, "tpick_jvp"), table=T, dot_table=dev(dt, gpu), where=W, x=X, dot_y=dy)
    assert host(dy).tobytes() == evaluate(fwd.program, {**env, "dot_table": dt}, n)["dot_y"].tobytes()

    m = 8 * 4 * 3
    t2, xg = g.normal(size=(8, 4)), g.normal(size=m)
    out = dev(np.zeros(m), gpu)
    hawk.run(hawk.load(tmp_path, "tgrid"), t=dev(t2, gpu), x=dev(xg, gpu), out=out)
    i = np.arange(m)
    e, a = i // 4, i % 4
    want2 = t2[np.clip(e, 0, 7), a] * xg + t2[np.clip(a, 0, 7), np.clip(e, 0, 3)] + t2.reshape(-1)[i % 5]
    assert host(out).tobytes() == want2.tobytes()
    with pytest.raises(HawkError, match="needs a cell"):
        hawk.run(hawk.load(tmp_path, "tpick"), table=dev(np.zeros(0), gpu), where=W, x=X, y=y)


# -- the ordered gradient's log fold ----------------------------------------------

def _log_fold(gpu, v, c, rows, init):
    """Run hk_keyed_log_fold_f64 (hk_keyed_log_fold_f32 for float32 ``v``) on
    copies of ``v``, ``c`` and ``init``; return (out, status) on the host."""
    import torch
    from hawk_amd import _core
    width, keys = c.shape
    cells = init.size
    V, C, out = dev(v, gpu), dev(c, gpu), dev(init, gpu)
    scratch = torch.empty(max(1, _core.keyed_log_fold_scratch_bytes(cells)), dtype=torch.uint8, device=gpu)
    status = torch.empty(2, dtype=torch.int32, device=gpu)
    fold = _core.keyed_log_fold_f32 if v.dtype == np.float32 else _core.keyed_log_fold
    fold(V.data_ptr(), keys * rows, C.data_ptr(), keys, rows, width, out.data_ptr(), cells,
         scratch.data_ptr(), status.data_ptr(), torch.cuda.current_stream().cuda_stream)
    torch.cuda.synchronize()
    return host(out), host(status).tolist()


@pytest.mark.parametrize("keys,rows,width", [(1, 1, 1), (1000, 1, 3), (5000, 40, 24), (777, 64, 2),
                                             (300, 65, 5), (40, 300, 3), (3, 5000, 2), (40000, 100, 2),
                                             (70000, 72, 1), (2000, 23, 7)])
def test_keyed_log_fold_is_the_oracle_bitwise(gpu, keys, rows, width):
    """The ordered gradient's fold through the C-ABI (a thread per (key, slot)
    for runs of up to 64 rows or 65536 pairs and more, a wave per pair
    otherwise): bit for bit the oracle's serial loop; cells no pair names keep
    their values."""
    g = rng(keys + 7 * rows + 31 * width)
    v = g.normal(size=(width, keys * rows)) * np.exp(3 * g.normal(size=(width, keys * rows)))
    cells = keys * width + 13
    c = g.permutation(cells)[:keys * width].reshape(width, keys).astype(np.int32)
    init = g.normal(size=cells)
    want = init.copy()
    assert O.keyed_log_fold(v, c, rows, want) == 0
    print(f"log fold keys={keys} rows={rows} width={width}", flush=True)
    out, status = _log_fold(gpu, v, c, rows, init)
    assert out.tobytes() == want.tobytes()
    assert status == [0, 2 ** 31 - 1]


@pytest.mark.parametrize("rows", [10, 100])
def test_keyed_log_fold_reports_a_cell_named_twice_and_one_outside(gpu, rows):
    keys, width = 100, 2
    g = rng(rows)
    v = g.normal(size=(width, keys * rows))
    cells = keys * width
    c = g.permutation(cells).reshape(width, keys).astype(np.int32)
    twice = c.copy()
    twice[1, 7] = c[0, 3]
    print(f"log fold collision rows={rows}", flush=True)
    out, status = _log_fold(gpu, v, twice, rows, np.zeros(cells))
    assert status == [2, int(c[0, 3])]
    sums = [sum(float(x) for x in v[e, k * rows:(k + 1) * rows]) for e, k in ((0, 3), (1, 7))]
    assert out[c[0, 3]] in sums
    outside = c.copy()
    outside[0, 5] = cells + 4
    out, status = _log_fold(gpu, v, outside, rows, np.full(cells, 9.0))
    assert status[0] == 1 and out[c[0, 5]] == 9.0


@pytest.mark.parametrize("s", [40, 48, 96])
def test_net_gradients_through_the_ordered_fold(gpu, tmp_path, s):
    """16384 nets in one launch (reference tests/test_net_axis.py:163-177):
    the ordered loss equals the numpy loop and the C oracle; the gradient wrt
    the per-net weights is the same bits on three launches, equals the loop
    at 256 nets and the oracle at all of them within the reference's 1e-10,
    and is exactly 0 on masked units.  The stage that folds in LDS and the
    stage that logs for a fold stage give the same bits, and those are the
    oracle's fold of the log, bit for bit (the logged contributions and cells
    are the IR's, within 1e-10 and exactly)."""
    import hawk_amd as hawk
    from hawk_amd import examples as E
    from hawk_amd.diff import vjp
    from hawk_amd.trace import Kernel
    from ir_eval import evaluate
    from net_axis import net_problem
    net = E.net_loss_for(s)
    back = Kernel(f"net_grad_{s}", vjp(net, wrt=("W",)))
    hawk.build([net, back], tmp_path / "fused")
    hawk.build([back], tmp_path / "logged", fuse_folds=False)
    k = 16384
    n = k * s
    pick = rng(1).choice(k, 256, replace=False)
    w, x, y, mask, loss, grad = net_problem(k, s, 3, pick)
    W, M, X, Y = dev(w.ravel(), gpu), dev(mask.ravel(), gpu), dev(x.ravel(), gpu), dev(y.ravel(), gpu)
    out = dev(np.zeros(k), gpu)
    print(f"net loss s={s}", flush=True)
    hawk.run(hawk.load(tmp_path / "fused", net.name), W=W, mask=M, x=X, y=Y, out=out)
    np.testing.assert_allclose(host(out)[pick], loss, rtol=1e-12)
    np.testing.assert_allclose(host(out), O.net_loss(w, mask, x, y, threads=8), rtol=1e-12)
    kf, kl = hawk.load(tmp_path / "fused", back.name), hawk.load(tmp_path / "logged", back.name)
    assert [t["op"] for t in kf.team] == ["fused_fold"] and [t["op"] for t in kl.team] == ["ordered_fold"]
    seen = []
    for kern in (kf, kf, kf, kl):
        bw = dev(np.zeros(k * E.NET_WEIGHTS), gpu)
        print(f"net grad s={s} {kern.team[0]['op']}", flush=True)
        hawk.run(kern, W=W, mask=M, x=X, y=Y, bar_out=dev(np.ones(k), gpu), bar_W=bw)
        seen.append(host(bw).reshape(k, -1))
    assert seen[0].tobytes() == seen[1].tobytes() == seen[2].tobytes() == seen[3].tobytes()
    np.testing.assert_allclose(seen[0][pick], grad, rtol=1e-10, atol=1e-10)
    np.testing.assert_allclose(seen[0], O.net_grad(w, mask, x, y, np.ones(k), threads=8), rtol=1e-10, atol=1e-10)
    dead = np.repeat(mask == 0.0, 3, axis=1)
    assert (seen[0][dead] == 0.0).all() and (seen[0][~dead] != 0.0).all()
    logv = host(kl._scratch[("plane", "hk_logv_bar_W", n)])
    logc = host(kl._scratch[("plane", "hk_logc_bar_W", n)])
    refold = np.zeros(k * E.NET_WEIGHTS)
    assert O.keyed_log_fold(logv, logc, s, refold) == 0
    assert refold.tobytes() == seen[0].tobytes()
    env = {"W": w.ravel(), "mask": mask.ravel(), "x": x.ravel(), "y": y.ravel(), "bar_out": np.ones(k)}
    values, cells = evaluate(back.program, env, n)["bar_W"]
    np.testing.assert_allclose(logv, np.stack(values), rtol=1e-10, atol=1e-12)
    assert (logc == np.stack([c[::s] for c in cells])).all()


def _keyed_table_kernel(group):
    import hawk_amd as hawk
    from hawk_amd import Grid, Scalar, Table

    @hawk.kernel
    def kt(lane: Grid["key", "sample":group], t: Table["key", "w":3], x: Scalar) -> Scalar:
        a, b, c = t.at(key=lane.key, w=0), t.at(key=lane.key, w=1), t.at(key=lane.key, w=2)
        return hawk.sum(a * x * x + b * x + c, over="sample", policy="ordered")
    return kt


@pytest.mark.parametrize("keys,group", [(1000, 40), (777, 64), (500, 48), (3001, 5), (5000, 1), (300, 100),
                                        (9, 2000), (4099, 64)])
def test_ordered_fold_in_lds_and_through_a_log_are_the_oracles_bits(gpu, tmp_path, keys, group):
    """A keyed kernel whose contributions are products (numpy has their bits):
    the gradient wrt a per-key table, folded in the stage's LDS where the
    keys fit a block (groups 40, 64, 48, 5, 1) and through the log and the
    fold stage otherwise (100, 2000), is the oracle's fold of the IR's
    contributions, bit for bit, on a full and a partial last block."""
    import hawk_amd as hawk
    from hawk_amd.diff import vjp
    from hawk_amd.emit_hip import fold_block
    from hawk_amd.trace import Kernel
    from ir_eval import evaluate
    back = Kernel("kt_vjp", vjp(_keyed_table_kernel(group), wrt=("t",)))
    hawk.build([back], tmp_path)
    kern = hawk.load(tmp_path, "kt_vjp")
    assert kern.team[0]["op"] == ("fused_fold" if fold_block(group) else "ordered_fold")
    n = keys * group
    g = rng(keys + group)
    t, x, bar = g.normal(size=keys * 3), g.normal(size=n), g.normal(size=keys)
    bt = dev(np.full(keys * 3, np.nan), gpu)
    print(f"fold keys={keys} group={group} {kern.team[0]['op']}", flush=True)
    hawk.run(kern, t=dev(t, gpu), x=dev(x, gpu), bar_out=dev(bar, gpu), bar_t=bt)
    values, cells = evaluate(back.program, {"t": t, "x": x, "bar_out": bar}, n)["bar_t"]
    want = np.full(keys * 3, np.nan)
    assert O.keyed_log_fold(np.stack(values), np.stack([c[::group] for c in cells]), group, want) == 0
    assert host(bt).tobytes() == want.tobytes()


def _shared_cell_kernel():
    import hawk_amd as hawk
    from hawk_amd import Grid, Scalar, Table

    @hawk.kernel
    def shared_cell(lane: Grid["key", "sample":4], t: Table[Scalar], x: Scalar) -> Scalar:
        return hawk.sum(t.at(0) * x + t.at(lane.key) * x, over="sample", policy="ordered")
    return shared_cell


def test_a_table_cell_every_key_reads_is_reported(gpu, tmp_path):
    """Under an ordered keyed sum each cell's gradient is stored from one
    key's sum (reference hawk/emit/team.py:281-312): a cell every key reads
    (t.at(0)) would race, so the run names it instead of returning its bits."""
    import hawk_amd as hawk
    from hawk_amd import HawkError
    from hawk_amd.diff import vjp
    from hawk_amd.trace import Kernel
    back = Kernel("shared_cell_vjp", vjp(_shared_cell_kernel(), wrt=("t",)))
    hawk.build([back], tmp_path)
    keys = 50
    x = rng(5).normal(size=keys * 4)
    bt = dev(np.zeros(keys), gpu)
    print("shared cell vjp", flush=True)
    with pytest.raises(HawkError, match="cell 0 of bar_t is read by more than one key"):
        hawk.run(hawk.load(tmp_path, back.name), t=dev(np.ones(keys), gpu), x=dev(x, gpu),
                 bar_out=dev(np.ones(keys), gpu), bar_t=bt)


# -- hawk.chain -------------------------------------------------------------------

def test_chain_is_its_members_launched_in_turn(gpu, tmp_path):
    """One fused launch of the chain (reference tests/test_chain.py:150-177)
    gives the bits of the four members launched one after another through
    planes, twice, within the fp64 bar of the C oracle's chain of the same
    members; its JVP and VJP are within the reference's bound of the
    long-double chain rule."""
    import chain_members as C
    import hawk_amd as hawk
    from hawk_amd.diff import jvp, vjp
    from hawk_amd.trace import Kernel
    chained = hawk.chain(*C.MEMBERS, name="fixture")
    tangent = Kernel("fixture_jvp", jvp(hawk.chain(C.unit_circle, C.decay, C.scale_vec, name="d"), wrt=("x",)))
    adjoint = Kernel("fixture_vjp", vjp(hawk.chain(C.unit_circle, C.decay, C.scale_vec, name="d"), wrt=("x",)))
    hawk.build([chained, *C.MEMBERS, tangent, adjoint], tmp_path)
    n = 100_003
    g = rng(5)
    x, acc0 = g.uniform(0.1, 2.0, n), g.uniform(0.0, 1.0, n)
    X = dev(x, gpu)
    runs = []
    for _ in range(2):
        acc, y = dev(acc0, gpu), dev(np.zeros((3, n)), gpu)
        print("chain fused", flush=True)
        hawk.run(hawk.load(tmp_path, "fixture"), x=X, acc=acc, y=y)
        runs.append((host(acc), host(y)))
    assert runs[0][0].tobytes() == runs[1][0].tobytes() and runs[0][1].tobytes() == runs[1][1].tobytes()
    a, b = dev(np.zeros((3, n)), gpu), dev(np.zeros(n), gpu)
    acc, y = dev(acc0, gpu), dev(np.zeros((3, n)), gpu)
    print("chain members", flush=True)
    hawk.run(hawk.load(tmp_path, "unit_circle"), x=X, a=a)
    hawk.run(hawk.load(tmp_path, "decay"), a=a, x=X, b=b)
    hawk.run(hawk.load(tmp_path, "accumulate"), b=b, acc=acc)
    hawk.run(hawk.load(tmp_path, "scale_vec"), a=a, b=b, y=y)
    assert runs[0][0].tobytes() == host(acc).tobytes() and runs[0][1].tobytes() == host(y).tobytes()
    want_acc = acc0.copy()
    want_y = O.chain_members(x, want_acc)             # the C oracle (glibc sin/cos/exp), acc updated in place
    assert within_contract(runs[0][1], want_y).all() and within_contract(runs[0][0], want_acc).all()
    # the derivatives against the long-double chain rule, within the reference's bound: 16 eps of the
    # output's largest magnitude (tests/test_chain.py:47-54; the terms of dy/dx cancel)
    ld = np.longdouble
    xl = x.astype(ld)
    a = np.stack([np.sin(xl), np.cos(xl), xl * ld("0.5")])
    da = np.stack([np.cos(xl), -np.sin(xl), np.full(n, ld("0.5"))])
    e = np.exp(-(a * a).sum(axis=0))
    dydx = da * (e + xl) + a * (e * (-2 * (a * da).sum(axis=0)) + 1)
    bound = lambda ref: 16 * np.finfo(np.float64).eps * float(np.max(np.abs(ref)))
    dy = dev(np.zeros((3, n)), gpu)
    hawk.run(hawk.load(tmp_path, "fixture_jvp"), x=X, dot_x=dev(np.ones(n), gpu), dot_y=dy)
    assert float(np.max(np.abs(host(dy).astype(ld) - dydx))) <= bound(dydx)
    seed = g.uniform(0.5, 1.5, (3, n))
    bx = dev(np.zeros(n), gpu)
    hawk.run(hawk.load(tmp_path, "fixture_vjp"), x=X, bar_y=dev(seed, gpu), bar_x=bx)
    want = (seed.astype(ld) * dydx).sum(axis=0)
    assert float(np.max(np.abs(host(bx).astype(ld) - want))) <= bound(want)


# -- the default policy over some axes --------------------------------------------

def _keyed_default_kernel(group):
    import hawk_amd as hawk
    from hawk_amd import Grid, Scalar

    @hawk.kernel
    def kdefault(lane: Grid["key", "sample":group], x: Scalar) -> Scalar:
        return hawk.sum(x, over="sample")
    return kdefault


@pytest.mark.parametrize("keys,group", [(4, 8), (1000, 40), (65536, 64), (3, 4096 * 32 + 5), (5000, 1),
                                        (10, 100_000), (1, 1000), (777, 33), (50, 2048), (50, 2049), (7, 8191)])
def test_keyed_default_sum_is_the_oracle_bitwise(gpu, tmp_path, keys, group):
    """hawk.sum(x, over=<trailing axes>) under the default policy: each key's
    run is a default-policy sample sum of its own (compensated rows of 32 from
    the key's first sample, the canonical finish), bit for bit the oracle's,
    the same bits on a second launch; one key is the whole run's default sum.
    Keys of up to 2048 samples take a wave each, longer ones a workgroup."""
    import hawk_amd as hawk
    hawk.build([_keyed_default_kernel(group)], tmp_path)
    kern = hawk.load(tmp_path, "kdefault")
    assert [t["op"] for t in kern.team] == ["keyed_comp"]
    n = keys * group
    x = rng(keys + group).normal(size=n) * np.exp(rng(3).normal(size=n))
    X = dev(x, gpu)
    print(f"keyed default sum keys={keys} group={group}", flush=True)
    outs = []
    for _ in range(2):
        out = dev(np.full(keys, np.nan), gpu)
        hawk.run(kern, x=X, out=out)
        outs.append(host(out))
    want = O.keyed_sample_sum(x, group)
    assert outs[0].tobytes() == want.tobytes() == outs[1].tobytes()
    if keys == 1:
        assert outs[0][0] == O.sample_sum(x)


def test_net_loss_and_gradient_under_the_default_policy(gpu, tmp_path):
    """The reference's default net axis (tests/test_net_axis.py:103-110,
    :208-223): 16384 nets of 40 samples, the loss equal to the loop (rtol
    1e-12) and to the ordered loss within 8 S eps, the same bits on a second
    launch; its gradient wrt W (an ordered scatter of each read's
    contribution: no ordered keyed sum to fold under) equal to the loop at
    256 nets within 1e-10 and the same bits on a second launch."""
    import hawk_amd as hawk
    from hawk_amd import examples as E
    from hawk_amd.diff import vjp
    from hawk_amd.trace import Kernel
    from net_axis import net_problem
    s, k = 40, 16384
    net, ordered = E.net_loss_for(s, "auto"), E.net_loss_for(s)
    back = Kernel("net_grad_default", vjp(net, wrt=("W",)))
    hawk.build([net, ordered, back], tmp_path)
    assert [t["op"] for t in hawk.load(tmp_path, back.name).team] == ["ordered_scatter"] * E.NET_WEIGHTS
    pick = rng(1).choice(k, 256, replace=False)
    w, x, y, mask, loss, grad = net_problem(k, s, 3, pick)
    W, M, X, Y = dev(w.ravel(), gpu), dev(mask.ravel(), gpu), dev(x.ravel(), gpu), dev(y.ravel(), gpu)
    runs = []
    for name in (net.name, net.name, ordered.name):
        out = dev(np.zeros(k), gpu)
        print(f"net loss {name}", flush=True)
        hawk.run(hawk.load(tmp_path, name), W=W, mask=M, x=X, y=Y, out=out)
        runs.append(host(out))
    assert runs[0].tobytes() == runs[1].tobytes()
    np.testing.assert_allclose(runs[0][pick], loss, rtol=1e-12)
    np.testing.assert_allclose(runs[0], runs[2], rtol=8 * s * np.finfo(np.float64).eps)
    seen = []
    for _ in range(2):
        bw = dev(np.zeros(k * E.NET_WEIGHTS), gpu)
        print("net grad default", flush=True)
        hawk.run(hawk.load(tmp_path, back.name), W=W, mask=M, x=X, y=Y, bar_out=dev(np.ones(k), gpu), bar_W=bw)
        seen.append(host(bw).reshape(k, -1))
    assert seen[0].tobytes() == seen[1].tobytes()
    np.testing.assert_allclose(seen[0][pick], grad, rtol=1e-10, atol=1e-10)


def test_a_cut_chain_is_the_fused_chain(gpu, tmp_path):
    """A chain cut at every boundary (a register line of 32, reference
    tests/test_chain.py:298-334) runs as four segment kernels through hwc_
    planes and gives the fused chain's bits, by hawk.run and by prepare."""
    import chain_members as C
    import hawk_amd as hawk
    chained = hawk.chain(*C.MEMBERS, name="fixture")
    hawk.build([chained], tmp_path / "fused")
    hawk.build([chained], tmp_path / "cut", register_line=32)
    cut = hawk.load(tmp_path / "cut", "fixture")
    assert [s.name for s in cut.segments] == [f"fixture__s{i}" for i in range(4)]
    n = 100_003
    g = rng(8)
    x, acc0 = g.uniform(0.1, 2.0, n), g.uniform(0.0, 1.0, n)
    X = dev(x, gpu)
    got = []
    for kern, how in ((hawk.load(tmp_path / "fused", "fixture"), "run"), (cut, "run"), (cut, "prepare")):
        acc, y = dev(acc0, gpu), dev(np.zeros((3, n)), gpu)
        print(f"chain {how} {type(kern).__name__}", flush=True)
        if how == "run":
            hawk.run(kern, x=X, acc=acc, y=y)
        else:
            kern.prepare(x=X, acc=acc, y=y)()
        got.append((host(acc).tobytes(), host(y).tobytes()))
    assert got[0] == got[1] == got[2]
    # the cut chain with its Vector[3] output sample-major, (N, 3), under layout='samples_first'
    acc, y = dev(acc0, gpu), dev(np.zeros((n, 3)), gpu)
    print("chain run samples_first", flush=True)
    hawk.run(cut, x=X, acc=acc, y=y, layout="samples_first")
    assert host(acc).tobytes() == got[0][0]
    assert np.ascontiguousarray(host(y).T).tobytes() == got[0][1]


def test_folds_and_keyed_sums_keep_ieee_specials_and_empty_runs(gpu, tmp_path):
    """Inf, NaN and -0 through the ordered fold (in LDS and logged) and the
    keyed sums, against the oracle bit for bit (NaN as NaN); a run of no
    samples leaves the outputs as they were."""
    import hawk_amd as hawk
    from hawk_amd.diff import vjp
    from hawk_amd.trace import Kernel
    from ir_eval import evaluate
    group, keys = 40, 300
    back = Kernel("kt_vjp", vjp(_keyed_table_kernel(group), wrt=("t",)))
    hawk.build([back], tmp_path / "fused")
    hawk.build([back], tmp_path / "logged", fuse_folds=False)
    hawk.build([_keyed_default_kernel(group), _keyed_kernels(group)], tmp_path / "sums")
    n = keys * group
    g = rng(17)
    t, x, bar = g.normal(size=keys * 3), g.normal(size=n), g.normal(size=keys)
    x[5], x[n // 2], x[n - 1], x[77] = np.inf, -np.inf, np.nan, -0.0
    t[4] = np.inf
    values, cells = evaluate(back.program, {"t": t, "x": x, "bar_out": bar}, n)["bar_t"]
    want = np.zeros(keys * 3)
    assert O.keyed_log_fold(np.stack(values), np.stack([c[::group] for c in cells]), group, want) == 0
    for sub in ("fused", "logged"):
        bt = dev(np.zeros(keys * 3), gpu)
        print(f"fold specials {sub}", flush=True)
        hawk.run(hawk.load(tmp_path / sub, "kt_vjp"), t=dev(t, gpu), x=dev(x, gpu), bar_out=dev(bar, gpu), bar_t=bt)
        got = host(bt)
        assert np.array_equal(np.isnan(got), np.isnan(want))
        assert got[~np.isnan(got)].tobytes() == want[~np.isnan(want)].tobytes()
    for name, oracle in (("kdefault", O.keyed_sample_sum), ("ksum", O.keyed_ordered_sum)):
        out = dev(np.full(keys, 3.0), gpu)
        print(f"keyed specials {name}", flush=True)
        hawk.run(hawk.load(tmp_path / "sums", name), x=dev(x, gpu), out=out)
        got, w = host(out), oracle(x, group)
        assert np.array_equal(np.isnan(got), np.isnan(w)) and got[~np.isnan(got)].tobytes() == w[~np.isnan(w)].tobytes()
    # no samples: nothing written
    bt = dev(np.full(keys * 3, 7.0), gpu)
    hawk.run(hawk.load(tmp_path / "fused", "kt_vjp"), t=dev(t, gpu), x=dev(np.zeros(0), gpu),
             bar_out=dev(np.zeros(0), gpu), bar_t=bt)
    assert (host(bt) == 7.0).all()


# -- banded reductions ------------------------------------------------------------

def _band_data(kind, n):
    V = 65536
    if kind == "cancel_lanes":          # each virtual lane of the ordered tree cancels 2^60 against itself
        reps = -(-n // (4 * V))
        block = np.concatenate([np.full(V, 2.0 ** 60), np.ones(V), np.full(V, -(2.0 ** 60)), np.ones(V)])
        return np.tile(block, reps)[:n]
    if kind == "reference_series":      # the reference's float32-exact 2^30 cancelling series
        return np.tile([2.0 ** 30, 1.0, -(2.0 ** 30), 1.0], n // 4 + 1)[:n].astype(np.float32).astype(np.float64)
    if kind == "exact_integers":        # every partial fits a double-double
        k = rng(n).integers(-(1 << 40), 1 << 40, n, dtype=np.int64)
        return k.astype(np.float64) * 2.0 ** -20
    if kind == "one_lane":              # seven terms on one virtual lane's rows (l, l + 8192, ...), zeros elsewhere
        from test_oracle import BAND_LANE_TERMS
        x = np.zeros(n)
        rows = 5 + 8192 * np.arange(7)
        x[rows[rows < n]] = np.array(BAND_LANE_TERMS)[rows < n]
        return x
    g = rng(n + 7)
    return g.normal(size=n) * np.exp(g.normal(size=n) * 8)


@pytest.mark.parametrize("kind", ["cancel_lanes", "reference_series", "exact_integers", "wide", "one_lane"])
@pytest.mark.parametrize("n", [1, 31, 33, 1000, 8193, 65537, 3 * 65536 + 777, (1 << 20) + 5])
def test_banded_sums_are_the_oracles_bits_and_replay(unit_banded, gpu, kind, n):
    """The banded mode's sample sums on the device (band rows in the stage, the
    banded canonical finish, the banded ordered tree) are the oracle's bits,
    on every one of three launches."""
    import hawk_amd as hawk
    x = _band_data(kind, n)
    X = dev(x, gpu)
    k = _load(unit_banded, "band_total")
    want = (O.band_sample_sum(x), O.band_sample_sum(x * x), O.band_ordered_sum(x))
    print(f"band_total {kind} n={n}", flush=True)
    for _ in range(3):
        cells = {c: dev(np.full(1, np.nan), gpu) for c in ("s", "s_sq", "s_ord")}
        hawk.run(k, x=X, **cells)
        got = tuple(float(host(cells[c])[0]) for c in ("s", "s_sq", "s_ord"))
        assert np.array(got).tobytes() == np.array(want).tobytes(), (got, want)
    if kind == "one_lane" and n > 6 * 8192 + 5:
        from test_oracle import BAND_LANE_TERMS
        assert want[2] == BAND_LANE_TERMS[1]          # the reference's geometry: one band of seven terms


@pytest.mark.parametrize("kind", ["cancel_lanes", "wide"])
@pytest.mark.parametrize("n", [9 * 8192 * 32 + 12345, (1 << 24) + 3])
def test_band_ordered_sum_across_many_stages(unit_banded, gpu, kind, n):
    """The banded ordered sum where each virtual lane's walk spans many
    32-row stages of the lanes kernel's ring (10 stages, the last partial and
    not a multiple of the four loader register sets; and 64 stages): the
    oracle's bits."""
    import hawk_amd as hawk
    x = _band_data(kind, n)
    k = _load(unit_banded, "band_total")
    print(f"band_total stages {kind} n={n}", flush=True)
    cells = {c: dev(np.full(1, np.nan), gpu) for c in ("s", "s_sq", "s_ord")}
    hawk.run(k, x=dev(x, gpu), **cells)
    assert float(host(cells["s_ord"])[0]) == O.band_ordered_sum(x)


def test_banded_sums_on_the_device_hold_the_reference_bounds(unit_banded, gpu):
    """Against exact rational sums: the reference's cancelling series within
    0.01 ULP53 (tests/test_banded_sum.py), a lane-cancelling series the plain
    fixed tree gets wrong held exactly, and exact-integer data rounded once."""
    from fractions import Fraction

    import hawk_amd as hawk
    k = _load(unit_banded, "band_total")

    def run(x):
        cells = {c: dev(np.zeros(1), gpu) for c in ("s", "s_sq", "s_ord")}
        hawk.run(k, x=dev(x, gpu), **cells)
        return {c: float(host(v)[0]) for c, v in cells.items()}
    x = _band_data("reference_series", 3 * 65536 + 777)
    exact = sum(Fraction(float(v)) for v in x)
    got = run(x)
    for c in ("s", "s_ord"):
        assert abs(Fraction(got[c]) - exact) <= Fraction(1, 100) * Fraction(float(np.spacing(float(exact))))
    x = _band_data("cancel_lanes", 4 * 65536)
    got = run(x)
    assert got["s_ord"] == got["s"] == 2.0 * 65536
    assert O.ordered_sum(x) == 65536.0                       # the plain fixed tree loses a term a lane
    x = _band_data("exact_integers", (1 << 20) + 5)
    k_int = (x * 2.0 ** 20).astype(np.int64)
    want = float(Fraction(int(k_int.sum()), 1 << 20))
    got = run(x)
    assert got["s"] == got["s_ord"] == want


# -- the float32 mode's ordered reductions ----------------------------------

@pytest.mark.parametrize("n", golden("ordered_sum_sizes")["sizes"])
def test_float32_ordered_sum_is_the_float32_tree_bitwise(unit32, gpu, n):
    """hawk.sum(x, policy="ordered") in a float32 build: every lane sum and
    tree level a float addition (the reference's team stages add `Real`s):
    the float32 oracle's bits, NumPy's float32 tree, on three launches."""
    import hawk_amd as hawk
    g = rng(n + 32)
    x = (g.normal(size=n) * np.exp(g.normal(size=n))).astype(np.float32)
    k = _load(unit32, "ordered_total")
    runs = []
    for _ in range(3):
        total = dev(np.zeros(1, np.float32), gpu)
        hawk.run(k, x=dev(x, gpu), total=total)
        runs.append(host(total))
    assert runs[0].dtype == np.float32
    assert runs[0].tobytes() == runs[1].tobytes() == runs[2].tobytes()
    assert runs[0][0].tobytes() == O.ordered_sum(x).tobytes() == np.float32(tree_sum(x)).tobytes()


@pytest.mark.parametrize("cells, n, heavy", [(7, 30_000, False), (1000, 30_000, False), (7, 20_000, True),
                                             (3, 1000, False), (65536, 400_000, False), (12289, 300_001, False),
                                             (40_000, 2_000_003, True), (70_000, 300_000, False),
                                             (600_000, 1_300_000, False)])
def test_float32_ordered_scatter_is_the_float32_walk_bitwise(unit32, gpu, cells, n, heavy):
    """hawk.scatter(acc, policy="ordered")[key] += x in a float32 build, through
    every form of the walk (split walk with and without tail ranges, sorted
    walk, serial walk): the float32 oracle's bits, the same on a replay."""
    import hawk_amd as hawk
    g = rng(cells + n + 32)
    key = g.integers(0, cells, n).astype(np.int32)
    if heavy:
        key[g.random(n) < 0.9] = cells // 2
    key[::7] = -1
    print(f"float32 scatter cells={cells} n={n} heavy={heavy}", flush=True)
    x = (g.normal(size=n) * np.exp(g.normal(size=n))).astype(np.float32)
    acc0 = np.linspace(1.0, 2.0, cells).astype(np.float32)
    k = _load(unit32, "ordered_add")
    outs = []
    for _ in range(2):
        acc = dev(acc0, gpu)
        hawk.run(k, key=dev(key, gpu), x=dev(x, gpu), acc=acc)
        outs.append(host(acc))
    want, status = O.ordered_scatter(key, x, acc0)
    assert not status[1:].any() and want.dtype == np.float32
    assert outs[0].tobytes() == outs[1].tobytes() == want.tobytes()


def test_float32_scatter_of_a_computed_value_and_zipf_keys(unit32, gpu):
    """A float32 stage computes x*x into its own plane and the float32 scatter
    folds it at config 5's Zipf keys into 65536 cells: the oracle's bits."""
    import hawk_amd as hawk
    n, cells = 1 << 20, 1 << 16
    g = rng(321)
    key = ((g.zipf(1.1, n) - 1) % cells).astype(np.int32)
    x = g.normal(size=n).astype(np.float32)
    acc0 = g.normal(size=cells).astype(np.float32)
    acc = dev(acc0, gpu)
    hawk.run(_load(unit32, "add_sq"), key=dev(key, gpu), x=dev(x, gpu), acc=acc)
    want, _ = O.ordered_scatter(key, (x * x).astype(np.float32), acc0)
    assert host(acc).tobytes() == want.tobytes()


@pytest.mark.parametrize("keys, group", [(4, 8), (1000, 5000), (3, 200003), (70000, 7), (17, 1025), (3000, 2)])
def test_float32_keyed_ordered_sum_bitwise(gpu, tmp_path, keys, group):
    """hawk.sum(x, over=<trailing axes>, policy="ordered") in a float32 build:
    each key's run by the fixed tree in float, the float32 oracle's bits."""
    import hawk_amd as hawk
    hawk.build([_keyed_kernels(group)], tmp_path, mode="float32")
    kern = hawk.load(tmp_path, "ksum")
    n = keys * group
    x = (rng(70 + group).uniform(-2.0, 2.0, n) * np.exp(rng(8).normal(size=n))).astype(np.float32)
    print(f"float32 keyed sum keys={keys} group={group}", flush=True)
    out = dev(np.full(keys, np.nan, np.float32), gpu)
    hawk.run(kern, x=dev(x, gpu), out=out)
    assert host(out).tobytes() == O.keyed_ordered_sum(x, group).tobytes()


@pytest.mark.parametrize("keys,group", [(4, 8), (1000, 40), (3, 4096 * 32 + 5), (5000, 1), (10, 100_000),
                                        (777, 33), (50, 2049)])
def test_float32_keyed_default_sum_is_the_oracle_bitwise(gpu, tmp_path, keys, group):
    """The default policy over some axes in a float32 build: each key's run a
    float32 default-policy sample sum of its own (float rows and compensation,
    the canonical finish in float32), the float32 oracle's bits; one key is
    the whole run's float32 default sum."""
    import hawk_amd as hawk
    hawk.build([_keyed_default_kernel(group)], tmp_path, mode="float32")
    kern = hawk.load(tmp_path, "kdefault")
    assert [t["op"] for t in kern.team] == ["keyed_comp"]
    n = keys * group
    x = (rng(keys + group + 32).normal(size=n) * np.exp(rng(3).normal(size=n))).astype(np.float32)
    print(f"float32 keyed default sum keys={keys} group={group}", flush=True)
    out = dev(np.full(keys, np.nan, np.float32), gpu)
    hawk.run(kern, x=dev(x, gpu), out=out)
    got = host(out)
    assert got.dtype == np.float32 and got.tobytes() == O.keyed_sample_sum(x, group).tobytes()


@pytest.mark.parametrize("keys,rows,width", [(1000, 1, 3), (5000, 40, 24), (300, 65, 5), (3, 5000, 2),
                                             (70000, 72, 1)])
def test_float32_keyed_log_fold_is_the_oracle_bitwise(gpu, keys, rows, width):
    """The float32 fold through the C-ABI, on both of its forms (a thread a
    pair, a wave a pair): each run added in float from +0 in lane order, the
    float32 oracle's bits; cells no pair names keep their values."""
    g = rng(keys + 7 * rows + 31 * width + 32)
    v = (g.normal(size=(width, keys * rows)) * np.exp(3 * g.normal(size=(width, keys * rows)))).astype(np.float32)
    cells = keys * width + 13
    c = g.permutation(cells)[:keys * width].reshape(width, keys).astype(np.int32)
    init = g.normal(size=cells).astype(np.float32)
    want = init.copy()
    assert O.keyed_log_fold(v, c, rows, want) == 0
    print(f"float32 log fold keys={keys} rows={rows} width={width}", flush=True)
    out, status = _log_fold(gpu, v, c, rows, init)
    assert out.dtype == np.float32 and out.tobytes() == want.tobytes()
    assert status == [0, 2 ** 31 - 1]


@pytest.mark.parametrize("keys,group", [(1000, 40), (777, 64), (3001, 5), (300, 100), (9, 2000)])
def test_float32_ordered_fold_in_lds_and_through_a_log(gpu, tmp_path, keys, group):
    """The gradient wrt a per-key table under an ordered keyed sum in a
    float32 build, folded in the stage's LDS (groups 40, 64, 5) and through
    the log and the fold stage (100, 2000).  Integer inputs keep every
    product and sum exact in float32, so the float32 gradient equals the
    IR's contributions folded exactly."""
    import hawk_amd as hawk
    from hawk_amd.diff import vjp
    from hawk_amd.emit_hip import fold_block
    from hawk_amd.trace import Kernel
    from ir_eval import evaluate
    back = Kernel("kt_vjp", vjp(_keyed_table_kernel(group), wrt=("t",)))
    hawk.build([back], tmp_path, mode="float32")
    kern = hawk.load(tmp_path, "kt_vjp")
    assert kern.team[0]["op"] == ("fused_fold" if fold_block(group) else "ordered_fold")
    n = keys * group
    g = rng(keys + group + 32)
    t = g.integers(-4, 5, keys * 3).astype(np.float32)
    x = g.integers(-8, 9, n).astype(np.float32)
    bar = g.integers(-4, 5, keys).astype(np.float32)
    bt = dev(np.full(keys * 3, np.nan, np.float32), gpu)
    print(f"float32 fold keys={keys} group={group} {kern.team[0]['op']}", flush=True)
    hawk.run(kern, t=dev(t, gpu), x=dev(x, gpu), bar_out=dev(bar, gpu), bar_t=bt)
    values, cells = evaluate(back.program, {"t": t.astype(np.float64), "x": x.astype(np.float64),
                                            "bar_out": bar.astype(np.float64)}, n)["bar_t"]
    want = np.full(keys * 3, np.nan)
    assert O.keyed_log_fold(np.stack(values), np.stack([c[::group] for c in cells]), group, want) == 0
    assert (np.abs(want) < 2.0 ** 24).all()                       # exact in float32
    assert host(bt).tobytes() == want.astype(np.float32).tobytes()


def test_sample_major_planes_through_hawk_run(unit, gpu):
    """hawk.run with (N, w) planes (reference hawk/runtime.py:542-566): the
    energy forward and VJP on sample-major v give the component-major run's
    bits, the VJP's sample-major bar_v is written back, layout= resolves a
    plane that reads both ways, and prepare refuses a marked plane."""
    import hawk_amd as hawk
    n = 10_007
    v = rng(61).normal(size=(3, n))
    bar_out = rng(62).normal(size=n)
    want = dev(np.zeros(n), gpu)
    hawk.run(_load(unit, "energy"), v=dev(v, gpu), out=want)
    got = dev(np.zeros(n), gpu)
    hawk.run(_load(unit, "energy"), v=dev(np.ascontiguousarray(v.T), gpu), out=got)
    assert host(got).tobytes() == host(want).tobytes()
    bv_soa = dev(np.zeros((3, n)), gpu)
    hawk.run(_load(unit, "energy_vjp"), v=dev(v, gpu), bar_out=dev(bar_out, gpu), bar_v=bv_soa)
    bv_aos = dev(np.zeros((n, 3)), gpu)
    hawk.run(_load(unit, "energy_vjp"), v=hawk.samples_first(dev(np.ascontiguousarray(v.T), gpu)),
             bar_out=dev(bar_out, gpu), bar_v=bv_aos)
    assert host(bv_aos).tobytes() == np.ascontiguousarray(host(bv_soa).T).tobytes()
    three = rng(63).normal(size=(3, 3))
    out3 = dev(np.zeros(3), gpu)
    with pytest.raises(hawk.HawkError, match="reads both as"):
        hawk.run(_load(unit, "energy"), v=dev(three, gpu), out=out3)
    hawk.run(_load(unit, "energy"), v=dev(three, gpu), out=out3, layout="samples_first")
    assert np.allclose(host(out3), 0.5 * (three * three).sum(axis=1), rtol=1e-15, atol=0)
    with pytest.raises(hawk.HawkError, match="prepare binds planes by address"):
        _load(unit, "energy").prepare(v=hawk.samples_first(dev(three, gpu)), out=out3)
