"""The target's own fp64 exp, sin, cos and tanh (``hawk_amd/emit_hip.py``
``_MATH_HELPERS``), built from the same text by the host compiler and held to
glibc, the reference's host math (reference tests/test_math_parity.py:279:
host ``native`` is glibc bit for bit; the device is held within ULP of it).

The helpers use only IEEE operations, so a host build (tests/math_host.py)
computes the device's bits; tests/test_gpu_parity.py holds the device to
the host build's bits and to the same glibc values."""

import numpy as np
import pytest

from conftest import ulp_diff


@pytest.fixture(scope="module")
def helpers(tmp_path_factory):
    import math_host
    return math_host.build(tmp_path_factory.mktemp("math"))


def _sweep(which, g):
    if which == "tanh":
        return np.concatenate([g.uniform(-2, 2, 300_000), g.normal(size=50_000) * 1e-3, g.uniform(-30, 30, 100_000),
                               np.exp(g.uniform(-700, 3, 50_000)) * np.sign(g.normal(size=50_000)),
                               np.arange(-23, 23, 1e-3)])
    if which == "exp":
        return np.concatenate([g.normal(size=300_000) * 5, g.uniform(-745.2, 709.8, 300_000),
                               g.uniform(-1e-8, 1e-8, 20_000), np.arange(-745, 710, 0.25)])
    return np.concatenate([np.exp(g.normal(size=300_000)), g.uniform(-200, 200, 200_000),
                           g.uniform(-1.4e5, 1.4e5, 100_000), np.pi / 2 * np.arange(-3000, 3000),
                           g.uniform(-1e-7, 1e-7, 20_000)])


@pytest.mark.parametrize("which, bound", [("exp", 1), ("sin", 2), ("cos", 2), ("tanh", 3)])
def test_helpers_are_within_ulp_of_glibc(helpers, which, bound):
    """Max 1 ulp (exp), 2 ulp (sin and cos, at arguments of some 10^4) and 3
    ulp (tanh: glibc's own tanh is up to 2 ulp from the true value near
    |x| = 0.2, where this one is up to 2 ulp the other way) from glibc over
    sweeps of half a million points or more, within the 4-ulp fp64 bar."""
    import oracle_lib as O
    x = _sweep(which, np.random.default_rng(7))
    got, want = helpers(which, x), O.libm(which, x)
    big = np.isinf(want)
    assert (got[big] == want[big]).all()
    u = ulp_diff(got[~big], want[~big])
    assert u.max() <= bound, f"{which}: max {u.max()} ulp at {x[~big][np.argmax(u)]!r}"


@pytest.mark.parametrize("which", ["exp", "sin", "cos", "tanh"])
def test_helpers_on_special_values(helpers, which):
    """Signed zeros, infinities, NaN, subnormals, the overflow and underflow
    edges of exp and the library hand-over of sin/cos at 2^17: NaN where glibc
    gives NaN, zeros of glibc's sign, infinities exactly, the rest within 2 ulp."""
    import oracle_lib as O
    x = np.array([0.0, -0.0, np.inf, -np.inf, np.nan, 5e-324, -5e-324, 2.2250738585072014e-308, 1e-310, -1e-310,
                  709.782712893384, 709.7827128933841, 710.0, -745.1332191019411, -745.1332191019412, -745.2,
                  -708.39641853226408, -1000.0, 1e300, -1e300, 131071.99, 131072.0, -131072.0, 1e22,
                  3.141592653589793, 1.5707963267948966, -1.5707963267948966, 2.0 ** -26, -2.0 ** -27, 1e-8])
    got, want = helpers(which, x), O.libm(which, x)
    for xi, g_, w_ in zip(x, got, want):
        if np.isnan(w_):
            assert np.isnan(g_), (which, xi, g_)
        elif w_ == 0.0:
            assert g_ == 0.0 and np.signbit(g_) == np.signbit(w_), (which, xi, g_, w_)
        elif np.isinf(w_):
            assert g_ == w_, (which, xi, g_)
        else:
            assert ulp_diff(np.array([g_]), np.array([w_]))[0] <= 2.0, (which, xi, g_, w_)


def _same_bits(a, b):
    return np.array_equal(a.view(np.int64), b.view(np.int64)) or (
        np.array_equal(np.isnan(a), np.isnan(b)) and np.array_equal(a[~np.isnan(a)].view(np.int64),
                                                                    b[~np.isnan(b)].view(np.int64)))


def test_domain_forms_are_the_general_forms_on_their_domains(helpers):
    """The forms the emitter picks for a bounded operand give the general
    form's bits on their domain: exp on x <= 0, tanh on [-20, 20] (NaN stays
    NaN in both), sin on [0, inf), and the rsq-seeded square root is the
    correctly rounded sqrt on [2^-700, DBL_MAX] (the host seed here is
    1/sqrt(x) rounded; the device's is its reciprocal square root, and the
    GPU test holds that form to numpy's sqrt too).  The tanh's quotient
    e / (e + 2) without the division's scaling and fixup is the correctly
    rounded quotient over its whole range, tiny and subnormal e included."""
    g = np.random.default_rng(11)
    x = np.concatenate([-np.abs(g.normal(size=200_000)) * 30, -np.exp(g.uniform(-700, 7, 100_000)),
                        np.arange(-746, 0, 0.125), [0.0, -0.0, -5e-324, -1e-310, -745.2, -1200.0, -1e300,
                                                    -np.inf, np.nan]])
    assert _same_bits(helpers("exp_nonpos", x), helpers("exp", x))
    t = np.concatenate([g.uniform(-20, 20, 300_000), g.normal(size=50_000) * 1e-4, np.arange(-20, 20, 1e-3),
                        np.exp(g.uniform(-700, 2.99, 50_000)) * np.sign(g.normal(size=50_000)),
                        [0.0, -0.0, 5e-324, -5e-324, 19.999, -20.0, 20.0, np.nan]])
    assert _same_bits(helpers("tanh_mid", t), helpers("tanh", t))
    s = np.concatenate([1.0 + g.uniform(0, 1, 300_000), np.exp(g.uniform(-480, 709, 300_000)),
                        np.nextafter(1.0, 2.0) + np.arange(2000) * 2.0 ** -52, 4.0 - np.arange(2000) * 2.0 ** -51,
                        [2.0 ** -700, 1.7e308, 1.0, 2.0, 3.0, np.nan]])
    assert _same_bits(helpers("sqrt_normal", s), np.sqrt(s))
    p = np.concatenate([np.exp(g.normal(size=200_000)) * 3, g.uniform(0, 200, 200_000),
                        np.exp(g.uniform(-700, 20, 100_000)), np.arange(0, 2000, 0.01), g.uniform(0, 1e-8, 20_000),
                        [0.0, 5e-324, 1e-310, 2.0 ** -26, 2.0 ** -27, 131071.99, 131072.0, 1e300, np.inf, np.nan]])
    assert _same_bits(helpers("sin_nonneg", p), helpers("sin", p))
    e = np.concatenate([np.expm1(g.uniform(0, 128, 300_000)), np.exp(g.uniform(-745, 0, 100_000)),
                        g.uniform(0, 1, 100_000), [0.0, 5e-324, 1e-310, 2.0 ** -52, 6.2e27, np.nan]])
    assert _same_bits(helpers("div_mid", e), e / (e + 2.0))


def test_emitter_picks_the_domain_forms_from_value_ranges():
    """Interval arithmetic over the IR: the chain's sqrt(|tanh| + 1) is on
    [1, 2], its tanh argument 1.5 sin + 0.25 is on [-1.25, 1.75], its sin
    argument exp(x) is >= 0 and its last exp argument -|t6| is <= 0, so each
    gets its bounded form; an unbounded operand keeps the general form."""
    from hawk_amd import Scalar, kernel
    from hawk_amd import math as m
    from hawk_amd.emit_hip import plan_kernel
    from hawk_amd.examples import chain

    src = plan_kernel(chain.program, "chain").source
    for form in ("hk_sqrt_normal(", "hk_tanh_mid(", "hk_exp_nonpos(", "hk_sin_nonneg("):
        assert src.count("= " + form) == 1, form
    assert src.count("= hk_exp(") == 1

    @kernel
    def free(x: Scalar) -> Scalar:
        return m.sqrt(x) + m.tanh(x * 2.0) + m.exp(x) + m.sqrt(m.exp(x)) + m.tanh(m.sin(x) * 25.0)

    src = plan_kernel(free.program, "free").source
    assert "= hk_sqrt_normal(" not in src and "= hk_tanh_mid(" not in src and "= hk_exp_nonpos(" not in src
    assert "= hk_sin_nonneg(" not in src
    assert src.count("= sqrt(") == 2 and src.count("= hk_tanh(") == 2


def test_float32_builds_call_the_float_overloads(helpers):
    """The IR's dtype is f64 in a float32 build as well, where Real is float:
    there the emitter spells sqrt, exp, tanh, sin and cos as the float
    overloads and picks no bounded form, whose bounds assume double
    arithmetic.  sqrt(|sin x| + 1e-50) is the case that would break: 1e-50
    rounds to 0.0f, and at x = 0 the bounded square root (seeded by the
    reciprocal square root) gives NaN where sqrt(0) is 0."""
    from hawk_amd import Scalar, kernel
    from hawk_amd import math as m
    from hawk_amd.emit_hip import plan_kernel

    @kernel
    def tiny(x: Scalar) -> Scalar:
        return m.sqrt(m.abs(m.sin(x)) + 1e-50) + m.exp(-m.abs(x)) + m.tanh(m.sin(x) * 2.0) + m.cos(x)

    src64 = plan_kernel(tiny.program, "tiny").source
    assert "= hk_sqrt_normal(" in src64 and "= hk_exp_nonpos(" in src64 and "= hk_tanh_mid(" in src64
    src32 = plan_kernel(tiny.program, "tiny", mode="float32").source
    assert "hk_sqrt_normal(" not in src32.split("extern \"C\"")[-1]
    body = src32.split("extern \"C\"")[-1]
    for helper in ("hk_exp", "hk_sin", "hk_cos", "hk_tanh", "hk_sqrt_normal", "hk_exp_nonpos", "hk_tanh_mid",
                   "hk_sin_nonneg"):
        assert helper + "(" not in body, helper
    for call in ("= sqrt(", "= exp(", "= tanh(", "= sin(", "= cos("):
        assert call in body, call
    # the failure the gate prevents, on the host: the bounded form at 0
    assert np.isnan(helpers("sqrt_normal", np.array([0.0]))[0])
