"""The config-5 chain's per-element parity bound — TEST INFRASTRUCTURE.

The chain (``hawk_amd.examples.chain``, the oracle's ``hko_chain``) is

    t1 = exp(x);  t2 = sin(t1);  a = 1.5 t2;  t3 = a + 0.25;  t4 = tanh(t3);
    w = |t4| + 1;  t5 = sqrt(w);  s = t5 t5;  t6 = s - x;  t7 = exp(-|t6|);
    m = t7 x;  y = m + t4.

The device computes every IEEE operation (+, -, *, sqrt, |.|) correctly
rounded, as the oracle does, and each transcendental within 4 ulp of glibc.
Where ``y`` cancels (``t7 x`` against ``t4``) a 4-ulp difference in one
transcendental becomes many ulps of ``y``, so a plain 4-ulp bar on ``y`` is the
wrong contract.  The bound here is the first-order propagation of each
operation's allowance to ``y``:

    |y_dev - y_oracle| <= 2 * sum_k |dy/dv_k| * a_k * ulp(v_k)

over every operation result ``v_k``, with ``a_k`` = 4 for a transcendental
(its contract against glibc) and 1 for an IEEE operation (the same correctly
rounded operation on inputs that already differ rounds to at most one ulp
more than the exact difference of its results).  ``|dy/dv_k|`` is bounded by
products of absolute values (|.| is Lipschitz 1, so the kinks at ``t4 = 0``
and ``t6 = 0`` are covered from both sides); the factor 2 covers the second
order and an ulp measured on the other side of a power of two.
"""

from __future__ import annotations

import numpy as np

import oracle_lib as O


def parts(x: np.ndarray, perturb: dict | None = None) -> dict:
    """The chain's operation results, the oracle's operations one by one (glibc
    for the transcendentals, numpy's IEEE ufuncs elsewhere).  ``perturb``
    maps a result's name to a function applied to it (a planted mistake, for
    the tests of the bound itself)."""
    f = perturb or {}
    ident = lambda v: v          # noqa: E731
    p = {}
    p["t1"] = f.get("t1", ident)(O.libm("exp", x))
    p["t2"] = f.get("t2", ident)(O.libm("sin", p["t1"]))
    p["a"] = 1.5 * p["t2"]
    p["t3"] = p["a"] + 0.25
    p["t4"] = f.get("t4", ident)(O.libm("tanh", p["t3"]))
    p["w"] = np.abs(p["t4"]) + 1.0
    p["t5"] = np.sqrt(p["w"])
    p["s"] = p["t5"] * p["t5"]
    p["t6"] = p["s"] - x
    p["t7"] = f.get("t7", ident)(O.libm("exp", -np.abs(p["t6"])))
    p["m"] = p["t7"] * x
    p["y"] = f.get("y", ident)(p["m"] + p["t4"])
    return p


def element_bound(x: np.ndarray, p: dict | None = None) -> np.ndarray:
    """Per element, the largest |y_dev - y_oracle| the operations' allowances
    admit (see the module docstring)."""
    p = parts(x) if p is None else p
    ulp = lambda v: np.spacing(np.abs(v))        # noqa: E731
    d = {"y": np.ones_like(x), "m": np.ones_like(x)}
    d["t7"] = np.abs(x)                           # m = t7 x
    d["t6"] = d["t7"] * p["t7"]                   # t7 = exp(-|t6|)
    d["s"] = d["t6"]                              # t6 = s - x
    d["t5"] = 2.0 * p["t5"] * d["s"]              # s = t5 t5
    d["w"] = d["t5"] / (2.0 * p["t5"])            # t5 = sqrt(w)
    d["t4"] = 1.0 + d["w"]                        # y = m + t4 and w = |t4| + 1
    d["t3"] = d["t4"] * (1.0 - p["t4"] * p["t4"])  # t4 = tanh(t3)
    d["a"] = d["t3"]                              # t3 = a + 0.25
    d["t2"] = 1.5 * d["t3"]                       # a = 1.5 t2
    d["t1"] = d["t2"] * np.abs(np.cos(p["t1"]))   # t2 = sin(t1)
    allowance = {"t1": 4, "t2": 4, "t4": 4, "t7": 4}
    total = np.zeros_like(x)
    for name, dv in d.items():
        total += allowance.get(name, 1) * ulp(p[name]) * dv
    return 2.0 * total


def within(got: np.ndarray, want: np.ndarray, bound: np.ndarray) -> np.ndarray:
    """Elementwise: equal (NaN with NaN), or within the bound."""
    same = (got == want) | (np.isnan(got) & np.isnan(want))
    return same | (np.abs(got - want) <= bound)
