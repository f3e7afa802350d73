"""A host build of the target's fp64 math helpers (``hawk_amd/emit_hip.py``
``_MATH_HELPERS``) — TEST INFRASTRUCTURE.

The helpers use only IEEE operations (fused multiply-add, rint, ldexp, a
correctly rounded add, multiply and divide), so a host build computes the
device's bits, with two exceptions each form documents: the reciprocal and
reciprocal-square-root seeds are the correctly rounded 1/x and 1/sqrt(x)
here and the hardware's estimates on the device, which the Newton-Raphson
steps that follow make no difference to; and sin/cos hand |x| >= 2^17 to
the library."""

from __future__ import annotations

import ctypes
import subprocess
from pathlib import Path

import numpy as np

_DRIVER = """
extern "C" void hk_eval(int which, const double* x, double* y, long n) {
    for (long i = 0; i < n; ++i)
        y[i] = which == 0 ? hk_exp(x[i]) : which == 1 ? hk_sin(x[i]) : which == 2 ? hk_cos(x[i])
             : which == 3 ? hk_tanh(x[i]) : which == 4 ? hk_exp_nonpos(x[i]) : which == 5 ? hk_sqrt_normal(x[i])
             : which == 6 ? hk_tanh_mid(x[i]) : which == 7 ? hk_sin_nonneg(x[i]) : hk_div_mid(x[i], x[i] + 2.0);
}
"""

WHICH = {"exp": 0, "sin": 1, "cos": 2, "tanh": 3, "exp_nonpos": 4, "sqrt_normal": 5, "tanh_mid": 6, "sin_nonneg": 7,
         "div_mid": 8}


def build(directory: Path):
    """Compile the helpers with g++ into ``directory``; returns ``run(which, x)``
    (``div_mid`` evaluates x / (x + 2))."""
    from hawk_amd.emit_hip import _MATH_HELPERS
    src = Path(directory) / "helpers.cpp"
    src.write_text("#include <cmath>\nusing std::fma; using std::rint; using std::ldexp; using std::fabs;\n"
                   "#define HK_MATH_QUAL static inline\n#define HK_MATH_PIN(c) (void)(c)\n"
                   "#define HK_RSQ(x) (1.0 / std::sqrt(x))\n#define HK_RCP(x) (1.0 / (x))\n" + _MATH_HELPERS + _DRIVER)
    lib = Path(directory) / "helpers.so"
    subprocess.run(["g++", "-O2", "-ffp-contract=off", "-fno-math-errno", "-shared", "-fPIC", str(src), "-o",
                    str(lib)], check=True)
    handle = ctypes.CDLL(str(lib))

    def run(which, x):
        x = np.ascontiguousarray(x, dtype=np.float64)
        y = np.empty_like(x)
        handle.hk_eval(WHICH[which], x.ctypes.data_as(ctypes.c_void_p), y.ctypes.data_as(ctypes.c_void_p),
                       ctypes.c_long(x.size))
        return y
    return run
