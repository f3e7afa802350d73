"""The five benchmark kernels, written as a hawk user writes them.

These are the workloads the benchmark and the parity tests run (one per
benchmark configuration): a pure streaming kernel, a vector kernel with its
reverse and forward derivatives, a rolled 32-substep leapfrog with its
reverse-mode derivative, per-sample linear algebra (a 6x6 SPD solve; a
16x16 fp32 product), and a fused elementwise chain feeding a fixed-tree
ordered sum and a keyed ordered scatter.
"""

from __future__ import annotations

from . import diff
from . import trace as _trace
from .math import abs as _abs
from .math import cho_solve, cholesky, cos, dot, exp, sin, sqrt, tanh, vec
from .trace import Kernel, kernel
from .types import Grid, Index, Matrix, Mutable, Param, Scalar, Table, Terminated, Vector

#: Leapfrog step and substep count of the two-body kernel.
DT = 1e-3
SUBSTEPS = 32


@kernel
def scale(x: Scalar, a: Param, b: Param) -> Scalar:
    return a * x + b


@kernel
def energy(v: Vector[3], out: Mutable[Scalar]):
    out = 0.5 * dot(v, v)


energy_vjp = Kernel("energy_vjp", diff.vjp(energy, wrt=("v",)))
energy_jvp = Kernel("energy_jvp", diff.jvp(energy, wrt=("v",)))


@kernel
def twobody(r0: Vector[3], v0: Vector[3], mu: Param, r: Mutable[Vector[3]], v: Mutable[Vector[3]]):
    rr = r0
    vv = v0
    for k in range(SUBSTEPS):
        r2 = dot(rr, rr)
        acc = (-mu / (r2 * sqrt(r2))) * rr
        vh = vv + (0.5 * DT) * acc
        rr = rr + DT * vh
        r2n = dot(rr, rr)
        accn = (-mu / (r2n * sqrt(r2n))) * rr
        vv = vh + (0.5 * DT) * accn
    r = rr
    v = vv


twobody_vjp = Kernel("twobody_vjp", diff.vjp(twobody, wrt=("r0", "v0")))
#: The two-body VJP with the gravitational parameter's gradient too: a cell
#: summed over every sample.
twobody_vjp_mu = Kernel("twobody_vjp_mu", diff.vjp(diff.param_planes(twobody), wrt=("r0", "v0", "mu")))


@kernel
def spd_solve(A: Matrix[6, 6], b: Vector[6], x: Mutable[Vector[6]]):
    L, info = cholesky(A)
    x = cho_solve(L, b)


spd_solve_vjp = Kernel("spd_solve_vjp", diff.vjp(spd_solve, wrt=("A", "b")))


@kernel
def mm16(A: Matrix[16, 16], B: Matrix[16, 16], C: Mutable[Matrix[16, 16]]):
    C = A @ B


mm16_vjp = Kernel("mm16_vjp", diff.vjp(mm16, wrt=("A", "B")))


@kernel
def chain(x: Scalar, key: Index, y: Mutable[Scalar], total: Mutable[Scalar], bins: Mutable[Scalar]):
    t1 = exp(x)
    t2 = sin(t1)
    t3 = 1.5 * t2 + 0.25
    t4 = tanh(t3)
    t5 = sqrt(_abs(t4) + 1.0)
    t6 = t5 * t5 - x
    t7 = exp(-_abs(t6))
    y = t7 * x + t4
    total = _trace.sum(y, policy="ordered")
    _trace.scatter(bins, policy="ordered")[key] += y


@kernel
def chain_steps(x: Scalar, e1: Mutable[Scalar], s2: Mutable[Scalar], h4: Mutable[Scalar], e7: Mutable[Scalar],
                y: Mutable[Scalar]):
    """The chain's per-sample stage with the outputs of its four
    transcendentals stored beside ``y`` (the same operations, so ``y`` has
    the fused chain's bits): each operation can then be checked on its own
    inputs."""
    t1 = exp(x)
    t2 = sin(t1)
    t3 = 1.5 * t2 + 0.25
    t4 = tanh(t3)
    t5 = sqrt(_abs(t4) + 1.0)
    t6 = t5 * t5 - x
    t7 = exp(-_abs(t6))
    e1 = t1
    s2 = t2
    h4 = t4
    e7 = t7
    y = t7 * x + t4


@kernel
def ordered_total(x: Scalar, total: Mutable[Scalar]):
    total = _trace.sum(x, policy="ordered")


@kernel
def ordered_add(key: Index, x: Scalar, acc: Mutable[Scalar]):
    _trace.scatter(acc, policy="ordered")[key] += x


@kernel
def sample_total(x: Scalar, y: Mutable[Scalar], total: Mutable[Scalar]):
    y = 2.0 * x
    total = _trace.sum(x * x)


@kernel
def plain_total(x: Scalar, total: Mutable[Scalar]):
    total = _trace.sum(x)


@kernel
def add_sq(key: Index, x: Scalar, acc: Mutable[Scalar]):
    _trace.scatter(acc, policy="ordered")[key] += x * x


#: The VJP of a keyed add is a gather: bar_x = 2 x bar_acc[key] (reference
#: tests/test_scatter_ordered.py:42-51).
add_sq_grad = Kernel("add_sq_grad", diff.vjp(add_sq, wrt=("x",)))

#: The chain's derivatives through all three of its sinks: the reverse reads
#: bar_y (a plane), bar_total (a broadcast cell) and bar_bins[key] (a gather);
#: the forward writes dot_y and adds its tangents into dot_total and dot_bins
#: with the primal's ordered policies.
chain_vjp = Kernel("chain_vjp", diff.vjp(chain, wrt=("x",)))
chain_jvp = Kernel("chain_jvp", diff.jvp(chain, wrt=("x",)))


#: Hidden units and weights per net of :func:`net_loss_for`.
NET_UNITS, NET_WEIGHTS = 8, 24


def net_loss_for(samples: int, policy: str = "ordered") -> Kernel:
    """Many small models in one launch (the reference's net axis,
    tests/test_net_axis.py): lanes are (net, sample); net k's weights are row
    k of the table ``W`` (unit h uses w[3h], w[3h+1], w[3h+2]), a mask row
    switches its unused units off, and its loss is the ordered sum of the
    squared residuals over its own samples (``policy="auto"``: the default
    sum of each net's samples).  Under the ordered policy the VJP wrt ``W`` is
    the ordered log fold: each net's gradient is the sum of its samples'
    contributions in lane order."""
    @kernel
    def net_loss(lane: Grid["net", "sample":samples], W: Table["net", "w":NET_WEIGHTS],
                 mask: Table["net", "h":NET_UNITS], x: Scalar, y: Scalar) -> Scalar:
        pred = 0.0 * x
        for h in range(NET_UNITS):
            act = tanh(W.at(net=lane.net, w=3 * h) * x + W.at(net=lane.net, w=3 * h + 1))
            pred = pred + mask.at(net=lane.net, h=h) * W.at(net=lane.net, w=3 * h + 2) * act
        r = pred - y
        return _trace.sum(r * r, over="sample", policy=policy)
    return Kernel(f"net_loss_{samples}" + ("" if policy == "ordered" else f"_{policy}"), net_loss.program)


@kernel
def unit_circle(x: Scalar, a: Mutable[Vector[3]]):
    a = vec(sin(x), cos(x), x * 0.5)


@kernel
def decay(a: Vector[3], x: Scalar, b: Mutable[Scalar]):
    b = exp(-dot(a, a)) + x


@kernel
def accumulate(b: Scalar, acc: Mutable[Scalar]):
    acc = acc + b * b


@kernel
def scale_vec(a: Vector[3], b: Scalar, y: Mutable[Vector[3]]):
    y = a * b


#: Four kernels that pass values by name (the shape of the reference's
#: tests/test_chain.py fixture: a vector, a scalar read from it, an
#: accumulator updated in place, an output read from two earlier values):
#: ``hawk.chain(*CHAIN_MEMBERS, name=...)`` runs them as one kernel.
CHAIN_MEMBERS = (unit_circle, decay, accumulate, scale_vec)


# -- kernels that finish their own sample (reference tests/test_finish_own_sample.py:52-86)

#: The oscillator's explicit-Euler step (exact in binary: t stays a multiple of it).
OSC_DT = 0.125


@kernel(steps=1)
def osc_finish(dt: Param, t_final: Scalar, terminated: Terminated,
               x: Mutable[Scalar], v: Mutable[Scalar], t: Mutable[Scalar]):
    v_start = v
    a = -x
    v = v_start + dt * a
    x = x + dt * v_start
    tn = t + dt
    t = tn
    terminated = tn >= t_final


@kernel
def stop_only(t: Scalar, t_final: Param, terminated: Terminated):
    terminated = t >= t_final


@kernel(steps=1)
def smooth_finish(x: Scalar, terminated: Terminated, y: Mutable[Scalar]):
    y = x * x + 1.0
    terminated = x > 2.0


#: The oscillator taking up to 8 steps a launch.
osc_finish_x8 = _trace.steps(osc_finish, 8)
#: The oscillator taking the launch's word of steps, with its fast entries.
osc_finish_xauto = _trace.steps(osc_finish, "auto")


@kernel
def spin(c: Param, s: Param, limit: Scalar, terminated: Terminated, p: Mutable[Vector[2]], n: Mutable[Scalar]):
    """A rotation of a 2-vector per step until the step count reaches ``limit``:
    an automatic kernel carrying a vector and a scalar."""
    x = p[0]
    y = p[1]
    p = vec(c * x - s * y, s * x + c * y)
    n = n + 1.0
    terminated = n >= limit


@kernel
def decay_until(rate: Param, floor: Param, terminated: Terminated, y: Mutable[Scalar]):
    """A finishing kernel built with no ``steps=``: its automatic kernel, under its own name."""
    y = y * rate
    terminated = y < floor
smooth_finish_vjp = Kernel("smooth_finish_vjp", diff.vjp(smooth_finish, wrt=("x",)))
FINISHING = {k.name: k for k in (osc_finish, osc_finish_x8, osc_finish_xauto, stop_only, smooth_finish,
                                 smooth_finish_vjp, decay_until, spin)}


#: Every kernel above, by name.
ALL = {k.name: k for k in (scale, energy, energy_vjp, energy_jvp, twobody, twobody_vjp, spd_solve,
                            spd_solve_vjp, chain, chain_steps, ordered_total, ordered_add, sample_total, plain_total,
                            twobody_vjp_mu, add_sq, add_sq_grad, chain_vjp, chain_jvp, mm16, mm16_vjp)}
#: The float32 unit (built with mode="float32").
FLOAT32 = {k.name: k for k in (mm16, mm16_vjp, sample_total, plain_total, ordered_total, ordered_add, add_sq)}


@kernel
def band_total(x: Scalar, s: Mutable[Scalar], s_sq: Mutable[Scalar], s_ord: Mutable[Scalar]):
    """The sample sums of the banded mode (the reference's banded row sum
    kernel, tests/test_banded_sum.py, plus the ordered sum): the default
    policy over x and over the computed x*x, and the ordered policy over x."""
    s = _trace.sum(x)
    s_sq = _trace.sum(x * x)
    s_ord = _trace.sum(x, policy="ordered")


#: The banded unit (built with mode="banded").
BANDED = {k.name: k for k in (band_total,)}
