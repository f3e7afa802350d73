"""Member kernels for the ``hawk.chain`` tests — TEST INFRASTRUCTURE: the
four members of :data:`hawk_amd.examples.CHAIN_MEMBERS`, and kernels each
chain refusal needs."""

from __future__ import annotations

import hawk_amd as hawk
from hawk_amd import Grid, Mutable, Scalar, Table


from hawk_amd.examples import CHAIN_MEMBERS as MEMBERS, accumulate, decay, scale_vec, unit_circle  # noqa: F401


@hawk.kernel
def flat_a(a: Scalar, z: Mutable[Scalar]):
    z = a * 2.0


@hawk.kernel
def blind_b(x: Scalar, b: Mutable[Scalar]):
    b = x * 3.0


@hawk.kernel
def fill(x: Scalar, table: Mutable[Scalar]):
    table = x * 2.0


@hawk.kernel
def pick(table: Table[Scalar], x: Scalar, out: Mutable[Scalar]):
    out = table.at(0) * x


@hawk.kernel
def total_of(x: Scalar, t: Mutable[Scalar]):
    t = hawk.sum(x, policy="ordered")


@hawk.kernel
def reads_total(t: Scalar, x: Scalar, z: Mutable[Scalar]):
    z = t * x


@hawk.kernel
def on_grid(lane: Grid["key", "s":4], x: Scalar, b: Mutable[Scalar]):
    b = x * 2.0
