"""Benchmark of hawk's gfx950 target on one MI355X.

``python bench.py [--steps K] [--warmup W] [--config C]`` prints ONE JSON line.
A step is one pass of the hot path over one batch of synthetic inputs already
resident in HBM.  The default workload is BASELINE.json's ``configs[1]``: the
``energy`` kernel's forward, VJP and JVP over N = 2^25 samples (fp64).  Other
configurations (``--config 1|3|4a|4b|5``) time the remaining workloads the same
way; ``--config 4b64`` is config 4b's product in the float64 mode; ``--config 5k`` times config 5's ordered sum in the reference's keyed
spelling (``hawk.sum(x, over=...)``) over 16384 keys, ``--config 5t`` a
``Table`` read at config 5's keys and its VJP (an ordered scatter), and
``--config 5n`` 65536 small models in one launch (the net axis): each net's
ordered loss and its gradient wrt its weights (the ordered log fold);
``--config chain`` four kernels chained into one launch (``hawk.chain``), and
``--config steps`` an oscillator that finishes its own sample, 8 steps a
launch (``hawk.steps``), over 2^24 samples, and ``--config persist`` 2^22 such
oscillators of 1-256 steps each run to their finish in one launch of the
persistent entry (the plain and range entries timed beside it).
``--config sum`` times config 5's sums in the default policy (the compensated
row sums, in float64) over the same 2^26 samples.
``python bench.py --latency`` prints the CU latencies the ordered scatter is
built around instead (a single-workgroup probe kernel), and
``python bench.py --pattern-sweep`` the per-sample 16x16 product's copy
ceilings over tilings (a K-sliced copy per tile shape).

Each stage launch of the timed steps (a per-sample kernel, or a team stage:
the ordered sum or the ordered scatter) is bracketed by HIP events on the
stream it is launched on (torch's current stream), so the per-stage durations,
the achieved algorithmic GB/s (bytes per sample x samples / duration) and the
roofline fraction come from the timed run itself.  ``roofline.traffic`` is the
dominant stage's HBM bytes per launch from two child ``rocprofv3 --pmc`` passes
(FETCH_SIZE, then WRITE_SIZE), each scaled by what that counter reads for a
plain 1 GiB copy (``--no-traffic`` skips them).  The CPU baseline is the C
oracle (the host-target restatement, hawk's ``native`` profile) on the same
workload, on this host's cores: every core of this process's affinity mask,
then one core, then the same build with ``-ffp-contract=fast``, with the CPU
model named.

The default run (config 2, without ``--only``) also records configs 1, 3, 4a,
4b and 5 under ``config.configs``: each one's stages (HIP events, median of 5
steps after warm-up steps for at least 0.25 s: each record follows a CPU
baseline, and a GPU that idled runs its first milliseconds of VALU-bound work
at a lower clock), its dominant stage against its roofline and the
oracle's rate on every host core (the median of at least 5 repetitions);
config 5's record also carries its dominant stage's HBM traffic.  An
FP64-bound stage (config 3) is set against the FP64 peak by the FLOPs it
executes, measured by one more ``rocprofv3 --pmc`` pass (the FP64 VALU
instruction counters over SQ_WAVES, per sample).
"""

from __future__ import annotations

import argparse
import json
import os
import statistics
import sys
import tempfile
import time
from pathlib import Path

import numpy as np

ROOT = Path(__file__).resolve().parent
sys.path.insert(0, str(ROOT))

METRIC = "samples/s + achieved HBM GB/s (% of 8 TB/s) for fwd and VJP kernels, 1 GPU"
HBM_PEAK_GBS = 8000.0
#: The CPU baseline repeats the step until this much wall time has passed
#: (at least 3, at most 2000 repetitions).
CPU_SECONDS = 10.0
FP64_PEAK_TFLOPS = 78.6


def log(msg: str) -> None:
    print(f"[bench] {msg}", file=sys.stderr, flush=True)


def _dev(a, device):
    import torch
    return torch.from_numpy(np.ascontiguousarray(a)).to(device)


# ---------------------------------------------------------------------------
# workloads: inputs (seeded, config index as seed), the kernels of one step,
# algorithmic bytes per sample of each kernel, and the CPU baseline's step.


def ops(kernel) -> int:
    """Floating-point operations per sample of a loaded kernel's per-sample
    stage, as its build counted them in the emitted code."""
    return int(kernel.sidecar.get("fp_ops_per_sample", 0))


def twobody_vjp_algorithmic_ops() -> int:
    """The two-body VJP's algorithmic operations per sample: its traced forward
    and reverse with one tape (no checkpoint replay, whose recomputation the
    built kernel adds), counted in the rendered stage as the build counts
    every kernel's operations."""
    from hawk_amd import diff
    from hawk_amd import examples as E
    from hawk_amd.emit_hip import plan_kernel
    saved = diff.CHECKPOINT_SEGMENT
    diff.CHECKPOINT_SEGMENT = 1 << 30          # larger than any trip count: the loop keeps one tape
    try:
        program = diff.vjp(E.twobody, wrt=("r0", "v0"))
    finally:
        diff.CHECKPOINT_SEGMENT = saved
    return plan_kernel(program, "twobody_vjp_one_tape").algorithmic_ops


def _xcd(unit: Path, name: str) -> bool:
    """Whether a built per-sample stage hands its blocks out XCD by XCD."""
    return "hk_xcd_order = true" in (unit / f"{name}.hip").read_text()


def workload(config: str, device):
    import torch

    import hawk_amd as hawk
    from hawk_amd import examples as E

    unit = Path(tempfile.mkdtemp(prefix="hawk_bench_"))
    if config == "1":
        n = 1 << 26
        x = np.random.default_rng(1).uniform(-1.0, 1.0, n)
        hawk.build([E.scale], unit)
        k = hawk.load(unit, "scale")
        X, OUT = _dev(x, device), torch.zeros(n, dtype=torch.float64, device=device)
        kernels = [k.prepare(x=X, a=2.0, b=1.0, out=OUT)]
        work = {"scale": (16, ops(k))}

        def cpu(threads):
            import oracle_lib as O
            out = np.empty(n)
            O.lib().hko_tiled(1, O._p(x), None, None, None, O._p(out), None, 2.0, 1.0, n, threads)
        # the stage's HBM pattern (one row read, one written) in its own launch shape, for pattern_ceiling
        sh = k.launch_shape
        return dict(name="scale fwd (config 1)", n=n, kernels=kernels, work=work, cpu=cpu, dtype="f64",
                    pattern={"scale": (1, 1, sh["block"], sh["block"], sh["per_thread"], _xcd(unit, "scale"),
                                       "hk_pair_" in (unit / "scale.hip").read_text())},
                    esize=8)
    if config == "2":
        n = 1 << 25
        g = np.random.default_rng(2)
        v = g.normal(size=(3, n))
        gt = np.random.default_rng(102)
        dv = gt.normal(size=(3, n))
        bar_out = np.ones(n)
        hawk.build([E.energy, E.energy_vjp, E.energy_jvp], unit)
        kf, kv, kj = (hawk.load(unit, s) for s in ("energy", "energy_vjp", "energy_jvp"))
        V, DV, BO = _dev(v, device), _dev(dv, device), _dev(bar_out, device)
        OUT = torch.zeros(n, dtype=torch.float64, device=device)
        BV = torch.zeros((3, n), dtype=torch.float64, device=device)
        DO = torch.zeros(n, dtype=torch.float64, device=device)
        kernels = [kf.prepare(v=V, out=OUT), kv.prepare(v=V, bar_out=BO, bar_v=BV),
                   kj.prepare(v=V, dot_v=DV, dot_out=DO)]
        work = {"energy": (32, ops(kf)), "energy_vjp": (56, ops(kv)), "energy_jvp": (56, ops(kj))}

        def cpu(threads):
            import oracle_lib as O
            L = O.lib()
            out, bv, do = np.empty(n), np.empty((3, n)), np.empty(n)
            L.hko_tiled(2, O._p(v), None, None, None, O._p(out), None, 0.0, 0.0, n, threads)
            L.hko_tiled(3, O._p(v), O._p(bar_out), None, None, O._p(bv), None, 0.0, 0.0, n, threads)
            L.hko_tiled(4, O._p(v), O._p(dv), None, None, O._p(do), None, 0.0, 0.0, n, threads)
        # each stage's HBM pattern (element rows read, rows written) in its own launch shape, for
        # pattern_ceiling
        sh = {k.name: (k.launch_shape["block"], k.launch_shape["per_thread"], _xcd(unit, k.name)) for k in (kf, kv, kj)}
        pattern = {"energy": (3, 1, sh["energy"][0], *sh["energy"]),
                   "energy_vjp": (4, 3, sh["energy_vjp"][0], *sh["energy_vjp"]),
                   "energy_jvp": (6, 1, sh["energy_jvp"][0], *sh["energy_jvp"])}
        return dict(name="energy fwd + VJP + JVP (config 2)", n=n, kernels=kernels, work=work, cpu=cpu, dtype="f64",
                    pattern=pattern, esize=8)
    if config == "3":
        n = 1 << 22
        g = np.random.default_rng(3)
        d = g.normal(size=(3, n))
        d /= np.linalg.norm(d, axis=0)
        r0 = d * g.uniform(0.5, 2.0, n)
        v0 = g.normal(0.0, 0.3, size=(3, n))
        gt = np.random.default_rng(103)
        bar_r, bar_v = gt.normal(size=(3, n)), gt.normal(size=(3, n))
        hawk.build([E.twobody, E.twobody_vjp], unit)
        kf, kv = hawk.load(unit, "twobody"), hawk.load(unit, "twobody_vjp")
        R0, V0, BR, BV = (_dev(a, device) for a in (r0, v0, bar_r, bar_v))
        R, VV, BR0, BV0 = (torch.zeros((3, n), dtype=torch.float64, device=device) for _ in range(4))
        kernels = [kf.prepare(r0=R0, v0=V0, mu=1.0, r=R, v=VV),
                   kv.prepare(r0=R0, v0=V0, mu=1.0, bar_r=BR, bar_v=BV, bar_r0=BR0, bar_v0=BV0)]
        work = {"twobody": (96, ops(kf)), "twobody_vjp": (144, twobody_vjp_algorithmic_ops())}
        outs = [np.empty((3, n)) for _ in range(4)]

        def cpu(threads):
            # the host target's shape for a rolled loop: tiles of samples stepping together (loop interchange)
            import oracle_lib as O
            L = O.lib()
            L.hko_tiled(9, O._p(r0), O._p(v0), None, None, O._p(outs[0]), O._p(outs[1]), 1.0, 0.0, n, threads)
            L.hko_tiled(10, O._p(r0), O._p(v0), O._p(bar_r), O._p(bar_v), O._p(outs[2]), O._p(outs[3]), 1.0, 0.0,
                        n, threads)
        return dict(name="two-body leapfrog fwd + VJP (config 3)", n=n, kernels=kernels, work=work, cpu=cpu,
                    dtype="f64", bound="fp64",
                    flops_basis="traced operations per sample (not measured in this run; the executed count "
                                "needs the rocprofv3 pass that --no-traffic skips): the forward's, and the VJP's "
                                "forward and reverse without its checkpoint replay")
    if config == "4a":
        n = 1 << 20
        g = np.random.default_rng(4)
        B = g.normal(size=(n, 6, 6))
        A = np.ascontiguousarray((np.matmul(B, B.transpose(0, 2, 1)) + 6.0 * np.eye(6)).transpose(1, 2, 0))
        b = np.ascontiguousarray(g.normal(size=(n, 6)).T)
        bar_x = np.random.default_rng(104).normal(size=(6, n))
        hawk.build([E.spd_solve, E.spd_solve_vjp], unit)
        kf, kv = hawk.load(unit, "spd_solve"), hawk.load(unit, "spd_solve_vjp")
        Ad, bd, BX = _dev(A, device), _dev(b, device), _dev(bar_x, device)
        X = torch.zeros((6, n), dtype=torch.float64, device=device)
        BA = torch.zeros((6, 6, n), dtype=torch.float64, device=device)
        BB = torch.zeros((6, n), dtype=torch.float64, device=device)
        kernels = [kf.prepare(A=Ad, b=bd, x=X), kv.prepare(A=Ad, b=bd, bar_x=BX, bar_A=BA, bar_b=BB)]
        work = {"spd_solve": (384, ops(kf)), "spd_solve_vjp": (720, ops(kv))}

        def cpu(threads):
            import oracle_lib as O
            O.spd_solve(A, b, threads=threads)
            O.spd_solve_vjp(A, b, bar_x, threads=threads)
        # each stage's HBM pattern: element rows read and written, in the stage's launch shape
        sf, sv = kf.launch_shape, kv.launch_shape
        pattern = {"spd_solve": (42, 6, sf["block"], sf["block"], sf["per_thread"], _xcd(unit, "spd_solve")),
                   "spd_solve_vjp": (48, 42, sv["block"], sv["block"], sv["per_thread"], _xcd(unit, "spd_solve_vjp"))}
        return dict(name="6x6 SPD solve fwd + VJP (config 4a)", n=n, kernels=kernels, work=work, cpu=cpu, dtype="f64",
                    pattern=pattern, esize=8)
    if config in ("4b", "4b64"):
        # 4b64: the same product in the float64 mode (fp64 planes, v_mfma_f64_16x16x4f64)
        f64 = config == "4b64"
        nt, tdt, esize = (np.float64, torch.float64, 8) if f64 else (np.float32, torch.float32, 4)
        n = 1 << 20
        g = np.random.default_rng(4)
        A = g.normal(0.0, 0.25, size=(16, 16, n)).astype(nt)
        B = g.normal(0.0, 0.25, size=(16, 16, n)).astype(nt)
        bar_C = np.random.default_rng(104).normal(0.0, 0.25, size=(16, 16, n)).astype(nt)
        hawk.build([E.mm16, E.mm16_vjp], unit, mode="float64" if f64 else "float32")
        kf, kv = hawk.load(unit, "mm16"), hawk.load(unit, "mm16_vjp")
        Ad, Bd, BC = _dev(A, device), _dev(B, device), _dev(bar_C, device)
        C, BA, BB = (torch.zeros((16, 16, n), dtype=tdt, device=device) for _ in range(3))
        kernels = [kf.prepare(A=Ad, B=Bd, C=C), kv.prepare(A=Ad, B=Bd, bar_C=BC, bar_A=BA, bar_B=BB)]
        # labels are the team stage's: the forward's mm16 launch, then the VJP's;
        # bytes are 768 (fwd) and 1280 (VJP) elements a sample
        work = {"mm16": (768 * esize, 8192), "mm16#2": (1280 * esize, 16384)}

        def cpu(threads):
            import oracle_lib as O
            O.mm16(A, B, threads=threads)
            O.mm16_vjp(A, B, bar_C, threads=threads)
        what = "fp64 16x16 product fwd + VJP (config 4b in float64)" if f64 else "fp32 16x16 product fwd + VJP (config 4b)"
        # each stage's HBM pattern (element rows read, rows written, tile samples, threads), for pattern_ceiling
        tile = 256 // esize      # hawk_linalg.hip's shapes: 16 threads a sample (fp32), 32 (fp64 forward)
        pattern = {"mm16": (512, 256, tile, (32 if f64 else 16) * tile, 1, True),
                   "mm16#2": (768, 512, tile // 2, 8 * tile, 1, True)}
        return dict(name=what, n=n, kernels=kernels, work=work, cpu=cpu, dtype="f64" if f64 else "f32",
                    pattern=pattern, esize=esize)
    if config == "5":
        n = 1 << 26
        g = np.random.default_rng(5)
        x = g.normal(size=n)
        cells = 1 << 16
        key = ((g.zipf(1.1, n) - 1) % cells).astype(np.int32)
        hawk.build([E.chain], unit)
        k = hawk.load(unit, "chain")
        X, KEY = _dev(x, device), _dev(key, device)
        Y = torch.zeros(n, dtype=torch.float64, device=device)
        TOT = torch.zeros(1, dtype=torch.float64, device=device)
        BINS = torch.zeros(cells, dtype=torch.float64, device=device)
        kernels = [k.prepare(x=X, key=KEY, y=Y, total=TOT, bins=BINS)]
        # per stage: the chain reads x, writes y; the sum reads y; the scatter reads key and y and
        # reads + writes every bin once
        work = {"chain": (16, ops(k)), "ordered_sum": (8, 1), "ordered_scatter": (12 + 16 * cells / n, 1)}

        def cpu(threads):
            import oracle_lib as O
            y = O.chain(x, threads=threads)
            O.ordered_sum(y, threads=threads)
            O.ordered_scatter(key, y, np.zeros(cells), threads=threads)
        return dict(name="chain + ordered sum + ordered scatter (config 5)", n=n, kernels=kernels, work=work, cpu=cpu,
                    dtype="f64")
    if config == "band":
        # the banded mode's sample sums over config 5's input size: the default policy over x and over
        # x*x (band rows in the stage, the banded canonical finish) and the ordered policy over x (the
        # banded fixed tree), reference tests/test_banded_sum.py's kernel plus the ordered sum
        n = 1 << 26
        x = np.random.default_rng(5).normal(size=n)
        hawk.build([E.band_total], unit, mode="banded")
        k = hawk.load(unit, "band_total")
        X = _dev(x, device)
        cells = {c: torch.zeros(1, dtype=torch.float64, device=device) for c in ("s", "s_sq", "s_ord")}
        kernels = [k.prepare(x=X, **cells)]
        rows = 16 / 32                          # a (hi, lo) band row per 32 samples
        work = {"band_total": (8 + 2 * rows, 0), "row_sum": (rows, 1), "row_sum#2": (rows, 1),
                "band_ordered_sum": (8, 1)}

        def cpu(threads):
            import oracle_lib as O
            O.band_sample_sum(x)
            O.band_sample_sum(x * x)
            O.band_ordered_sum(x)
        return dict(name="banded sample sums: default policy over x and x*x, ordered over x (mode='banded')",
                    n=n, kernels=kernels, work=work, cpu=cpu, dtype="f64 (double-double bands)", cpu_threads=1)
    if config == "sum":
        # the default-policy sample sums in the float64 mode over config 5's input size: band_total's
        # kernel (the default policy over x and over x*x, the ordered policy over x) without the bands:
        # compensated 32-sample rows in the stage, then the canonical finish of each row plane
        n = 1 << 26
        x = np.random.default_rng(5).normal(size=n)
        hawk.build([E.band_total], unit)
        k = hawk.load(unit, "band_total")
        X = _dev(x, device)
        cells = {c: torch.zeros(1, dtype=torch.float64, device=device) for c in ("s", "s_sq", "s_ord")}
        kernels = [k.prepare(x=X, **cells)]
        rows = 16 / 32                          # a (hi, comp) row per 32 samples
        work = {"band_total": (8 + 2 * rows, 0), "row_sum": (rows, 1), "row_sum#2": (rows, 1),
                "ordered_sum": (8, 1)}

        def cpu(threads):
            import oracle_lib as O
            O.sample_sum(x)
            O.sample_sum(x * x)
            O.ordered_sum(x, threads=threads)
        return dict(name="default-policy sample sums over x and x*x, ordered over x (float64)", n=n,
                    kernels=kernels, work=work, cpu=cpu, dtype="f64")
    if config == "5k":
        # config 5b in the reference's keyed spelling (tests/test_ordered_fixed_tree.py:43-47), over
        # 16384 keys of 4096 samples: hawk.sum(x, over="sample", policy="ordered") per key
        n, group = 1 << 26, 4096
        x = np.random.default_rng(5).normal(size=n)

        @hawk.kernel
        def keyed_total(lane: hawk.Grid["key", "sample":4096], x: hawk.Scalar) -> hawk.Scalar:
            return hawk.sum(x, over="sample", policy="ordered")
        hawk.build([keyed_total], unit)
        k = hawk.load(unit, "keyed_total")
        X = _dev(x, device)
        OUT = torch.zeros(n // group, dtype=torch.float64, device=device)
        kernels = [k.prepare(x=X, out=OUT)]
        work = {"keyed_sum": (8 + 8 / group, 1)}    # every x once, every cell once

        def cpu(threads):
            import oracle_lib as O
            O.keyed_ordered_sum(x, group, threads=threads, profile=None)
        return dict(name="keyed ordered sum, 16384 keys x 4096 samples (config 5b, keyed)", n=n, kernels=kernels,
                    work=work, cpu=cpu, dtype="f64")
    if config == "5t":
        # a Table read at config 5's Zipf keys, y = table.at(key) * x, and its VJP wrt the table: the
        # ordered scatter of bar_y * x at the cells read (reference tests/test_diff_cross_sample.py:40-63)
        from hawk_amd.diff import vjp
        from hawk_amd.trace import Kernel
        n, cells = 1 << 26, 1 << 16
        g = np.random.default_rng(5)
        x = g.normal(size=n)
        key = ((g.zipf(1.1, n) - 1) % cells).astype(np.int32)
        table = np.random.default_rng(105).normal(size=cells)
        bar_y = np.random.default_rng(205).normal(size=n)

        @hawk.kernel
        def lookup_scale(table: hawk.Table[hawk.Scalar], key: hawk.Index, x: hawk.Scalar,
                         y: hawk.Mutable[hawk.Scalar]):
            y = table.at(key) * x
        back = Kernel("lookup_scale_vjp", vjp(lookup_scale, wrt=("table",)))
        hawk.build([lookup_scale, back], unit)
        kf, kv = hawk.load(unit, "lookup_scale"), hawk.load(unit, "lookup_scale_vjp")
        T, K, X, BY = _dev(table, device), _dev(key, device), _dev(x, device), _dev(bar_y, device)
        Y = torch.zeros(n, dtype=torch.float64, device=device)
        BT = torch.zeros(cells, dtype=torch.float64, device=device)
        kernels = [kf.prepare(table=T, key=K, x=X, y=Y), kv.prepare(table=T, key=K, x=X, bar_y=BY, bar_table=BT)]
        # forward: key and x in, y out (the table stays in cache); the VJP's stage reads key, x and
        # bar_y and writes the cell and the contribution the scatter reads (as config 5's scatter
        # reads its key and y), and the scatter reads + writes every cell once
        work = {"lookup_scale": (20, ops(kf)), "lookup_scale_vjp": (20 + 12, ops(kv)),
                "ordered_scatter": (12 + 16 * cells / n, 1)}

        def cpu(threads):
            import oracle_lib as O
            y = table[np.clip(key, 0, cells - 1)] * x
            O.ordered_scatter(np.clip(key, 0, cells - 1).astype(np.int32), bar_y * x, np.zeros(cells),
                              threads=threads)
            return y
        return dict(name="Table read at Zipf keys + its VJP wrt the table (config 5, tables)", n=n,
                    kernels=kernels, work=work, cpu=cpu, dtype="f64")
    if config == "chain":
        # hawk.chain (reference hawk/trace/chain.py): four kernels passing a vector and a scalar by
        # name, run as ONE launch; the intermediates a (3 reals) and b never reach HBM
        members = E.CHAIN_MEMBERS
        n = 1 << 25
        g = np.random.default_rng(9)
        x, acc0 = g.uniform(0.1, 2.0, n), g.uniform(0.0, 1.0, n)
        chained = hawk.chain(*members, name="fixture")
        hawk.build([chained, *members], unit)
        kc = hawk.load(unit, "fixture")
        X, ACC = _dev(x, device), _dev(acc0, device)
        Y = torch.zeros((3, n), dtype=torch.float64, device=device)
        kernels = [kc.prepare(x=X, acc=ACC, y=Y)]
        work = {"fixture": (48, ops(kc))}          # x and acc in, acc and y out

        def members_ms():
            # the same work as four launches through planes, for comparison (not the measured step)
            A = torch.zeros((3, n), dtype=torch.float64, device=device)
            B = torch.zeros(n, dtype=torch.float64, device=device)
            preps = [hawk.load(unit, "unit_circle").prepare(x=X, a=A), hawk.load(unit, "decay").prepare(a=A, x=X, b=B),
                     hawk.load(unit, "accumulate").prepare(b=B, acc=ACC), hawk.load(unit, "scale_vec").prepare(a=A, b=B, y=Y)]
            for p in preps:
                p()
            torch.cuda.synchronize()
            a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            a.record()
            for _ in range(10):
                for p in preps:
                    p()
            b.record()
            torch.cuda.synchronize()
            return a.elapsed_time(b) / 10

        def cpu(threads):
            import oracle_lib as O
            O.chain_members(x, acc0.copy(), threads=threads, profile=None)
        return dict(name="hawk.chain of four kernels (vector and scalar passed by name), one launch", n=n,
                    kernels=kernels, work=work, cpu=cpu, dtype="f64", compare=members_ms)
    if config == "steps":
        # a kernel finishing its own sample, stepped 8 times a launch (reference hawk/trace/steps.py):
        # the explicit-Euler oscillator, every sample live (t_final past every timed step), so
        # each launch takes 8 steps of every sample with its state in registers between them
        k8 = E.osc_finish_x8
        n = 1 << 24
        g = np.random.default_rng(17)
        x, v = g.uniform(-1.0, 1.0, n), g.uniform(-1.0, 1.0, n)
        t_final = np.full(n, 1e30)
        hawk.build([k8], unit)
        kk = hawk.load(unit, k8.name)
        planes = {"x": _dev(x, device), "v": _dev(v, device), "t": torch.zeros(n, dtype=torch.float64, device=device),
                  "t_final": _dev(t_final, device), "terminated": torch.zeros(n, dtype=torch.bool, device=device)}
        kernels = [kk.prepare(dt=E.OSC_DT, **planes)]
        work = {k8.name: (33 + 24, ops(kk))}      # x, v, t, t_final and the mask in; x, v, t out

        def cpu(threads):
            import oracle_lib as O
            O.osc_launch(8, E.OSC_DT, t_final, x.copy(), v.copy(), np.zeros(n), np.zeros(n, dtype=bool),
                         profile=None)
        return dict(name="oscillator finishing its own sample, 8 steps a launch (hawk.steps)", n=n,
                    kernels=kernels, work=work, cpu=cpu, dtype="f64", cpu_threads=1)
    if config == "persist":
        # hawk.steps(k, "auto") through its persistent entry (reference hawk/emit/cuda.py:465-689): 2^22
        # oscillators of 1 to 256 steps each, every one run to its finish in one launch.  Each step
        # first restores the inputs (the "reset" stage: four plane copies), then runs the launch.
        ka = E.osc_finish_xauto
        n = 1 << 22
        g = np.random.default_rng(41)
        t_final = E.OSC_DT * g.integers(1, 257, n).astype(float)
        x, v = g.uniform(-1.0, 1.0, n), g.uniform(-1.0, 1.0, n)
        hawk.build([ka], unit)
        kk = hawk.load(unit, ka.name)
        X0, V0, TF = _dev(x, device), _dev(v, device), _dev(t_final, device)
        planes = {"x": X0.clone(), "v": V0.clone(), "t": torch.zeros(n, dtype=torch.float64, device=device),
                  "t_final": TF, "terminated": torch.zeros(n, dtype=torch.bool, device=device)}

        class Reset:
            def stages(self):
                def reset():
                    planes["x"].copy_(X0)
                    planes["v"].copy_(V0)
                    planes["t"].zero_()
                    planes["terminated"].zero_()
                return [("reset", reset)]
        kernels = [Reset(), kk.prepare(dt=E.OSC_DT, steps=256, entry="persist", **planes)]
        mean_steps = float(np.rint(t_final / E.OSC_DT).mean())
        step_ops = 6                               # a trip: 2 mul, 3 add, 1 compare
        work = {"reset": (2 * (8 + 8 + 8 + 1), 0),
                f"{ka.name}_persist": (33 + 25, step_ops * mean_steps)}

        def other_entries():
            # the same launch through the plain and the range entries (one lane a sample, each wave
            # held by its longest sample), for comparison
            out = {}
            for entry in ("plain", "range"):
                prep = kk.prepare(dt=E.OSC_DT, steps=256, entry=entry, **planes)
                reset = Reset().stages()[0][1]
                times = []
                for _ in range(6):
                    reset()
                    a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
                    a.record()
                    prep()
                    b.record()
                    torch.cuda.synchronize()
                    times.append(a.elapsed_time(b))
                out[f"{entry}_entry_ms"] = round(statistics.median(times[1:]), 5)
            return out

        def cpu(threads):
            import oracle_lib as O
            O.osc_launch(256, E.OSC_DT, t_final, x.copy(), v.copy(), np.zeros(n), np.zeros(n, dtype=bool),
                         profile=None)
        return dict(name="oscillators of 1-256 steps run to their finish in one launch of the persistent "
                         "entry (hawk.steps 'auto')", n=n, kernels=kernels, work=work, cpu=cpu, dtype="f64",
                    cpu_threads=1, bound="fp64", compare_entries=other_entries)
    if config == "5n":
        # the net axis (reference tests/test_net_axis.py): 65536 small models of 64 samples in one
        # launch, each net's loss an ordered keyed sum and its gradient wrt its 24 weights the
        # ordered log fold (reference hawk/diff/ordered.py)
        from hawk_amd.diff import vjp
        from hawk_amd.trace import Kernel
        k, s = 1 << 16, 64
        n = k * s
        P, H = E.NET_WEIGHTS, E.NET_UNITS
        g = np.random.default_rng(7)
        w = g.normal(size=(k, P)) * 0.7
        x, y = g.normal(size=(k, s)), g.normal(size=(k, s))
        mask = (np.arange(H)[None, :] < np.resize([8, 3, 5, 1, 6], k)[:, None]).astype(np.float64)
        net = E.net_loss_for(s)
        back = Kernel(f"net_grad_{s}", vjp(net, wrt=("W",)))
        hawk.build([net, back], unit, fuse_folds=os.environ.get("HAWK_BENCH_LOGGED_FOLD") != "1")
        kf, kv = hawk.load(unit, net.name), hawk.load(unit, back.name)
        W, M, X, Y = (_dev(a.ravel(), device) for a in (w, mask, x, y))
        OUT, BO = torch.zeros(k, dtype=torch.float64, device=device), torch.ones(k, dtype=torch.float64, device=device)
        BW = torch.zeros(k * P, dtype=torch.float64, device=device)
        kernels = [kf.prepare(W=W, mask=M, x=X, y=Y, out=OUT),
                   kv.prepare(W=W, mask=M, x=X, y=Y, bar_out=BO, bar_W=BW)]
        tables = 8 * (P + H) / s                  # a net's weights and mask, read once per net
        # loss: x, y in, the term out; keyed sum: every term once, every cell once.  The gradient folds
        # in the stage's LDS (fold_clear: the claim counts zeroed; the stage: x, y and the net's cells
        # in, bar_W out); built with fuse_folds=False it logs each contribution for a fold stage instead
        work = {net.name: (24 + tables, ops(kf)), "keyed_sum": (8 + 8 / s, 1)}
        if kv.team[0]["op"] == "fused_fold":
            work.update({"fold_clear": (4 * P / s, 0), back.name: (16 + tables + (8 + 8 * P) / s, ops(kv))})
        else:
            work.update({back.name: (16 + 8 * P + tables + (8 + 4 * P) / s, ops(kv)),
                         "ordered_fold": (8 * P + (4 * P + 8 * P) / s, 1)})

        def cpu(threads):
            import oracle_lib as O
            O.net_loss(w, mask, x, y, threads=threads, profile=None)
            O.net_grad(w, mask, x, y, np.ones(k), threads=threads, profile=None)
        return dict(name="net axis: 65536 nets x 64 samples, ordered loss and its gradient (ordered log fold)",
                    n=n, kernels=kernels, work=work, cpu=cpu, dtype="f64",
                    bound="fp64" if kv.team[0]["op"] == "fused_fold" else None)
    raise SystemExit(f"unknown --config {config!r}")


#: The kernels a team stage launches, as rocprofv3 names them (the per-sample
#: stage is one kernel named after the hawk kernel).  A full stage label
#: ("mm16#2": the VJP's two products, which share bar_C) names kernels its
#: step launches once; a base label's kernels may serve several stages.
STAGE_KERNELS = {"ordered_sum": ("hawk_sum_lanes", "hawk_sum_fold"),
                 "band_ordered_sum": ("hawk_band_sum_lanes", "hawk_band_sum_fold"),
                 "ordered_scatter": ("hawk_scatter_status", "hawk_split_hot", "hawk_split_tail", "hawk_fill_zero",
                                     "hawk_scatter_walk", "hawk_scatter_serial", "hawk_scatter_cells"),
                 "mm16": ("hawk_mm16_f32", "hawk_mm16_f64"),
                 "keyed_sum": ("hawk_keyed_rows",),      # keys of at most 65536 samples (config 5k: 4096)
                 "mm16#2": ("hawk_mm16_f32_shared", "hawk_mm16_f64_shared"),
                 "ordered_fold": ("hawk_log_fold_lanes", "hawk_log_fold_waves")}
COPY_PROBE_BYTES = 1 << 30


def _kernel_base(name: str) -> str:
    """A kernel's name without namespace, template arguments, signature and the
    return type a demangled template function carries ("void f<2>(...)")."""
    name = name.replace("(anonymous namespace)::", "")
    name = name.split("(")[0].split("<")[0].strip()
    return name[len("void "):] if name.startswith("void ") else name


_PATTERN_SOURCE = """
typedef {elem} E;
struct GRefMirror {{ void* data_; unsigned long long samples_, compStride_, sampleStride_; int deviceType_, deviceId_; }};
extern "C" __attribute__((used)) __device__ char eagle_abi_tag[] = "aether-abi/2";
extern "C" __attribute__((used)) __device__ unsigned long long eagle_layout_sizes[5] = {{40, 32, 32, 8, 24}};
// A stage's HBM pattern without its arithmetic: a workgroup reads {per} tiles
// of {tile} consecutive samples from {rows_in} element rows (rows nSamples
// apart) and writes {rows_out} rows, every load issued before the first is
// used.  Tile v of workgroup w is tile w*{per} + v, the per-sample stages'
// order (several samples a thread, a block apart); with {xcd}, workgroups are
// handed out XCD by XCD (a stage with its XCD order, the 16x16 product).
extern "C" __global__ void __launch_bounds__({threads}) hawk_pattern_copy(
        GRefMirror in_m, GRefMirror out_m, long long base, long long count, long long nSamples) {{
    const E* in = static_cast<const E*>(in_m.data_);
    E* out = static_cast<E*>(out_m.data_);
    constexpr int kStep = {threads} / {tile}, kIn = {rows_in} / kStep, kOut = {rows_out} / kStep, kPer = {per};
    const long long groups = count / ({tile} * kPer);
    const long long per_xcd = (groups + 7) / 8;
    const long long group = {xcd} ? static_cast<long long>(blockIdx.x % 8) * per_xcd + blockIdx.x / 8
                                  : static_cast<long long>(blockIdx.x);
    if (group >= groups) return;
    const int e_own = threadIdx.x / {tile};
    E x[kPer][kIn];
#pragma unroll
    for (int v = 0; v < kPer; ++v) {{
        const long long s0 = base + (group * kPer + v) * {tile} + threadIdx.x % {tile};
#pragma unroll
        for (int r = 0; r < kIn; ++r)
            x[v][r] = __builtin_nontemporal_load(in + static_cast<long long>(e_own + r * kStep) * nSamples + s0);
    }}
    if ({read_only}) {{           // the reads alone: one store a thread, never taken for finite data
        E a = E(0);
#pragma unroll
        for (int v = 0; v < kPer; ++v)
#pragma unroll
            for (int r = 0; r < kIn; ++r) a += x[v][r];
        if (a != a) out[threadIdx.x] = a;
        return;
    }}
#pragma unroll
    for (int v = 0; v < kPer; ++v) {{
        const long long s0 = base + (group * kPer + v) * {tile} + threadIdx.x % {tile};
#pragma unroll
        for (int r = 0; r < kOut; ++r) {{          // output row r folds input rows r, r + kOut, ...
            E o = x[v][r];
#pragma unroll
            for (int j = r + kOut; j < kIn; j += kOut) o += x[v][j];
            __builtin_nontemporal_store(o, out + static_cast<long long>(e_own + r * kStep) * nSamples + s0);
        }}
    }}
}}
"""


# The pattern of a stage that runs in pairs of adjacent samples (16 bytes a
# lane a row): thread t of workgroup g takes pairs (g*{per} + v)*{threads} + t.
_PAIR_SOURCE = """
typedef {elem} E;
typedef E V __attribute__((ext_vector_type(2)));
struct GRefMirror {{ void* data_; unsigned long long samples_, compStride_, sampleStride_; int deviceType_, deviceId_; }};
extern "C" __attribute__((used)) __device__ char eagle_abi_tag[] = "aether-abi/2";
extern "C" __attribute__((used)) __device__ unsigned long long eagle_layout_sizes[5] = {{40, 32, 32, 8, 24}};
extern "C" __global__ void __launch_bounds__({threads}) hawk_pattern_pairs(
        GRefMirror in_m, GRefMirror out_m, long long base, long long count, long long nSamples) {{
    const E* in = static_cast<const E*>(in_m.data_);
    E* out = static_cast<E*>(out_m.data_);
    const long long groups = count / (2 * {threads} * {per});
    const long long group = blockIdx.x;
    if (group >= groups) return;
    V x[{per}][{rows_in}];
#pragma unroll
    for (int v = 0; v < {per}; ++v) {{
        const long long s0 = base + ((group * {per} + v) * {threads} + threadIdx.x) * 2;
#pragma unroll
        for (int r = 0; r < {rows_in}; ++r)
            x[v][r] = __builtin_nontemporal_load(reinterpret_cast<const V*>(in + static_cast<long long>(r) * nSamples + s0));
    }}
    if ({read_only}) {{           // the reads alone: one store a thread, never taken for finite data
        E a = E(0);
#pragma unroll
        for (int v = 0; v < {per}; ++v)
#pragma unroll
            for (int r = 0; r < {rows_in}; ++r) a += x[v][r].x + x[v][r].y;
        if (a != a) out[threadIdx.x] = a;
        return;
    }}
#pragma unroll
    for (int v = 0; v < {per}; ++v) {{
        const long long s0 = base + ((group * {per} + v) * {threads} + threadIdx.x) * 2;
#pragma unroll
        for (int r = 0; r < {rows_out}; ++r) {{     // output row r folds input rows r, r + rows_out, ...
            V o = x[v][r];
#pragma unroll
            for (int j = r + {rows_out}; j < {rows_in}; j += {rows_out}) o += x[v][j];
            __builtin_nontemporal_store(o, reinterpret_cast<V*>(out + static_cast<long long>(r) * nSamples + s0));
        }}
    }}
}}
"""


def _gen(device):
    """A seeded generator on ``device`` for the pattern copies' input planes."""
    import torch
    g = torch.Generator(device=device)
    g.manual_seed(7)
    return g


def _time_copy(src: str, name: str, ab, grid: int, threads: int, n: int, reps: int) -> float:
    """Milliseconds a launch of copy kernel ``name`` (built from ``src`` by
    hipRTC, launched through ``hk_launch_grid``) takes over ``n`` samples."""
    import torch

    from hawk_amd import _core
    from hawk_amd.compile import compile_source
    stream = torch.cuda.current_stream()
    code, _key, _hit = compile_source(src, name)
    entry = _core.DeviceLibrary(code).entry(name)
    launch = lambda: entry.run_grid(ab, 0, n, n, grid, threads, stream.cuda_stream)  # noqa: E731
    for _ in range(3):
        launch()
    a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    a.record(stream)
    for _ in range(reps):
        launch()
    b.record(stream)
    b.synchronize()
    return a.elapsed_time(b) / reps


def pattern_ceiling(w, device, reps: int = 10) -> dict:
    """Per stage of ``w`` that names its HBM pattern: the rate (algorithmic
    GB/s) of a copy kernel with exactly that pattern and no arithmetic:
    the ceiling that layout and tile shape leave the stage.  A tiled
    product's pattern (several threads a sample) is also copied in 2, 4 and
    8 K slices, the next slice's loads in flight, as the product streams its
    operands; the best of these is its ceiling."""
    import torch

    from hawk_amd import _core
    out = {}
    n, esize = w["n"], w["esize"]
    dt = torch.float64 if esize == 8 else torch.float32
    elem = "double" if esize == 8 else "float"
    for label, (rows_in, rows_out, tile, threads, per, xcd, *pairs) in w["pattern"].items():
        if n % (tile * per):
            raise ValueError(f"pattern_ceiling: N={n} is not a multiple of the tiles ({per} x {tile})")
        if pairs and pairs[0]:
            # a stage in pairs of adjacent samples: its pattern, 16 bytes a lane a row
            src_t = torch.randn((rows_in, n), dtype=dt, device=device, generator=_gen(device))
            dst_t = torch.empty((rows_out, n), dtype=dt, device=device)
            ab = _core.ArgBlock(["gref", "gref"])
            ab.bind(0, src_t.data_ptr(), n)
            ab.bind(1, dst_t.data_ptr(), n)
            rate = {}
            for read_only in (0, 1):
                src = _PAIR_SOURCE.format(elem=elem, rows_in=rows_in, rows_out=rows_out, threads=threads,
                                          per=per // 2, read_only=read_only)
                ms = _time_copy(src, "hawk_pattern_pairs", ab, n // (threads * per), threads, n, reps)
                moved = rows_in if read_only else rows_in + rows_out
                rate[read_only] = (ms, moved * esize * n / (ms * 1e-3) / 1e9)
            out[label] = {"pattern": f"{rows_in} rows in, {rows_out} out, pairs of adjacent samples on "
                                     f"{threads} threads, {per // 2} a thread",
                          "ms": round(rate[0][0], 5), "copy_GBs": round(rate[0][1], 1),
                          "reads_only_GBs": round(rate[1][1], 1)}
            del src_t, dst_t, ab
            continue
        # normal variates like the workloads' planes: a plane of zeros copies some 5 % faster (the
        # energy forward's pattern: 7.52 TB/s from zeros, 7.15 from its own v), so zeros overstate the
        # ceiling
        src_t = torch.randn((rows_in, n), dtype=dt, device=device, generator=_gen(device))
        dst_t = torch.empty((rows_out, n), dtype=dt, device=device)
        ab = _core.ArgBlock(["gref", "gref"])
        ab.bind(0, src_t.data_ptr(), n)
        ab.bind(1, dst_t.data_ptr(), n)
        groups = n // (tile * per)
        grid = 8 * ((groups + 7) // 8) if xcd else groups
        rate = {}
        for read_only in (0, 1):
            src = _PATTERN_SOURCE.format(elem=elem, rows_in=rows_in, rows_out=rows_out, tile=tile, threads=threads,
                                         per=per, xcd="true" if xcd else "false", read_only=read_only)
            ms = _time_copy(src, "hawk_pattern_copy", ab, grid, threads, n, reps)
            moved = rows_in if read_only else rows_in + rows_out
            rate[read_only] = (ms, moved * esize * n / (ms * 1e-3) / 1e9)
        best = (rate[0][0], 1)
        step = threads // tile
        if step > 1:
            for slices in (2, 4, 8):
                if rows_in % (step * slices) or 2 * (rows_in // step // slices) + rows_out // step > 160:
                    continue
                src = _SWEEP_SOURCE.format(elem=elem, tile=tile, threads=threads, slices=slices, rows_in=rows_in,
                                           rows_out=rows_out)
                ms = _time_copy(src, "hawk_pattern_sweep", ab, grid, threads, n, reps)
                best = min(best, (ms, slices))
        ms, slices = best
        out[label] = {"pattern": f"{rows_in} rows in, {rows_out} out, {tile}-sample tiles of {threads} threads, "
                                 f"{per} a workgroup" + (", XCD order" if xcd else "")
                                 + (f", {slices} K slices" if slices > 1 else ""),
                      "ms": round(ms, 5), "copy_GBs": round((rows_in + rows_out) * esize * n / (ms * 1e-3) / 1e9, 1),
                      "reads_only_GBs": round(rate[1][1], 1)}
        del src_t, dst_t, ab
    torch.cuda.synchronize()
    torch.cuda.empty_cache()
    return out


_SWEEP_SOURCE = """
typedef {elem} E;
struct GRefMirror {{ void* data_; unsigned long long samples_, compStride_, sampleStride_; int deviceType_, deviceId_; }};
extern "C" __attribute__((used)) __device__ char eagle_abi_tag[] = "aether-abi/2";
extern "C" __attribute__((used)) __device__ unsigned long long eagle_layout_sizes[5] = {{40, 32, 32, 8, 24}};
// The 16x16 product's HBM pattern in {slices} K slices: a workgroup of
// {threads} threads reads a tile of {tile} consecutive samples from {rows_in}
// element rows, a slice of them at a time with the next slice's loads in
// flight, and writes {rows_out} rows; tiles are handed out XCD by XCD.
extern "C" __global__ void __launch_bounds__({threads}) hawk_pattern_sweep(
        GRefMirror in_m, GRefMirror out_m, long long base, long long count, long long nSamples) {{
    const E* in = static_cast<const E*>(in_m.data_);
    E* out = static_cast<E*>(out_m.data_);
    constexpr int kStep = {threads} / {tile}, kIn = {rows_in} / kStep / {slices}, kOut = {rows_out} / kStep;
    const long long tiles = count / {tile};
    const long long per_xcd = (tiles + 7) / 8;
    const long long tile = static_cast<long long>(blockIdx.x % 8) * per_xcd + blockIdx.x / 8;
    if (tile >= tiles) return;
    const long long s0 = base + tile * {tile} + threadIdx.x % {tile};
    const int e_own = threadIdx.x / {tile};
    E acc[kOut];
#pragma unroll
    for (int r = 0; r < kOut; ++r) acc[r] = E(0);
    E x[kIn], y[kIn];
#pragma unroll
    for (int r = 0; r < kIn; ++r)
        x[r] = __builtin_nontemporal_load(in + static_cast<long long>(e_own + r * kStep) * nSamples + s0);
#pragma unroll
    for (int q = 0; q < {slices}; ++q) {{
        if (q + 1 < {slices}) {{
#pragma unroll
            for (int r = 0; r < kIn; ++r)
                y[r] = __builtin_nontemporal_load(in + static_cast<long long>(e_own + ((q + 1) * kIn + r) * kStep) *
                                                  nSamples + s0);
        }}
#pragma unroll
        for (int r = 0; r < kIn; ++r) acc[r % kOut] += x[r];
#pragma unroll
        for (int r = 0; r < kIn; ++r) x[r] = y[r];
    }}
#pragma unroll
    for (int r = 0; r < kOut; ++r)
        __builtin_nontemporal_store(acc[r], out + static_cast<long long>(e_own + r * kStep) * nSamples + s0);
}}
"""


def pattern_sweep(device, n: int = 1 << 20, reps: int = 10) -> dict:
    """The fp32 16x16 product's forward (512 element rows in, 256 out) and
    VJP (768 in, 512 out) HBM patterns at N = 2^20, copied with no
    arithmetic over every run length (tiles of 32 to 256 samples: 128 B to
    1 KB a row), workgroup size (256 to 1024 threads) and number of K slices
    (1 to 8) whose staged rows fit a thread's registers: the rate the
    layout allows each tiling, against which the product's own tiling is
    chosen."""
    import itertools

    import torch

    from hawk_amd import _core
    rows = []
    for name, rows_in, rows_out in (("mm16", 512, 256), ("mm16#2", 768, 512)):
        src_t = torch.randn((rows_in, n), dtype=torch.float32, device=device, generator=_gen(device))
        dst_t = torch.empty((rows_out, n), dtype=torch.float32, device=device)
        ab = _core.ArgBlock(["gref", "gref"])
        ab.bind(0, src_t.data_ptr(), n)
        ab.bind(1, dst_t.data_ptr(), n)
        for tile, threads, slices in itertools.product((32, 64, 128, 256), (256, 512, 1024), (1, 2, 4, 8)):
            step = threads // tile
            if threads % tile or rows_in % (step * slices) or rows_out % step:
                continue
            regs = 2 * (rows_in // step // slices) + rows_out // step
            if regs > 160:                  # more staged rows than a thread's registers hold
                continue
            src = _SWEEP_SOURCE.format(elem="float", tile=tile, threads=threads, slices=slices, rows_in=rows_in,
                                       rows_out=rows_out)
            ms = _time_copy(src, "hawk_pattern_sweep", ab, 8 * ((n // tile + 7) // 8), threads, n, reps)
            gbs = (rows_in + rows_out) * 4 * n / (ms * 1e-3) / 1e9
            rows.append({"pattern": name, "run_bytes": tile * 4, "threads": threads, "slices": slices,
                         "ms": round(ms, 5), "GBs": round(gbs, 1), "hbm_frac": round(gbs / HBM_PEAK_GBS, 4)})
            log(f"pattern sweep: {rows[-1]}")
        del src_t, dst_t, ab
        torch.cuda.empty_cache()
    best = {}
    for r in rows:
        key = f"{r['pattern']} {r['run_bytes']} B"
        if key not in best or r["GBs"] > best[key]["GBs"]:
            best[key] = r
    return {"n": n, "dtype": "f32", "best_per_run": best, "all": rows}


def _with_pattern(w, device, per_stage: dict) -> dict:
    """``pattern_ceiling`` of ``w``'s stages, each with the stage's fraction of it."""
    if "pattern" not in w:
        return {}
    ceil = pattern_ceiling(w, device)
    for label, c in ceil.items():
        if label in per_stage:
            c["stage_of_pattern"] = round(per_stage[label]["achieved_GBs"] / c["copy_GBs"], 4)
    log(f"pattern ceilings: {ceil}")
    return ceil


def _pmc_pass(counter: str, config: str) -> dict:
    """One ``rocprofv3 --pmc <counter ...>`` pass over a short run of this bench
    (plus the 1 GiB copy probe) in a child process: ``{kernel: [value per
    dispatch]}`` for one counter, ``{counter: {kernel: [...]}}`` for several
    (space-separated, one hardware pass)."""
    import csv
    import shutil
    import signal
    import subprocess

    prof = shutil.which("rocprofv3")
    if prof is None:
        raise RuntimeError("rocprofv3 is not on PATH")
    out = Path(tempfile.mkdtemp(prefix="hawk_pmc_"))
    names = counter.split()
    cmd = [prof, "--pmc", *names, "--output-format", "csv", "-d", str(out), "-o", "run", "--",
           sys.executable, str(ROOT / "bench.py"), "--config", config, "--steps", "2", "--warmup", "1",
           "--no-cpu", "--no-traffic", "--copy-probe"]
    proc = subprocess.Popen(cmd, stdout=subprocess.DEVNULL, stderr=subprocess.PIPE, text=True,
                            start_new_session=True)
    try:
        _, err = proc.communicate(timeout=180)
    except subprocess.TimeoutExpired:
        os.killpg(proc.pid, signal.SIGKILL)
        proc.communicate()
        raise RuntimeError(f"rocprofv3 --pmc {counter} did not finish in 180 s")
    table = out / "run_counter_collection.csv"
    if not table.exists():       # the profiler can end badly after a complete run; only a missing table counts
        raise RuntimeError(f"rocprofv3 --pmc {counter} wrote no counters (exit {proc.returncode}): {err[-300:]}")
    seen: dict = {c: {} for c in names}
    with table.open() as f:
        for row in csv.DictReader(f):
            if row["Counter_Name"] in seen:
                seen[row["Counter_Name"]].setdefault(_kernel_base(row["Kernel_Name"]), []).append(
                    float(row["Counter_Value"]))
    return seen[names[0]] if len(names) == 1 else seen


#: The FP64 VALU instruction counters; FLOPs = 64 lanes x (ADD + MUL + TRANS + 2 FMA).
FP64_COUNTERS = ("SQ_INSTS_VALU_ADD_F64", "SQ_INSTS_VALU_MUL_F64", "SQ_INSTS_VALU_FMA_F64",
                 "SQ_INSTS_VALU_TRANS_F64", "SQ_WAVES")


def measure_fp64(config: str, kernels: list) -> dict:
    """Executed FP64 FLOPs per sample of each per-sample kernel (one sample a
    lane): one ``rocprofv3 --pmc`` pass with the FP64 instruction counters and
    SQ_WAVES; per wave, 64 x (ADD + MUL + TRANS + 2 FMA) / 64 lanes.  Dividing
    by the waves the same pass counted keeps the figure right whichever share
    of the chip's counters the pass samples."""
    log(f"fp64: rocprofv3 --pmc {' '.join(FP64_COUNTERS)} pass over --config {config}")
    seen = _pmc_pass(" ".join(FP64_COUNTERS), config)
    out = {}
    for k in kernels:
        if not all(k in seen[c] for c in FP64_COUNTERS):
            raise RuntimeError(f"fp64 counters: {k} was not seen")
        med = {c: statistics.median(seen[c][k]) for c in FP64_COUNTERS}
        per_wave = (med["SQ_INSTS_VALU_ADD_F64"] + med["SQ_INSTS_VALU_MUL_F64"] + med["SQ_INSTS_VALU_TRANS_F64"]
                    + 2.0 * med["SQ_INSTS_VALU_FMA_F64"]) / med["SQ_WAVES"]
        out[k] = {"flops_per_sample": per_wave, "counts_per_wave": {c.replace("SQ_INSTS_VALU_", ""): round(
            med[c] / med["SQ_WAVES"], 2) for c in FP64_COUNTERS[:4]}}
    return out


def measure_traffic(config: str, kernels: list, occurrence: int = 0, per_step: int = 1) -> dict:
    """HBM bytes per launch of the stage whose kernels are ``kernels``: FETCH_SIZE
    and WRITE_SIZE (KiB per dispatch, one pass each), each scaled by what the same
    counter reads for a plain copy of 1 GiB.  When a step launches the same
    kernel ``per_step`` times, the stage's dispatches are every ``per_step``-th
    from ``occurrence``."""
    total = 0.0
    factors = {}
    for counter in ("FETCH_SIZE", "WRITE_SIZE"):
        log(f"traffic: rocprofv3 --pmc {counter} pass over --config {config}")
        seen = _pmc_pass(counter, config)
        copies = [v for k, vs in seen.items() if "copyBuffer" in k for v in vs]
        if not copies or max(copies) <= 0:
            raise RuntimeError(f"{counter}: the copy probe was not seen")
        factor = COPY_PROBE_BYTES / (max(copies) * 1024.0)
        factors[counter] = round(factor, 4)
        present = [k for k in kernels if k in seen]     # a stage may launch one of two forms
        if not present:
            raise RuntimeError(f"{counter}: none of the kernels {kernels} was seen")
        for k in present:
            total += statistics.median(seen[k][occurrence::per_step]) * 1024.0 * factor
    return {"bytes": total, "factors": factors}


def _stages_of(w) -> list:
    stages = []
    for prep in w["kernels"]:
        for label, launch in prep.stages():
            while label in (x for x, _ in stages):     # a stage label taken by an earlier kernel
                label = label.split("#")[0] + "#" + str(int(label.split("#")[1]) + 1 if "#" in label else 2)
            stages.append((label, launch))
    return stages


def use_fp64_counts(w, per_stage: dict, counts: dict) -> None:
    """Replace each FP64-bound stage's FLOPs per sample by the executed count
    measured by :func:`measure_fp64` (the roofline's numerator)."""
    n = w["n"]
    for label, rec in per_stage.items():
        c = counts.get(label)
        if not c:
            continue
        f_per = c["flops_per_sample"]
        tf = f_per * n / (rec["ms"] * 1e-3) / 1e12
        rec.update({"flops_per_sample": round(f_per, 2), "fp64_counts_per_wave": c["counts_per_wave"],
                    "achieved_TFLOPs": tf, "fp64_frac": tf / FP64_PEAK_TFLOPS})
    w["flops_basis"] = ("FP64 FLOPs executed, per sample: 64 x (ADD + MUL + TRANS + 2 FMA) VALU instructions "
                        "per wave over SQ_WAVES, one rocprofv3 --pmc pass of this bench")


def time_steps(w, steps: int, warmup: int, settle_s: float = 0.0) -> dict:
    """Warm up, then time ``steps`` steps of workload ``w``: every stage launch
    bracketed by HIP events on the stream it runs on (torch's current stream,
    the stream the launchers were prepared on), the whole run by two more.
    With ``settle_s``, the warm-up goes on past ``warmup`` steps until that
    many seconds of them have run: a GPU that sat idle (during a CPU
    baseline) comes back at a lower shader clock, and its first milliseconds
    of work run 10-15 % slower in the VALU- and LDS-bound stages."""
    import torch
    stages = _stages_of(w)
    done = 0
    t_warm = time.perf_counter()
    while done < warmup or (settle_s > 0.0 and time.perf_counter() - t_warm < settle_s):
        for _label, launch in stages:
            launch()
        done += 1
        if done >= warmup and settle_s > 0.0 and done % 8 == 0:
            torch.cuda.synchronize()
    torch.cuda.synchronize()
    stream = torch.cuda.current_stream()
    events = {label: [] for label, _ in stages}
    t0 = time.perf_counter()
    start_all = torch.cuda.Event(enable_timing=True)
    end_all = torch.cuda.Event(enable_timing=True)
    start_all.record(stream)
    for _ in range(steps):
        for label, launch in stages:
            a = torch.cuda.Event(enable_timing=True)
            b = torch.cuda.Event(enable_timing=True)
            a.record(stream)
            launch()
            b.record(stream)
            events[label].append((a, b))
    end_all.record(stream)
    torch.cuda.synchronize()
    wall = time.perf_counter() - t0
    n = w["n"]
    per_stage = {}
    for label in events:
        b_per, f_per = w["work"][label]
        med = statistics.median(a.elapsed_time(b) for a, b in events[label])
        per_stage[label] = {"ms": round(med, 5), "samples_per_s": n / (med * 1e-3),
                            "bytes_per_sample": b_per, "flops_per_sample": f_per,
                            "achieved_GBs": b_per * n / (med * 1e-3) / 1e9,
                            "hbm_frac": b_per * n / (med * 1e-3) / 1e9 / HBM_PEAK_GBS}
        if w.get("bound") == "fp64" and f_per:
            tf = f_per * n / (med * 1e-3) / 1e12
            per_stage[label].update({"achieved_TFLOPs": tf, "fp64_frac": tf / FP64_PEAK_TFLOPS})
    return {"ms_step": start_all.elapsed_time(end_all) / steps, "per_stage": per_stage, "wall": wall,
            "warmup": done}


def roofline_of(w, per_stage: dict, traffic=None) -> dict:
    dominant = max(per_stage, key=lambda k: per_stage[k]["ms"])
    d = per_stage[dominant]
    if w.get("bound") == "fp64":
        return {"bound": "fp64-valu", "kernel": dominant, "achieved": round(d["achieved_TFLOPs"], 3),
                "peak": FP64_PEAK_TFLOPS, "unit": "TFLOP/s", "frac": round(d["fp64_frac"], 4), "traffic": traffic,
                "flops_basis": w.get("flops_basis", "operations counted in the emitted code")}
    return {"bound": "hbm", "kernel": dominant, "achieved": round(d["achieved_GBs"], 1),
            "peak": HBM_PEAK_GBS, "unit": "GB/s", "frac": round(d["hbm_frac"], 4), "traffic": traffic}


def host_cores() -> int:
    """The cores this process may run on (its affinity mask)."""
    try:
        return len(os.sched_getaffinity(0))
    except AttributeError:
        return os.cpu_count() or 1


def cpu_model() -> str:
    try:
        for line in Path("/proc/cpuinfo").read_text().splitlines():
            if line.startswith("model name"):
                return line.split(":", 1)[1].strip()
    except OSError:
        pass
    import platform
    return platform.processor() or "unknown"


def cpu_rate(w, threads: int, profile: str, seconds: float, min_reps: int = 5) -> tuple:
    """Samples/s of the oracle's step on ``threads`` threads in build
    ``profile`` (one warm-up, then repetitions for about ``seconds``; at
    least ``min_reps``): ``(rate, repetitions, seconds of CPU work)``; the
    rate is the median repetition's."""
    import oracle_lib as O
    O.use_profile(profile)
    cores = w.get("cpu_threads") or threads
    w["cpu"](cores)
    times = []
    begin = time.perf_counter()
    while len(times) < min_reps or (time.perf_counter() - begin < seconds and len(times) < 2000):
        t = time.perf_counter()
        w["cpu"](cores)
        times.append(time.perf_counter() - t)
    return w["n"] / statistics.median(times), len(times), sum(times)


#: The configurations the default run records beside its headline (config 2).
OTHER_CONFIGS = ("1", "3", "4a", "4b", "5")


#: Configurations whose record measures the dominant stage's HBM traffic too.
TRAFFIC_CONFIGS = ("5",)


def _fp64_stages(w, per_stage: dict) -> list:
    """The FP64-bound per-sample stages (one sample a lane), by label."""
    if w.get("bound") != "fp64":
        return []
    return [label for label in per_stage if label.split("#")[0] not in STAGE_KERNELS]


def _traffic_of(config: str, per_stage: dict, dominant: str):
    if dominant in STAGE_KERNELS:
        kernels, occurrence, per_step = STAGE_KERNELS[dominant], 0, 1
    else:
        base_label = dominant.split("#")[0]
        kernels = STAGE_KERNELS.get(base_label, (base_label,))
        occurrence = int(dominant.split("#")[1]) - 1 if "#" in dominant else 0
        per_step = sum(1 for x in per_stage if x.split("#")[0] == base_label)
    return measure_traffic(config, kernels, occurrence, per_step)


def config_record(config: str, device, steps: int = 5, warmup: int = 2, pmc: bool = True,
                  settle_s: float = 0.25) -> dict:
    """One configuration's record for the default run: its stages timed on
    the GPU (HIP events, median of ``steps``, after warm-up steps for at least
    ``settle_s`` seconds: the record follows a CPU baseline, during which the
    GPU idles), the dominant stage against its
    roofline (an FP64-bound one by its executed FLOPs, and for
    :data:`TRAFFIC_CONFIGS` with its HBM traffic, when ``pmc``), and the
    oracle on every host core (the median of at least 5 repetitions after a
    warm-up)."""
    import torch
    log(f"config {config}: record")
    w = workload(config, device)
    t = time_steps(w, steps, warmup, settle_s)
    ceiling = _with_pattern(w, device, t["per_stage"])
    traffic = None
    if pmc:
        try:
            fp64 = _fp64_stages(w, t["per_stage"])
            if fp64:
                use_fp64_counts(w, t["per_stage"], measure_fp64(config, fp64))
            if config in TRAFFIC_CONFIGS:
                dominant = max(t["per_stage"], key=lambda k: t["per_stage"][k]["ms"])
                traffic = round(_traffic_of(config, t["per_stage"], dominant)["bytes"])
                log(f"config {config}: traffic of {dominant}: {traffic / 1e6:.1f} MB per launch")
        except Exception as exc:        # counters are evidence, not the measurement
            log(f"config {config}: counters not measured: {exc}")
    rate, reps, cpu_s = cpu_rate(w, host_cores(), "native", 0.0, min_reps=5)
    rec = {"workload": w["name"], "N": w["n"], "dtype": w["dtype"], "ms_per_step": round(t["ms_step"], 5),
           "steps": steps, "warmup": t["warmup"],
           "samples_per_s": w["n"] / (t["ms_step"] * 1e-3),
           "stages": {k: {kk: (round(vv, 6) if isinstance(vv, float) else vv) for kk, vv in v.items()}
                      for k, v in t["per_stage"].items()},
           "roofline": roofline_of(w, t["per_stage"], traffic),
           **({"pattern_ceiling": ceiling} if ceiling else {}),
           "cpu_baseline": {"value": rate, "unit": "samples/s", "cores": w.get("cpu_threads") or host_cores(),
                            "kind": "port", "sample": f"the full step on the C oracle (native profile), median of "
                                                      f"{reps} repetitions ({cpu_s:.1f} s of CPU work) after 1 "
                                                      "warm-up"}}
    del w
    torch.cuda.synchronize()
    torch.cuda.empty_cache()
    return rec


# ---------------------------------------------------------------------------
# --latency: the gfx950 latencies the team stages are designed around, one
# probe kernel built through the package's hipRTC path and launched as a
# single workgroup through hk_launch_grid; one JSON object of shader-clock
# cycles (clock64) per operation:
# * add_chain_registers: a dependent fp64 add whose operand is a register;
# * add_chain_lds_alone: the same chain with its operands read from LDS,
#   eight reads ahead, by one wave on an otherwise idle CU;
# * add_chain_lds_loaded: that chain while fifteen other waves of the
#   workgroup read LDS without pause;
# * add_chain_lds_deep_alone / _loaded: the same two with 24 values read
#   ahead (four rotating blocks of eight);
# * add_chain_readlane / add_chain_dpp: operands taken from the other lanes
#   of one register by readlane or by a DPP wave_shl rotation;
# * lds_round_trip / lds_round_trip_loaded: dependent LDS reads (each address
#   the previous read's value) by one wave, alone or while fifteen other
#   waves read LDS;
# * ds_or_same_address: a 64-bit ds_or by all 64 lanes into one slot, per
#   instruction.
# Only the probe kernel's own buffers are touched (4096 doubles in, two
# doubles a wave out).

LATENCY_SOURCE = r"""
struct GRefMirror { void* data_; unsigned long long samples_, compStride_, sampleStride_; int deviceType_, deviceId_; };
extern "C" __attribute__((used)) __device__ char eagle_abi_tag[] = "aether-abi/2";
extern "C" __attribute__((used)) __device__ unsigned long long eagle_layout_sizes[5] = {40, 32, 32, 8, 24};

__device__ __forceinline__ double lane_shl(double x) {
    const long long b = __double_as_longlong(x);
    const int lo = __builtin_amdgcn_update_dpp(0, static_cast<int>(b), 0x130, 0xf, 0xf, false);
    const int hi = __builtin_amdgcn_update_dpp(0, static_cast<int>(b >> 32), 0x130, 0xf, 0xf, false);
    return __longlong_as_double((static_cast<long long>(hi) << 32) | static_cast<unsigned>(lo));
}

// src: 4096 doubles; out: two doubles a wave (cycles, a value that keeps the
// work alive).  Wave 0 runs the probe; in mode 2 the other waves read LDS.
extern "C" __global__ void __launch_bounds__(1024) hawk_latency(
        GRefMirror src_m, GRefMirror out_m, long long mode, long long reps,
        long long base, long long count, long long nSamples) {
    (void)count; (void)nSamples;
    const double* src = static_cast<const double*>(src_m.data_);
    double* out = static_cast<double*>(out_m.data_);
    __shared__ double buf[4096 + 64];               // 64 zeros past the end for the deep feed's last loads
    __shared__ int next[4096];
    __shared__ unsigned long long tab[64];
    __shared__ volatile int done;
    const int t = threadIdx.x, wave = t >> 6, lane = t & 63;
    for (int i = t; i < 4096; i += blockDim.x) {
        buf[i] = src[i];
        next[i] = (i * 1021 + 7) & 4095;          // 1021 is odd: a permutation of [0, 4096)
    }
    if (t < 64) buf[4096 + t] = 0.0;
    if (t < 64) tab[t] = 0;
    if (t == 0) done = 0;
    __syncthreads();
    double a = 0.0;
    long long c0 = clock64();
    if (wave != 0) {
        if (mode == 2 || mode == 7 || mode == 9) {  // loaders: LDS reads until wave 0's probe ends
            // (bounded as well: at most 4096 * reps rounds, more than the chain takes)
            for (long long r = 0; r < reps * 4096 && !done; ++r)
#pragma unroll
                for (int q = 0; q < 8; ++q) a += buf[(static_cast<int>(r) * 512 + q * 64 + lane) & 4095];
        }
    } else if (mode == 0) {
        const double x = buf[lane];
        for (long long r = 0; r < reps; ++r)
#pragma unroll
            for (int q = 0; q < 64; ++q) a = a + x;
    } else if (mode == 1 || mode == 2) {
        for (long long r = 0; r < reps; ++r) {
            double cur[8];
#pragma unroll
            for (int q = 0; q < 8; ++q) cur[q] = buf[q];
            for (int m = 8; m < 4096; m += 8) {
                double nxt[8];
#pragma unroll
                for (int q = 0; q < 8; ++q) nxt[q] = buf[m + q];
#pragma unroll
                for (int q = 0; q < 8; ++q) a = a + cur[q];
#pragma unroll
                for (int q = 0; q < 8; ++q) cur[q] = nxt[q];
            }
#pragma unroll
            for (int q = 0; q < 8; ++q) a = a + cur[q];
        }
    } else if (mode == 8 || mode == 9) {
        // four rotating blocks of 8: three blocks (24 values) in flight while one is added
        for (long long r = 0; r < reps; ++r) {
            double b0[8], b1[8], b2[8], b3[8];
#pragma unroll
            for (int q = 0; q < 8; ++q) { b0[q] = buf[q]; b1[q] = buf[8 + q]; b2[q] = buf[16 + q]; }
            for (int m = 24; m < 4096 + 24; m += 32) {
#pragma unroll
                for (int q = 0; q < 8; ++q) b3[q] = buf[m + q];
#pragma unroll
                for (int q = 0; q < 8; ++q) a = a + b0[q];
#pragma unroll
                for (int q = 0; q < 8; ++q) b0[q] = buf[m + 8 + q];
#pragma unroll
                for (int q = 0; q < 8; ++q) a = a + b1[q];
#pragma unroll
                for (int q = 0; q < 8; ++q) b1[q] = buf[m + 16 + q];
#pragma unroll
                for (int q = 0; q < 8; ++q) a = a + b2[q];
#pragma unroll
                for (int q = 0; q < 8; ++q) b2[q] = buf[m + 24 + q];
#pragma unroll
                for (int q = 0; q < 8; ++q) a = a + b3[q];
            }
        }
    } else if (mode == 3) {
        for (long long r = 0; r < reps; ++r) {
            const double x = buf[(static_cast<int>(r) * 64 + lane) & 4095];
            const long long b = __double_as_longlong(x);
#pragma unroll
            for (int q = 0; q < 64; ++q) {
                const int lo = __builtin_amdgcn_readlane(static_cast<int>(b), q);
                const int hi = __builtin_amdgcn_readlane(static_cast<int>(b >> 32), q);
                a = a + __longlong_as_double((static_cast<long long>(hi) << 32) | static_cast<unsigned>(lo));
            }
        }
    } else if (mode == 4) {
        for (long long r = 0; r < reps; ++r) {
            double x = buf[(static_cast<int>(r) * 64 + lane) & 4095];
#pragma unroll
            for (int q = 0; q < 64; ++q) { a = a + x; x = lane_shl(x); }
        }
    } else if (mode == 5 || mode == 7) {
        int j = lane & 0;
        for (long long r = 0; r < reps * 64; ++r) j = next[j];
        a = j;
    } else if (mode == 6) {
        // every lane's slot is lane * base = 0 (base is 0 at run time, which
        // the compiler cannot see, so it keeps one ds_or per lane)
        unsigned long long* slot = &tab[(lane * static_cast<int>(base)) & 63];
        for (long long r = 0; r < reps; ++r) {
            atomicOr(slot, 1ull << lane);
            __builtin_amdgcn_wave_barrier();
        }
        a = static_cast<double>(tab[0]);
    }
    const long long c1 = clock64();
    if (wave == 0 && lane == 0) done = 1;
    if (lane == 0) {
        out[2 * wave] = static_cast<double>(c1 - c0);
        out[2 * wave + 1] = a;
    }
}
"""

#: mode -> (name, waves, operations per repetition)
LATENCY_PROBES = {
    0: ("add_chain_registers", 1, 64),
    1: ("add_chain_lds_alone", 1, 4096),
    2: ("add_chain_lds_loaded", 16, 4096),
    3: ("add_chain_readlane", 1, 64),
    4: ("add_chain_dpp", 1, 64),
    5: ("lds_round_trip", 1, 64),
    6: ("ds_or_same_address", 1, 1),
    7: ("lds_round_trip_loaded", 16, 64),
    8: ("add_chain_lds_deep_alone", 1, 4096),
    9: ("add_chain_lds_deep_loaded", 16, 4096),
}


def latency_probes(device=None, reps: int = 64) -> dict:
    """Cycles per operation of every probe of :data:`LATENCY_SOURCE` (median of
    five launches each, after one), one workgroup on one CU."""
    import statistics

    import torch

    from hawk_amd import _core
    from hawk_amd.compile import compile_source

    device = torch.device("cuda:0") if device is None else device
    code, _key, _hit = compile_source(LATENCY_SOURCE, "hawk_latency")
    entry = _core.DeviceLibrary(code).entry("hawk_latency")
    src = torch.arange(4096, dtype=torch.float64, device=device) * 1e-3
    out = torch.zeros(32, dtype=torch.float64, device=device)
    stream = torch.cuda.current_stream()
    result = {}
    for mode, (name, waves, per_rep) in LATENCY_PROBES.items():
        ab = _core.ArgBlock(["gref", "gref", "int", "int"])
        ab.bind(0, src.data_ptr(), 4096)
        ab.bind(1, out.data_ptr(), 32)
        ab.bind_value(2, mode)
        ab.bind_value(3, reps)
        cycles = []
        for _ in range(6):
            entry.run_grid(ab, 0, 1, 1, 1, 64 * waves, stream.cuda_stream)
            stream.synchronize()
            cycles.append(float(out[0].item()))
        result[name] = round(statistics.median(cycles[1:]) / (reps * per_rep), 2)
    return result



def main() -> int:
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=3)
    ap.add_argument("--config", default="2")
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline")
    ap.add_argument("--no-traffic", action="store_true",
                    help="skip the two rocprofv3 --pmc passes that measure the dominant stage's HBM traffic")
    ap.add_argument("--only", action="store_true",
                    help="time the chosen configuration alone (the default run of config 2 also records "
                         "configs " + ", ".join(OTHER_CONFIGS) + ")")
    ap.add_argument("--latency", action="store_true",
                    help="print the CU latencies the ordered scatter is built around (one probe kernel on one "
                         "CU) as one JSON object, and nothing else")
    ap.add_argument("--pattern-sweep", action="store_true",
                    help="print the 16x16 product's HBM pattern copy rates over run lengths, workgroup sizes and "
                         "K slices as one JSON object, and nothing else")
    ap.add_argument("--copy-probe", action="store_true",
                    help="after the timed steps, run one plain 1 GiB device copy (untimed): the "
                         "known-size kernel that scales HBM counters read by rocprofv3 --pmc")
    args = ap.parse_args()
    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) != 1:
        print("bench.py measures one GPU: this build's hot path runs on a single MI355X "
              "(sharding over several GPUs is a design, not launched)", file=sys.stderr)
        return 2
    import torch
    device = torch.device("cuda:0")
    if args.latency:
        print(json.dumps({"device": torch.cuda.get_device_name(0), "cycles_per_op": latency_probes(device)}),
              flush=True)
        return 0
    if args.pattern_sweep:
        print(json.dumps({"device": torch.cuda.get_device_name(0), **pattern_sweep(device)}), flush=True)
        return 0
    log(f"config {args.config}: building and uploading inputs")
    w = workload(args.config, device)
    n = w["n"]
    log(f"timing {args.steps} steps after {args.warmup} warm-up steps")
    t = time_steps(w, args.steps, args.warmup)
    ms_step, per_stage, wall = t["ms_step"], t["per_stage"], t["wall"]
    if args.copy_probe:
        src = torch.ones(COPY_PROBE_BYTES // 8, dtype=torch.float64, device=device)
        dst = torch.empty_like(src)
        dst.copy_(src)
        torch.cuda.synchronize()
        log("copy probe: 1 GiB read + 1 GiB written by one copy kernel")
        del src, dst
    ceiling = _with_pattern(w, device, per_stage)
    dominant = max(per_stage, key=lambda k: per_stage[k]["ms"])
    d = per_stage[dominant]
    traffic = None
    if not args.no_traffic and _fp64_stages(w, per_stage):
        try:
            use_fp64_counts(w, per_stage, measure_fp64(args.config, _fp64_stages(w, per_stage)))
        except Exception as exc:        # counters are evidence, not the measurement
            log(f"fp64 FLOPs not measured: {exc}")
    if not args.no_traffic:
        try:
            tr = _traffic_of(args.config, per_stage, dominant)
            traffic = round(tr["bytes"])
            log(f"traffic of {dominant}: {traffic / 1e6:.1f} MB per launch "
                f"(algorithmic {d['bytes_per_sample'] * n / 1e6:.1f} MB; counter factors {tr['factors']})")
        except Exception as exc:        # counters are evidence, not the measurement: report null
            log(f"traffic not measured: {exc}")
    roofline = roofline_of(w, per_stage, traffic)
    cpu_baseline = None
    if not args.no_cpu:
        cores = w.get("cpu_threads") or host_cores()
        log(f"CPU baseline: the oracle on {cores} threads (native profile), then 1 thread, then -ffp-contract=fast")
        rate, reps, spent = cpu_rate(w, cores, "native", CPU_SECONDS)
        one, one_reps, one_spent = cpu_rate(w, 1, "native", CPU_SECONDS / 2)
        fast, fast_reps, _ = cpu_rate(w, cores, "fast", CPU_SECONDS / 4)
        cpu_baseline = {"value": rate, "unit": "samples/s", "cores": cores, "kind": "port",
                        "cpu_model": cpu_model(),
                        "sample": f"the full step ({w['name']}, N={n}) on the C oracle (native profile: gcc -O3 "
                                  f"-march=native -ffp-contract=off, {cores} threads, one contiguous tile each), "
                                  f"median of {reps} repetitions ({spent:.1f} s of CPU work) after 1 warm-up",
                        "one_core": {"value": one, "cores": 1, "sample": f"median of {one_reps} repetitions "
                                                                          f"({one_spent:.1f} s)"},
                        "fp_contract_fast": {"value": fast, "cores": cores,
                                             "sample": f"-ffp-contract=fast build, median of {fast_reps} "
                                                       "repetitions (its bits are not the exact profile's)"}}
    compare = {}
    if "compare" in w:
        compare["members_launched_one_by_one_ms"] = round(w["compare"](), 5)
        log(f"the same members as separate launches: {compare['members_launched_one_by_one_ms']} ms a step")
    if "compare_entries" in w:
        compare.update(w["compare_entries"]())
        log(f"the same launch through the other entries: {compare}")
    records = {}
    name, dtype = w["name"], w["dtype"]
    if args.config == "2" and not args.only:
        del w
        torch.cuda.synchronize()
        torch.cuda.empty_cache()
        for c in OTHER_CONFIGS:
            records[c] = config_record(c, device, pmc=not args.no_traffic)
    line = {
        "metric": METRIC, "value": n / (ms_step * 1e-3), "unit": "samples/s", "n_gpus": 1,
        "steps": args.steps, "warmup": args.warmup, "ms_per_step": round(ms_step, 5),
        "higher_is_better": True, "scaling": "weak", "vs_baseline": None, "dtype": dtype,
        "data": "synthetic (seeded numpy, resident in HBM before timing)",
        "config": {"workload": name, "N": n, **compare,
                   "stages": {k: {kk: (round(vv, 6) if isinstance(vv, float) else vv) for kk, vv in v.items()}
                              for k, v in per_stage.items()},
                   **({"pattern_ceiling": ceiling} if ceiling else {}),
                   **({"configs": records} if records else {})},
        "roofline": roofline, "cpu_baseline": cpu_baseline, "wall_s": round(wall, 3),
    }
    print(json.dumps(line), flush=True)
    return 0


if __name__ == "__main__":
    sys.path.insert(0, str(ROOT / "tests"))
    raise SystemExit(main())
