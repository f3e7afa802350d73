"""Benchmark of hawk's gfx950 target on one MI355X.

``python bench.py [--steps K] [--warmup W] [--config C]`` prints ONE JSON line.
A step is one pass of the hot path over one batch of synthetic inputs already
resident in HBM.  The default workload is BASELINE.json's ``configs[1]``: the
``energy`` kernel's forward, VJP and JVP over N = 2^25 samples (fp64).  Other
configurations (``--config 1|3|4a|5``) time the remaining workloads the same way.

Each kernel launch of the timed steps is bracketed by HIP events on the stream
it is launched on (torch's current stream), so the per-kernel durations, the
achieved algorithmic GB/s (bytes per sample x samples / duration) and the
roofline fraction come from the timed run itself.  The CPU baseline is the C
oracle (the host-target restatement, hawk's ``native`` profile) on the same
workload, on this host's cores.
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
FP64_PEAK_TFLOPS = 78.6


def log(msg: str) -> None:
    print(f"[bench] {msg}", file=sys.stderr, flush=True)


def _dev(a, device):
    import torch
    return torch.from_numpy(np.ascontiguousarray(a)).to(device)


# ---------------------------------------------------------------------------
# workloads: inputs (seeded, config index as seed), the kernels of one step,
# algorithmic bytes per sample of each kernel, and the CPU baseline's step.


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
        kernels = [("scale", k.prepare(x=X, a=2.0, b=1.0, out=OUT), 16, 2)]

        def cpu(threads):
            import oracle_lib as O
            out = np.empty(n)
            O.lib("native").hko_tiled(1, O._p(x), None, None, None, O._p(out), None, 2.0, 1.0, n, threads)
        return dict(name="scale fwd (config 1)", n=n, kernels=kernels, cpu=cpu, dtype="f64")
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
        kernels = [("energy", kf.prepare(v=V, out=OUT), 32, 6),
                   ("energy_vjp", kv.prepare(v=V, bar_out=BO, bar_v=BV), 56, 4),
                   ("energy_jvp", kj.prepare(v=V, dot_v=DV, dot_out=DO), 56, 12)]

        def cpu(threads):
            import oracle_lib as O
            L = O.lib("native")
            out, bv, do = np.empty(n), np.empty((3, n)), np.empty(n)
            L.hko_tiled(2, O._p(v), None, None, None, O._p(out), None, 0.0, 0.0, n, threads)
            L.hko_tiled(3, O._p(v), O._p(bar_out), None, None, O._p(bv), None, 0.0, 0.0, n, threads)
            L.hko_tiled(4, O._p(v), O._p(dv), None, None, O._p(do), None, 0.0, 0.0, n, threads)
        return dict(name="energy fwd + VJP + JVP (config 2)", n=n, kernels=kernels, cpu=cpu, dtype="f64")
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
        kernels = [("twobody", kf.prepare(r0=R0, v0=V0, mu=1.0, r=R, v=VV), 96, 42 * 32),
                   ("twobody_vjp", kv.prepare(r0=R0, v0=V0, mu=1.0, bar_r=BR, bar_v=BV, bar_r0=BR0, bar_v0=BV0),
                    144, 3 * 42 * 32)]

        def cpu(threads):
            import oracle_lib as O
            O.twobody(r0, v0, 1.0, threads=threads)
            O.twobody_vjp(r0, v0, 1.0, bar_r, bar_v, threads=threads)
        return dict(name="two-body leapfrog fwd + VJP (config 3)", n=n, kernels=kernels, cpu=cpu,
                    dtype="f64", bound="fp64")
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
        kernels = [("spd_solve", kf.prepare(A=Ad, b=bd, x=X), 384, 230),
                   ("spd_solve_vjp", kv.prepare(A=Ad, b=bd, bar_x=BX, bar_A=BA, bar_b=BB), 720, 410)]

        def cpu(threads):
            import oracle_lib as O
            O.spd_solve(A, b, threads=threads)
            O.spd_solve_vjp(A, b, bar_x, threads=threads)
        return dict(name="6x6 SPD solve fwd + VJP (config 4a)", n=n, kernels=kernels, cpu=cpu, dtype="f64")
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
        kernels = [("chain", k.prepare(x=X, key=KEY, y=Y, total=TOT, bins=BINS), 20, 14)]

        def cpu(threads):
            import oracle_lib as O
            y = O.chain(x, threads=threads)
            O.ordered_sum(y, threads=threads)
            O.ordered_scatter(key, y, np.zeros(cells), threads=threads)
        return dict(name="chain + ordered sum + ordered scatter (config 5)", n=n, kernels=kernels, cpu=cpu,
                    dtype="f64")
    raise SystemExit(f"unknown --config {config!r}")


def main() -> int:
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=3)
    ap.add_argument("--config", default="2")
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline")
    args = ap.parse_args()
    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) != 1:
        print("bench.py measures one GPU: this build's hot path runs on a single MI355X "
              "(multi-GPU sharding is described in DESIGN.md, not launched)", file=sys.stderr)
        return 2
    import torch
    device = torch.device("cuda:0")
    log(f"config {args.config}: building and uploading inputs")
    w = workload(args.config, device)
    n = w["n"]
    for _ in range(args.warmup):
        for _name, fn, _b, _f in w["kernels"]:
            fn()
    torch.cuda.synchronize()
    log(f"warmup done ({args.warmup} steps); timing {args.steps} steps")
    stream = torch.cuda.current_stream()
    events = {name: [] for name, *_ in w["kernels"]}
    t0 = time.perf_counter()
    torch.cuda.synchronize()
    start_all = torch.cuda.Event(enable_timing=True)
    end_all = torch.cuda.Event(enable_timing=True)
    start_all.record(stream)
    for _ in range(args.steps):
        for name, fn, _b, _f in w["kernels"]:
            a = torch.cuda.Event(enable_timing=True)
            b = torch.cuda.Event(enable_timing=True)
            a.record(stream)
            fn()
            b.record(stream)
            events[name].append((a, b))
    end_all.record(stream)
    torch.cuda.synchronize()
    wall = time.perf_counter() - t0
    ms_step = start_all.elapsed_time(end_all) / args.steps
    per_kernel = {}
    for name, b_per, f_per in ((k[0], k[2], k[3]) for k in w["kernels"]):
        ms = [a.elapsed_time(b) for a, b in events[name]]
        med = statistics.median(ms)
        per_kernel[name] = {"ms": round(med, 5), "samples_per_s": n / (med * 1e-3),
                            "bytes_per_sample": b_per, "flops_per_sample": f_per,
                            "achieved_GBs": b_per * n / (med * 1e-3) / 1e9,
                            "hbm_frac": b_per * n / (med * 1e-3) / 1e9 / HBM_PEAK_GBS}
    dominant = max(per_kernel, key=lambda k: per_kernel[k]["ms"])
    d = per_kernel[dominant]
    if w.get("bound") == "fp64":
        achieved = d["flops_per_sample"] * n / (d["ms"] * 1e-3) / 1e12
        roofline = {"bound": "fp64-valu", "kernel": dominant, "achieved": round(achieved, 3),
                    "peak": FP64_PEAK_TFLOPS, "unit": "TFLOP/s", "frac": round(achieved / FP64_PEAK_TFLOPS, 4),
                    "traffic": None}
    else:
        roofline = {"bound": "hbm", "kernel": dominant, "achieved": round(d["achieved_GBs"], 1),
                    "peak": HBM_PEAK_GBS, "unit": "GB/s", "frac": round(d["hbm_frac"], 4), "traffic": None}
    cpu_baseline = None
    if not args.no_cpu:
        threads = os.cpu_count() or 1
        threads = min(threads, 16)
        log(f"CPU baseline: oracle (native profile) on {threads} threads")
        import oracle_lib as O
        O.build("native")
        w["cpu"](threads)
        times = []
        for _ in range(3):
            t = time.perf_counter()
            w["cpu"](threads)
            times.append(time.perf_counter() - t)
        tc = statistics.median(times)
        cpu_baseline = {"value": n / tc, "unit": "samples/s", "cores": threads, "kind": "port",
                        "sample": f"the full step ({w['name']}, N={n}) on the C oracle, median of 3 after 1 warm-up"}
    line = {
        "metric": METRIC, "value": n / (ms_step * 1e-3), "unit": "samples/s", "n_gpus": 1,
        "steps": args.steps, "warmup": args.warmup, "ms_per_step": round(ms_step, 5),
        "higher_is_better": True, "scaling": "weak", "vs_baseline": None, "dtype": w["dtype"],
        "data": "synthetic (seeded numpy, resident in HBM before timing)",
        "config": {"workload": w["name"], "N": n,
                   "kernels": {k: {kk: (round(vv, 6) if isinstance(vv, float) else vv) for kk, vv in v.items()}
                               for k, v in per_kernel.items()}},
        "roofline": roofline, "cpu_baseline": cpu_baseline, "wall_s": round(wall, 3),
    }
    print(json.dumps(line), flush=True)
    return 0


if __name__ == "__main__":
    sys.path.insert(0, str(ROOT / "tests"))
    raise SystemExit(main())
