"""The launch-crossing contract of reference tests/test_launch_crossings.py:125-178
and tests/cards/CARD_LAUNCH_CROSSINGS.md, on the gfx950 target: a loop that
keeps its binding crosses the C-ABI once per launch; a loop that moves every
pointer each step crosses twice (one bulk rebind, one launch), whatever the
number of pointer slots.  ``hawk.run`` keeps the same budget: over the planes
of its last run it adds no crossing to its launch, over moved planes one."""

from __future__ import annotations

import time

import numpy as np
import pytest

from conftest import rng

pytestmark = pytest.mark.gpu

N = 256
LAUNCHES = 2000


def _crossings_per_launch(body, launches: int = LAUNCHES) -> float:
    """``body`` called ``launches`` times between two readings; the closing
    reading's own crossing is taken off."""
    from hawk_amd import _core
    before = _core.crossings()
    for _ in range(launches):
        body()
    after = _core.crossings()
    return (after - before - 1) / launches


def _pointer_slots(kernel) -> list:
    return [i for i, k in enumerate(kernel.block.descriptor) if k not in ("f64", "f32", "int", "nsamples")]


def _cases(gpu):
    """(kernel name, planes, a second set of planes of the same shapes) for a
    kernel with 2 pointer slots and one with 4."""
    import torch

    def d(a):
        return torch.from_numpy(np.ascontiguousarray(a)).to(gpu)
    g = rng(71)
    scale = ({"x": d(g.uniform(-1, 1, N)), "a": 2.0, "b": 1.0, "out": d(np.zeros(N))},
             {"x": d(g.uniform(-1, 1, N)), "a": 2.0, "b": 1.0, "out": d(np.zeros(N))})
    r0 = g.normal(size=(3, N))
    r0 /= np.linalg.norm(r0, axis=0)
    twobody = tuple({"r0": d(r0), "v0": d(g.normal(0.0, 0.3, (3, N))), "mu": 1.0,
                     "r": d(np.zeros((3, N))), "v": d(np.zeros((3, N)))} for _ in range(2))
    return [("scale", *scale), ("twobody", *twobody)]


def test_stable_and_rebind_loops_cross_once_and_twice_per_launch(unit, gpu):
    import torch

    import hawk_amd as hawk
    stream = torch.cuda.current_stream().cuda_stream
    counts = {}
    for name, planes, other in _cases(gpu):
        k = hawk.load(unit, name)
        hawk.run(k, **planes)                           # the validated bind
        slots = _pointer_slots(k)
        print(f"crossings {name}: {len(slots)} pointer slots", flush=True)
        stable = _crossings_per_launch(lambda: k.launch(0, N, N, stream))
        ptrs = [planes[k.arg_spec[s][1]].data_ptr() for s in slots]

        def step():
            k.rebind(slots, ptrs)
            k.launch(0, N, N, stream)
        moved = _crossings_per_launch(step)
        torch.cuda.synchronize()
        assert stable == 1.0, f"{name}: the stable-binding loop crossed {stable} times per launch"
        assert moved == 2.0, f"{name}: the rebind-every-slot loop crossed {moved} times per launch"
        counts[name] = len(slots)
    assert counts == {"scale": 2, "twobody": 4}         # 2, not slots + 1, at two slot counts


def test_hawk_run_rebinds_only_what_moved(unit, gpu):
    """hawk.run over the planes of its last run: one crossing (the launch);
    alternating between two sets of planes: two (the bulk rebind and the
    launch); the results follow the planes bound."""
    import torch

    import hawk_amd as hawk
    for name, planes, other in _cases(gpu):
        k = hawk.load(unit, name)
        hawk.run(k, **planes)
        same = _crossings_per_launch(lambda: hawk.run(k, **planes), 200)
        turn = [0]

        def alternate():
            turn[0] ^= 1
            hawk.run(k, **(other if turn[0] else planes))
        moved = _crossings_per_launch(alternate, 200)
        torch.cuda.synchronize()
        assert (same, moved) == (1.0, 2.0), (name, same, moved)
    scale_a, scale_b = _cases(gpu)[0][1:]
    k = hawk.load(unit, "scale")
    hawk.run(k, **scale_a)
    hawk.run(k, **scale_b)
    torch.cuda.synchronize()
    for p in (scale_a, scale_b):
        assert p["out"].cpu().numpy().tobytes() == ((2.0 * p["x"].cpu().numpy()) + 1.0).tobytes()


def test_seconds_per_launch_beside_the_card(unit, gpu):
    """Host seconds per launch of both arms, interleaved, five repeats (the
    card's measurement; printed, gating nothing but a sanity ceiling)."""
    import torch

    import hawk_amd as hawk
    stream = torch.cuda.current_stream().cuda_stream
    for name, planes, other in _cases(gpu):
        k = hawk.load(unit, name)
        hawk.run(k, **planes)
        slots = _pointer_slots(k)
        ptrs = [planes[k.arg_spec[s][1]].data_ptr() for s in slots]
        arms = {"stable_binding": [], "rebind_every_slot": []}
        for _ in range(5):
            t0 = time.perf_counter()
            for _ in range(LAUNCHES):
                k.launch(0, N, N, stream)
            arms["stable_binding"].append((time.perf_counter() - t0) / LAUNCHES)
            torch.cuda.synchronize()
            t0 = time.perf_counter()
            for _ in range(LAUNCHES):
                k.rebind(slots, ptrs)
                k.launch(0, N, N, stream)
            arms["rebind_every_slot"].append((time.perf_counter() - t0) / LAUNCHES)
            torch.cuda.synchronize()
        for arm, xs in arms.items():
            print(f"launch seconds {name} {arm}: min {min(xs):.3g} median {sorted(xs)[2]:.3g} max {max(xs):.3g} "
                  f"({len(slots)} pointer slots, N={N})", flush=True)
            assert sorted(xs)[2] < 1e-3
