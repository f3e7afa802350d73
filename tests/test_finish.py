"""Kernels that finish their own sample, and ``hawk.steps`` (the shape of
reference ``tests/test_finish_own_sample.py``).

``terminated = cond`` makes the sample's mask ``mask | cond`` and adds one to
the ``finished_count`` cell per newly finished sample; a kernel declaring
``terminated: Terminated`` skips the samples its mask holds.  ``hawk.steps``
takes up to K such steps a launch.

Rows:

* the oracle, pinned by the closed form of the explicit-Euler oscillator
  (``x + i v`` is multiplied by ``1 - i dt`` each step) and by the step
  count ``t_final / dt`` (exact: every ``t`` is a multiple of ``dt = 1/8``);
  K steps a launch give the bits of K single-step launches;
* the tracer's record (the mask and counter slots, the sidecar's ``finish``),
  its refusals (each names the kernel) and the rendered epilogue;
* the IR evaluator running the stepped program equals the oracle, bit for bit;
* on the GPU (``-m gpu``): the oscillator stepped until its counter reaches N,
  one step and eight steps a launch, bit for bit against the oracle with the
  launch count exact; a pre-set mask skipped and never counted; a stop-only
  kernel; a derived kernel guarded by the same mask; 2^22 samples.
"""

from __future__ import annotations

import numpy as np
import pytest

import oracle_lib as O
from conftest import rng

from hawk_amd import Mutable, Scalar, Terminated

DT = 0.125
N = 40


def _inputs(n=N, seed=7):
    g = np.random.default_rng(seed)
    t_final = DT * g.integers(3, 30, n).astype(float)
    x = g.uniform(-1.0, 1.0, n)
    v = g.uniform(-1.0, 1.0, n)
    return t_final, x, v


def _oracle_until_done(K, t_final, x, v, mask=None, limit=400):
    """Launch the oracle until every sample is finished: the planes, the count
    each launch added, and the number of launches."""
    n = x.size
    x, v, t = x.copy(), v.copy(), np.zeros(n)
    mask = np.zeros(n, dtype=bool) if mask is None else mask.copy()
    counts = []
    while not mask.all() and len(counts) < limit:
        counts.append(O.osc_launch(K, DT, t_final, x, v, t, mask))
    return x, v, t, mask, counts


# -- the oracle, pinned -----------------------------------------------------------

def test_the_oracle_follows_the_closed_form_and_stops_on_time():
    t_final, x0, v0 = _inputs(200, seed=3)
    x, v, t, mask, counts = _oracle_until_done(1, t_final, x0, v0)
    steps = np.rint(t_final / DT).astype(int)
    assert mask.all() and sum(counts) == x0.size
    assert len(counts) == steps.max()
    # every t is a multiple of 1/8, so the additions are exact and t stops at t_final
    assert np.array_equal(t, steps * DT) and np.array_equal(t, t_final)
    # x' + i v' = (1 - i dt)(x + i v): after m steps, (1 - i dt)^m (x0 + i v0)
    z = (1.0 - 1j * DT) ** steps * (x0 + 1j * v0)
    scale = np.abs(z)
    assert np.all(np.abs(x - z.real) <= 64 * steps * np.finfo(float).eps * scale)
    assert np.all(np.abs(v - z.imag) <= 64 * steps * np.finfo(float).eps * scale)
    # each launch counts exactly the samples whose last step it took
    assert counts == [int((steps == m).sum()) for m in range(1, steps.max() + 1)]


def test_the_oracle_after_the_first_step_by_hand():
    """One step of one sample, worked by hand: x=1, v=0, dt=1/8 gives
    v = -1/8, x = 1, t = 1/8; a second gives x = 1 - 1/64, v = -1/4."""
    x, v, t = np.array([1.0]), np.array([0.0]), np.array([0.0])
    mask, t_final = np.zeros(1, dtype=bool), np.array([0.25])
    assert O.osc_launch(1, DT, t_final, x, v, t, mask) == 0
    assert (x[0], v[0], t[0], bool(mask[0])) == (1.0, -0.125, 0.125, False)
    assert O.osc_launch(1, DT, t_final, x, v, t, mask) == 1
    assert (x[0], v[0], t[0], bool(mask[0])) == (1.0 - 1.0 / 64, -0.25, 0.25, True)


@pytest.mark.parametrize("K", [2, 8, 64])
def test_k_steps_a_launch_are_k_single_steps(K):
    t_final, x0, v0 = _inputs(300, seed=5)
    one = _oracle_until_done(1, t_final, x0, v0)
    many = _oracle_until_done(K, t_final, x0, v0)
    for a, b in zip(one[:4], many[:4]):
        assert a.tobytes() == b.tobytes()
    assert len(many[4]) == -(-len(one[4]) // K)
    assert sum(many[4]) == x0.size


def test_a_set_mask_is_skipped_and_never_counted_by_the_oracle():
    t_final, x0, v0 = _inputs()
    preset = np.zeros(N, dtype=bool)
    preset[[0, 3, 7, 11]] = True
    x, v, t, mask, counts = _oracle_until_done(1, t_final, x0, v0, preset)
    assert sum(counts) == N - preset.sum()
    assert np.array_equal(x[preset], x0[preset]) and np.all(t[preset] == 0.0)


# -- the tracer -------------------------------------------------------------------

def test_the_trace_records_the_finish_and_binds_the_counter():
    from hawk_amd import examples as E
    from hawk_amd.ir import Finish
    spec = E.osc_finish.arg_spec
    assert ("lookup", "finished_count") in spec and ("terminated", "terminated") in spec
    assert E.osc_finish.decls["finished_count"].ttype.dtype == "u32"
    fin = [s for s in E.osc_finish.sinks if isinstance(s, Finish)]
    assert len(fin) == 1 and fin[0].steps == 1 and E.osc_finish.sinks[-1] is fin[0]
    assert ("lookup", "finished_count") in E.stop_only.arg_spec
    assert E.osc_finish_x8.sinks[-1].steps == 8 and E.osc_finish_x8.step is E.osc_finish


def test_a_derived_kernel_drops_the_finish_and_keeps_the_guard():
    from hawk_amd import examples as E
    from hawk_amd.diff import jvp, vjp
    from hawk_amd.ir import Finish
    from hawk_amd.trace import Kernel
    for transform in (vjp, jvp):
        prog = transform(E.smooth_finish, wrt=("x",))
        assert not any(isinstance(s, Finish) for s in prog.sinks)
        spec = Kernel("d", prog).arg_spec
        assert ("lookup", "finished_count") not in spec and ("terminated", "terminated") in spec


def test_the_sidecar_declares_the_finish(tmp_path):
    import hawk_amd as hawk
    from hawk_amd import examples as E
    b = hawk.build([E.osc_finish, E.osc_finish_x8, E.smooth_finish_vjp, E.stop_only], tmp_path)
    sc = b.sidecar("osc_finish")
    assert sc["finish"] == {"mask": "terminated", "counter": "finished_count", "steps": 1}
    assert sc["terminated_readonly"] is False
    assert ["lookup", "finished_count"] in sc["arg_spec"]
    assert b.sidecar("osc_finish_x8")["finish"]["steps"] == 8
    d = b.sidecar("smooth_finish_vjp")
    assert "finish" not in d and d["terminated_readonly"] is True
    assert ["lookup", "finished_count"] not in d["arg_spec"]
    assert "hk_finish_count" not in (tmp_path / "smooth_finish_vjp.hip").read_text()


def test_the_epilogue_is_the_last_text_of_the_guarded_scope():
    from hawk_amd import examples as E
    from hawk_amd.emit_hip import plan_kernel
    src = plan_kernel(E.osc_finish.program, "osc_finish").source
    lines = [ln.strip() for ln in src[src.index("hk_in = "):].splitlines()]
    guard = lines.index("if (hk_in && hk_p_terminated[hk_i] == 0) {")
    close = lines.index("}", guard)
    assert lines[close - 1].startswith("if (") and lines[close - 1].endswith(
        "{ hk_p_terminated[hk_i] = 1; hk_new = true; }")
    stores = [k for k, ln in enumerate(lines[:close]) if ln.startswith("hk_p_") and "] = " in ln]
    assert stores and max(stores) < close - 1
    assert lines[close + 1] == "hk_finish_count(hk_p_finished_count, hk_new);"


def test_a_guarded_kernel_that_never_finishes_reads_its_mask_only():
    import hawk_amd as hawk
    from hawk_amd.emit_hip import plan_kernel

    @hawk.kernel
    def guarded(x: Scalar, terminated: Terminated, y: Mutable[Scalar]):
        y = x + 1.0
    src = plan_kernel(guarded.program, "guarded").source
    assert "const unsigned char* __restrict__ hk_p_terminated" in src
    assert "hk_finish_count" not in src and "finished_count" not in src
    assert ("terminated", "terminated") in guarded.arg_spec


def _refused(src_fn, match):
    import hawk_amd as hawk
    from hawk_amd.ir import HawkError
    with pytest.raises(HawkError, match=match):
        hawk.kernel(src_fn)


def test_a_second_finish_refuses():

    def twice(x: Scalar, terminated: Terminated, y: Mutable[Scalar]):
        y = x
        terminated = x > 1.0
        terminated = x > 2.0
    _refused(twice, r"'twice'.*finished twice")


def test_a_finish_on_both_sides_of_an_if_is_two_statements_and_refuses():

    def both(x: Scalar, terminated: Terminated, y: Mutable[Scalar]):
        y = x
        if x > 0.0:
            terminated = x > 1.0
        else:
            terminated = x < -1.0
    _refused(both, r"'both'.*finished twice")


@pytest.mark.parametrize("literal", ["True", "False"])
def test_a_bool_literal_refuses(literal, tmp_path):
    src = (f"def lit(x: Scalar, terminated: Terminated, y: Mutable[Scalar]):\n"
           f"    y = x\n"
           f"    terminated = {literal}\n")
    scope = {"Scalar": Scalar, "Terminated": Terminated, "Mutable": Mutable}
    path = tmp_path / f"lit_{literal}.py"          # the trace reads the source file
    path.write_text(src)
    exec(compile(src, str(path), "exec"), scope)
    _refused(scope["lit"], r"'lit'.*Python literal")


def test_a_mask_the_guard_does_not_gate_on_refuses():

    def other(x: Scalar, terminated: Terminated, rejected: Terminated, y: Mutable[Scalar]):
        y = x
        rejected = x > 1.0
    _refused(other, r"'other'.*'rejected'.*guard")


def test_an_undeclared_terminated_refuses():

    def undeclared(x: Scalar, y: Mutable[Scalar]):
        y = x
        Terminated[...] = x > 1.0
    _refused(undeclared, r"'undeclared'.*did not declare")


def test_a_finish_inside_a_for_refuses():

    def looped(x: Scalar, terminated: Terminated, y: Mutable[Scalar]):
        y = x
        for _ in range(3):
            terminated = x > 1.0
    _refused(looped, r"'looped'.*inside a `for`")


def test_a_guarded_kernel_with_a_sum_refuses_at_build():
    import hawk_amd as hawk
    from hawk_amd.emit_hip import plan_kernel
    from hawk_amd.ir import HawkError

    @hawk.kernel
    def summed(x: Scalar, terminated: Terminated, total: Mutable[Scalar]):
        total = hawk.sum(x, policy="ordered")
        terminated = x > 1.0
    with pytest.raises(HawkError, match="guarded kernel"):
        plan_kernel(summed.program, "summed")


# -- hawk.steps -------------------------------------------------------------------

def test_steps_refusals():
    import hawk_amd as hawk
    from hawk_amd import examples as E
    from hawk_amd.diff import jvp
    from hawk_amd.ir import HawkError
    with pytest.raises(HawkError, match="never finishes"):
        hawk.steps(E.scale, 4)
    with pytest.raises(HawkError, match="K is an int"):
        hawk.steps(E.osc_finish, 0)
    with pytest.raises(HawkError, match="K is an int"):
        hawk.steps(E.osc_finish, "several")

    @hawk.kernel
    def reserved(fused_steps: Scalar, terminated: Terminated, x: Mutable[Scalar]):
        x = x + fused_steps
        terminated = x > 1.0
    with pytest.raises(HawkError, match="'fused_steps' is reserved"):
        hawk.steps(reserved, "auto")
    with pytest.raises(HawkError, match="derive from the single step"):
        hawk.steps(E.osc_finish_x8, 2)
    with pytest.raises(HawkError, match="commits no Mutable"):
        hawk.steps(E.stop_only, 2)

    @hawk.kernel
    def returns(x: Scalar, terminated: Terminated) -> Scalar:
        terminated = x > 1.0
        return x * 2.0
    with pytest.raises(HawkError, match="not a step kernel's commit"):
        hawk.steps(returns, 2)
    with pytest.raises(HawkError, match="differentiate the single step"):
        jvp(E.osc_finish_x8, wrt=("t_final",))

    @hawk.kernel
    def inner_loop(terminated: Terminated, x: Mutable[Scalar]):
        y = x
        for _ in range(3):
            y = y * 0.5
        x = y
        terminated = y < 0.1
    with pytest.raises(HawkError, match="loop of the step reads the carried state"):
        hawk.steps(inner_loop, 2)


@pytest.mark.parametrize("K", [1, 3, 8])
def test_the_stepped_program_evaluates_to_the_oracle(K):
    """The IR of ``hawk.steps(osc_finish, K)``, evaluated in NumPy (the guard
    applied by hand), launch by launch, equals the oracle bit for bit."""
    import hawk_amd as hawk
    from hawk_amd import examples as E
    from ir_eval import evaluate
    k = E.osc_finish if K == 1 else hawk.steps(E.osc_finish, K)
    t_final, x, v = _inputs(64, seed=9)
    t, mask = np.zeros(x.size), np.zeros(x.size, dtype=bool)
    ox, ov, ot, om = x.copy(), v.copy(), t.copy(), mask.copy()
    for _ in range(40):
        env = {"dt": DT, "t_final": t_final, "x": x, "v": v, "t": t, "terminated": mask}
        got = evaluate(k.program, env, x.size)
        live = ~mask
        x, v, t = (np.where(live, got[n], old) for n, old in (("x", x), ("v", v), ("t", t)))
        newly = live & got["terminated"]
        mask = mask | newly
        counted = O.osc_launch(K, DT, t_final, ox, ov, ot, om)
        assert int(newly.sum()) == counted
        for a, b in ((x, ox), (v, ov), (t, ot), (mask, om)):
            assert a.tobytes() == b.tobytes()
        if mask.all():
            break
    assert mask.all()


def test_an_automatic_kernel_records_its_word_and_fast_entries(tmp_path):
    import hawk_amd as hawk
    from hawk_amd import examples as E
    ka = E.osc_finish_xauto
    assert ka.name == "osc_finish_xauto" and ka.sinks[-1].steps == "auto"
    assert ("lookup", "fused_steps") in ka.arg_spec
    b = hawk.build([ka], tmp_path)
    sc = b.sidecar(ka.name)
    assert sc["finish"] == {"mask": "terminated", "counter": "finished_count", "steps": "auto", "steps_max": 64}
    assert sc["fast_entries"] == {"range": "osc_finish_xauto_range", "persist": "osc_finish_xauto_persist"}
    src = (tmp_path / f"{ka.name}.hip").read_text()
    persist = src[src.index("osc_finish_xauto_persist("):]
    # one claim a wave: a ballot, one atomic add by the first needy lane; no barrier
    assert "atomicAdd(hk_next," in persist and "__syncthreads" not in persist
    assert "hk_span = hk_chunk < 1 ? 1 : hk_chunk" in persist        # every chunk runs a trip
    from hawk_amd.resources import kernel_resources
    res = kernel_resources((tmp_path / f"{ka.name}.hsaco").read_bytes())
    assert set(res) == {ka.name, f"{ka.name}_range", f"{ka.name}_persist"}
    assert all(r["private_segment_fixed_size"] == 0 for r in res.values())


@pytest.mark.parametrize("word", [1, 5, 0, -3, 64, 100])
def test_the_automatic_program_runs_the_word_of_trips(word):
    from hawk_amd import examples as E
    from ir_eval import evaluate
    t_final, x, v = _inputs(64, seed=19)
    t, mask = np.zeros(x.size), np.zeros(x.size, dtype=bool)
    env = {"dt": DT, "t_final": t_final, "x": x, "v": v, "t": t, "terminated": mask,
           "fused_steps": np.array([word], dtype=np.int32)}
    got = evaluate(E.osc_finish_xauto.program, env, x.size)
    ox, ov, ot, om = x.copy(), v.copy(), t.copy(), mask.copy()
    trips = np.zeros(x.size, dtype=np.int32)
    O.osc_launch(word, DT, t_final, ox, ov, ot, om, trips=trips)
    for key, ref in (("x", ox), ("v", ov), ("t", ot), ("terminated", om)):
        assert np.asarray(got[key]).tobytes() == ref.tobytes(), key
    assert np.array_equal(trips, np.clip(np.minimum(word, np.rint(t_final / DT)), 0, None))


def test_a_finishing_kernel_is_its_automatic_kernel_by_default():
    import hawk_amd as hawk
    from hawk_amd import examples as E
    k = E.decay_until
    assert k.name == "decay_until" and k.sinks[-1].steps == "auto" and k.step.name == "decay_until"
    assert ("lookup", "fused_steps") in k.arg_spec
    assert hawk.steps(k, 4).name == "decay_until_x4" and hawk.steps(k, 4).step is k.step
    assert E.osc_finish.sinks[-1].steps == 1                     # steps=1 keeps the single step
    assert E.stop_only.sinks[-1].steps == 1                      # commits no plane: not admitted

    @hawk.kernel(steps=3)
    def three(terminated: Terminated, y: Mutable[Scalar]):
        y = y * 0.5
        terminated = y < 0.1
    assert three.name == "three_x3" and three.sinks[-1].steps == 3


def test_a_chain_of_a_guarded_member_refuses():
    import hawk_amd as hawk
    from hawk_amd import examples as E
    from hawk_amd.ir import HawkError
    with pytest.raises(HawkError, match="'osc_finish' declares a Terminated mask"):
        hawk.chain(E.osc_finish, E.scale, name="c")


# -- on the GPU -------------------------------------------------------------------

@pytest.fixture(scope="module")
def finishing(tmp_path_factory):
    import hawk_amd as hawk
    from hawk_amd import examples as E
    directory = tmp_path_factory.mktemp("finishing")
    hawk.build(list(E.FINISHING.values()), directory)
    return directory


def _dev(a, gpu):
    import torch
    return torch.from_numpy(np.ascontiguousarray(a)).to(gpu)


def _step_on_gpu(finishing, gpu, name, t_final, x, v, preset=None, limit=400):
    import hawk_amd as hawk
    import torch
    k = hawk.load(finishing, name)
    n = x.size
    mask = np.zeros(n, dtype=bool) if preset is None else preset.copy()
    planes = {"t_final": _dev(t_final, gpu), "x": _dev(x, gpu), "v": _dev(v, gpu),
              "t": _dev(np.zeros(n), gpu), "terminated": _dev(mask, gpu)}
    counter = torch.tensor([int(mask.sum())], dtype=torch.int32, device=gpu)
    launches = 0
    while int(counter.item()) < n and launches < limit:
        hawk.run(k, dt=DT, finished_count=counter, **planes)
        launches += 1
    got = {key: val.cpu().numpy() for key, val in planes.items()}
    return got, int(counter.item()), launches


@pytest.mark.gpu
@pytest.mark.parametrize("name,K", [("osc_finish", 1), ("osc_finish_x8", 8)])
def test_the_device_finishes_counts_and_matches_the_oracle(finishing, gpu, name, K):
    t_final, x, v = _inputs()
    got, counted, launches = _step_on_gpu(finishing, gpu, name, t_final, x, v)
    rx, rv, rt, rmask, counts = _oracle_until_done(K, t_final, x, v)
    assert counted == N and got["terminated"].all() and rmask.all()
    assert launches == len(counts) == -(-int(round(t_final.max() / DT)) // K)
    for key, ref in (("x", rx), ("v", rv), ("t", rt)):
        assert got[key].tobytes() == ref.tobytes(), key


@pytest.mark.gpu
@pytest.mark.parametrize("name", ["osc_finish", "osc_finish_x8"])
def test_a_preset_mask_is_skipped_and_never_counted(finishing, gpu, name):
    t_final, x, v = _inputs()
    preset = np.zeros(N, dtype=bool)
    preset[[0, 3, 7, 11]] = True
    got, counted, _ = _step_on_gpu(finishing, gpu, name, t_final, x, v, preset=preset)
    assert counted == N, f"a pre-set sample was counted again ({counted})"
    assert np.array_equal(got["x"][preset], x[preset])
    assert np.array_equal(got["t"][preset], np.zeros(preset.sum()))


@pytest.mark.gpu
def test_a_stop_only_kernel_finishes_and_counts(finishing, gpu):
    import hawk_amd as hawk
    import torch
    k = hawk.load(finishing, "stop_only")
    n = 100_003
    t = np.linspace(0.0, 1.0, n)
    mask = torch.zeros(n, dtype=torch.bool, device=gpu)
    counter = torch.zeros(1, dtype=torch.int32, device=gpu)
    hawk.run(k, t=_dev(t, gpu), t_final=0.5, terminated=mask, finished_count=counter)
    assert np.array_equal(mask.cpu().numpy(), t >= 0.5)
    assert int(counter.item()) == int((t >= 0.5).sum())
    hawk.run(k, t=_dev(t, gpu), t_final=0.5, terminated=mask, finished_count=counter)
    assert int(counter.item()) == int((t >= 0.5).sum()), "a set mask was counted again"
    # unbound, the runtime counts each run afresh: a lower t_final finishes more
    hawk.run(k, t=_dev(t, gpu), t_final=0.25, terminated=mask)
    assert int(k.finished.item()) == int(((t >= 0.25) & (t < 0.5)).sum())


@pytest.mark.gpu
def test_a_derived_kernel_skips_the_masked_samples(finishing, gpu):
    import hawk_amd as hawk
    k = hawk.load(finishing, "smooth_finish_vjp")
    n = 4099
    g = rng(21)
    x, bar_y = g.uniform(-3.0, 3.0, n), g.normal(size=n)
    mask = g.uniform(size=n) < 0.3
    bar_x = _dev(np.full(n, -7.0), gpu)
    term = _dev(mask, gpu)
    hawk.run(k, x=_dev(x, gpu), bar_y=_dev(bar_y, gpu), terminated=term, bar_x=bar_x)
    got = bar_x.cpu().numpy()
    assert np.all(got[mask] == -7.0)
    assert got[~mask].tobytes() == (bar_y * (x + x))[~mask].tobytes() or \
        np.allclose(got[~mask], (2.0 * x * bar_y)[~mask], rtol=1e-15, atol=0)
    assert np.array_equal(term.cpu().numpy(), mask)          # read only


@pytest.mark.gpu
def test_two_to_the_22_samples_step_to_the_oracle(finishing, gpu):
    """At 2^22 samples, eight steps a launch: every plane equal to the
    oracle's bit for bit, the counter exactly N, the launch count exact."""
    n = 1 << 22
    t_final, x, v = _inputs(n, seed=13)
    got, counted, launches = _step_on_gpu(finishing, gpu, "osc_finish_x8", t_final, x, v)
    rx, rv, rt, rmask, counts = _oracle_until_done(8, t_final, x, v)
    assert counted == n and launches == len(counts)
    for key, ref in (("x", rx), ("v", rv), ("t", rt), ("terminated", rmask)):
        assert got[key].tobytes() == ref.tobytes(), key


def _run_auto(finishing, gpu, t_final, x, v, mask, word, entry="plain", chunk=8):
    """One launch of the automatic oscillator; the planes, the runtime's
    counter and, for a fast entry, its reports."""
    import hawk_amd as hawk
    k = hawk.load(finishing, "osc_finish_xauto")
    planes = {"t_final": _dev(t_final, gpu), "x": _dev(x, gpu), "v": _dev(v, gpu),
              "t": _dev(np.zeros(x.size), gpu), "terminated": _dev(mask, gpu)}
    hawk.run(k, dt=DT, steps=word, entry=entry, chunk=chunk, **planes)
    got = {key: val.cpu().numpy() for key, val in planes.items()}
    reports = None if entry == "plain" else (int(k.steps_max.item()), int(k.steps_sum.item()))
    return got, int(k.finished.item()), reports


@pytest.mark.gpu
@pytest.mark.parametrize("word", [1, 8, 0, -3, 100])
def test_the_automatic_kernel_runs_its_word(finishing, gpu, word):
    t_final, x, v = _inputs(5000, seed=23)
    mask = np.zeros(x.size, dtype=bool)
    got, counted, _ = _run_auto(finishing, gpu, t_final, x, v, mask, word)
    ox, ov, ot, om = x.copy(), v.copy(), np.zeros(x.size), mask.copy()
    want = O.osc_launch(word, DT, t_final, ox, ov, ot, om)
    assert counted == want
    for key, ref in (("x", ox), ("v", ov), ("t", ot), ("terminated", om)):
        assert got[key].tobytes() == ref.tobytes(), key


@pytest.mark.gpu
@pytest.mark.parametrize("entry,word,chunk", [("range", 7, 8), ("range", 64, 8), ("persist", 1, 8),
                                              ("persist", 7, 1), ("persist", 64, 3), ("persist", 64, 64),
                                              ("persist", 0, 8)])
def test_the_fast_entries_are_the_plain_entrys_bits(finishing, gpu, entry, word, chunk):
    """The range and persistent entries give the plain entry's bits, report
    the largest and the total trips, and count the samples finished on entry
    too (reference hawk/emit/cuda.py:373-380)."""
    n = 100_003
    t_final, x, v = _inputs(n, seed=29)
    g = rng(31)
    mask = g.uniform(size=n) < 0.1
    got, counted, (most, total) = _run_auto(finishing, gpu, t_final, x, v, mask, word, entry, chunk)
    ox, ov, ot, om = x.copy(), v.copy(), np.zeros(n), mask.copy()
    trips = np.zeros(n, dtype=np.int32)
    newly = O.osc_launch(word, DT, t_final, ox, ov, ot, om, trips=trips)
    for key, ref in (("x", ox), ("v", ov), ("t", ot), ("terminated", om)):
        assert got[key].tobytes() == ref.tobytes(), key
    assert counted == newly + int(mask.sum())
    assert (most, total) == (int(trips.max()), int(trips.sum()))


@pytest.mark.gpu
@pytest.mark.parametrize("entry", ["persist", "range"])
def test_fast_entries_twice_on_a_side_stream(finishing, gpu, entry):
    """Two runs in a row on a stream that is not torch's current one: the
    claim counter, the report cells and the finish counter are reset on that
    stream, so each run is the oracle's launch bit for bit (a reset left on
    the current stream could let the grid claim from the last run's count)."""
    import torch

    import hawk_amd as hawk
    k = hawk.load(finishing, "osc_finish_xauto")
    n = 50_021
    t_final, x, v = _inputs(n, seed=61)
    mask = rng(62).uniform(size=n) < 0.05
    planes = {"t_final": _dev(t_final, gpu), "x": _dev(x, gpu), "v": _dev(v, gpu),
              "t": _dev(np.zeros(n), gpu), "terminated": _dev(mask, gpu)}
    torch.cuda.synchronize()
    side = torch.cuda.Stream()
    ox, ov, ot, om = x.copy(), v.copy(), np.zeros(n), mask.copy()
    for word in (5, 9):
        hawk.run(k, dt=DT, steps=word, entry=entry, chunk=4, stream=side, **planes)
        side.synchronize()
        trips = np.zeros(n, dtype=np.int32)
        O.osc_launch(word, DT, t_final, ox, ov, ot, om, trips=trips)
        got = {key: val.cpu().numpy() for key, val in planes.items()}
        for key, ref in (("x", ox), ("v", ov), ("t", ot), ("terminated", om)):
            assert got[key].tobytes() == ref.tobytes(), (word, key)
        assert int(k.finished.item()) == int(om.sum())
        assert (int(k.steps_max.item()), int(k.steps_sum.item())) == (int(trips.max()), int(trips.sum()))


@pytest.mark.gpu
def test_a_prepared_persistent_launcher_counts_each_call_afresh(finishing, gpu):
    """A prepared persistent launcher on a side stream, called twice: each
    call runs the oracle's launch bit for bit; after each, ``finished`` is the
    batch's finished count (not the first call's count added again) and the
    reports are that call's trips.  A second launcher of the same kernel holds
    cells of its own."""
    import torch

    import hawk_amd as hawk
    k = hawk.load(finishing, "osc_finish_xauto")
    n = 40_009
    t_final, x, v = _inputs(n, seed=67)
    planes = {"t_final": _dev(t_final, gpu), "x": _dev(x, gpu), "v": _dev(v, gpu),
              "t": _dev(np.zeros(n), gpu), "terminated": _dev(np.zeros(n, dtype=bool), gpu)}
    torch.cuda.synchronize()
    side = torch.cuda.Stream()
    launch = k.prepare(dt=DT, steps=6, entry="persist", chunk=2, stream=side, **planes)
    other = k.prepare(dt=DT, steps=6, entry="persist", chunk=2, stream=side, **planes)
    assert launch.steps_sum.data_ptr() != other.steps_sum.data_ptr()
    ox, ov, ot, om = x.copy(), v.copy(), np.zeros(n), np.zeros(n, dtype=bool)
    for call in range(2):
        launch()
        side.synchronize()
        trips = np.zeros(n, dtype=np.int32)
        O.osc_launch(6, DT, t_final, ox, ov, ot, om, trips=trips)
        for key, ref in (("x", ox), ("v", ov), ("t", ot), ("terminated", om)):
            assert planes[key].cpu().numpy().tobytes() == ref.tobytes(), (call, key)
        assert int(launch.finished.item()) == int(om.sum()), call
        assert (int(launch.steps_max.item()), int(launch.steps_sum.item())) == (int(trips.max()), int(trips.sum()))
    assert om.sum() > 0 and not om.all()


@pytest.mark.gpu
def test_the_persistent_entry_over_two_to_the_22_samples(finishing, gpu):
    """2^22 samples of 1 to 256 steps each, run whole in one launch of the
    persistent grid: the oracle's bits, every sample finished and counted."""
    n = 1 << 22
    g = np.random.default_rng(37)
    t_final = DT * g.integers(1, 257, n).astype(float)
    x, v = g.uniform(-1.0, 1.0, n), g.uniform(-1.0, 1.0, n)
    got, counted, (most, total) = _run_auto(finishing, gpu, t_final, x, v, np.zeros(n, dtype=bool), 256,
                                            "persist", 8)
    ox, ov, ot, om = x.copy(), v.copy(), np.zeros(n), np.zeros(n, dtype=bool)
    O.osc_launch(256, DT, t_final, ox, ov, ot, om)
    assert counted == n and got["terminated"].all()
    for key, ref in (("x", ox), ("v", ov), ("t", ot)):
        assert got[key].tobytes() == ref.tobytes(), key
    steps = np.rint(t_final / DT).astype(np.int64)
    assert (most, total) == (int(steps.max()), int(steps.sum()))


@pytest.mark.gpu
@pytest.mark.parametrize("word", [None, 5])
def test_a_default_automatic_kernel_runs_one_step_unless_told(finishing, gpu, word):
    """``decay_until`` (no ``steps=``) runs one step a launch by default and
    the word's steps when given: y * rate each step, in NumPy's order."""
    import hawk_amd as hawk
    k = hawk.load(finishing, "decay_until")
    n = 3001
    y0 = rng(43).uniform(0.5, 2.0, n)
    y, mask = _dev(y0, gpu), _dev(np.zeros(n, dtype=bool), gpu)
    hawk.run(k, rate=0.75, floor=0.3, terminated=mask, y=y, **({} if word is None else {"steps": word}))
    want, done = y0.copy(), np.zeros(n, dtype=bool)
    for _ in range(1 if word is None else word):
        live = ~done
        want = np.where(live, want * 0.75, want)
        done = done | (live & (want < 0.3))
    assert y.cpu().numpy().tobytes() == want.tobytes()
    assert np.array_equal(mask.cpu().numpy(), done) and int(k.finished.item()) == int(done.sum())


@pytest.mark.gpu
@pytest.mark.parametrize("entry", ["plain", "range", "persist"])
def test_a_vector_carry_steps_to_numpy_on_every_entry(finishing, gpu, entry):
    """``spin`` carries a 2-vector and a scalar: each entry, 100 steps a
    launch, against NumPy's operation order bit for bit, with the reports."""
    import hawk_amd as hawk
    k = hawk.load(finishing, "spin")
    n = 20_011
    g = rng(47)
    p0 = g.uniform(-1.0, 1.0, (2, n))
    limit = g.integers(1, 151, n).astype(float)
    c, s = float(np.cos(0.3)), float(np.sin(0.3))
    P, N, M = _dev(p0, gpu), _dev(np.zeros(n), gpu), _dev(np.zeros(n, dtype=bool), gpu)
    hawk.run(k, c=c, s=s, limit=_dev(limit, gpu), terminated=M, p=P, n=N, steps=100, entry=entry)
    x, y, cnt, done = p0[0].copy(), p0[1].copy(), np.zeros(n), np.zeros(n, dtype=bool)
    trips = np.zeros(n, dtype=np.int64)
    for _ in range(100):
        live = ~done
        x, y = np.where(live, c * x - s * y, x), np.where(live, s * x + c * y, y)
        cnt = np.where(live, cnt + 1.0, cnt)
        trips += live
        done = done | (live & (cnt >= limit))
    got = P.cpu().numpy()
    assert got[0].tobytes() == x.tobytes() and got[1].tobytes() == y.tobytes()
    assert N.cpu().numpy().tobytes() == cnt.tobytes() and np.array_equal(M.cpu().numpy(), done)
    assert int(k.finished.item()) == int(done.sum())
    if entry != "plain":
        assert (int(k.steps_max.item()), int(k.steps_sum.item())) == (int(trips.max()), int(trips.sum()))


@pytest.mark.gpu
def test_the_runtime_refuses_steps_and_entries_it_cannot_run(finishing, gpu):
    import hawk_amd as hawk
    from hawk_amd.ir import HawkError
    n = 1000
    t_final, x, v = _inputs(n, seed=53)

    def planes():
        return {"t_final": _dev(t_final, gpu), "x": _dev(x, gpu), "v": _dev(v, gpu),
                "t": _dev(np.zeros(n), gpu), "terminated": _dev(np.zeros(n, dtype=bool), gpu)}
    single, auto = hawk.load(finishing, "osc_finish"), hawk.load(finishing, "osc_finish_xauto")
    with pytest.raises(HawkError, match="steps= sets the trip count"):
        hawk.run(single, dt=DT, steps=3, **planes())
    with pytest.raises(HawkError, match="fast entries are built for"):
        hawk.run(single, dt=DT, entry="persist", **planes())
    with pytest.raises(HawkError, match="entry= is 'plain', 'range' or 'persist'"):
        hawk.run(auto, dt=DT, entry="fast", **planes())
    with pytest.raises(HawkError, match="chunk= is an int"):
        hawk.run(auto, dt=DT, entry="persist", chunk=0, **planes())
    with pytest.raises(HawkError, match="steps= is an int"):
        hawk.run(auto, dt=DT, steps=2.5, **planes())
    with pytest.raises(HawkError, match="not planes it declares"):
        hawk.run(auto, dt=DT, fused_steps=_dev(np.ones(1, dtype=np.int32), gpu), **planes())
