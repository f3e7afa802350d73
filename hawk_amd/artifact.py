"""``hawk.build``: kernels -> a deployment unit on disk for the hip target.

For each kernel: its per-sample stage as HIP source (``<name>.hip``) and the
gfx950 code object hipRTC made of it (``<name>.hsaco``), and a sidecar
``<name>.json`` the runtime reads (arg_spec, slot kinds, planes, the team
stages after the per-sample stage, the launch shape).  A ``manifest.json``
lists the unit.  The layout follows reference ``hawk/artifact/bundle.py:1349-1575``
and ``hawk/artifact/sidecar.py:412-476`` with the ``hip`` row in place of the
host and cuda rows.
"""

from __future__ import annotations

import hashlib
import json
import os
from dataclasses import dataclass
from pathlib import Path

from . import compile as _compile
from . import policy as _policy
from .emit_hip import fp_ops_per_sample
from .resources import kernel_resources
from .emit_hip import plan_kernel
from .ir import AUTO_K_MAX, FINISHED_PLANE, Finish, HawkError
from .targets import TARGETS, row
from .trace import Kernel


@dataclass
class Artifact:
    name: str
    sidecar: dict


@dataclass
class Bundle:
    directory: Path
    artifacts: list
    digest: str

    def sidecar(self, name: str) -> dict:
        for a in self.artifacts:
            if a.name == name:
                return a.sidecar
        raise HawkError(f"the unit holds no kernel {name!r}")


def _write(path: Path, data: bytes) -> None:
    tmp = path.with_suffix(path.suffix + f".tmp{os.getpid()}")
    tmp.write_bytes(data)
    os.replace(tmp, path)


#: Per-sample plane bytes and operations at or below which a stage is a pure
#: stream: four samples a thread keep more loads in flight (measured on
#: MI355X: a*x+b 5.7 -> 6.4 TB/s).  Other stages run one sample a thread:
#: in workgroups of 128 up to 32 bytes a sample (energy 6.5 -> 6.8 TB/s) and
#: beyond 64 (the 6x6 SPD solve 5.1 -> 5.5), of 256 in between (the energy
#: VJP and JVP, 56 bytes: 6.2 -> 6.45).
STREAM_BYTES, STREAM_OPS = 16, 4


def _stage_bytes(plan, mode: str) -> int:
    size = 4 if mode == "float32" else 8
    total = 0
    for info in plan.stage.planes.values():
        if info["role"] in ("uniform", "rows_out", "nsamples", "lookup", "key_out", "fold_scratch",
                            "accum_out"):                  # per cell / per key
            continue
        count = 1
        for e in info["shape"]:
            count *= e
        total += count * {"i32": 4, "u32": 4, "bool": 1}.get(info["dtype"], size)
    return total


#: The launch shape of a plain stage that gathers from a table: each sample's
#: table read waits on its key, and 1024 threads of two samples each
#: measured fastest for such a stage (config 5t's lookup: 0.42 ms at 128 x 1,
#: 0.36 at 512 x 2, 0.28 at 1024 x 2, 0.41 at 1024 x 4).
GATHER_SHAPE = (1024, 2)

#: The launch shape of a light stream whose planes are all scalar float64
#: planes: 64 threads of one pair of adjacent samples, read and written 16
#: bytes a lane (``emit_hip._pair_lines``).  A copy of ``scale``'s pattern
#: measured 0.1634 ms at 64 threads x 16 B, 0.1655-0.1666 at 128-512 x 16 B,
#: and 0.1683-0.1703 for 8 B a lane at 256 x 4, 512 x 2 and 128 x 4 (2^26
#: samples, one box).
PAIR_SHAPE = (64, 2)
STREAM_SHAPE = (256, 4)


def launch_shape(plan, mode: str) -> tuple:
    """``(block, per_thread)`` a stage runs with when the build does not fix them."""
    from .emit_hip import fp_ops_per_sample, pair_candidate
    stage = plan.stage
    if (any(info["role"] == "lookup" for info in stage.planes.values()) and not stage.row_sums
            and not stage.fused_folds and not stage.key_writes and stage.guard is None and stage.finish is None):
        return GATHER_SHAPE
    nbytes = _stage_bytes(plan, mode)
    if nbytes <= STREAM_BYTES and fp_ops_per_sample(plan.source) <= STREAM_OPS:
        return PAIR_SHAPE if pair_candidate(stage, mode) else STREAM_SHAPE
    shape = (256, 1) if 32 < nbytes <= 64 else (128, 1)
    if stage.row_sums and not stage.fused_folds:
        # row reductions take two samples a lane (the paired layout)
        shape = (shape[0], 2)
    return shape


def _chain_record(k, sidecar: dict, mode: str) -> None:
    """A chain's members, outputs, register estimate and fence in its sidecar
    (reference ``hawk/ir/fusion.py``); one past its fence is reported."""
    import warnings

    from .chaining import estimate, fence
    est = estimate(k.program, mode)
    res = sidecar.get("resources") or {}
    vgprs, scratch = res.get("vgpr_count"), res.get("private_segment_fixed_size") or 0
    inside = None if vgprs is None else fence(vgprs, scratch, est)
    sidecar["chain"] = {"members": [m.name for m in k.members], "outputs": list(k.outputs),
                        "estimate_vgprs": est, "within_fence": inside}
    if inside is False:
        warnings.warn(f"chain {k.name!r} compiled to {vgprs} VGPRs and {scratch} B of scratch a lane, past "
                      f"its fence (1.6 x the estimate {est} + 16): split it into shorter chains", stacklevel=3)


def _cut_chains(kernels, mode: str, register_line: int | None, target) -> tuple:
    """``(kernels, chains)``: each chain the cut rule cuts replaced by its
    segments (``<name>__s<i>``), and ``{chain name: its sidecar}``."""
    from .chaining import REGISTER_LINE, cuts, segments
    from .trace import Kernel as _Kernel
    out, chains = [], {}
    for k in kernels:
        members = getattr(k, "members", None)
        at = cuts(members, mode, register_line or REGISTER_LINE) if members else []
        if not at:
            out.append(k)
            continue
        names, crossing, planes = [], {}, {}
        for i, (program, writes, _reads) in enumerate(segments(members, at)):
            seg = _Kernel(f"{k.name}__s{i}", program)
            out.append(seg)
            names.append(seg.name)
            for w in writes:
                d = program.decls[w]
                crossing[w] = {"shape": list(d.ttype.shape), "dtype": d.ttype.dtype}
        chains[k.name] = {"kernel": k.name, "target": target.id, "offload_arch": target.offload_arch, "mode": mode,
                          "segments": names, "crossing": crossing, "cuts": at,
                          "chain": {"members": [m.name for m in members], "outputs": list(k.outputs)},
                          "planes": planes, "entry": None, "team": []}
    return out, chains


#: The reference's build options and the values it accepts
#: (reference hawk/emit/policy.py FORMS / LINALG_FORMS / WIDE_FORMS,
#: hawk/compile/toolchain.py:625 and :928).
EMIT_FORMS = _policy.FORMS
LINALG_FORMS = _policy.LINALG_FORMS
WIDE_FORMS = _policy.WIDE_FORMS
HOST_PROFILES = ("native", "portable", "native-vector-math", "native-vector-math-nofma")
OPT_LEVELS = ("O0", "O1", "O2", "O3")


def _reference_options(kind, layout_sizes_override, defines, device_arch, host_profile, opt_level,
                       literal_table, embedded_profile, emit_form, linalg_form, wide_form,
                       launch_bounds) -> tuple:
    """Check the reference's build options (reference
    hawk/artifact/bundle.py:1349-1420) and return ``(compile options, block
    fixed by launch_bounds or None, what the sidecar records, launch_bounds'
    blocks or 1)``.  The forms
    choose how the reference spells a site; this target's stages add in the
    order they are written whatever the spelling, so they are checked and
    recorded.  ``opt_level`` and ``defines`` reach hipRTC; ``launch_bounds``
    fixes the block as the reference's ``launch.block = threads`` does, and
    its ``blocks`` becomes each entry's waves-per-EU floor
    (:func:`waves_per_eu`)."""
    if kind is not None:
        raise HawkError("kind=: an execution kind (hawk.ext lanes or an active-set guard) has no hip form in this "
                        "build")
    if layout_sizes_override is not None:
        raise HawkError("layout_sizes_override= is the reference host build's test-only door; the hip target's "
                        "mirror sizes are the library's (hk_layout_sizes)")
    if embedded_profile is not None:
        raise HawkError("embedded_profile= belongs to the reference's MISRA C target, which this build does not have")
    if device_arch not in ("", "gfx950"):
        raise HawkError(f"device_arch={device_arch!r}: the hip target builds gfx950")
    for what, value, allowed in (("emit_form", emit_form, EMIT_FORMS), ("linalg_form", linalg_form, LINALG_FORMS),
                                 ("wide_form", wide_form, WIDE_FORMS)):
        if value is not None and value not in allowed:
            raise HawkError(f"{what} must be one of {allowed}, got {value!r}")
    if host_profile and host_profile not in HOST_PROFILES:
        raise HawkError(f"host_profile must be one of {HOST_PROFILES}, got {host_profile!r}")
    if opt_level and opt_level not in OPT_LEVELS:
        raise HawkError(f"opt_level must be one of {OPT_LEVELS}, got {opt_level!r}")
    block = None
    blocks = 1
    launch_bounds = _policy.check_launch_bounds(launch_bounds)
    if launch_bounds is not None:
        threads, blocks = launch_bounds
        if threads % 64 or threads > 1024:
            raise HawkError(f"launch_bounds={launch_bounds!r}: gfx950 runs wave64 workgroups of at most 1024 "
                            "threads, so threads must be a multiple of 64 up to 1024")
        block = int(threads)
    options = list(_compile.RTC_OPTIONS)
    if opt_level:
        options = [f"-{opt_level}" if o.startswith("-O") else o for o in options]
    for d in defines or ():
        d = str(d)
        if not d or d.startswith("-") or any(c.isspace() for c in d):
            raise HawkError(f"defines: {d!r} is not NAME or NAME=VALUE")
        options.append(f"-D{d}")
    contraction = _policy.contraction()
    record = {k: v for k, v in (("emit_form", emit_form), ("linalg_form", linalg_form), ("wide_form", wide_form),
                                ("contraction", contraction if contraction != "direct" else None),
                                ("launch_bounds", list(launch_bounds) if launch_bounds else None),
                                ("host_profile", host_profile or None), ("opt_level", opt_level or None),
                                ("literal_table", bool(literal_table) or None),
                                ("defines", [str(d) for d in defines] if defines else None)) if v is not None}
    return tuple(options), block, record, int(blocks)


def waves_per_eu(block: int, blocks: int) -> int:
    """The occupancy floor that ``launch_bounds=(threads, blocks)`` asks of a
    stage launched with ``block`` threads: ``blocks`` workgroups resident on
    one CU are ``blocks * block / 64`` waves over its four SIMDs, so each
    SIMD (execution unit) must hold that many / 4, at most 8 on gfx950.  The
    compiler then caps the stage's registers to fit (the CUDA minimum
    blocks per multiprocessor, spelled as amdgpu waves per EU)."""
    return max(1, min(8, -(-blocks * block // 256)))


def _with_waves(source: str, block: int, waves: int) -> str:
    """Every entry's ``__launch_bounds__(block)`` given the occupancy floor."""
    if waves <= 1:
        return source
    return source.replace(f"__launch_bounds__({block})", f"__launch_bounds__({block}, {waves})")


def build_bundle(kernels, directory, *, targets=("hip",), mode: str = "float64", cache_dir=None,
                 block: int | None = None, per_thread: int | None = None, nontemporal: bool = True,
                 fuse_folds: bool = True, register_line: int | None = None, kind=None,
                 layout_sizes_override=None, defines=(), device_arch: str = "", name: str | None = None,
                 derivative=None, host_profile: str = "", opt_level: str = "", literal_table: bool = False,
                 embedded_profile=None, emit_form: str | None = None, linalg_form: str | None = None,
                 wide_form: str | None = None, launch_bounds=None) -> Bundle:
    """Build ``kernels`` (a Kernel or a list of them) into ``directory``.
    ``block`` / ``per_thread`` fix every stage's launch shape; left ``None``
    each stage gets :func:`launch_shape`'s.  A stage that folds an ordered
    gradient in LDS keeps the block its keys need, one sample a thread
    (``fuse_folds=False`` logs and folds in a team stage instead).  A
    ``hawk.chain`` is cut where its fused estimate passes ``register_line``
    VGPRs (default: the spill line, 512): its segments build as kernels of
    their own and its sidecar lists them in order.  The reference's own
    options (``emit_form`` ... ``launch_bounds``, ``name``, ``derivative``)
    are taken as :func:`_reference_options` describes."""
    if isinstance(kernels, Kernel):
        kernels = [kernels]
    # an option left unset is the ambient hawk_amd.policy.using value (reference
    # hawk/artifact/bundle.py:1359-1360: an explicit argument wins)
    ambient = _policy.form(), _policy.linalg_form(), _policy.wide_form(), _policy.launch_bounds()
    emit_form = emit_form if emit_form is not None else (ambient[0] if ambient[0] != "auto" else None)
    linalg_form = linalg_form if linalg_form is not None else (ambient[1] if ambient[1] != "auto" else None)
    wide_form = wide_form if wide_form is not None else (ambient[2] if ambient[2] != "auto" else None)
    launch_bounds = launch_bounds if launch_bounds is not None else ambient[3]
    options, bounds_block, recorded, min_blocks = _reference_options(
        kind, layout_sizes_override, defines, device_arch, host_profile, opt_level, literal_table,
        embedded_profile, emit_form, linalg_form, wide_form, launch_bounds)
    if block is None and bounds_block is not None:
        block = bounds_block
    if derivative is not None and not isinstance(derivative, dict):
        raise HawkError("derivative= maps kernel names to their primal's name (or (name, unit digest))")
    targets = tuple(targets)
    bad = [t for t in targets if t not in TARGETS]
    if bad:
        raise HawkError(f"targets={bad}: this build's target row is 'hip' (gfx950); the reference's host "
                        "and cuda rows are not part of it")
    (target,) = [row(t) for t in dict.fromkeys(targets)] or [row("hip")]
    kernels, chains = _cut_chains(list(kernels), mode, register_line, target)
    if block is not None and (block % 64 or not 64 <= block <= 1024):
        raise HawkError(f"block={block}: a multiple of 64 in [64, 1024] (wave64)")
    if per_thread is not None and not 1 <= per_thread <= 64:
        raise HawkError(f"per_thread={per_thread}: 1 .. 64 samples a thread")
    directory = Path(directory)
    directory.mkdir(parents=True, exist_ok=True)
    artifacts = []
    names = [k.name for k in kernels]
    if len(set(names)) != len(names):
        raise HawkError(f"two kernels share a name in {names}")
    plans = []
    for k in kernels:
        plan = plan_kernel(k.program, k.name, mode=mode, block=block or 256, per_thread=per_thread or 1,
                           nontemporal=nontemporal, fuse_folds=fuse_folds, target=target)
        shape = (block or 256, per_thread or 1)
        if plan.block is not None:
            shape = (plan.block, 1)
        elif plan.stage is not None and (block is None or per_thread is None):
            auto = launch_shape(plan, mode)
            shape = (block or auto[0], per_thread or auto[1])
            if shape != (256, 1):
                plan = plan_kernel(k.program, k.name, mode=mode, block=shape[0], per_thread=shape[1],
                                   nontemporal=nontemporal, fuse_folds=fuse_folds, target=target)
            if auto == PAIR_SHAPE and "hk_pair_" not in plan.source:
                # the body reads a plane other than at its own sample: the
                # one-sample stream shape (for what the build left open)
                shape = (block or STREAM_SHAPE[0], per_thread or STREAM_SHAPE[1])
                plan = plan_kernel(k.program, k.name, mode=mode, block=shape[0], per_thread=shape[1],
                                   nontemporal=nontemporal, fuse_folds=fuse_folds, target=target)
        if plan.stage is not None and min_blocks > 1:
            plan.source = _with_waves(plan.source, shape[0], waves_per_eu(shape[0], min_blocks))
        plans.append((k, plan, shape))
    staged = [(k, p) for k, p, _ in plans if p.stage is not None]
    compiled = dict(zip([k.name for k, _ in staged],
                        _compile.compile_units([(k.name, p.source) for k, p in staged], options=options,
                                               cache_dir=cache_dir)))
    for k, plan, shape in plans:
        sidecar = {
            "kernel": k.name, "target": target.id, "offload_arch": target.offload_arch, "mode": mode,
            "scalar_type": mode, "planes": plan.planes, "team": plan.team,
            "launch": {"block": shape[0], "per_thread": shape[1], "nontemporal": nontemporal,
                       **({"waves_per_eu": waves_per_eu(shape[0], min_blocks)}
                          if waves_per_eu(shape[0], min_blocks) > 1 else {})},
            "grid": [list(a) for a in k.program.grid.axes] if k.program.grid is not None else None,
            "tables": {t: [list(a) for a in axes] for t, axes in k.program.tables.items()},
            "entry": None, "arg_spec": [], "descriptor": [],
        }
        if plan.stage is not None:
            code, key, _hit = compiled[k.name]
            _write(directory / f"{k.name}{target.source}", plan.source.encode())
            _write(directory / f"{k.name}{target.artifact}", code)
            sidecar.update({
                "entry": k.name,
                "arg_spec": [list(p) for p in plan.stage.arg_spec],
                "descriptor": [plan.stage.planes[n]["kind"] for _, n in plan.stage.arg_spec],
                "source": f"{k.name}{target.source}", "code_object": f"{k.name}{target.artifact}",
                "format": target.format, "entry_kind": target.entry,
                "source_sha256": hashlib.sha256(plan.source.encode()).hexdigest(),
                "code_sha256": hashlib.sha256(code).hexdigest(),
                "cache_key": key, "compile_options": list(options),
                "toolchain": _compile.toolchain(),
                "resources": kernel_resources(code).get(k.name, {}),
                # the program's ops as traced (the algorithmic count), and what
                # the emitted stage executes after carried reuse
                "fp_ops_per_sample": plan.algorithmic_ops,
                "fp_ops_emitted": fp_ops_per_sample(plan.source),
            })
        finish = next((s for s in k.program.sinks if isinstance(s, Finish)), None)
        if plan.stage is not None and plan.stage.guard is not None:
            # reference tests/test_finish_own_sample.py:98-106
            sidecar["terminated_readonly"] = finish is None
            if finish is not None:
                sidecar["finish"] = {"mask": finish.name, "counter": FINISHED_PLANE, "steps": finish.steps}
            if finish is not None and finish.steps == "auto":
                # reference hawk/trace/steps.py:31-37 and hawk/emit/cuda.py:465-784
                sidecar["finish"]["steps_max"] = AUTO_K_MAX
                sidecar["fast_entries"] = {"range": f"{k.name}_range", "persist": f"{k.name}_persist"}
        if getattr(k, "members", None) is not None:
            _chain_record(k, sidecar, mode)
        if recorded:
            sidecar["build_options"] = recorded
        if derivative and k.name in derivative:
            sidecar["primal"] = derivative[k.name] if isinstance(derivative[k.name], str) else list(derivative[k.name])
        _write(directory / f"{k.name}.json", json.dumps(sidecar, indent=1, sort_keys=True).encode())
        artifacts.append(Artifact(k.name, sidecar))
    for name, sidecar in chains.items():
        by_name = {a.name: a.sidecar for a in artifacts}
        for seg in sidecar["segments"]:
            for pname, info in by_name[seg]["planes"].items():
                if not info.get("scratch") and pname not in sidecar["crossing"]:
                    sidecar["planes"].setdefault(pname, info)
        _write(directory / f"{name}.json", json.dumps(sidecar, indent=1, sort_keys=True).encode())
        artifacts.append(Artifact(name, sidecar))
    digest = hashlib.sha256(json.dumps([a.sidecar for a in artifacts], sort_keys=True).encode()).hexdigest()
    manifest = {"target": target.id, "offload_arch": target.offload_arch, "mode": mode, "digest": digest,
                "kernels": [a.name for a in artifacts]}
    if name is not None:
        manifest["name"] = str(name)
    _write(directory / "manifest.json", json.dumps(manifest, indent=1, sort_keys=True).encode())
    return Bundle(directory, artifacts, digest)
