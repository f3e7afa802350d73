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
from .emit_hip import fp_ops_per_sample
from .resources import kernel_resources
from .emit_hip import plan_kernel
from .ir import HawkError
from .trace import Kernel

TARGETS = ("hip",)


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


def build_bundle(kernels, directory, *, targets=("hip",), mode: str = "float64", cache_dir=None,
                 block: int = 256, per_thread: int = 1, nontemporal: bool = True) -> Bundle:
    """Build ``kernels`` (a Kernel or a list of them) into ``directory``."""
    if isinstance(kernels, Kernel):
        kernels = [kernels]
    targets = tuple(targets)
    bad = [t for t in targets if t not in TARGETS]
    if bad:
        raise HawkError(f"targets={bad}: this build's target row is 'hip' (gfx950); the reference's host "
                        "and cuda rows are not part of it")
    if block % 64 or not 64 <= block <= 1024:
        raise HawkError(f"block={block}: a multiple of 64 in [64, 1024] (wave64)")
    directory = Path(directory)
    directory.mkdir(parents=True, exist_ok=True)
    artifacts = []
    names = [k.name for k in kernels]
    if len(set(names)) != len(names):
        raise HawkError(f"two kernels share a name in {names}")
    plans = [(k, plan_kernel(k.program, k.name, mode=mode, block=block, per_thread=per_thread,
                             nontemporal=nontemporal)) for k in kernels]
    staged = [(k, p) for k, p in plans if p.stage is not None]
    compiled = dict(zip([k.name for k, _ in staged],
                        _compile.compile_units([(k.name, p.source) for k, p in staged], cache_dir=cache_dir)))
    for k, plan in plans:
        sidecar = {
            "kernel": k.name, "target": "hip", "offload_arch": "gfx950", "mode": mode,
            "scalar_type": mode, "planes": plan.planes, "team": plan.team,
            "launch": {"block": block, "per_thread": per_thread, "nontemporal": nontemporal},
            "entry": None, "arg_spec": [], "descriptor": [],
        }
        if plan.stage is not None:
            code, key, _hit = compiled[k.name]
            _write(directory / f"{k.name}.hip", plan.source.encode())
            _write(directory / f"{k.name}.hsaco", code)
            sidecar.update({
                "entry": k.name,
                "arg_spec": [list(p) for p in plan.stage.arg_spec],
                "descriptor": [plan.stage.planes[n]["kind"] for _, n in plan.stage.arg_spec],
                "source": f"{k.name}.hip", "code_object": f"{k.name}.hsaco",
                "source_sha256": hashlib.sha256(plan.source.encode()).hexdigest(),
                "code_sha256": hashlib.sha256(code).hexdigest(),
                "cache_key": key, "compile_options": list(_compile.RTC_OPTIONS),
                "toolchain": _compile.toolchain(),
                "resources": kernel_resources(code).get(k.name, {}),
                "fp_ops_per_sample": fp_ops_per_sample(plan.source),
            })
        _write(directory / f"{k.name}.json", json.dumps(sidecar, indent=1, sort_keys=True).encode())
        artifacts.append(Artifact(k.name, sidecar))
    digest = hashlib.sha256(json.dumps([a.sidecar for a in artifacts], sort_keys=True).encode()).hexdigest()
    manifest = {"target": "hip", "offload_arch": "gfx950", "mode": mode, "digest": digest,
                "kernels": [a.name for a in artifacts]}
    _write(directory / "manifest.json", json.dumps(manifest, indent=1, sort_keys=True).encode())
    return Bundle(directory, artifacts, digest)
