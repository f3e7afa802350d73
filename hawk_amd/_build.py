"""Build step of hawk's gfx950 target: compile ``libhawk_core.so`` in-tree.

The library is the C-ABI launcher (``csrc/hawk_core.cpp``) plus the
hand-written team-stage kernels (``csrc/hawk_team.hip``, ``csrc/hawk_linalg.hip``), built by ``hipcc``
for gfx950 only.  Its build digest is the sha256 of its own sources (each
file's name and sha256, in sorted order), stamped into the library and
recomputed by :mod:`hawk_amd._core` at load, the same self-check the
reference runs at import (reference ``hawk/__init__.py:146-212``).
"""

from __future__ import annotations

import hashlib
import os
import subprocess
import sys
from pathlib import Path

PACKAGE = Path(__file__).resolve().parent
ROOT = PACKAGE.parent
CSRC = PACKAGE / "csrc"
INCLUDE = ROOT / "include"
LIBRARY = PACKAGE / "libhawk_core.so"
HIPCC = os.environ.get("HAWK_HIPCC", "/opt/rocm/bin/hipcc")

#: Flags every HIP translation unit of this target is built with: gfx950
#: only, no floating-point contraction (the host oracle's ``native`` profile
#: is built with -ffp-contract=off, reference hawk/compile/toolchain.py:956-987),
#: and packed-FP32 instruction selection switched off.
HIP_FLAGS = ("--offload-arch=gfx950", "-O3", "-ffp-contract=off",
             "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops")


def digest_sources() -> list:
    """The files the build digest covers, relative to the repository root."""
    files = sorted(p for p in CSRC.iterdir() if p.is_file() and p.suffix in (".cpp", ".hip", ".h"))
    return files + [INCLUDE / "hawk_core.h"]


def source_digest() -> str:
    """sha256 over ``name\\nsha256(file)\\n`` of every covered file, sorted by name."""
    stream = []
    for path in sorted(digest_sources(), key=lambda p: p.relative_to(ROOT).as_posix()):
        stream.append(f"{path.relative_to(ROOT).as_posix()}\n{hashlib.sha256(path.read_bytes()).hexdigest()}\n")
    return hashlib.sha256("".join(stream).encode()).hexdigest()


def build_library(verbose: bool = False) -> Path:
    """Compile ``libhawk_core.so`` next to this file; returns its path."""
    digest = source_digest()
    info = "compiler=" + HIPCC + "\\nflags=" + " ".join(HIP_FLAGS) + "\\noffload_arch=gfx950"
    tmp = LIBRARY.with_suffix(".so.tmp")
    cmd = [HIPCC, *HIP_FLAGS, "-fPIC", "-shared", "-std=c++17",
           f"-I{INCLUDE}", f"-I{CSRC}",
           f'-DHAWK_BUILD_DIGEST="{digest}"', f'-DHAWK_BUILD_INFO="{info}"',
           str(CSRC / "hawk_core.cpp"), str(CSRC / "hawk_team.hip"), str(CSRC / "hawk_linalg.hip"),
           "-o", str(tmp), "-lhiprtc", "-lamdhip64"]
    if verbose:
        print(" ".join(cmd), flush=True)
    proc = subprocess.run(cmd, capture_output=True, text=True)
    if proc.returncode != 0:
        raise RuntimeError(f"hipcc failed building {LIBRARY.name}:\n{proc.stdout}\n{proc.stderr}")
    os.replace(tmp, LIBRARY)
    return LIBRARY


if __name__ == "__main__":
    print(build_library(verbose="-v" in sys.argv))
