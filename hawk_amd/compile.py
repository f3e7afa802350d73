"""The hipRTC build-and-cache path of the gfx950 target.

``compile_units`` compiles HIP translation units with hipRTC for
``--offload-arch=gfx950`` (through ``hk_rtc_compile`` of the C-ABI) and keeps
the code objects in a content-addressed cache, the shape of reference
``hawk/compile/cache.py:347-459``: the key is the sha256 of the source, the
options, the compiler's identity and the target, so a changed compiler or
flag is a miss and an unchanged kernel is one file read.  Entries are
published atomically (write to a temporary name, then rename).

The compile itself runs in a worker process that never imports torch
(:mod:`hawk_amd._rtc_worker`), so it uses the system ROCm toolchain rather
than the copy PyTorch-ROCm bundles; ``HAWK_RTC_IN_PROCESS=1`` compiles in this
process with whichever hipRTC is loaded here.
"""

from __future__ import annotations

import base64
import hashlib
import json
import os
import subprocess
import sys
import threading
from pathlib import Path

from . import _core
from .ir import HawkError

#: Options every device unit is compiled with: no floating-point contraction
#: (the device computes the host oracle's ``native``-profile operations),
#: packed-FP32 instruction selection off, C++17.
RTC_OPTIONS = ("-O3", "-std=c++17", "-ffp-contract=off",
               "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops")

_stats = {"hits": 0, "misses": 0}
_stats_lock = threading.Lock()


def default_cache_dir() -> Path:
    env = os.environ.get("HAWK_CACHE_DIR")
    return Path(env) if env else Path(__file__).resolve().parent / "_cache"


_toolchain_lock = threading.Lock()
_toolchain: dict = {}


def _in_process() -> bool:
    return os.environ.get("HAWK_RTC_IN_PROCESS") == "1"


def _run_worker(units: list, options) -> dict:
    job = json.dumps({"options": list(options), "units": [list(u) for u in units]})
    env = dict(os.environ, HAWK_NO_TORCH_PRELOAD="1")
    root = str(Path(__file__).resolve().parent.parent)
    env["PYTHONPATH"] = root + (os.pathsep + env["PYTHONPATH"] if env.get("PYTHONPATH") else "")
    proc = subprocess.run([sys.executable, "-m", "hawk_amd._rtc_worker"], input=job, capture_output=True,
                          text=True, env=env)
    if proc.returncode != 0:
        raise HawkError(f"the hipRTC worker failed (exit {proc.returncode}): {proc.stderr[-2000:]}")
    reply = json.loads(proc.stdout)
    if not reply.get("ok"):
        raise HawkError(reply.get("error", "the hipRTC worker failed"))
    return reply


def toolchain() -> str:
    """The identity of the compiler the build uses (part of every cache key)."""
    key = "in-process" if _in_process() else "worker"
    with _toolchain_lock:
        if key not in _toolchain:
            if _in_process():
                from ._rtc_worker import toolchain_identity
                _toolchain[key] = toolchain_identity(_core.lib())
            else:
                _toolchain[key] = _run_worker([], RTC_OPTIONS)["toolchain"]
        return _toolchain[key]


def cache_key(source: str, options) -> str:
    blob = json.dumps({"source": source, "options": list(options), "target": "gfx950",
                       "toolchain": toolchain()}, sort_keys=True)
    return hashlib.sha256(blob.encode()).hexdigest()


def cache_stats() -> dict:
    with _stats_lock:
        return dict(_stats)


def _publish(path: Path, data: bytes) -> None:
    """Write ``data`` to ``path`` atomically: a reader sees the old file, or
    the whole new one."""
    tmp = path.with_suffix(path.suffix + f".tmp{os.getpid()}_{threading.get_ident()}")
    tmp.write_bytes(data)
    os.replace(tmp, path)


def _cached(cache: Path, key: str):
    """The code object stored under ``key``, or ``None`` when the entry is
    absent or not whole.  An entry is the code object ``<key>.hsaco`` and its
    validity record ``<key>.json`` (its size and sha256), published after
    the object: a missing record, or an object that does not match it (a
    truncated or damaged file), is a miss and gets rebuilt (reference
    ``hawk/compile/cache.py:385-444``: a record beside the artifact, a miss
    the safe default)."""
    try:
        record = json.loads((cache / f"{key}.json").read_text())
        code = (cache / f"{key}.hsaco").read_bytes()
    except (OSError, ValueError):
        return None
    if record.get("size") != len(code) or record.get("sha256") != hashlib.sha256(code).hexdigest():
        return None
    return code


def compile_units(units: list, options=RTC_OPTIONS, cache_dir=None) -> list:
    """``[(code object bytes, cache key, hit)]`` for ``units`` = ``[(name, source)]``,
    compiling every miss in one hipRTC worker call."""
    cache = Path(cache_dir) if cache_dir is not None else default_cache_dir()
    keys = [cache_key(src, options) for _, src in units]
    out: list = [None] * len(units)
    misses = []
    for i, key in enumerate(keys):
        code = _cached(cache, key)
        if code is not None:
            out[i] = (code, key, True)
        else:
            misses.append(i)
    if misses:
        todo = [(f"{units[i][0]}.hip", units[i][1]) for i in misses]
        if _in_process():
            codes = [_core.rtc_compile(src, name, list(options))[0] for name, src in todo]
        else:
            codes = [base64.b64decode(c) for _n, c, _log in _run_worker(todo, options)["units"]]
        cache.mkdir(parents=True, exist_ok=True)
        for i, code in zip(misses, codes):
            _publish(cache / f"{keys[i]}.hsaco", code)
            record = {"size": len(code), "sha256": hashlib.sha256(code).hexdigest(), "unit": units[i][0],
                      "options": list(options), "toolchain": toolchain()}
            _publish(cache / f"{keys[i]}.json", json.dumps(record, sort_keys=True).encode())
            out[i] = (code, keys[i], False)
    with _stats_lock:
        _stats["hits"] += len(units) - len(misses)
        _stats["misses"] += len(misses)
    return out


def compile_source(source: str, name: str, options=RTC_OPTIONS, cache_dir=None) -> tuple:
    """``(code object bytes, cache key, hit)`` for one unit."""
    return compile_units([(name, source)], options, cache_dir)[0]
