"""The hipRTC build-and-cache path of the gfx950 target.

``compile_source`` compiles one HIP translation unit with hipRTC for
``--offload-arch=gfx950`` (through ``hk_rtc_compile`` of the C-ABI) and keeps
the code object in a content-addressed cache, the shape of reference
``hawk/compile/cache.py:347-459``: the key is the sha256 of the source, the
options, the hipRTC version and the target, so a changed compiler or flag is a
miss and an unchanged kernel is one file read.  Entries are published
atomically (write to a temporary name, then rename).
"""

from __future__ import annotations

import hashlib
import json
import os
import threading
from pathlib import Path

from . import _core

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


def cache_key(source: str, options) -> str:
    blob = json.dumps({"source": source, "options": list(options), "target": "gfx950",
                       "hiprtc": _core.rtc_version()}, sort_keys=True)
    return hashlib.sha256(blob.encode()).hexdigest()


def cache_stats() -> dict:
    with _stats_lock:
        return dict(_stats)


def compile_source(source: str, name: str, options=RTC_OPTIONS, cache_dir=None) -> tuple:
    """``(code object bytes, cache key, hit)`` for ``source``."""
    cache = Path(cache_dir) if cache_dir is not None else default_cache_dir()
    key = cache_key(source, options)
    path = cache / f"{key}.hsaco"
    if path.exists():
        with _stats_lock:
            _stats["hits"] += 1
        return path.read_bytes(), key, True
    code, _log = _core.rtc_compile(source, f"{name}.hip", list(options))
    cache.mkdir(parents=True, exist_ok=True)
    tmp = path.with_suffix(f".tmp{os.getpid()}_{threading.get_ident()}")
    tmp.write_bytes(code)
    os.replace(tmp, path)
    with _stats_lock:
        _stats["misses"] += 1
    return code, key, False
