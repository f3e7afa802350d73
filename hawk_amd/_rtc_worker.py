"""hipRTC compile worker: ``python -m hawk_amd._rtc_worker`` reads a JSON job
on stdin and writes the code objects on stdout.

PyTorch-ROCm ships its own HIP runtime and comgr (the compiler hipRTC drives),
and once torch is imported in a process every hipRTC call there uses torch's
copy.  The gfx950 target compiles its kernels with the ROCm toolchain of the
system instead — the one ``libhawk_core.so`` itself is built with — so the
compile runs here, in a process that never imports torch.

Job: ``{"options": [...], "units": [[name, source], ...]}``.  Reply:
``{"ok": true, "toolchain": "...", "units": [[name, base64 code, log], ...]}``
or ``{"ok": false, "error": "..."}``.
"""

from __future__ import annotations

import base64
import json
import os
import sys


def toolchain_identity(lib) -> str:
    """The hipRTC API version and the comgr library this process compiles with."""
    version = lib.hk_rtc_version()
    from hawk_amd import _core
    _core.rtc_compile('extern "C" __global__ void hawk_probe() {}', "hawk_probe.hip", [])   # loads comgr
    comgr = "?"
    try:
        for line in open(f"/proc/{os.getpid()}/maps"):
            if "libamd_comgr" in line:
                path = line.split()[-1]
                st = os.stat(path)
                comgr = f"{os.path.realpath(path)}:{st.st_size}"
                break
    except OSError:
        pass
    return f"hiprtc-{version};comgr={comgr}"


def main() -> int:
    os.environ["HAWK_NO_TORCH_PRELOAD"] = "1"
    job = json.loads(sys.stdin.read())
    from hawk_amd import _core
    try:
        lib = _core.lib()
        units = []
        for name, source in job["units"]:
            code, log = _core.rtc_compile(source, name, job["options"])
            units.append([name, base64.b64encode(code).decode(), log])
        reply = {"ok": True, "toolchain": toolchain_identity(lib), "units": units}
    except Exception as exc:  # the parent re-raises the text as HawkError
        reply = {"ok": False, "error": str(exc)}
    sys.stdout.write(json.dumps(reply))
    return 0


if __name__ == "__main__":
    raise SystemExit(main())
