"""Resource usage of a gfx950 code object, read from its own metadata.

Every AMDGPU code object carries an ``NT_AMDGPU_METADATA`` note (msgpack)
listing each kernel's VGPR/AGPR/SGPR counts, spills, private (scratch) and
group (LDS) segment sizes.  The build records them in the sidecar — the role
the reference gives its ptxas ``-v`` figures (reference
``hawk/compile/drivers.py:279-300``, ``hawk/artifact/bundle.py:533-571``) — and
derives the waves a SIMD can hold at that register count.
"""

from __future__ import annotations

import struct

_NT_AMDGPU_METADATA = 32
#: gfx950: 512 VGPRs per SIMD lane (the unified VGPR+AGPR file), allocated in
#: granules of 8, at most 8 waves per SIMD.
_VGPR_FILE = 512
_VGPR_GRANULE = 8
_MAX_WAVES = 8

_FIELDS = (".vgpr_count", ".agpr_count", ".sgpr_count", ".vgpr_spill_count", ".sgpr_spill_count",
           ".private_segment_fixed_size", ".group_segment_fixed_size", ".wavefront_size",
           ".max_flat_workgroup_size")


def _notes(blob: bytes):
    if blob[:4] != b"\x7fELF" or blob[4] != 2:
        return
    shoff = struct.unpack_from("<Q", blob, 0x28)[0]
    shentsize, shnum = struct.unpack_from("<HH", blob, 0x3A)
    for i in range(shnum):
        base = shoff + i * shentsize
        sh_type = struct.unpack_from("<I", blob, base + 4)[0]
        if sh_type != 7:                     # SHT_NOTE
            continue
        off, size = struct.unpack_from("<QQ", blob, base + 0x18)
        pos, end = off, off + size
        while pos + 12 <= end:
            namesz, descsz, ntype = struct.unpack_from("<III", blob, pos)
            pos += 12
            name = blob[pos:pos + namesz]
            pos += (namesz + 3) & ~3
            desc = blob[pos:pos + descsz]
            pos += (descsz + 3) & ~3
            yield name, ntype, desc


def kernel_resources(code: bytes) -> dict:
    """``{kernel symbol: {field: value, ..., "waves_per_simd": w}}``; empty when
    the object carries no readable metadata."""
    try:
        import msgpack
    except ImportError:          # the figures are diagnostics; a missing decoder only drops them
        return {}
    out = {}
    for name, ntype, desc in _notes(code):
        if ntype != _NT_AMDGPU_METADATA or not name.startswith(b"AMDGPU"):
            continue
        meta = msgpack.unpackb(desc, raw=False, strict_map_key=False)
        for k in meta.get("amdhsa.kernels", []):
            row = {f.lstrip("."): k.get(f) for f in _FIELDS if f in k}
            regs = row.get("vgpr_count") or 0         # the unified count: AGPRs included
            granted = max(_VGPR_GRANULE, -(-regs // _VGPR_GRANULE) * _VGPR_GRANULE)
            row["waves_per_simd"] = min(_MAX_WAVES, _VGPR_FILE // granted)
            out[k.get(".name", "?")] = row
    return out
