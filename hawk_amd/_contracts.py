"""The ABI contract's constants, stated once on the Python side.

The layout table every gfx950 artifact exports as ``eagle_layout_sizes`` and
``libhawk_core.so`` marshals (reference ``hawk/_contracts.py:40-92``): the
40-byte ``GRefMirror``, the 32-byte ``ScalarHandle`` / ``IntHandle``, the
8-byte index of the ``nsamples`` role and the 24-byte partition triple.
"""

ABI_TAG = "aether-abi/2"

LAYOUT = (
    ("GRefMirror", 40),
    ("ScalarHandle", 32),
    ("IntHandle", 32),
    ("index_t", 8),
    ("PartitionTriple", 24),
)

GREF_MIRROR_SIZE = 40
SCALAR_HANDLE_SIZE = 32
INT_HANDLE_SIZE = 32
PARTITION_TRIPLE_SIZE = 24

#: DLPack device codes a mirror carries.
DEVICE_CPU = 1
DEVICE_ROCM = 10
