"""``hawk.load`` / ``hawk.run`` for the gfx950 target.

The thin Python face over ``libhawk_core.so`` (reference ``hawk/runtime.py``):
``load`` opens a built unit's kernel (code object loaded and ABI-checked by
``hk_load``), ``run`` validates and binds the caller's planes — PyTorch-ROCm
tensors, bound by their device pointers, never copied — launches the
per-sample stage over ``[base, base+count)``, then the team stages (the
fixed-tree ordered sum, the ordered scatter) on the same HIP stream.

Ownership as in the reference (``hawk/runtime.py:20-22``, ``:655-696``): the
planes are the caller's and are written in place; the runtime owns only its
scratch (term planes of a split kernel, the sum's lane partials, the
scatter's chunk partials and status plane), made once per sample count.

Threading: one :class:`DeviceKernel` shared by threads is safe: ``run`` holds
the kernel's lock over bind and launch (reference ``hawk/runtime.py:46-53``).
"""

from __future__ import annotations

import json
import threading
from pathlib import Path

from . import _contracts, _core
from .ir import HawkError

def _bound_length(role: str, x, n: int) -> int:
    """The length a slot is bound with: its cells for a lookup plane (the
    gather's bound), its keys for a per-key plane, the sample count otherwise."""
    if role in ("lookup", "accum_out", "fold_scratch"):
        return int(x.numel())
    return int(x.shape[-1]) if role == "key_out" else n


_PER_SAMPLE = ("per_sample", "vec_in", "mat_in", "mutable", "out", "wide_out", "terminated")
#: The per-sample roles a launch writes.
_WRITTEN = ("mutable", "out", "wide_out", "terminated")

#: The finish counter (reference ``hawk/ir/nodes.py:839``): one cell a
#: finishing kernel adds its newly finished samples to.  The caller may bind
#: it (an int32 tensor of one element, added to); left unbound the runtime
#: binds its own, zeroed before each ``hawk.run`` and readable afterwards as
#: the kernel's ``finished``.
FINISHED_PLANE = "finished_count"
#: The trip-count word of a ``hawk.steps(k, "auto")`` kernel: the runtime's
#: own one-cell int32, set from ``steps=`` (reference ``hawk/ir/nodes.py:841-845``).
FUSED_STEPS_PLANE = "fused_steps"
#: The fast entries of an automatic kernel and the slots each adds to the
#: kernel's own (reference ``hawk/emit/cuda.py:262-281``): the range entry's
#: steps max (u32) and steps sum (u64); the persistent entry's claim counter,
#: steps max, steps sum and chunk length.
FAST_SLOTS = {"range": ("int_handle", "handle"), "persist": ("int_handle", "int_handle", "handle", "int")}
#: The persistent entry's most workgroups: 256 CUs x 8 workgroups of 256
#: threads (32 waves a CU, gfx950's most); a smaller run takes one a block of samples.
PERSIST_BLOCKS = 2048
#: Trips between two claims of the persistent entry.  Measured on MI355X
#: (2^22 samples of 1-256 steps of the oscillator, one launch): chunks of 1,
#: 4, 8, 16, 32, 64 and 256 trips take 1.35, 0.82, 0.65, 0.56, 0.49, 0.50 and
#: 0.64 ms (the plain entry 0.93 ms): a short chunk spends its time claiming,
#: a long one holds finished lanes idle until the chunk ends.
PERSIST_CHUNK = 32
#: The fast entries' most samples a launch: the persistent grid claims from a
#: 32-bit counter in batches past the end, so it stays well below 2^32.
FAST_MAX = 1 << 30


def _torch():
    import torch
    return torch


def _on(stream: int):
    """A context in which torch's own work (a counter's ``zero_()``, a cell's
    ``fill_()``) is issued on ``stream``, the stream the next launch uses, so
    the reset is ordered before that launch and after the previous one."""
    torch = _torch()
    return torch.cuda.stream(torch.cuda.ExternalStream(stream)) if stream else _nullcontext()


class DeviceKernel:
    """One kernel of a built unit, loaded for the gfx950 target."""

    def __init__(self, directory: Path, sidecar: dict):
        from .targets import ENTRY_DEVICE, TARGETS
        built_for = TARGETS.get(sidecar.get("target"))
        if built_for is None or built_for.entry != ENTRY_DEVICE:
            raise HawkError(f"{sidecar.get('kernel')!r} was not built for the hip target")
        self.directory = Path(directory)
        self.sidecar = sidecar
        self.name = sidecar["kernel"]
        self.planes = sidecar["planes"]
        self.team = sidecar.get("team") or []
        self.arg_spec = [tuple(p) for p in sidecar.get("arg_spec") or []]
        self.mode = sidecar.get("mode", "float64")
        self.launch_shape = sidecar.get("launch", {"block": 256, "per_thread": 1})
        self.entry = None
        self.block = None
        if sidecar.get("entry"):
            code = (self.directory / sidecar["code_object"]).read_bytes()
            self.library = _core.DeviceLibrary(code)
            self.entry = self.library.entry(sidecar["entry"])
            self.block = _core.ArgBlock(sidecar["descriptor"])
        # What each slot of self.block holds: ("p", ptr, samples, device) or
        # ("v", value); None before the first bind.
        self._held_slots: list = [None] * len(self.arg_spec)
        self._scratch: dict = {}
        self._lock = threading.Lock()
        self.scatter_chunks = None
        self.finished = None      # the runtime's finish counter when the caller binds none
        self.steps_max = None     # a fast entry's largest trips a sample (one int32 cell)
        self.steps_sum = None     # a fast entry's trips over every sample (one int64 cell)

    # -- validation ----------------------------------------------------------
    def _real_dtype(self):
        torch = _torch()
        return torch.float32 if self.mode == "float32" else torch.float64

    def caller_planes(self) -> list:
        return [n for n, p in self.planes.items() if not p.get("scratch") and n != FUSED_STEPS_PLANE]

    @property
    def automatic(self) -> bool:
        """Whether the kernel reads its trip count at launch (``hawk.steps(k, "auto")``)."""
        return (self.sidecar.get("finish") or {}).get("steps") == "auto"

    def _word(self, steps, device, stream: int):
        """The trip-count word, set to ``steps`` on ``stream`` (held; rewritten
        only when the value changes)."""
        torch = _torch()
        if isinstance(steps, bool) or not isinstance(steps, int):
            raise HawkError(f"kernel {self.name!r}: steps= is an int (the trips this launch runs), got {steps!r}")
        held = self._scratch.get(("word", device))
        if held is None:
            held = torch.zeros(1, dtype=torch.int32, device=device)
            self._scratch[("word", device)] = held
            self._word_value = None
        value = max(-(1 << 31), min(steps, (1 << 31) - 1))
        if getattr(self, "_word_value", None) != value:
            with _on(stream):
                held.fill_(value)
            self._word_value = value
        return held

    def _held(self, key, dtype, device):
        torch = _torch()
        t = self._scratch.get((key, device))
        if t is None:
            t = torch.zeros(1, dtype=dtype, device=device)
            self._scratch[(key, device)] = t
        return t

    def _fast(self, entry: str, bound: dict, n: int, chunk: int, device, stream: int, cells=None):
        """``(DeviceEntry, ArgBlock, cells)`` of the fast entry ``entry`` bound
        to ``bound``.  ``cells`` are its claim counter (the persistent entry's
        only) and report cells (steps max, steps sum), zeroed here on
        ``stream``; by default the kernel's own (then its ``steps_max`` /
        ``steps_sum``), or those a :class:`Prepared` holds for itself."""
        torch = _torch()
        if entry not in FAST_SLOTS:
            raise HawkError(f"kernel {self.name!r}: entry= is 'plain', 'range' or 'persist', got {entry!r}")
        if not self.automatic:
            raise HawkError(f"kernel {self.name!r}: the fast entries are built for hawk.steps(k, 'auto') kernels")
        if entry == "persist" and (isinstance(chunk, bool) or not isinstance(chunk, int) or not 1 <= chunk <= 1 << 20):
            raise HawkError(f"kernel {self.name!r}: chunk= is an int in [1, 2^20], got {chunk!r}")
        names = self.sidecar["fast_entries"]
        fn = self.library.entry(names[entry])
        block = _core.ArgBlock(list(self.sidecar["descriptor"]) + list(FAST_SLOTS[entry]))
        self._bind(block, bound, n)
        if cells is None:
            cells = (self._held("claims", torch.int32, device), self._held("steps_max", torch.int32, device),
                     self._held("steps_sum", torch.int64, device))
            self.steps_max, self.steps_sum = cells[1], cells[2]
        with _on(stream):
            for c in cells:
                c.zero_()
        extra = list(cells) if entry == "persist" else list(cells[1:])
        slot = len(self.arg_spec)
        for x in extra:
            block.bind(slot, x.data_ptr(), 1, 1, _contracts.DEVICE_ROCM, x.device.index or 0)
            slot += 1
        if entry == "persist":
            block.bind_value(slot, int(chunk))
        return fn, block, cells

    def _bind(self, block, bound: dict, n: int) -> None:
        for slot, (role, name) in enumerate(self.arg_spec):
            kind = block.descriptor[slot]
            x = bound[name]
            if kind in ("f64", "f32"):
                block.bind_value(slot, float(x))
                continue
            block.bind(slot, x.data_ptr(), _bound_length(role, x, n), 1, _contracts.DEVICE_ROCM,
                       x.device.index or 0)

    def _launch_fast(self, entry: str, fn, block, base: int, count: int, n: int, stream: int) -> None:
        threads = self.launch_shape["block"]
        if entry == "range":
            fn.run(block, base, count, n, threads=threads, per_thread=self.launch_shape["per_thread"], stream=stream)
            return
        grid = max(1, min(-(-count // threads), PERSIST_BLOCKS))
        fn.run_grid(block, base, count, n, grid, threads, stream=stream)

    def _counter(self, arrays: dict, device):
        """``arrays`` with the finish counter bound: the caller's, else the
        runtime's own (zeroed by the caller of this method when it wants a count
        per run)."""
        if FINISHED_PLANE not in self.planes or FINISHED_PLANE in arrays:
            return arrays, None
        torch = _torch()
        held = self._scratch.get(("finished", device))
        if held is None:
            held = torch.zeros(1, dtype=torch.int32, device=device)
            self._scratch[("finished", device)] = held
        self.finished = held
        return {**arrays, FINISHED_PLANE: held}, held

    def check_planes(self, arrays: dict, n_samples=None) -> int:
        """Validate every bound plane against the sidecar; return the sample count."""
        torch = _torch()
        grid = self.sidecar.get("grid")
        n_grid = None
        if grid:
            # a Grid's extents may be given by label (reference hawk/trace/decl.py:135-145:
            # "the caller gives it as node=N"): the first axis's sets the lane count
            static = 1
            for _, e in grid:
                static *= e if e is not None else 1
            for pos, (label, extent) in enumerate(grid):
                if label not in arrays:
                    continue
                value = arrays.pop(label)
                if isinstance(value, bool) or not isinstance(value, int) or value < 0:
                    raise HawkError(f"kernel {self.name!r}: the Grid extent {label}= is an int >= 0, got {value!r}")
                if extent is not None and value != extent:
                    raise HawkError(f"kernel {self.name!r}: the Grid declares {label}:{extent}, the call gives "
                                    f"{label}={value}")
                if pos == 0:
                    n_grid = value * (static // (extent or 1)) if extent else value * static
        declared = set(self.caller_planes())
        unknown = sorted(set(arrays) - declared)
        if unknown:
            raise HawkError(f"kernel {self.name!r}: {unknown} are not planes it declares "
                            f"(declared: {sorted(declared)})")
        missing = sorted(declared - set(arrays) - {FINISHED_PLANE})
        if missing:
            raise HawkError(f"kernel {self.name!r}: bind {missing}")
        n = n_samples
        problems = []
        keyed = []
        for name in sorted(declared & set(arrays)):
            info = self.planes[name]
            x = arrays[name]
            role = info["role"]
            if role == "uniform":
                if isinstance(x, bool) or not isinstance(x, (int, float)):
                    problems.append(f"{name!r} is a Param: pass a Python number, got {type(x).__name__}")
                continue
            if not isinstance(x, torch.Tensor):
                problems.append(f"{name!r} must be a torch tensor on the GPU (the hip target binds device "
                                f"pointers), got {type(x).__name__}")
                continue
            if not x.is_cuda:
                problems.append(f"{name!r} is on {x.device}; the hip target binds device planes")
                continue
            if not x.is_contiguous():
                problems.append(f"{name!r} is not contiguous; pass x.contiguous()")
                continue
            # a cell or scatter target holds its declared type (a float32
            # build's default sum has a float32 cell); a per-sample plane the
            # build's Real
            want = torch.int32 if info["dtype"] in ("i32", "u32") else torch.bool if info["dtype"] == "bool" else (
                (torch.float32 if info["dtype"] == "f32" else torch.float64) if role in ("cell", "accum_out")
                else self._real_dtype())
            if x.dtype != want:
                problems.append(f"{name!r} has dtype {x.dtype}, the kernel reads {want}")
                continue
            if role in _PER_SAMPLE:
                lead = tuple(info["shape"])
                if x.dim() != len(lead) + 1 or tuple(x.shape[:-1]) != lead:
                    problems.append(f"{name!r} has shape {tuple(x.shape)}; a {lead or 'scalar'} plane is "
                                    f"({', '.join(str(e) for e in lead + ('N',))})")
                    continue
                if n is None:
                    n = int(x.shape[-1])
                elif int(x.shape[-1]) != n:
                    problems.append(f"{name!r} holds {int(x.shape[-1])} samples, other planes {n}")
            elif role == "cell" and info.get("group"):
                keyed.append((name, x, info["group"]))
            elif role == "cell":
                cells = 1
                for e in info["shape"]:
                    cells *= e
                if x.numel() != cells:
                    problems.append(f"{name!r} is " + (f"the {tuple(info['shape'])} result of a reduction over "
                                    f"the samples: bind {cells} elements" if info["shape"] else
                                    "a one-cell result of a reduction over the samples: bind 1 element")
                                    + f", got {x.numel()}")
            elif role == "accum_out":
                if x.dim() != 1:
                    problems.append(f"{name!r} is the 1-D plane of cells hawk.scatter adds into")
            elif name == FINISHED_PLANE:
                if x.numel() != 1:
                    problems.append(f"{name!r} is the one-cell finish counter: bind 1 element, got {x.numel()}")
            elif role == "lookup":
                axes = (self.sidecar.get("tables") or {}).get(name)
                if x.dim() != 1 and axes is None:
                    problems.append(f"{name!r} is a 1-D plane of cells read at a key (the adjoint of a "
                                    "hawk.scatter target): bind one value per cell")
                elif axes is not None:
                    rest, first = 1, axes[0][1]
                    for _, e in axes[1:]:
                        rest *= e
                    cells = int(x.numel())
                    if cells == 0 or cells % rest or (first is not None and cells != first * rest):
                        problems.append(f"{name!r} is a Table{[tuple(a) for a in axes]}: bind "
                                        + (f"{first * rest}" if first is not None else f"a nonzero multiple of {rest}")
                                        + f" cells, got {cells} (a read clamps into the table, so it needs a cell)")
        if n_grid is not None:
            if n is not None and n != n_grid:
                problems.append(f"the Grid's extents give {n_grid} lanes, the planes {n}")
            n = n_grid
        if n is not None and grid:
            static = 1
            for _, e in grid:
                static *= e if e is not None else 1
            if n % static:
                problems.append(f"{n} lanes are not a whole number of Grid{[tuple(a) for a in grid]} rows "
                                f"of {static}")
        for name, x, group in keyed:
            if n is not None and x.numel() != n // group:
                problems.append(f"{name!r} holds hawk.sum over the trailing lane axes, one cell per {group} "
                                f"lanes: bind {n // group} elements, got {x.numel()}")
        if problems:
            raise HawkError(f"kernel {self.name!r}: " + "; ".join(problems))
        if n is None:
            raise HawkError(f"kernel {self.name!r}: no per-sample plane is bound, so the sample count is "
                            "unknown; pass n_samples=" + (f" or the Grid's {grid[0][0]}=" if grid else ""))
        return n

    # -- scratch -------------------------------------------------------------
    def _is_f32(self, plane: str) -> bool:
        """Whether a team stage's cell or target plane holds float32 (a float32
        build's sums and scatters run in float32)."""
        return self.planes[plane]["dtype"] == "f32"

    def _buffer(self, key, nbytes: int, device, zero: bool = True):
        torch = _torch()
        held = self._scratch.get(key)
        if held is None or held.numel() < max(1, nbytes) or held.device != device:
            held = (torch.zeros if zero else torch.empty)(max(1, nbytes), dtype=torch.uint8, device=device)
            self._scratch[key] = held
        return held

    @staticmethod
    def _cell_ptr(t: dict, out) -> int:
        """The address of a team stage's cell: entry ``column`` of a vector
        cell (``hawk.sum`` of a vector commits one entry a column)."""
        return out.data_ptr() + (t.get("column") or 0) * out.element_size()

    def _row_sum(self, t: dict, bound: dict, n: int, device, stream: int) -> None:
        """Fold the stage's row partials into the cell: compensated (hi, comp)
        rows, band rows (hi, lo) in the banded mode, or one extreme a row
        (``hawk.max`` / ``hawk.min``).  A run of no samples leaves the
        reduction's identity: 0, -inf (max), +inf (min)."""
        out = bound[t["out"]]
        rows = -(-n // 32)
        col = t.get("column")
        if rows == 0:
            empty = {"max": float("-inf"), "min": float("inf")}.get(t.get("red"), 0.0)
            with _on(stream):
                (out.view(-1)[col:col + 1] if col is not None else out).fill_(empty)
            return
        band = t["op"] == "band_rows"
        f32 = self.planes[t["hi"]]["dtype"] == "f32"      # the rows are the stage's Real: the finish runs in it
        with _on(stream):
            nbytes = (_core.band_rows_finish_scratch_bytes if band else _core.rows_finish_scratch_bytes)(rows)
            scratch = self._buffer(("rows", t["hi"], rows), nbytes, device, zero=False)
        if t["op"] == "row_extreme":
            (_core.rows_extreme_f32 if f32 else _core.rows_extreme)(
                bound[t["hi"]].data_ptr(), rows, 1 if t["red"] == "max" else 2, self._cell_ptr(t, out),
                scratch.data_ptr(), stream)
            return
        finish = _core.band_rows_finish if band else _core.rows_finish_f32 if f32 else _core.rows_finish
        finish(bound[t["hi"]].data_ptr(), bound[t["comp"]].data_ptr(), rows, self._cell_ptr(t, out),
               scratch.data_ptr(), stream)

    def _term_plane(self, name: str, n: int, device):
        torch = _torch()
        info = self.planes[name]
        lead = tuple(info["shape"])
        key = ("plane", name, n)
        held = self._scratch.get(key)
        if held is None or held.device != device:
            if info.get("rows"):                       # one row partial per `rows` samples, in the stage's Real
                held = torch.empty(max(1, -(-n // info["rows"])),
                                   dtype=torch.float32 if info["dtype"] == "f32" else torch.float64, device=device)
            elif info.get("group"):                    # one entry per key (`group` samples)
                held = torch.empty(lead + (n // info["group"],), dtype=torch.int32, device=device)
            else:
                held = torch.empty(lead + (n,), dtype=torch.int32 if info["dtype"] == "i32" else self._real_dtype(),
                                   device=device)
            self._scratch[key] = held
        return held

    def _fold_scratch(self, name: str, bound: dict, device):
        """The claims and status of a fused fold: 64 status words, then one
        claim count per cell of its gradient plane."""
        torch = _torch()
        cells = int(bound[self.planes[name]["cells_of"]].numel())
        return self._buffer(("fold_scratch", name, cells), 4 * (64 + cells), device, zero=False).view(torch.int32)

    def _fold_clear_args(self, t: dict, bound: dict) -> tuple:
        """``(args, status, cells)`` of the set-up of a fused fold: its claims and
        status cleared (the fold entry with no keys), before the stage runs."""
        scratch = bound[t["scratch"]]
        cells = int(bound[t["out"]].numel())
        args = (0, 0, 0, 0, 1, 1, bound[t["out"]].data_ptr(), cells, scratch.data_ptr() + 256, scratch.data_ptr())
        return args, scratch, cells

    def _fold_args(self, t: dict, bound: dict, n: int, device) -> tuple:
        """``(args, status, cells)`` of the ordered fold ``t`` (the stage's log
        planes, the gradient plane, its claim counts and its status words)."""
        out = bound[t["out"]]
        cells = int(out.numel())
        scratch = self._buffer(("fold", t["out"], cells), _core.keyed_log_fold_scratch_bytes(cells), device,
                               zero=False)
        status = self._buffer(("fold_status", t["out"]), 8, device, zero=False)
        args = (bound[t["v"]].data_ptr(), n, bound[t["c"]].data_ptr(), n // t["group"], t["group"], t["width"],
                out.data_ptr(), cells, scratch.data_ptr(), status.data_ptr())
        return args, status, cells

    # -- launch --------------------------------------------------------------
    def bind_all(self, arrays: dict, n: int) -> None:
        """Bind the per-sample stage's slots to validated ``arrays``, crossing
        the C-ABI only for what changed since the last bind: a slot whose
        length, device or by-value number changed is bound on its own; every
        slot whose pointer alone moved is swapped in ONE bulk rebind.  So a
        run over the planes of the last run adds no crossing to its launch,
        and a run over moved planes adds one (reference ``hawk/runtime.py:330-345``,
        the stable-binding and rebind arms of its launch-crossing contract)."""
        moved_slots, moved_ptrs = [], []
        for slot, (role, name) in enumerate(self.arg_spec):
            kind = self.block.descriptor[slot]
            x = arrays[name]
            held = self._held_slots[slot]
            if kind in ("f64", "f32"):
                value = float(x)
                if held != ("v", value):
                    self.block.bind_value(slot, value)
                    self._held_slots[slot] = ("v", value)
                continue
            ptr, samples, device = x.data_ptr(), _bound_length(role, x, n), x.device.index or 0
            if held is not None and held[0] == "p" and held[2:] == (samples, device):
                if held[1] != ptr:
                    moved_slots.append(slot)
                    moved_ptrs.append(ptr)
                continue
            self.block.bind(slot, ptr, samples, 1, _contracts.DEVICE_ROCM, device)
            self._held_slots[slot] = ("p", ptr, samples, device)
        if moved_slots:
            self.rebind(moved_slots, moved_ptrs)

    def rebind(self, slots, ptrs) -> None:
        """The bulk pointer swap: every (slot, pointer) pair in ONE crossing
        (``hk_rebind``; reference ``hawk/runtime.py:330-345``).  Unchecked by
        design: it only moves slots a validated bind already shaped, so each
        slot keeps the length and device it was bound with.  A by-value slot
        is refused (by the C-ABI, naming the slot)."""
        slots = [int(s) for s in slots]
        ptrs = [int(p) for p in ptrs]
        self.block.rebind(slots, ptrs)
        for slot, ptr in zip(slots, ptrs):
            held = self._held_slots[slot]
            if held is not None and held[0] == "p":
                self._held_slots[slot] = ("p", ptr, held[2], held[3])

    def _run(self, arrays: dict, base: int, count: int, n: int, stream: int, check: bool, steps=None,
             entry: str = "plain", chunk: int = PERSIST_CHUNK) -> None:
        # every reset, scratch fill and status read is issued on the launch's stream
        with _on(stream):
            self._run_on(arrays, base, count, n, stream, check, steps, entry, chunk)

    def _run_on(self, arrays: dict, base: int, count: int, n: int, stream: int, check: bool, steps,
                entry: str, chunk: int) -> None:
        torch = _torch()
        device = next((x.device for x in arrays.values() if isinstance(x, torch.Tensor)), None)
        if device is None:
            raise HawkError(f"kernel {self.name!r}: no plane is a tensor, so there is no device to run on")
        bound, held = self._counter(dict(arrays), device)
        if held is not None:
            with _on(stream):
                held.zero_()                      # a count per run
        if self.automatic:
            bound[FUSED_STEPS_PLANE] = self._word(1 if steps is None else steps, device, stream)
        elif steps is not None:
            raise HawkError(f"kernel {self.name!r}: steps= sets the trip count of a hawk.steps(k, 'auto') kernel; "
                            "this one takes a fixed number of steps")
        if entry != "plain":
            if count >= FAST_MAX:
                raise HawkError(f"kernel {self.name!r}: the fast entries take fewer than 2^30 samples a launch")
            fn, block, _cells = self._fast(entry, bound, n, chunk, device, stream)
            self._launch_fast(entry, fn, block, base, count, n, stream)
            return
        for name, info in self.planes.items():
            if info.get("cells_of"):
                bound[name] = self._fold_scratch(name, bound, device)
            elif info.get("scratch"):
                bound[name] = self._term_plane(name, n, device)
        statuses = []
        for t in self.team:
            if t.get("before"):                  # a fused fold's claims and status, cleared first
                args, status, cells = self._fold_clear_args(t, bound)
                _core.keyed_log_fold(*args, stream)
                statuses.append((t, status, cells))
        if self.entry is not None:
            self.bind_all(bound, n)
            self.entry.run(self.block, base, count, n, threads=self.launch_shape["block"],
                           per_thread=self.launch_shape["per_thread"], stream=stream)
        for t in self.team:
            if t.get("before"):
                continue
            if t["op"] == "ordered_sum":
                u = bound[t["u"]]
                scratch = self._buffer(("sum", t["out"]), _core.ordered_sum_scratch_bytes(), device)
                fn = _core.ordered_sum_f32 if self._is_f32(t["out"]) else _core.ordered_sum
                fn(u.data_ptr(), n, self._cell_ptr(t, bound[t["out"]]), scratch.data_ptr(), stream)
            elif t["op"] == "ordered_scatter":
                target = bound[t["target"]]
                cells = int(target.numel())
                if cells == 0:
                    continue              # an ordered scatter into no cells adds nothing
                scratch = self._buffer(("scatter", t["target"], n, cells),
                                       _core.ordered_scatter_scratch_bytes(n, cells), device, zero=False)
                status = self._buffer(("status", t["target"]), 4 * 257, device)
                fn = _core.ordered_scatter_f32 if self._is_f32(t["target"]) else _core.ordered_scatter
                fn(bound[t["key"]].data_ptr(), bound[t["v"]].data_ptr(), n, target.data_ptr(), cells,
                   scratch.data_ptr(), status.data_ptr(), stream)
                self.scatter_chunks = _core.scatter_chunks(n, cells)
                statuses.append((t, status, cells))
            elif t["op"] == "mm16":
                _core.mm16([bound[p].data_ptr() for p in t["in"]], [bound[p].data_ptr() for p in t["out"]],
                           t["products"], n, stream, t.get("dtype", "f32"))
            elif t["op"] in ("row_sum", "band_rows", "row_extreme"):
                self._row_sum(t, bound, n, device, stream)
            elif t["op"] == "band_ordered_sum":
                u = bound[t["u"]]
                scratch = self._buffer(("band_sum", t["out"]), _core.band_ordered_sum_scratch_bytes(), device,
                                       zero=False)
                _core.band_ordered_sum(u.data_ptr(), n, self._cell_ptr(t, bound[t["out"]]), scratch.data_ptr(),
                                       stream)
            elif t["op"] == "keyed_sum":
                scratch = self._buffer(("keyed", t["out"], n), _core.keyed_ordered_sum_scratch_bytes(n, t["group"]),
                                       device)
                fn = _core.keyed_ordered_sum_f32 if self._is_f32(t["out"]) else _core.keyed_ordered_sum
                fn(bound[t["u"]].data_ptr(), n, t["group"], bound[t["out"]].data_ptr(), scratch.data_ptr(), stream)
            elif t["op"] == "ordered_fold":
                args, status, cells = self._fold_args(t, bound, n, device)
                (_core.keyed_log_fold_f32 if self._is_f32(t["out"]) else _core.keyed_log_fold)(*args, stream)
                statuses.append((t, status, cells))
            elif t["op"] == "keyed_comp":
                fn = _core.keyed_sample_sum_f32 if self._is_f32(t["out"]) else _core.keyed_sample_sum
                fn(bound[t["u"]].data_ptr(), n, t["group"], bound[t["out"]].data_ptr(), stream)
            else:
                raise HawkError(f"kernel {self.name!r}: unknown team stage {t['op']!r}")
        if check:
            for t, status, cells in statuses:
                problem = _status_problem(self.name, t, status, cells)
                if problem:
                    raise HawkError(problem)

    def prepare(self, *, stream=None, steps=None, entry: str = "plain", chunk: int = PERSIST_CHUNK,
                **arrays) -> Prepared:
        """Validate and bind ``arrays`` once and return a :class:`Prepared`
        launcher that re-runs the whole kernel (per-sample stage and team
        stages) over every sample with no per-call validation: the stable-binding
        path of reference ``tests/cards/CARD_LAUNCH_CROSSINGS.md`` (one crossing
        per launch).  The planes must stay alive and unmoved while it is used.
        ``steps`` / ``entry`` / ``chunk`` are :func:`run`'s; a prepared
        automatic kernel holds its own trip-count word, and its reports and
        finish count add up over calls."""
        return Prepared(self, arrays, stream, steps=steps, entry=entry, chunk=chunk)

    def launch(self, base: int, count: int, n_samples: int, stream: int = 0) -> None:
        """The per-sample stage alone over ``[base, base+count)`` (planes already bound)."""
        with self._lock:
            if self.entry is None:
                raise HawkError(f"kernel {self.name!r} has no per-sample stage")
            self.entry.run(self.block, base, count, n_samples, threads=self.launch_shape["block"],
                           per_thread=self.launch_shape["per_thread"], stream=stream)


def _status_problem(name: str, t: dict, status, cells: int) -> str | None:
    """What a team stage's status words report after a run, or ``None``."""
    torch = _torch()
    if t["op"] in ("ordered_fold", "fused_fold"):
        flags = status.view(torch.int32)[:2].cpu().tolist()
        if flags[0] & 1:
            return (f"{name}: the gradient {t['out']} has {cells} cells, fewer than the table it is the "
                    "gradient of; the reads past its end were not stored")
        if flags[0] & 2:
            return (f"{name}: cell {flags[1]} of {t['out']} is read by more than one key (or twice by one key): "
                    "under an ordered keyed sum each cell's gradient is stored from one key's sum, so those "
                    "stores raced; read a table by the kept lane axes, one cell per key and read")
        return None
    flags = status.view(torch.int32)[:257].cpu()
    if bool((flags[1:] != 0).any()):
        return (f"{name}: hawk.scatter({t['target']}, policy='ordered') got a key outside "
                f"[0, {cells}) that is not the skip key -1; those adds were dropped, the rest are "
                f"in {t['target']}")
    return None


class ChainedKernel:
    """A ``hawk.chain`` the build cut into segments: each segment is a kernel
    of its own, run in order; a value one segment passes to a later one
    crosses in a plane the runtime holds (``hwc_<name>``), made once per
    sample count (reference ``hawk/ir/chain.py:133-179``)."""

    def __init__(self, directory: Path, sidecar: dict):
        self.directory = Path(directory)
        self.sidecar = sidecar
        self.name = sidecar["kernel"]
        self.planes = sidecar["planes"]
        self.team = []
        self.segments = [load(directory, s) for s in sidecar["segments"]]
        self.crossing = sidecar["crossing"]
        self._held: dict = {}
        self._lock = threading.Lock()

    def caller_planes(self) -> list:
        return list(self.planes)

    def _bindings(self, arrays: dict, n_samples=None) -> list:
        """Each segment's planes: the caller's and the crossing planes it reads or writes."""
        torch = _torch()
        declared = set(self.planes)
        unknown = sorted(set(arrays) - declared)
        if unknown:
            raise HawkError(f"kernel {self.name!r}: {unknown} are not planes it declares "
                            f"(declared: {sorted(declared)})")
        missing = sorted(declared - set(arrays))
        if missing:
            raise HawkError(f"kernel {self.name!r}: bind {missing}")
        ns = {int(x.shape[-1]) for name, x in arrays.items()
              if isinstance(x, torch.Tensor) and self.planes[name]["role"] in _PER_SAMPLE}
        n = n_samples if n_samples is not None else (ns.pop() if len(ns) == 1 else None)
        if n is None:
            raise HawkError(f"kernel {self.name!r}: its planes disagree on the sample count, or none is bound")
        device = next((x.device for x in arrays.values() if isinstance(x, torch.Tensor)), None)
        if device is None:
            raise HawkError(f"kernel {self.name!r}: no plane is a tensor, so there is no device to run on")
        cross = {}
        for name, info in self.crossing.items():
            key = (name, n, device)
            held = self._held.get(key)
            if held is None:
                dt = torch.int32 if info["dtype"] == "i32" else torch.float64
                held = torch.empty(tuple(info["shape"]) + (n,), dtype=dt, device=device)
                self._held[key] = held
            cross[name] = held
        out = []
        for seg in self.segments:
            names = seg.caller_planes()
            out.append((seg, {p: (cross[p] if p in cross else arrays[p]) for p in names}))
        return out

    def resolve_call(self, arrays: dict, layout=None, n_samples=None) -> tuple:
        """``(bindings, write_back)`` of one call: the caller's planes made
        component-major once (:func:`hawk_amd.layout.resolve`), then each
        segment's planes (:meth:`_bindings`); ``write_back`` lists the
        sample-major planes the chain writes, with their component-major
        copies, to copy back after the last segment."""
        from . import layout as _layout
        arrays, write_back = _layout.resolve(self, dict(arrays), layout, _PER_SAMPLE, _WRITTEN)
        return self._bindings(arrays, n_samples), write_back

    def prepare(self, *, stream=None, **arrays):
        return _PreparedChain(self, arrays, stream)


class _PreparedChain:
    """The segments of a cut chain, each bound once (see :meth:`DeviceKernel.prepare`)."""

    def __init__(self, chain: ChainedKernel, arrays: dict, stream=None):
        self.kernel = chain
        self.parts = [seg.prepare(stream=stream, **planes) for seg, planes in chain._bindings(dict(arrays))]

    def __call__(self) -> None:
        for part in self.parts:
            part()

    def stages(self) -> list:
        return [step for part in self.parts for step in part.stages()]

    def check(self) -> None:
        for part in self.parts:
            part.check()


def load(directory, kernel: str, sidecar: dict | None = None):
    """Open ``<directory>/<kernel>`` of a unit built for the hip target."""
    directory = Path(directory)
    if sidecar is None:
        path = directory / f"{kernel}.json"
        if not path.exists():
            raise HawkError(f"{directory} holds no kernel {kernel!r} (no {path.name})")
        sidecar = json.loads(path.read_text())
    if sidecar.get("segments"):
        return ChainedKernel(directory, sidecar)
    return DeviceKernel(directory, sidecar)


class _nullcontext:
    def __enter__(self):
        return self

    def __exit__(self, *exc):
        return False


def run(kernel: DeviceKernel, *, base: int = 0, count: int | None = None, n_samples: int | None = None,
        layout: str | None = None, stream=None, check: bool = True, steps=None, entry: str = "plain",
        chunk: int = PERSIST_CHUNK, **arrays) -> None:
    """Bind ``arrays`` and run the kernel once, in place, on the current HIP
    stream (or ``stream``).  ``count`` defaults to every sample from ``base``.
    A kernel with team stages (``hawk.sum`` / ``hawk.scatter`` with
    policy='ordered') runs over every sample (no ``base``/``count``).

    A ``hawk.steps(k, "auto")`` kernel runs ``steps`` trips (default 1) and
    may run through a fast entry: ``entry="range"`` (one lane a sample) or
    ``"persist"`` (a persistent grid whose waves claim samples, ``chunk``
    trips between claims, default :data:`PERSIST_CHUNK`).  Both give the
    plain entry's bits, count samples finished on entry too (the counter then
    holds the batch's finished count), and leave the largest and the total
    trips run in the kernel's ``steps_max`` and ``steps_sum``.

    ``layout`` (``"samples_first"`` / ``"samples_last"``) and the markers
    :func:`hawk_amd.samples_first` / :func:`~hawk_amd.samples_last` say which
    axis of a per-sample plane holds the samples (:mod:`hawk_amd.layout`)."""
    from . import layout as _layout
    torch = _torch()
    if isinstance(kernel, ChainedKernel):
        if base != 0 or count is not None:
            raise HawkError(f"{kernel.name}: a cut chain runs over every sample (no base= or count=)")
        # The caller's planes are resolved to component-major once, at the
        # chain: the crossing planes are (w, N), so every segment then runs
        # on component-major planes, and a sample-major plane the chain
        # writes is copied back after the last segment.
        sid = torch.cuda.current_stream().cuda_stream if stream is None else getattr(stream, "cuda_stream", stream)
        with _on(int(sid)):
            bindings, write_back = kernel.resolve_call(arrays, layout, n_samples)
        for seg, planes in bindings:
            run(seg, n_samples=n_samples, stream=stream, check=check, **planes)
        if write_back:
            with _on(int(sid)):
                for dst, copy in write_back:
                    dst.copy_(copy.movedim(-1, 0))
        return
    if not isinstance(kernel, DeviceKernel):
        raise HawkError("hawk.run takes a kernel loaded with hawk.load")
    if stream is None:
        stream = torch.cuda.current_stream().cuda_stream
    elif hasattr(stream, "cuda_stream"):
        stream = stream.cuda_stream
    with _on(int(stream)):
        arrays, write_back = _layout.resolve(kernel, arrays, layout, _PER_SAMPLE, _WRITTEN)
    n = kernel.check_planes(arrays, n_samples)
    if kernel.team and (base != 0 or count not in (None, n)):
        raise HawkError(f"{kernel.name}: this kernel reduces over every sample, so it runs over every "
                        "sample (no base= or count=)")
    if count is None:
        count = n - base
    if base < 0 or count < 0 or base + count > n:
        raise HawkError(f"{kernel.name}: [base, base+count) = [{base}, {base + count}) is outside [0, {n})")
    with kernel._lock:
        kernel._run(arrays, int(base), int(count), int(n), int(stream), check, steps=steps, entry=entry,
                    chunk=chunk)
    if write_back:
        with _on(int(stream)):
            for dst, copy in write_back:       # a sample-major plane the kernel wrote
                dst.copy_(copy.movedim(-1, 0))


class Prepared:
    """A kernel bound once to fixed planes (see :meth:`DeviceKernel.prepare`).

    Everything it resets runs on its own stream, ordered with its launches.
    Through a fast entry it holds its own claim counter and report cells
    (another launcher of the same kernel never shares them), and each call
    starts them, and the runtime's finish counter, from zero: after a call,
    ``steps_max`` / ``steps_sum`` are that call's trips and ``finished`` is
    the batch's finished count (the fast entries count a sample finished on
    entry too).  Through the plain entry the finish count adds up over calls
    (each call counts only the samples it finishes), so it too holds the
    batch's finished count after every call."""

    def __init__(self, kernel: DeviceKernel, arrays: dict, stream=None, steps=None, entry: str = "plain",
                 chunk: int = PERSIST_CHUNK):
        from .layout import Marked
        torch = _torch()
        self.kernel = kernel
        marked = [name for name, x in arrays.items() if isinstance(x, Marked)]
        if marked:
            raise HawkError(f"{kernel.name}: prepare binds planes by address, so it takes component-major (w, N) "
                            f"planes only; {marked} are marked (hawk.run takes a sample-major plane through a copy)")
        self.n = kernel.check_planes(arrays)
        self.arrays = dict(arrays)
        if stream is None:
            stream = torch.cuda.current_stream().cuda_stream
        elif hasattr(stream, "cuda_stream"):
            stream = stream.cuda_stream
        self.stream = int(stream)
        with _on(self.stream):
            self._setup(kernel, arrays, steps, entry, chunk)

    def _setup(self, kernel, arrays: dict, steps, entry: str, chunk: int) -> None:
        torch = _torch()
        device = next((x.device for x in arrays.values() if isinstance(x, torch.Tensor)), None)
        if device is None:
            raise HawkError(f"kernel {self.name!r}: no plane is a tensor, so there is no device to run on")
        bound, held = kernel._counter(dict(arrays), device)
        self.held_counter = held
        if held is not None:
            held.zero_()
        self.finished = bound.get(FINISHED_PLANE)
        if kernel.automatic:
            w = 1 if steps is None else steps
            if isinstance(w, bool) or not isinstance(w, int):
                raise HawkError(f"kernel {kernel.name!r}: steps= is an int, got {w!r}")
            bound[FUSED_STEPS_PLANE] = torch.full((1,), max(-(1 << 31), min(w, (1 << 31) - 1)),
                                                  dtype=torch.int32, device=device)
        elif steps is not None:
            raise HawkError(f"kernel {kernel.name!r}: steps= sets the trip count of a hawk.steps(k, 'auto') kernel")
        self.fast = None
        if entry != "plain":
            if self.n >= FAST_MAX:
                raise HawkError(f"kernel {kernel.name!r}: the fast entries take fewer than 2^30 samples a launch")
            own = (torch.zeros(1, dtype=torch.int32, device=device), torch.zeros(1, dtype=torch.int32, device=device),
                   torch.zeros(1, dtype=torch.int64, device=device))
            fn, block, cells = kernel._fast(entry, bound, self.n, chunk, device, self.stream, cells=own)
            self.fast = (entry, fn, block, cells)
            self.steps_max, self.steps_sum = cells[1], cells[2]
        for name, info in kernel.planes.items():
            if info.get("cells_of"):
                bound[name] = kernel._fold_scratch(name, bound, device)
            elif info.get("scratch"):
                bound[name] = kernel._term_plane(name, self.n, device)
        self.bound = bound
        self.block = None
        if kernel.entry is not None:
            self.block = _core.ArgBlock(kernel.sidecar["descriptor"])
            for slot, (role, name) in enumerate(kernel.arg_spec):
                kind = self.block.descriptor[slot]
                x = bound[name]
                if kind in ("f64", "f32"):
                    self.block.bind_value(slot, float(x))
                else:
                    self.block.bind(slot, x.data_ptr(), _bound_length(role, x, self.n), 1, _contracts.DEVICE_ROCM,
                                    x.device.index or 0)
        self.steps = []
        self.before = []
        self.statuses = []
        for t in kernel.team:
            if t.get("before"):
                args, status, cells = kernel._fold_clear_args(t, bound)
                self.before.append((_core.keyed_log_fold, args))
                self.statuses.append((t, status, cells))
                continue
            if t["op"] == "ordered_sum":
                scratch = kernel._buffer(("sum", t["out"]), _core.ordered_sum_scratch_bytes(), device)
                args = (bound[t["u"]].data_ptr(), self.n, kernel._cell_ptr(t, bound[t["out"]]), scratch.data_ptr())
                self.steps.append((_core.ordered_sum_f32 if kernel._is_f32(t["out"]) else _core.ordered_sum, args))
            elif t["op"] == "ordered_scatter":
                target = bound[t["target"]]
                cells = int(target.numel())
                if cells == 0:
                    continue
                scratch = kernel._buffer(("scatter", t["target"], self.n, cells),
                                         _core.ordered_scatter_scratch_bytes(self.n, cells), device, zero=False)
                status = kernel._buffer(("status", t["target"]), 4 * 257, device)
                args = (bound[t["key"]].data_ptr(), bound[t["v"]].data_ptr(), self.n, target.data_ptr(), cells,
                        scratch.data_ptr(), status.data_ptr())
                self.steps.append((_core.ordered_scatter_f32 if kernel._is_f32(t["target"]) else _core.ordered_scatter,
                                   args))
                self.statuses.append((t, status, cells))
            elif t["op"] == "mm16":
                args = ([bound[p].data_ptr() for p in t["in"]], [bound[p].data_ptr() for p in t["out"]],
                        t["products"], self.n)
                self.steps.append((_core.mm16_f64 if t.get("dtype") == "f64" else _core.mm16, args))
            elif t["op"] in ("row_sum", "band_rows", "row_extreme"):
                self.steps.append((kernel._row_sum, (t, bound, self.n, device)))
            elif t["op"] == "band_ordered_sum":
                scratch = kernel._buffer(("band_sum", t["out"]), _core.band_ordered_sum_scratch_bytes(), device,
                                         zero=False)
                args = (bound[t["u"]].data_ptr(), self.n, kernel._cell_ptr(t, bound[t["out"]]), scratch.data_ptr())
                self.steps.append((_core.band_ordered_sum, args))
            elif t["op"] == "keyed_sum":
                scratch = kernel._buffer(("keyed", t["out"], self.n),
                                         _core.keyed_ordered_sum_scratch_bytes(self.n, t["group"]), device)
                args = (bound[t["u"]].data_ptr(), self.n, t["group"], bound[t["out"]].data_ptr(), scratch.data_ptr())
                self.steps.append((_core.keyed_ordered_sum_f32 if kernel._is_f32(t["out"]) else _core.keyed_ordered_sum,
                                   args))
            elif t["op"] == "ordered_fold":
                args, status, cells = kernel._fold_args(t, bound, self.n, device)
                self.steps.append((_core.keyed_log_fold_f32 if kernel._is_f32(t["out"]) else _core.keyed_log_fold,
                                   args))
                self.statuses.append((t, status, cells))
            elif t["op"] == "keyed_comp":
                args = (bound[t["u"]].data_ptr(), self.n, t["group"], bound[t["out"]].data_ptr())
                self.steps.append((_core.keyed_sample_sum_f32 if kernel._is_f32(t["out"]) else _core.keyed_sample_sum,
                                   args))
            else:
                raise HawkError(f"kernel {kernel.name!r}: unknown team stage {t['op']!r}")

    def __call__(self) -> None:
        for _label, launch in self.stages():
            launch()

    def stages(self) -> list:
        """``[(label, launch)]`` in run order: a fused fold's set-up
        (``"fold_clear"``), the per-sample stage (labelled with the kernel's
        name) and each team stage (``"ordered_sum"``, ``"ordered_scatter"``,
        ...); calling every ``launch`` in order is one run."""
        k = self.kernel
        out = [("fold_clear", lambda fn=fn, args=args: fn(*args, self.stream)) for fn, args in self.before]
        if self.fast is not None:
            entry, fn, block, cells = self.fast
            resets = list(cells) + ([self.held_counter] if self.held_counter is not None else [])

            def fast_stage():
                with _on(self.stream):          # claims from sample 0 again; this call's reports and count
                    for c in resets:
                        c.zero_()
                k._launch_fast(entry, fn, block, 0, self.n, self.n, self.stream)
            out.append((f"{k.name}_{entry}", fast_stage))
            return out
        if k.entry is not None:
            def stage():
                k.entry.run(self.block, 0, self.n, self.n, threads=k.launch_shape["block"],
                            per_thread=k.launch_shape["per_thread"], stream=self.stream)
            out.append((k.name, stage))
        labels = {_core.ordered_sum: "ordered_sum", _core.ordered_sum_f32: "ordered_sum",
                  _core.band_ordered_sum: "band_ordered_sum",
                  _core.ordered_scatter: "ordered_scatter", _core.ordered_scatter_f32: "ordered_scatter",
                  _core.mm16: "mm16", _core.mm16_f64: "mm16",
                  _core.keyed_ordered_sum: "keyed_sum", _core.keyed_ordered_sum_f32: "keyed_sum", _core.keyed_log_fold: "ordered_fold", _core.keyed_log_fold_f32: "ordered_fold",
                  _core.keyed_sample_sum: "keyed_comp", _core.keyed_sample_sum_f32: "keyed_comp"}
        for fn, args in self.steps:
            label = labels.get(fn, "row_sum")
            out.append((label, lambda fn=fn, args=args: fn(*args, self.stream)))
        return out

    def check(self) -> None:
        """Refuse, by name, a run whose ordered scatter met a bad key or whose
        ordered fold met a cell named twice (synchronises with its stream)."""
        for t, status, cells in self.statuses:
            with _on(self.stream):
                problem = _status_problem(self.kernel.name, t, status, cells)
            if problem:
                raise HawkError(problem)
