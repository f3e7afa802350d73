"""The entry point that allocates nothing, hk_ordered_sum_f64_noalloc, against
hk_ordered_sum_f64 on allocated scratch: the same bits (the fixed tree is
bit-exact), on two calls in a row, the second with fewer samples, and against
the oracle.  It runs through the C-ABI (ctypes)."""

from __future__ import annotations

import ctypes

import numpy as np
import pytest

import oracle_lib as O
from conftest import rng

pytestmark = pytest.mark.gpu


def _sum_with_scratch(u, n, gpu):
    import torch

    from hawk_amd import _core
    out = torch.full((1,), np.nan, dtype=torch.float64, device=gpu)
    scratch = torch.zeros(_core.ordered_sum_scratch_bytes(), dtype=torch.uint8, device=gpu)
    _core.ordered_sum(u.data_ptr(), n, out.data_ptr(), scratch.data_ptr(), torch.cuda.current_stream().cuda_stream)
    return out


def test_the_no_alloc_sum_is_the_allocating_sums_bits_twice_in_a_row(gpu):
    import torch

    from hawk_amd import _core
    L = _core.lib()
    assert L.hk_ordered_sum_noalloc_scratch_bytes() == L.hk_ordered_sum_scratch_bytes() == 524288 + 768
    stream = torch.cuda.current_stream().cuda_stream
    for n in ((1 << 22) + 12345, 70_001):         # the second call is smaller: no stale lanes may leak in
        x = rng(n).normal(size=n) * np.exp(rng(n + 1).normal(size=n))
        u = torch.from_numpy(x).to(gpu)
        out = torch.full((1,), np.nan, dtype=torch.float64, device=gpu)
        print(f"no-alloc ordered sum n={n}", flush=True)
        rc = L.hk_ordered_sum_f64_noalloc(ctypes.c_void_p(u.data_ptr()), n, ctypes.c_void_p(out.data_ptr()),
                                          ctypes.c_void_p(stream))
        assert rc == 0, L.hk_last_error().decode()
        want = _sum_with_scratch(u, n, gpu)
        got = out.cpu().numpy()
        assert got.tobytes() == want.cpu().numpy().tobytes()
        assert got[0] == O.ordered_sum(x)


def test_the_no_alloc_sum_of_nothing_and_its_refusals(gpu):
    import torch

    from hawk_amd import _core
    L = _core.lib()
    out = torch.full((1,), np.nan, dtype=torch.float64, device=gpu)
    _core.ordered_sum_noalloc(0, 0, out.data_ptr())
    assert out.item() == 0.0 and not np.signbit(out.item())
    rc = L.hk_ordered_sum_f64_noalloc(None, -1, ctypes.c_void_p(out.data_ptr()), None)
    assert rc == 1 and "n must be >= 0" in L.hk_last_error().decode()
    rc = L.hk_ordered_sum_f64_noalloc(None, 5, ctypes.c_void_p(out.data_ptr()), None)
    assert rc == 1 and "u and out are required" in L.hk_last_error().decode()


def test_the_no_alloc_sum_on_a_side_stream_and_the_null_stream(gpu):
    """Its per-device scratch address is the same whatever stream the call
    names; in order on one stream, calls do not race."""
    import torch

    from hawk_amd import _core
    side = torch.cuda.Stream()
    x = rng(91).normal(size=300_007)
    u = torch.from_numpy(x).to(gpu)
    a = torch.zeros(1, dtype=torch.float64, device=gpu)
    b = torch.zeros(1, dtype=torch.float64, device=gpu)
    torch.cuda.synchronize()
    _core.ordered_sum_noalloc(u.data_ptr(), x.size, a.data_ptr(), side.cuda_stream)
    side.synchronize()
    _core.ordered_sum_noalloc(u.data_ptr(), x.size, b.data_ptr(), 0)
    torch.cuda.synchronize()
    assert a.item() == b.item() == O.ordered_sum(x)
