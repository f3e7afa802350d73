"""Shared fixtures: the ``gpu`` marker, the built unit of benchmark kernels,
and the seeded synthetic inputs of the five configurations."""

from __future__ import annotations

import json
import sys
from functools import lru_cache
from pathlib import Path

import numpy as np
import pytest

ROOT = Path(__file__).resolve().parent.parent
sys.path.insert(0, str(ROOT))
sys.path.insert(0, str(Path(__file__).resolve().parent))


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs a real MI355X (runs the hip target)")


def _gpu_available() -> bool:
    try:
        import torch
        return bool(torch.cuda.is_available())
    except Exception:
        return False


@pytest.fixture(scope="session")
def gpu():
    if not _gpu_available():
        pytest.fail("this test is marked gpu and needs a ROCm device (run with -m 'not gpu' elsewhere)")
    import torch
    return torch.device("cuda:0")


@pytest.fixture(scope="session")
def unit(tmp_path_factory):
    """Every example kernel built for the hip target (float64), once."""
    import hawk_amd as hawk
    from hawk_amd import examples as E

    directory = tmp_path_factory.mktemp("unit64")
    hawk.build(list(E.ALL.values()), directory)
    return directory


@pytest.fixture(scope="session")
def unit32(tmp_path_factory):
    import hawk_amd as hawk
    from hawk_amd import examples as E

    directory = tmp_path_factory.mktemp("unit32")
    hawk.build(list(E.FLOAT32.values()), directory, mode="float32")
    return directory


@pytest.fixture(scope="session")
def unit_banded(tmp_path_factory):
    """The banded example kernels, built in the banded mode."""
    import hawk_amd as hawk
    from hawk_amd import examples as E

    directory = tmp_path_factory.mktemp("unit_banded")
    hawk.build(list(E.BANDED.values()), directory, mode="banded")
    return directory


@lru_cache(maxsize=None)
def _golden() -> dict:
    return json.loads((Path(__file__).resolve().parent / "golden" / "known_answers.json").read_text())


def golden(name: str) -> dict:
    """One entry of tests/golden/known_answers.json: known answers and case
    lists transcribed from the reference's README and tests (each entry cites
    its source file:line)."""
    return _golden()[name]


def rng(seed: int):
    return np.random.default_rng(seed)


def ulp_diff(a: np.ndarray, b: np.ndarray) -> np.ndarray:
    """|a - b| in units in the last place of b (float64)."""
    a = np.asarray(a, dtype=np.float64)
    b = np.asarray(b, dtype=np.float64)
    return np.abs(a - b) / np.spacing(np.maximum(np.abs(b), np.finfo(np.float64).tiny))


def within_contract(got: np.ndarray, want: np.ndarray, ulps: float = 4.0, rel: float = 1e-13) -> np.ndarray:
    """The fp64 parity bar of the north star: within 4 ulp OR 1e-13 relative."""
    got = np.asarray(got, dtype=np.float64)
    want = np.asarray(want, dtype=np.float64)
    same = (got == want) | (np.isnan(got) & np.isnan(want))
    close_ulp = ulp_diff(got, want) <= ulps
    close_rel = np.abs(got - want) <= rel * np.abs(want)
    return same | close_ulp | close_rel
