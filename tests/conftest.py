"""Shared test configuration.

Markers:
  gpu - needs an MI355X (or any gfx950) visible to torch; run with `-m gpu`.
        Without a GPU these are skipped, so `-m "not gpu"` stays green on a
        CPU-only host, as the reference's `cuda` marker does
        (tests/python/conftest.py:18-25).
"""

from __future__ import annotations

import os
import sys
from pathlib import Path

import numpy as np
import pytest
import torch

ROOT = Path(__file__).resolve().parents[1]
GOLDEN = ROOT / "tests" / "golden"
if str(ROOT) not in sys.path:
    sys.path.insert(0, str(ROOT))

# Operators must never silently fall back to PyTorch on a GPU during tests.
os.environ.setdefault("CUDAFORGE_STRICT", "1")


def pytest_configure(config: pytest.Config) -> None:
    config.addinivalue_line("markers", "gpu: needs a gfx950 GPU visible to torch")


def pytest_collection_modifyitems(config: pytest.Config, items: list[pytest.Item]) -> None:
    if torch.cuda.is_available():
        return
    skip = pytest.mark.skip(reason="no GPU visible to torch on this host")
    for item in items:
        if "gpu" in item.keywords:
            item.add_marker(skip)


@pytest.fixture(autouse=True)
def deterministic_seed() -> None:
    torch.manual_seed(0)


def load_golden(name: str) -> dict[str, dict[str, np.ndarray]]:
    """{case: {field: array}} from tests/golden/<name>.npz (keys 'case__field')."""
    cases: dict[str, dict[str, np.ndarray]] = {}
    with np.load(GOLDEN / name, allow_pickle=False) as data:
        for key in data.files:
            case, field = key.split("__", 1)
            cases.setdefault(case, {})[field] = data[key]
    return cases


def rng(seed: int) -> np.random.Generator:
    return np.random.Generator(np.random.PCG64(seed))
