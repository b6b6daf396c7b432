"""Shared test setup.

* ``gpu`` marks a test that runs the HIP kernels on a ROCm GPU. Without a GPU
  such tests are skipped; with one, a missing library is a failure (the
  product has no CPU fallback).
* The package lives under ``gpt2-harness_amd/`` and the oracle under
  ``oracle/``; both are put on ``sys.path`` here.
"""

from __future__ import annotations

import json
import sys
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parents[1]
for p in (ROOT / "gpt2-harness_amd", ROOT):
    if str(p) not in sys.path:
        sys.path.insert(0, str(p))

GOLDEN = ROOT / "tests" / "golden"


def pytest_configure(config: pytest.Config) -> None:
    config.addinivalue_line("markers", "gpu: needs a ROCm GPU (MI355X); runs the HIP kernels")


def pytest_collection_modifyitems(config: pytest.Config, items: list[pytest.Item]) -> None:
    import torch

    if torch.cuda.is_available():
        return
    skip = pytest.mark.skip(reason="no ROCm GPU visible")
    for item in items:
        if "gpu" in item.keywords:
            item.add_marker(skip)


@pytest.fixture(scope="session")
def known_answers() -> dict:
    return json.loads((GOLDEN / "quant_known_answers.json").read_text())


@pytest.fixture(scope="session")
def reference_decode() -> dict:
    return json.loads((GOLDEN / "reference_decode.json").read_text())


@pytest.fixture(scope="session")
def c_oracle():
    from oracle import quant

    return quant.c_oracle()


@pytest.fixture(scope="session")
def dev():
    import torch

    return torch.device("cuda:0")
