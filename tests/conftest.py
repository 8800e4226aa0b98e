"""Shared test setup: markers, import paths, the package and GPU fixtures.

Tests marked ``gpu`` need a ROCm GPU and the built library; everything else
runs on the CPU (oracle pins, host logic, C-ABI exports)."""

from __future__ import annotations

import sys
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parents[1]
if str(ROOT) not in sys.path:
    sys.path.insert(0, str(ROOT))

import __graft_entry__  # noqa: E402

__graft_entry__.load_package()


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs a ROCm GPU (MI355X) and the built HIP library")


@pytest.fixture(scope="session")
def device():
    import torch

    if not torch.cuda.is_available():
        pytest.skip("no ROCm GPU visible")
    return torch.device("cuda:0")


@pytest.fixture(scope="session")
def ops():
    import importlib

    return importlib.import_module("taomate_h3_amd.ops")


@pytest.fixture(scope="session")
def oracle():
    from oracle import oracle as O

    O._load()
    return O
