"""Shared test setup: repo root on sys.path, the `gpu` marker, and GPU
fixtures.  Tests marked `gpu` need an MI355X; the rest run on any CPU."""
from __future__ import annotations

import sys
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parents[1]
if str(ROOT) not in sys.path:
    sys.path.insert(0, str(ROOT))


def pytest_configure(config):
    config.addinivalue_line(
        "markers", "gpu: needs a ROCm GPU (MI355X); run with -m gpu")


@pytest.fixture(scope="session")
def cuda():
    import torch
    if not torch.cuda.is_available():
        pytest.skip("no GPU visible")
    return torch.device("cuda:0")


@pytest.fixture(scope="session")
def ext4(cuda):
    from cudalab_amd.build import build
    return build("int4gemv")


@pytest.fixture(scope="session")
def ext8(cuda):
    from cudalab_amd.build import build
    return build("qgemv")


def announce(msg: str) -> None:
    """Print (and flush) what a GPU step is about to run."""
    print(f"[case] {msg}", flush=True)
