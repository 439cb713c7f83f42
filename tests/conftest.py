"""Shared pytest setup.  GPU tests are marked ``gpu`` and need an MI355X:
on a box without one they fail (the native path has no CPU fallback)."""

from __future__ import annotations

import sys
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parents[1]
if str(ROOT) not in sys.path:
    sys.path.insert(0, str(ROOT))


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (gfx950) GPU and the built libkudacuda.so")


@pytest.fixture(scope="session")
def torch_gpu():
    import torch

    assert torch.cuda.is_available(), "GPU test run without a visible GPU"
    return torch


@pytest.fixture(scope="session")
def native(torch_gpu):
    from kudacuda_amd._native import Native

    n = Native(0)
    yield n
    n.close()


@pytest.fixture(scope="session")
def stream(torch_gpu):
    return torch_gpu.cuda.Stream(device="cuda:0")
