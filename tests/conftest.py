"""Shared pytest setup: the `gpu` marker, import paths and device fixtures."""
from __future__ import annotations

import sys
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parents[1]
for p in (ROOT / "qwen38-metal_amd", ROOT / "oracle", ROOT):
    if str(p) not in sys.path:
        sys.path.insert(0, str(p))


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (runs the HIP kernels)")


@pytest.fixture(scope="session")
def torch_dev():
    import torch
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    return torch.device("cuda:0")


@pytest.fixture(scope="session")
def rt(torch_dev):
    import torch
    import qm38
    r = qm38.Runtime(0)
    r.set_stream(torch.cuda.current_stream())
    yield r
    torch.cuda.synchronize()
    r.close()
