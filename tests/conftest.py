"""pytest setup: import paths, the `gpu` marker and shared comparison helpers."""
from __future__ import annotations

import os
import sys
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parents[1]
PKG = ROOT / "joyai-video-edit_amd"
for p in (str(PKG), str(ROOT)):
    if p not in sys.path:
        sys.path.insert(0, p)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (gfx950) and the built libraries")


@pytest.fixture(scope="session")
def dev():
    import torch
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    return torch.device("cuda", 0)


@pytest.fixture(scope="session")
def abi():
    """The C ABI, loaded through ctypes; fails (not skips) if it was not built."""
    from joyomni_ops import _abi
    return _abi


@pytest.fixture(scope="session")
def stream_handle(dev):
    import torch
    return torch.cuda.current_stream(dev).cuda_stream
