import os
import sys
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parent.parent
PKG = ROOT / "paged-batch-engine_amd"
for p in (str(ROOT), str(PKG)):
    if p not in sys.path:
        sys.path.insert(0, p)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (gfx950) GPU")
    try:  # property tests draw the same examples on every run, and keep no database
        from hypothesis import settings
        settings.register_profile("repeatable", derandomize=True, database=None)
        settings.load_profile("repeatable")
    except ImportError:
        pass


@pytest.fixture(scope="session")
def torch_cuda():
    import torch
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    return torch


def say(msg: str) -> None:
    """Names the case before a GPU step so a crash log identifies it."""
    print(f"[case] {msg}", flush=True)
