"""Shared pytest set-up: the ``gpu`` marker, package import and GPU fixtures."""

from __future__ import annotations

import sys
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parents[1]
if str(ROOT) not in sys.path:
    sys.path.insert(0, str(ROOT))

from __graft_entry__ import load_package  # noqa: E402

load_package()


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (runs the HIP library on cuda:0)")


def _gpu_available() -> bool:
    try:
        import torch

        return torch.cuda.is_available()
    except Exception:
        return False


@pytest.fixture(scope="session")
def gpu_ctx():
    """One device context for the whole GPU session (cuda:0)."""
    if not _gpu_available():
        pytest.skip("no GPU")
    from raon_npu_amd.device import Context

    ctx = Context(0)
    yield ctx
    ctx.close()
