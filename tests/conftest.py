"""Shared pytest setup.

Markers:
  gpu -- needs a ROCm device (MI355X); run with ``-m gpu`` on the GPU box.

The repository root is put on sys.path so ``oracle`` (the parity checkers)
and ``torchmatch_amd`` import from the tree, and ``tests/`` so the shared
helpers (``sk_parity``) import by name.
"""

from __future__ import annotations

import sys
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parents[1]
for _p in (ROOT, ROOT / "tests"):
    if str(_p) not in sys.path:
        sys.path.insert(0, str(_p))


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs a ROCm GPU (gfx950)")


@pytest.fixture(scope="session")
def device():
    import torch

    if not torch.cuda.is_available():
        pytest.skip("no ROCm device visible")
    return torch.device("cuda:0")
