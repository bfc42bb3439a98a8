"""Shared pytest setup: the ``gpu`` marker and import paths.

CPU tests (``-m "not gpu"``) cover the oracle against the golden fixtures, the
host-side logic and the C-ABI library's exports.  ``@pytest.mark.gpu`` tests
are the parity tests proper; they need an MI355X and the built ``libqmoe.so``.
"""

import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
PKG_DIR = os.path.join(ROOT, "nki-moe-7013_amd")
for p in (ROOT, PKG_DIR):
    if p not in sys.path:
        sys.path.insert(0, p)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X GPU and the built HIP library")


def gpu_available() -> bool:
    try:
        import torch

        return torch.cuda.is_available()
    except Exception:
        return False


@pytest.fixture(scope="session")
def dev():
    import torch

    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    return torch.device("cuda:0")
