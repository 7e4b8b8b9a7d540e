"""Shared pytest setup.

* Registers the ``gpu`` marker: every test that needs an MI355X is marked
  ``@pytest.mark.gpu``; everything else runs on a CPU-only machine.
* Puts the repository root on ``sys.path`` so ``oracle`` (the CPU checker) and
  ``tests.golden_io`` import, and loads the product package from
  ``mini-cuda-kernel-engine_amd/`` under the module name ``mcke_amd``.
"""
from __future__ import annotations

import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)

from __graft_entry__ import load_package  # noqa: E402


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (gfx950) GPU")


@pytest.fixture(scope="session")
def mcke():
    """The product package (ctypes over libmcke_amd.so)."""
    return load_package()


@pytest.fixture(scope="session")
def orc():
    import oracle

    oracle.lib()
    return oracle


@pytest.fixture(scope="session")
def gpu(mcke):
    """A device context for GPU tests: fails loudly if the HIP library or the
    GPU is missing (no CPU fallback exists)."""
    mcke.require_gpu()
    return mcke
