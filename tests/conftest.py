"""Shared pytest configuration.

Markers: ``gpu`` — needs an MI355X (run with ``-m gpu``); everything else runs
on the CPU (``-m "not gpu"``).  The oracle package (test infrastructure) and
the product package are imported from the repository root.
"""
import sys
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parent.parent
if str(ROOT) not in sys.path:
    sys.path.insert(0, str(ROOT))


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: test needs a gfx950 GPU and the built HIP library")


@pytest.fixture(scope="session")
def port():
    import oracle
    return oracle.port()


@pytest.fixture(scope="session")
def ref():
    import oracle
    r = oracle.ref()
    if r is None:
        pytest.skip("oracle/_ref (the compiled reference) is not built here")
    return r


@pytest.fixture(scope="session")
def hs():
    """The product package on a GPU; fails (never skips) when either is missing."""
    import torch
    assert torch.cuda.is_available(), "gpu test started without a visible GPU"
    import hillserve_amd
    hillserve_amd.lib()
    return hillserve_amd
