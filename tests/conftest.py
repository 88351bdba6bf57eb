import os
import subprocess
import sys
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parents[1]
sys.path.insert(0, str(ROOT))
sys.path.insert(0, str(ROOT / "tests"))


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (gfx950) GPU; runs the HIP library")


@pytest.fixture(scope="session")
def oracle():
    from oracle_lib import Oracle
    return Oracle.load()


@pytest.fixture(scope="session")
def qh():
    """The HIP library; GPU tests fail (not skip) when it is missing.  torch's
    wheel bundles its own HIP runtime (a second copy beside /opt/rocm's, which
    the library links): when a process uses both, torch must bring the GPU up
    first, so tests that mix them work whatever order they run in."""
    try:
        import torch
        if torch.cuda.is_available():
            torch.cuda.init()
    except ImportError:
        pass
    from saient_quartz_amd import lib
    return lib()
