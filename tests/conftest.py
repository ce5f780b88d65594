import sys
from pathlib import Path

import pytest

REPO = Path(__file__).resolve().parent.parent
PKG = REPO / "local-ai-gpu-acceleration_amd"
for p in (REPO, PKG):
    if str(p) not in sys.path:
        sys.path.insert(0, str(p))


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (gfx950) GPU")
    config.addinivalue_line("markers", "slow: multi-second CPU oracle runs")


@pytest.fixture(scope="session")
def orc():
    from oracle import binding

    binding.lib()
    return binding


@pytest.fixture(scope="session")
def rlib():
    from rtxllm_amd import _lib

    return _lib.lib()
