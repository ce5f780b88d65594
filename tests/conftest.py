import shutil
import subprocess
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


def pytest_terminal_summary(terminalreporter):
    """Greedy tokens that differed from the oracle's at a near-tie (tests/token_rule.py)."""
    mod = sys.modules.get("token_rule")
    if mod is None:
        return
    rows = mod.DISAGREEMENTS
    terminalreporter.write_line(f"token disagreements at near-ties: {len(rows)}")
    for label, tok, ref, gap in rows:
        terminalreporter.write_line(f"  {label}: token {tok}, oracle {ref}, relative gap {gap:.3e}")


@pytest.fixture(scope="session")
def orc():
    from oracle import binding

    binding.lib()
    return binding


@pytest.fixture(scope="session")
def rlib():
    from rtxllm_amd import _lib

    return _lib.lib()


@pytest.fixture(scope="session")
def selftest(tmp_path_factory) -> Path:
    """The native runtime self-test (tests/native/runtime_selftest.cpp with the
    library's pack-manifest loaders), built here with g++."""
    gxx = shutil.which("g++")
    if gxx is None:
        pytest.skip("g++ not available")
    exe = tmp_path_factory.mktemp("native") / "runtime_selftest"
    subprocess.run([gxx, "-std=c++17", "-O1", "-Wall", "-Werror", "-I", str(REPO / "include"),
                    str(REPO / "tests" / "native" / "runtime_selftest.cpp"),
                    str(PKG / "csrc" / "pack_manifest.cpp"), "-o", str(exe)],
                   check=True, capture_output=True, timeout=300)
    return exe
