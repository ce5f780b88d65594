"""The decode runner's VRAM arena (rtxllm::VramSuperallocator in the library,
the reference allocator's interface, vram_superallocator.h:25-53), through
its native self-test build/rtxllm_arena_selftest (tests/native/
arena_selftest.cpp, built by the library's Makefile).

On the CPU: spec validation with the reference's exception types and
messages, the empty arena's lookups, and a failed allocation (no device)
leaving the arena empty. On the GPU: the 256-byte layout, lookup by name
(a repeated name resolves to its first spec), moves, reset and reset_async,
and a rejected spec list leaving a live pool unchanged."""

from __future__ import annotations

import subprocess
from pathlib import Path

import pytest

REPO = Path(__file__).resolve().parent.parent
EXE = REPO / "local-ai-gpu-acceleration_amd" / "build" / "rtxllm_arena_selftest"


def run(*args: str) -> subprocess.CompletedProcess:
    if not EXE.is_file():
        pytest.fail(f"{EXE} is missing: build the library (make -C local-ai-gpu-acceleration_amd)")
    r = subprocess.run([str(EXE), *args], capture_output=True, text=True, timeout=120)
    print(r.stdout)
    return r


def test_arena_selftest_cpu():
    r = run("--cpu")
    assert r.returncode == 0, r.stdout + r.stderr
    assert "FAIL" not in r.stdout and r.stdout.count("ok  ") >= 11


@pytest.mark.gpu
def test_arena_selftest_gpu():
    r = run("--gpu")
    assert r.returncode == 0, r.stdout + r.stderr
    assert "FAIL" not in r.stdout and r.stdout.count("ok  ") >= 25
