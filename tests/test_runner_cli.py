"""The decode-step command's argument handling, on the CPU (no GPU call is
made before the arguments are accepted): unknown or malformed arguments exit
1 with the usage line, --help exits 0 (the reference runner's error exit)."""

from __future__ import annotations

import subprocess

import pytest

from rtxllm_amd._lib import PKG_ROOT

RUNNER = PKG_ROOT / "build" / "rtxllm_decode_runner"


@pytest.mark.parametrize("args,message", [
    (["--bogus"], "unknown argument --bogus"),
    (["--batch", "9"], "--batch must be 1..8"),
    (["--batch", "0"], "--batch must be 1..8"),
    (["--steps"], "--steps needs a value"),
    (["--max-ctx", "99999999999"], "out of range"),
])
def test_runner_rejects_bad_arguments(args, message):
    r = subprocess.run([str(RUNNER)] + args, capture_output=True, text=True, timeout=60)
    assert r.returncode == 1 and message in r.stderr and "usage: rtxllm_decode_runner" in r.stderr
    assert r.stdout == ""


def test_runner_help():
    r = subprocess.run([str(RUNNER), "--help"], capture_output=True, text=True, timeout=60)
    assert r.returncode == 0 and "usage: rtxllm_decode_runner" in r.stderr
