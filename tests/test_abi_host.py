"""C-ABI library: loads without a GPU, exports every declared symbol, and its
host-side helpers (pack split, synthetic generator) agree with the oracle."""

from __future__ import annotations

import re
from pathlib import Path

import numpy as np
import pytest

from rtxllm_amd import formats as F
from rtxllm_amd import packs

REPO = Path(__file__).resolve().parent.parent


# entry points of the profiling build (build/librtxllm_timeline.so) only
PROFILING_HEADERS = ("timeline.h",)


def declared_functions(profiling: bool = False) -> list[str]:
    names = []
    for hdr in sorted((REPO / "include" / "rtxllm").glob("*.h")):
        if (hdr.name in PROFILING_HEADERS) != profiling:
            continue
        text = re.sub(r"/\*.*?\*/", "", hdr.read_text(), flags=re.S)
        names += re.findall(r"^\s*(?:hipError_t|int|uint32_t|size_t|void\s*\*|void)\s*(rtxllm_\w+)\s*\(", text,
                            flags=re.M)
    return names


def test_library_exports_every_declared_symbol(rlib):
    names = declared_functions()
    assert len(names) >= 30
    missing = [n for n in names if not hasattr(rlib, n)]
    assert not missing, missing


def test_profiling_build_exports_the_library_and_its_timeline():
    """build/librtxllm_timeline.so is the library plus the timeline entry
    points; the library proper does not export them."""
    import ctypes

    from rtxllm_amd import _lib

    prof = declared_functions(profiling=True)
    assert prof == ["rtxllm_timeline_read", "rtxllm_timeline_clear"]
    path = _lib.LIB_PATH.with_name("librtxllm_timeline.so")
    assert path.is_file(), path
    tl = ctypes.CDLL(str(path), mode=ctypes.RTLD_LOCAL)
    missing = [n for n in declared_functions() + prof if not hasattr(tl, n)]
    assert not missing, missing
    assert not any(hasattr(_lib.lib(), n) for n in prof)


def test_measurement_probe_is_not_in_the_library(rlib):
    """The streaming-read probe lives in the bench's own helper library."""
    from rtxllm_amd import _lib

    assert not hasattr(rlib, "rtxllm_stream_read")
    assert "rtxllm_stream_read" not in declared_functions()
    assert hasattr(_lib.probe_lib(), "rtxllm_stream_read")


def test_binding_covers_declared_symbols():
    from rtxllm_amd import _lib

    bound = set(_lib.exported_names())
    assert set(declared_functions()) <= bound | set(getattr(_lib, "_EXTRA_BOUND", ())), (
        set(declared_functions()) - bound)


@pytest.mark.parametrize("fmt", F.SPLIT_FORMATS)
def test_product_split_pack_matches_oracle(orc, fmt):
    raw = packs.synth_raw(F.Q4K_RAW, 8, 2048, seed=99)
    p, m = packs.q4k_split(fmt, raw)
    op, om = orc.q4k_split(fmt, raw, F.META_BYTES[fmt])
    assert np.array_equal(p, op) and np.array_equal(m, om)


def test_synth_deterministic_and_thread_independent():
    a = packs.synth_raw(F.IQ3S, 64, 4096, seed=5, threads=1)
    b = packs.synth_raw(F.IQ3S, 64, 4096, seed=5, threads=7)
    c = packs.synth_raw(F.IQ3S, 64, 4096, seed=6, threads=1)
    assert np.array_equal(a, b) and not np.array_equal(a, c)
    x1 = packs.normal_f32(1, 10001, threads=1)
    x2 = packs.normal_f32(1, 10001, threads=5)
    assert np.array_equal(x1, x2)


def test_synth_field_distributions():
    rows, cols = 256, 4096
    raw = packs.synth_raw(F.Q4K_RAW, rows, cols, seed=0x5EED0000).reshape(-1, 144)
    d = raw[:, 0:2].copy().view(np.float16).astype(np.float32).ravel()
    dmin = raw[:, 2:4].copy().view(np.float16).astype(np.float32).ravel()
    for v in (d, dmin):
        assert v.min() >= np.float16(1e-4) and v.max() <= np.float16(2e-3)
        assert abs(float(v.mean()) - 1.05e-3) < 2e-5
    nib = np.concatenate([raw[:, 16:] & 15, raw[:, 16:] >> 4]).ravel()
    counts = np.bincount(nib, minlength=16)
    assert counts.min() > 0.95 * nib.size / 16
    x = packs.normal_f32(7, 200_000)
    assert abs(float(x.mean())) < 0.01 and abs(float(x.std()) - 1.0) < 0.01
