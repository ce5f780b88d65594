"""Shared pieces of the float64 precision gates (GPU tests).

Two error measures against the float64 product y64 (the oracle's
orc_matvec_f64, a closed form over the bit-exact dequantised weights):
  * normwise   err(y)  = max_i |y_i - y64_i| / max_i |y64_i|;
  * per element elem(y) = max_i |y_i - y64_i| / max(|y64_i|, FLOOR max_j |y64_j|),
    the relative error of every output with a floor, so outputs near zero
    (where a plain relative error means nothing) are measured against
    FLOOR of the largest output instead.
A GPU result passes when each measure is at most GATE times the same measure
of the reference's own fp32 path: the oracle's sequential fp32 accumulation
(main.cpp:1261-1309), run on the same bytes and activation."""

from __future__ import annotations

import numpy as np

from rtxllm_amd import formats as F
from rtxllm_amd import packs

GATE = 2.0  # gpu error / fp32-sequential error, both against the float64 product
FLOOR = 1e-3  # of max|y64|: the per-element measure's floor
THREADS = 16


def err64(y: np.ndarray, y64: np.ndarray) -> float:
    return float(np.max(np.abs(y.astype(np.float64) - y64)) / np.max(np.abs(y64)))


def elem64(y: np.ndarray, y64: np.ndarray, floor: float = FLOOR) -> float:
    den = np.maximum(np.abs(y64), floor * np.max(np.abs(y64)))
    return float(np.max(np.abs(y.astype(np.float64) - y64) / den))


def oracle_args(pack: packs.Pack):
    """The oracle's format, payload and metadata for a pack (unit layouts map
    back to their GGUF blocks, raw + predecoded to split-predecoded)."""
    if pack.fmt == F.Q4K_RAW_PREDECODED:
        return F.Q4K_SPLIT_PREDECODED, pack.payload.reshape(-1, 144)[:, 16:].copy().reshape(-1), pack.meta
    if pack.fmt == F.IQ2S_UNITS:
        return F.IQ2S, packs.iq2s_from_units(pack.payload), None
    if pack.fmt == F.IQ3S_UNITS:
        return F.IQ3S, packs.iq3s_from_units(pack.payload), None
    return pack.fmt, pack.payload, pack.meta


def references(orc, pack, x):
    """(fp32 sequential, float64) products of the pack with x."""
    of, pl, mt = oracle_args(pack)
    y32 = orc.matvec_f32(of, pl, mt, x, pack.rows, pack.cols, THREADS)
    y64 = orc.matvec_f64(of, pl, mt, x, pack.rows, pack.cols, THREADS)
    return y32, y64


def activation(kind: str, cols: int, seed: int) -> np.ndarray:
    x = packs.normal_f32(seed, cols)
    if kind == "outlier":
        # one +-1e3 value per 16-value group, at a seeded position
        rng = np.random.default_rng(seed)
        pos = np.arange(0, cols, 16) + rng.integers(0, 16, cols // 16)
        x[pos] = np.where(rng.random(cols // 16) < 0.5, -1e3, 1e3).astype(np.float32)
    elif kind == "heavy":
        # log-normal magnitudes: values spread over ~8 decades
        x = (x * np.exp(3.0 * packs.normal_f32(seed + 1, cols))).astype(np.float32)
    return x


KINDS = ("normal", "outlier", "heavy")


def gate(label: str, y: np.ndarray, y32: np.ndarray, y64: np.ndarray) -> tuple[float, float]:
    """Assert both measures against the fp32-sequential path; returns (normwise, per-element) of y."""
    e_gpu, e_f32 = err64(y, y64), err64(y32, y64)
    p_gpu, p_f32 = elem64(y, y64), elem64(y32, y64)
    print(f"{label}: normwise gpu {e_gpu:.3e} fp32-seq {e_f32:.3e}; per-element (floor {FLOOR:g}) "
          f"gpu {p_gpu:.3e} fp32-seq {p_f32:.3e}")
    assert e_gpu <= GATE * e_f32, (label, "normwise", e_gpu, e_f32)
    assert p_gpu <= GATE * p_f32, (label, "per-element", p_gpu, p_f32)
    return e_gpu, p_gpu
