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


def references_staged(orc, pack, x):
    """(fp32 sequential, float64, float64 on the staged x) products of the pack
    with x: the last multiplies the batch-1 kernels' 22-bit staged activation
    (xq.h: one power-of-two scale per 16-value group) exactly."""
    y32, y64 = references(orc, pack, x)
    of, pl, mt = oracle_args(pack)
    return y32, y64, orc.matvec_staged_f64(of, pl, mt, x, pack.rows, pack.cols, THREADS)


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


def batch_staged(x: np.ndarray) -> np.ndarray:
    """The activation values the batched matrix-core matvec multiplies: per
    256-value block, e from max|x| = f 2^e (f in [0.5, 1)), t = x 2^-e in
    fp32, hi = fp16(t), lo = fp16(t - hi) (round to nearest even, fp16
    subnormals kept), value (hi + lo) 2^e. Returned as float32, which holds
    every such value exactly (asserted)."""
    xb = np.asarray(x, np.float32).reshape(-1, 256)
    m = np.max(np.abs(xb), axis=1).astype(np.float64)
    e = np.where((m > 0) & np.isfinite(m), np.frexp(m)[1], 0).astype(np.int64)
    t = np.ldexp(xb.astype(np.float64), -e[:, None]).astype(np.float32)  # exact: a power-of-two scaling
    hi = t.astype(np.float16)
    lo = (t - hi.astype(np.float32)).astype(np.float16)
    v = np.ldexp(hi.astype(np.float64) + lo.astype(np.float64), e[:, None])
    out = v.astype(np.float32)
    assert np.array_equal(out.astype(np.float64), v), "staged value not exact in fp32"
    return out.reshape(-1)


def gate_staged(label: str, y: np.ndarray, y32: np.ndarray, y64: np.ndarray, yst64: np.ndarray) -> tuple[float, float]:
    """Gate of a kernel that rounds its activation once on input (the batch-1
    kernels keep 22 bits per 16-value group, the batched matrix-core matvec
    ~22 bits per 256-value block, so a group whose values span many decades
    loses the small ones' low bits; fp32 keeps 24 bits per value). On
    heavy-tailed activations that rounding alone can exceed twice the fp32
    path's per-element error. yst64 is the float64 product with the rounded
    activation.
      * the kernel's arithmetic on its rounded input: both measures of y
        against yst64 at most GATE times the fp32-sequential path's against y64;
      * normwise against y64 at most GATE times the fp32-sequential path's;
      * per element against y64 at most GATE times the larger of the
        fp32-sequential path's and the input rounding's own (yst64 against y64).
    Returns (normwise, per-element) of y against y64."""
    e_gpu, e_f32 = err64(y, y64), err64(y32, y64)
    p_gpu, p_f32, p_st = elem64(y, y64), elem64(y32, y64), elem64(yst64, y64)
    e_ar, p_ar = err64(y, yst64), elem64(y, yst64)
    print(f"{label}: normwise gpu {e_gpu:.3e} fp32-seq {e_f32:.3e} arith {e_ar:.3e}; per-element (floor {FLOOR:g}) "
          f"gpu {p_gpu:.3e} fp32-seq {p_f32:.3e} staging {p_st:.3e} arith {p_ar:.3e}")
    assert e_ar <= GATE * e_f32, (label, "normwise arithmetic", e_ar, e_f32)
    assert p_ar <= GATE * p_f32, (label, "per-element arithmetic", p_ar, p_f32)
    assert e_gpu <= GATE * e_f32, (label, "normwise", e_gpu, e_f32)
    assert p_gpu <= GATE * max(p_f32, p_st), (label, "per-element", p_gpu, p_f32, p_st)
    return e_gpu, p_gpu
