"""Seeded synthetic resident packs in host memory (numpy), built by the C-ABI's
host-side generator so every consumer sees the same bytes."""

from __future__ import annotations

import ctypes
from dataclasses import dataclass

import numpy as np

from . import formats as F
from ._lib import lib

D_LO, D_HI = 1e-4, 2e-3


def _ptr(a: np.ndarray) -> int:
    return a.ctypes.data_as(ctypes.c_void_p).value


@dataclass
class Pack:
    fmt: int
    rows: int
    cols: int
    payload: np.ndarray  # uint8
    meta: np.ndarray | None  # uint8 or None

    @property
    def blocks(self) -> int:
        return self.rows * (self.cols // F.BLOCK_VALUES)


def synth_raw(fmt: int, rows: int, cols: int, seed: int, d_lo: float = D_LO, d_hi: float = D_HI,
              threads: int = 0) -> np.ndarray:
    if cols % F.BLOCK_VALUES:
        raise ValueError("cols must be a multiple of 256")
    n = rows * (cols // F.BLOCK_VALUES)
    out = np.empty(n * F.PAYLOAD_BYTES[fmt], dtype=np.uint8)
    rc = lib().rtxllm_synth_raw_blocks(fmt, seed, n, d_lo, d_hi, _ptr(out), threads)
    if rc != 0:
        raise ValueError(f"rtxllm_synth_raw_blocks rejected format {fmt}")
    return out


def q4k_split(fmt: int, raw: np.ndarray) -> tuple[np.ndarray, np.ndarray]:
    n = raw.size // 144
    payload = np.empty(n * 128, dtype=np.uint8)
    meta = np.empty(n * F.META_BYTES[fmt], dtype=np.uint8)
    if lib().rtxllm_q4k_split_pack(fmt, _ptr(raw), n, _ptr(payload), _ptr(meta)) != 0:
        raise ValueError(f"rtxllm_q4k_split_pack rejected format {fmt}")
    return payload, meta


def predecoded_pairs(raw: np.ndarray) -> np.ndarray:
    """f32 (d*sc, dmin*m) x 8 per raw Q4_K block, as uint8 bytes."""
    return q4k_split(F.Q4K_SPLIT_PREDECODED, raw)[1]


def make_pack(fmt: int, rows: int, cols: int, seed: int, threads: int = 0) -> Pack:
    if fmt in F.SPLIT_FORMATS:
        raw = synth_raw(F.Q4K_RAW, rows, cols, seed, threads=threads)
        payload, meta = q4k_split(fmt, raw)
        return Pack(fmt, rows, cols, payload, meta)
    if fmt == F.Q4K_RAW_PREDECODED:
        raw = synth_raw(F.Q4K_RAW, rows, cols, seed, threads=threads)
        return Pack(fmt, rows, cols, raw, predecoded_pairs(raw))
    return Pack(fmt, rows, cols, synth_raw(fmt, rows, cols, seed, threads=threads), None)


def normal_f32(seed: int, n: int, mean: float = 0.0, std: float = 1.0, threads: int = 0) -> np.ndarray:
    out = np.empty(n, dtype=np.float32)
    lib().rtxllm_synth_normal_f32(seed, n, mean, std, _ptr(out), threads)
    return out


def normal_f16_bits(seed: int, n: int, mean: float = 0.0, std: float = 1.0, threads: int = 0) -> np.ndarray:
    out = np.empty(n, dtype=np.uint16)
    lib().rtxllm_synth_normal_f16(seed, n, mean, std, _ptr(out), threads)
    return out
