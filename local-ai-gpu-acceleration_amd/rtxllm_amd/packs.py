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


def iq2s_unit_order(n_blocks: int) -> np.ndarray:
    """Index array P with units[P] = raw for n_blocks GGUF IQ2_S blocks (82 B:
    d, qs[32], signs[32], qh[8], scales[8]) in the IQ2S_UNITS layout: per unit
    k of block b, qs[4k..4k+3] and signs[4k..4k+3] at 64 b + 8 k, (qh[k],
    scales[k]) at 64 N + 16 b + 2 k, d at 80 N + 2 b."""
    n = int(n_blocks)
    b = np.arange(n, dtype=np.int64)[:, None]
    i = np.arange(82, dtype=np.int64)[None, :]
    k_qs, j_qs = (i - 2) // 4, (i - 2) % 4
    k_sg, j_sg = (i - 34) // 4, (i - 34) % 4
    pos = np.where(i < 2, 80 * n + 2 * b + i,
          np.where(i < 34, 64 * b + 8 * k_qs + j_qs,
          np.where(i < 66, 64 * b + 8 * k_sg + 4 + j_sg,
          np.where(i < 74, 64 * n + 16 * b + 2 * (i - 66), 64 * n + 16 * b + 2 * (i - 74) + 1))))
    return pos.reshape(-1)


def iq2s_units(raw: np.ndarray) -> np.ndarray:
    """GGUF IQ2_S blocks -> the IQ2S_UNITS layout (rtxllm_iq2s_units_pack on the host)."""
    raw = np.ascontiguousarray(raw, np.uint8).reshape(-1)
    out = np.empty_like(raw)
    out[iq2s_unit_order(raw.size // 82)] = raw
    return out


def iq2s_from_units(units: np.ndarray) -> np.ndarray:
    units = np.ascontiguousarray(units, np.uint8).reshape(-1)
    return units[iq2s_unit_order(units.size // 82)]


def iq3s_unit_order(n_blocks: int) -> np.ndarray:
    """Index array P with units[P] = raw for n_blocks GGUF IQ3_S blocks (110 B:
    d, qs[64], qh[8], signs[32], scales[4]) in the IQ3S_UNITS layout (114 B per
    block): per unit k of block b, qs[8k..8k+7] and signs[4k..4k+3] at
    96 b + 12 k, (qh[k], scales[k / 2]) at 96 N + 16 b + 2 k, d at 112 N + 2 b;
    a scale byte's place here is its copy in the even unit of its pair."""
    n = int(n_blocks)
    b = np.arange(n, dtype=np.int64)[:, None]
    i = np.arange(110, dtype=np.int64)[None, :]
    pos = np.where(i < 2, 112 * n + 2 * b + i,
          np.where(i < 66, 96 * b + 12 * ((i - 2) // 8) + (i - 2) % 8,
          np.where(i < 74, 96 * n + 16 * b + 2 * (i - 66),
          np.where(i < 106, 96 * b + 12 * ((i - 74) // 4) + 8 + (i - 74) % 4,
                   96 * n + 16 * b + 4 * (i - 106) + 1))))
    return pos.reshape(-1)


def iq3s_units(raw: np.ndarray) -> np.ndarray:
    """GGUF IQ3_S blocks -> the IQ3S_UNITS layout (rtxllm_iq3s_units_pack on the host)."""
    raw = np.ascontiguousarray(raw, np.uint8).reshape(-1)
    n = raw.size // 110
    out = np.empty(114 * n, np.uint8)
    order = iq3s_unit_order(n)
    out[order] = raw
    scales = order.reshape(n, 110)[:, 106:].reshape(-1)  # even-unit copies; the odd unit's is 2 bytes on
    out[scales + 2] = raw.reshape(n, 110)[:, 106:].reshape(-1)
    return out


def iq3s_from_units(units: np.ndarray) -> np.ndarray:
    units = np.ascontiguousarray(units, np.uint8).reshape(-1)
    return units[iq3s_unit_order(units.size // 114)]


def make_pack(fmt: int, rows: int, cols: int, seed: int, threads: int = 0) -> Pack:
    if fmt in F.SPLIT_FORMATS:
        raw = synth_raw(F.Q4K_RAW, rows, cols, seed, threads=threads)
        payload, meta = q4k_split(fmt, raw)
        return Pack(fmt, rows, cols, payload, meta)
    if fmt == F.Q4K_RAW_PREDECODED:
        raw = synth_raw(F.Q4K_RAW, rows, cols, seed, threads=threads)
        return Pack(fmt, rows, cols, raw, predecoded_pairs(raw))
    if fmt == F.IQ2S_UNITS:
        return Pack(fmt, rows, cols, iq2s_units(synth_raw(F.IQ2S, rows, cols, seed, threads=threads)), None)
    if fmt == F.IQ3S_UNITS:
        return Pack(fmt, rows, cols, iq3s_units(synth_raw(F.IQ3S, rows, cols, seed, threads=threads)), None)
    return Pack(fmt, rows, cols, synth_raw(fmt, rows, cols, seed, threads=threads), None)


def normal_f32(seed: int, n: int, mean: float = 0.0, std: float = 1.0, threads: int = 0) -> np.ndarray:
    out = np.empty(n, dtype=np.float32)
    lib().rtxllm_synth_normal_f32(seed, n, mean, std, _ptr(out), threads)
    return out


def normal_f16_bits(seed: int, n: int, mean: float = 0.0, std: float = 1.0, threads: int = 0) -> np.ndarray:
    out = np.empty(n, dtype=np.uint16)
    lib().rtxllm_synth_normal_f16(seed, n, mean, std, _ptr(out), threads)
    return out
