"""Vectorised numpy decode of GGUF blocks, written from the block layouts
(ggml Q4_K / Q5_K / IQ2_S / IQ3_S as used by the reference runtime), used to
cross-check the C oracle. It is structured differently from the oracle (whole
blocks at a time with array bit operations, no per-value function) so a
transposed index or wrong shift in either shows up as a mismatch."""

from __future__ import annotations

import numpy as np


def f16(lo: np.ndarray, hi: np.ndarray) -> np.ndarray:
    return (lo.astype(np.uint16) | (hi.astype(np.uint16) << 8)).view(np.float16).astype(np.float32)


def scale_min(sc12: np.ndarray) -> tuple[np.ndarray, np.ndarray]:
    """sc12: [n, 12] uint8 -> (sc [n, 8], m [n, 8]) as uint8 (6-bit fields)."""
    s = sc12.astype(np.uint16)
    sc = np.empty((s.shape[0], 8), np.uint16)
    m = np.empty((s.shape[0], 8), np.uint16)
    sc[:, :4] = s[:, 0:4] & 63
    m[:, :4] = s[:, 4:8] & 63
    sc[:, 4:] = (s[:, 8:12] & 15) | ((s[:, 0:4] >> 6) << 4)
    m[:, 4:] = (s[:, 8:12] >> 4) | ((s[:, 4:8] >> 6) << 4)
    return sc, m


def q4k_from_parts(S: np.ndarray, M: np.ndarray, qs: np.ndarray) -> np.ndarray:
    """S, M: [n, 8] float32 per sub-block; qs: [n, 128] -> [n, 256] float32, w = S*q - M."""
    n = qs.shape[0]
    q = np.empty((n, 8, 32), np.float32)
    grp = qs.reshape(n, 4, 32)
    q[:, 0::2, :] = grp & 15
    q[:, 1::2, :] = grp >> 4
    w = (S[:, :, None] * q).astype(np.float32) - M[:, :, None]
    return w.astype(np.float32).reshape(n, 256)


def q4k_raw(blocks: np.ndarray) -> np.ndarray:
    b = blocks.reshape(-1, 144)
    d, dmin = f16(b[:, 0], b[:, 1]), f16(b[:, 2], b[:, 3])
    sc, m = scale_min(b[:, 4:16])
    S = (d[:, None] * sc.astype(np.float32)).astype(np.float32)
    M = (dmin[:, None] * m.astype(np.float32)).astype(np.float32)
    return q4k_from_parts(S, M, b[:, 16:])


def q5k(blocks: np.ndarray) -> np.ndarray:
    b = blocks.reshape(-1, 176)
    n = b.shape[0]
    d, dmin = f16(b[:, 0], b[:, 1]), f16(b[:, 2], b[:, 3])
    sc, m = scale_min(b[:, 4:16])
    qh = b[:, 16:48]
    grp = b[:, 48:176].reshape(n, 4, 32)
    q = np.empty((n, 8, 32), np.float32)
    for j in range(8):
        g, high = j // 2, j % 2
        low = (grp[:, g, :] >> 4) if high else (grp[:, g, :] & 15)
        q[:, j, :] = low + 16 * ((qh >> j) & 1)
    S = (d[:, None] * sc.astype(np.float32)).astype(np.float32)
    M = (dmin[:, None] * m.astype(np.float32)).astype(np.float32)
    return ((S[:, :, None] * q).astype(np.float32) - M[:, :, None]).astype(np.float32).reshape(n, 256)


def iq2s(blocks: np.ndarray, kgrid: np.ndarray) -> np.ndarray:
    b = blocks.reshape(-1, 82)
    n = b.shape[0]
    d = f16(b[:, 0], b[:, 1])
    qs = b[:, 2:34].reshape(n, 8, 4).astype(np.uint32)  # [ib32][grp]
    sg = b[:, 34:66].reshape(n, 8, 4).astype(np.uint32)
    qh = b[:, 66:74].astype(np.uint32)
    scales = b[:, 74:82].astype(np.uint32)
    hi = np.stack([(qh >> (2 * g)) & 3 for g in range(4)], axis=2)  # [n, 8, 4]
    idx = qs | (hi << 8)
    words = kgrid[idx].astype(np.uint32)  # [n, 8, 4]
    lanes = np.arange(8, dtype=np.uint32)
    mag = 2 * ((words[..., None] >> (2 * lanes)) & 3) + 1  # [n, 8, 4, 8]
    neg = (sg[..., None] >> lanes) & 1
    nib = np.stack([scales & 15, scales & 15, scales >> 4, scales >> 4], axis=2)  # [n, 8, 4]
    scale = ((d[:, None, None] * (np.float32(0.5) + nib.astype(np.float32))).astype(np.float32) * np.float32(0.25)).astype(np.float32)
    signed = np.where(neg == 1, -mag.astype(np.float32), mag.astype(np.float32))
    return (scale[..., None] * signed).astype(np.float32).reshape(n, 256)


def iq3s(blocks: np.ndarray, grid: np.ndarray) -> np.ndarray:
    b = blocks.reshape(-1, 110)
    n = b.shape[0]
    d = f16(b[:, 0], b[:, 1])
    qs = b[:, 2:66].reshape(n, 8, 8).astype(np.uint32)  # [ib32][sel 0..7]
    qh = b[:, 66:74].astype(np.uint32)
    sg = b[:, 74:106].reshape(n, 8, 4).astype(np.uint32)  # [ib32][grp]
    scales = b[:, 106:110].astype(np.uint32)
    sel = np.arange(8, dtype=np.uint32)
    idx = qs | (((qh[:, :, None] >> sel) & 1) << 8)  # [n, 8, 8]
    words = grid[idx].astype(np.uint32)
    mags = np.stack([(words >> (8 * k)) & 0xFF for k in range(4)], axis=3)  # [n, 8, 8(sel), 4]
    mags = mags.reshape(n, 8, 32)  # value index within ib32 = 4*sel + k
    bits = np.arange(8, dtype=np.uint32)
    neg = ((sg[..., None] >> bits) & 1).reshape(n, 8, 32)  # value = 8*grp + lane
    nib = np.stack([scales & 15, scales >> 4], axis=2).reshape(n, 8)
    scale = (d[:, None] * (1 + 2 * nib).astype(np.float32)).astype(np.float32)
    signed = np.where(neg == 1, -mags.astype(np.float32), mags.astype(np.float32))
    return (scale[..., None] * signed).astype(np.float32).reshape(n, 256)
