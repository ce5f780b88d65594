"""Resident-pack format ids and block sizes (the C-ABI's numbering).

Sizes follow tools/bench/gguf_block_formats.py:14-22 (GGUF blocks of 256
values: Q4_K 144 B, Q5_K 176 B, IQ2_S 82 B, IQ3_S 110 B) and the Q4_K split
metadata sizes of tools/bench/q4k_resident_pack.py:91-97.
"""

from __future__ import annotations

Q4K_RAW = 0
Q4K_SPLIT_PREDECODED = 1
Q4K_SPLIT_HALF = 2
Q4K_SPLIT_COMPACT = 3
Q4K_SPLIT_NATIVE = 4
Q5K = 5
IQ2S = 6
IQ3S = 7
Q4K_RAW_PREDECODED = 8
IQ2S_UNITS = 9  # IQ2_S bytes regrouped per 32-value unit (packs.iq2s_units)
IQ3S_UNITS = 10  # IQ3_S bytes regrouped per 32-value unit (packs.iq3s_units), 114 B per block

BLOCK_VALUES = 256

PAYLOAD_BYTES = {
    Q4K_RAW: 144,
    Q4K_SPLIT_PREDECODED: 128,
    Q4K_SPLIT_HALF: 128,
    Q4K_SPLIT_COMPACT: 128,
    Q4K_SPLIT_NATIVE: 128,
    Q5K: 176,
    IQ2S: 82,
    IQ3S: 110,
    Q4K_RAW_PREDECODED: 144,
    IQ2S_UNITS: 82,
    IQ3S_UNITS: 114,
}
META_BYTES = {
    Q4K_SPLIT_PREDECODED: 64,
    Q4K_SPLIT_HALF: 32,
    Q4K_SPLIT_COMPACT: 20,
    Q4K_SPLIT_NATIVE: 16,
    Q4K_RAW_PREDECODED: 64,
}
# GGUF bytes per block of the source format: the roofline's algorithmic bytes.
GGUF_BLOCK_BYTES = {f: (144 if f in (0, 1, 2, 3, 4, 8) else PAYLOAD_BYTES[f]) for f in PAYLOAD_BYTES}
GGUF_BLOCK_BYTES[IQ3S_UNITS] = 110

NAMES = {
    Q4K_RAW: "q4k-raw",
    Q4K_SPLIT_PREDECODED: "q4k-split-predecoded",
    Q4K_SPLIT_HALF: "q4k-split-half",
    Q4K_SPLIT_COMPACT: "q4k-split-compact",
    Q4K_SPLIT_NATIVE: "q4k-split-native",
    Q5K: "q5k",
    IQ2S: "iq2s",
    IQ3S: "iq3s",
    Q4K_RAW_PREDECODED: "q4k-raw-predecoded",
    IQ2S_UNITS: "iq2s-units",
    IQ3S_UNITS: "iq3s-units",
}
SPLIT_FORMATS = (Q4K_SPLIT_PREDECODED, Q4K_SPLIT_HALF, Q4K_SPLIT_COMPACT, Q4K_SPLIT_NATIVE)


def meta_bytes(fmt: int) -> int:
    return META_BYTES.get(fmt, 0)


def algorithmic_bytes(fmt: int, rows: int, cols: int) -> int:
    """rows * (cols/256) * GGUF block bytes + fp32 x and y."""
    return rows * (cols // BLOCK_VALUES) * GGUF_BLOCK_BYTES[fmt] + 4 * (rows + cols)


def auto_policy(rows: int, cols: int, block_count: int) -> str:
    """Reference Q4_K pack policy (q4k_resident_pack.py:75-79)."""
    del rows, cols
    return "split-compact" if block_count <= 4096 else "split-predecoded"
