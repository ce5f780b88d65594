"""Greedy-token comparison for the GPU tests.

The reference gate fails on any token mismatch (iq_matvec_probe/main.cpp:
424-465). Here a token may differ from the oracle's only at a near-tie: when
the oracle's logit at the GPU's token is within `tie` (relative to the
largest logit) of the oracle's maximum, which the matvec's rounding can
reorder. Every such disagreement is recorded and the pytest summary prints
how many there were (tests/conftest.py), so they are counted, not hidden."""

from __future__ import annotations

import numpy as np

DISAGREEMENTS: list[tuple[str, int, int, float]] = []


def argmax_lowest(logits: np.ndarray) -> int:
    """Greedy argmax, the lowest index among equal maxima (decode_kernels.cu:2993-3031)."""
    return int(np.argmax(np.asarray(logits)))


def check_token(label: str, token: int, ref_logits: np.ndarray, tie: float) -> None:
    ref_logits = np.asarray(ref_logits, np.float64)
    ref_tok = argmax_lowest(ref_logits)
    if token == ref_tok:
        return
    top = float(ref_logits[ref_tok])
    gap = (top - float(ref_logits[token])) / abs(top)
    assert gap <= tie, f"{label}: token {token} vs oracle {ref_tok}, relative gap {gap:.3e} > {tie:g}"
    DISAGREEMENTS.append((label, int(token), ref_tok, gap))
