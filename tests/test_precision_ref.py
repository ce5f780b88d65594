"""CPU checks of the batch-staging restatement the batched precision gates use."""

from __future__ import annotations

import numpy as np

from precision_ref import batch_staged


def test_batch_staged_keeps_short_values_exact():
    # values of <= 22 significant bits relative to their block maximum survive
    rng = np.random.default_rng(1)
    x = (rng.integers(-(1 << 21), 1 << 21, 1024) * 2.0 ** -17).astype(np.float32)
    assert np.array_equal(batch_staged(x), x)


def test_batch_staged_error_bound_and_blocks():
    rng = np.random.default_rng(2)
    x = (rng.standard_normal(2048) * np.exp(3.0 * rng.standard_normal(2048))).astype(np.float32)
    xs = batch_staged(x)
    for b in range(8):
        blk, st = x[256 * b:256 * (b + 1)].astype(np.float64), xs[256 * b:256 * (b + 1)].astype(np.float64)
        e = np.frexp(np.max(np.abs(blk)))[1]
        # hi + lo keeps 22 significant bits, or half an fp16 subnormal step of the block scale
        assert np.all(np.abs(st - blk) <= np.maximum(np.abs(blk) * 2.0 ** -22, 2.0 ** (e - 25)))
        # values >= 2^-3 of the block scale keep at least 22 significant bits
        big = np.abs(blk) >= 2.0 ** (e - 3)
        assert np.all(np.abs(st - blk)[big] <= np.abs(blk)[big] * 2.0 ** -22)
    # a zero block stays zero, exponent 0
    assert np.array_equal(batch_staged(np.zeros(256, np.float32)), np.zeros(256, np.float32))
