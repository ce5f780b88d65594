"""CPU checks of the oracle's activation-staging restatement (the rule the GPU
staging kernel must match bit for bit): digit ranges, reconstruction error
bound, the group maximum mapping to +-16256, exact group sums, zero groups and a
hand-worked group."""

from __future__ import annotations

import numpy as np
import pytest


def test_stage_properties(orc):
    rng = np.random.default_rng(5)
    x = rng.standard_normal(4096).astype(np.float32) * np.repeat(rng.uniform(0.01, 30, 256), 16).astype(np.float32)
    h, l, s, t = orc.stage_activation(x)
    X = 128 * h.astype(np.int64) + l.astype(np.int64)
    assert h.min() >= -127 and h.max() <= 127
    assert l.min() >= -64 and l.max() <= 63
    assert np.abs(X).max() <= 16256
    xs = np.repeat(s.astype(np.float64), 16)
    # |x - s X| <= s / 2, up to the fp32 rounding of x * (16256 / m)
    err = np.abs(x.astype(np.float64) - xs * X)
    assert np.all(err <= xs * (0.5 + 1e-3))
    g = x.reshape(-1, 16)
    arg = np.abs(g).argmax(axis=1)
    assert np.all(np.abs(X.reshape(-1, 16)[np.arange(256), arg]) == 16256)
    np.testing.assert_array_equal(t, (s * X.reshape(-1, 16).sum(axis=1).astype(np.float32)).astype(np.float32))


def test_stage_weighted_and_zero_group(orc):
    x = np.zeros(256, np.float32)
    x[16:32] = np.arange(16, dtype=np.float32) - 7.5
    w = np.full(256, 2.0, np.float32)
    h, l, s, t = orc.stage_activation(x, w)
    assert s[0] == 0.0 and t[0] == 0.0 and not h[:16].any() and not l[:16].any()
    # group 1: v = 2 (j - 7.5), max |v| = 15 at j = 15 -> X = 16256; j = 0 -> -16256
    X = 128 * h[16:32].astype(int) + l[16:32].astype(int)
    assert X[15] == 16256 and X[0] == -16256
    assert s[1] == np.float32(15.0) / np.float32(16256.0)
    # j = 8: v = 1 -> X = rint(16256 / 15) = 1084 (1083.73)
    assert X[8] == 1084
    assert X.sum() == 0 and t[1] == 0.0


def test_stage_hand_worked():
    """X = 300 -> H = floor(364 / 128) = 2, L = 44; X = -65 -> H = floor(-1/128) = -1, L = 63."""
    for X, H, L in [(300, 2, 44), (-65, -1, 63), (63, 0, 63), (64, 1, -64), (-16256, -127, 0), (16256, 127, 0)]:
        assert (X + 64) // 128 == H and X - 128 * H == L


@pytest.mark.slow
def test_staged_f64_matvec_close_to_fp32_oracle(orc):
    from rtxllm_amd import formats as F
    from rtxllm_amd import packs

    for fmt in (F.Q4K_SPLIT_NATIVE, F.Q5K, F.IQ2S, F.IQ3S):
        pack = packs.make_pack(fmt, 64, 4096, seed=99 + fmt)
        x = packs.normal_f32(1234, 4096)
        ref = orc.matvec_f64(fmt, pack.payload, pack.meta, x, 64, 4096, 4)
        got = orc.matvec_staged_f64(fmt, pack.payload, pack.meta, x, 64, 4096, 4)
        assert np.max(np.abs(got - ref)) / np.max(np.abs(ref)) < 2e-4
