"""CPU checks of the oracle's activation-staging restatement (the rule the GPU
staging kernel must match bit for bit): digit ranges, reconstruction error
bound, the group maximum mapping to +-K (K = 127 * 256), exact group sums,
zero groups and hand-worked digits."""

from __future__ import annotations

import numpy as np
import pytest

K = 32512


def test_stage_properties(orc):
    rng = np.random.default_rng(5)
    x = rng.standard_normal(4096).astype(np.float32) * np.repeat(rng.uniform(0.01, 30, 256), 16).astype(np.float32)
    h, l, s, t = orc.stage_activation(x)
    X = 256 * h.astype(np.int64) + l.astype(np.int64)
    assert h.min() >= -127 and h.max() <= 127
    assert l.min() >= -128 and l.max() <= 127
    assert np.abs(X).max() <= K
    xs = np.repeat(s.astype(np.float64), 16)
    # |x - s X| <= s / 2 plus the fp32 rounding of x * (K / m) and of s = m / K,
    # each at most K * 2^-24 (below 0.002 steps)
    err = np.abs(x.astype(np.float64) - xs * X)
    assert np.all(err <= xs * 0.51)
    assert np.mean(err / xs) < 0.3  # rounding to nearest: mean error ~1/4 step
    g = x.reshape(-1, 16)
    arg = np.abs(g).argmax(axis=1)
    assert np.all(np.abs(X.reshape(-1, 16)[np.arange(256), arg]) == K)
    np.testing.assert_array_equal(t, (s * X.reshape(-1, 16).sum(axis=1).astype(np.float32)).astype(np.float32))


def test_stage_weighted_and_zero_group(orc):
    x = np.zeros(256, np.float32)
    x[16:32] = np.arange(16, dtype=np.float32) - 7.5
    w = np.full(256, 2.0, np.float32)
    h, l, s, t = orc.stage_activation(x, w)
    assert s[0] == 0.0 and t[0] == 0.0 and not h[:16].any() and not l[:16].any()
    # group 1: v = 2 (j - 7.5), max |v| = 15 at j = 15 -> X = K; j = 0 -> -K
    X = 256 * h[16:32].astype(int) + l[16:32].astype(int)
    assert X[15] == K and X[0] == -K
    assert s[1] == np.float32(15.0) / np.float32(K)
    # j = 8: v = 1 -> X = rint(K / 15) = 2167 (2167.47)
    assert X[8] == 2167
    assert X.sum() == 0 and t[1] == 0.0


def test_stage_digits_hand_worked(orc):
    """Digits of hand-picked X through the oracle (a group whose maximum is K so
    that X = v exactly): H = floor((X + 128) / 256), L = X - 256 H, e.g.
    X = 300 -> (1, 44); X = 128 -> (1, -128); X = 127 -> (0, 127);
    X = -129 -> (-1, 127); X = -K -> (-127, 0)."""
    cases = [(300, 1, 44), (-65, 0, -65), (128, 1, -128), (127, 0, 127), (-128, 0, -128), (-129, -1, 127),
             (-K, -127, 0), (K, 127, 0), (1, 0, 1), (-1, 0, -1), (383, 1, 127), (384, 2, -128)]
    x = np.zeros(16 * len(cases), np.float32)
    for i, (X, _, _) in enumerate(cases):
        x[16 * i] = K           # group maximum: scale exactly 1
        x[16 * i + 1] = X
    h, l, s, _ = orc.stage_activation(x)
    for i, (X, H, L) in enumerate(cases):
        assert s[i] == 1.0
        assert (h[16 * i + 1], l[16 * i + 1]) == (H, L), X
        assert 256 * H + L == X


@pytest.mark.slow
def test_staged_f64_matvec_close_to_fp32_oracle(orc):
    """The staging step (3.1e-5 of each group's maximum) moves a 4096-column
    product by ~1e-5 of its largest output: far inside the 1e-3 bar."""
    from rtxllm_amd import formats as F
    from rtxllm_amd import packs

    for fmt in (F.Q4K_SPLIT_NATIVE, F.Q5K, F.IQ2S, F.IQ3S):
        pack = packs.make_pack(fmt, 64, 4096, seed=99 + fmt)
        x = packs.normal_f32(1234, 4096)
        ref = orc.matvec_f64(fmt, pack.payload, pack.meta, x, 64, 4096, 4)
        got = orc.matvec_staged_f64(fmt, pack.payload, pack.meta, x, 64, 4096, 4)
        assert np.max(np.abs(got - ref)) / np.max(np.abs(ref)) < 1e-4
