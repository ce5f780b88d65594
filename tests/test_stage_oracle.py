"""CPU checks of the oracle's activation-staging restatement (the rule the GPU
staging kernel must match bit for bit): digit ranges, reconstruction error
bound, the group maximum mapping to +-K (K = 127 * 16384), exact group sums,
zero groups and hand-worked digits."""

from __future__ import annotations

import numpy as np
import pytest

K = 2080768


def test_stage_properties(orc):
    rng = np.random.default_rng(5)
    x = rng.standard_normal(4096).astype(np.float32) * np.repeat(rng.uniform(0.01, 30, 256), 16).astype(np.float32)
    h, m, l, s, t = orc.stage_activation(x)
    X = 16384 * h.astype(np.int64) + 128 * m.astype(np.int64) + l.astype(np.int64)
    assert h.min() >= -127 and h.max() <= 127
    assert m.min() >= -64 and m.max() <= 64
    assert l.min() >= -64 and l.max() <= 63
    assert np.abs(X).max() <= K
    xs = np.repeat(s.astype(np.float64), 16)
    # |x - s X| <= s / 2 plus the fp32 rounding of x * (K / m) and of s = m / K,
    # each at most K * 2^-24 = 0.124 steps
    err = np.abs(x.astype(np.float64) - xs * X)
    assert np.all(err <= xs * 0.75)
    assert np.mean(err / xs) < 0.3  # rounding to nearest: mean error ~1/4 step
    g = x.reshape(-1, 16)
    arg = np.abs(g).argmax(axis=1)
    assert np.all(np.abs(X.reshape(-1, 16)[np.arange(256), arg]) == K)
    np.testing.assert_array_equal(t, (s * X.reshape(-1, 16).sum(axis=1).astype(np.float32)).astype(np.float32))


def test_stage_weighted_and_zero_group(orc):
    x = np.zeros(256, np.float32)
    x[16:32] = np.arange(16, dtype=np.float32) - 7.5
    w = np.full(256, 2.0, np.float32)
    h, m, l, s, t = orc.stage_activation(x, w)
    assert s[0] == 0.0 and t[0] == 0.0 and not h[:16].any() and not m[:16].any() and not l[:16].any()
    # group 1: v = 2 (j - 7.5), max |v| = 15 at j = 15 -> X = K; j = 0 -> -K
    X = 16384 * h[16:32].astype(int) + 128 * m[16:32].astype(int) + l[16:32].astype(int)
    assert X[15] == K and X[0] == -K
    assert s[1] == np.float32(15.0) / np.float32(K)
    # j = 8: v = 1 -> X = rint(K / 15) = 138718 (138717.87)
    assert X[8] == 138718
    assert X.sum() == 0 and t[1] == 0.0


def test_stage_digits_hand_worked(orc):
    """Digits of hand-picked X through the oracle (a group whose maximum is K so
    that X = v exactly): X = 300 -> (0, 2, 44); X = -65 -> (0, -1, 63); X = 8192
    -> (1, -64, 0); X = 8191 -> (0, 64, -1); X = -K -> (-127, 0, 0)."""
    cases = [(300, 0, 2, 44), (-65, 0, -1, 63), (8192, 1, -64, 0), (8191, 0, 64, -1), (-K, -127, 0, 0),
             (K, 127, 0, 0), (1, 0, 0, 1), (-1, 0, 0, -1), (64, 0, 1, -64), (16383, 1, 0, -1)]
    x = np.zeros(16 * len(cases), np.float32)
    for i, (X, _, _, _) in enumerate(cases):
        x[16 * i] = K           # group maximum: scale exactly 1
        x[16 * i + 1] = X
    h, m, l, s, _ = orc.stage_activation(x)
    for i, (X, H, M, L) in enumerate(cases):
        assert s[i] == 1.0
        assert (h[16 * i + 1], m[16 * i + 1], l[16 * i + 1]) == (H, M, L), X
        assert 16384 * H + 128 * M + L == X


@pytest.mark.slow
def test_staged_f64_matvec_close_to_fp32_oracle(orc):
    from rtxllm_amd import formats as F
    from rtxllm_amd import packs

    for fmt in (F.Q4K_SPLIT_NATIVE, F.Q5K, F.IQ2S, F.IQ3S):
        pack = packs.make_pack(fmt, 64, 4096, seed=99 + fmt)
        x = packs.normal_f32(1234, 4096)
        ref = orc.matvec_f64(fmt, pack.payload, pack.meta, x, 64, 4096, 4)
        got = orc.matvec_staged_f64(fmt, pack.payload, pack.meta, x, 64, 4096, 4)
        assert np.max(np.abs(got - ref)) / np.max(np.abs(ref)) < 2e-6
