"""CPU checks of the oracle's activation-staging restatement (the rule the GPU
staging kernels must match bit for bit): an independent numpy restatement
(np.frexp / np.ldexp / np.rint), digit ranges, the exact reconstruction bound
|x - s X| <= s / 2, the group maximum landing in [2^21, 2^22], exact group
sums, zero / NaN / infinite groups and hand-worked digits."""

from __future__ import annotations

import numpy as np
import pytest

LIM = 1 << 22


def np_stage(x: np.ndarray):
    """numpy restatement: per 16-value group m = max|v| = f 2^e, s = 2^(e-22),
    X = rint(v 2^(22-e)), balanced base-256 digits."""
    g = x.astype(np.float32).reshape(-1, 16)
    m = np.max(np.abs(g), axis=1)
    _, e = np.frexp(m)
    X = np.rint(np.ldexp(g.astype(np.float64), (22 - e)[:, None])).astype(np.int64)
    s = np.where(m > 0, np.ldexp(np.float32(1.0), e - 22), 0).astype(np.float32)
    L = (X + 128) % 256 - 128
    X1 = (X - L) // 256
    M = (X1 + 128) % 256 - 128
    H = (X1 - M) // 256
    return H.reshape(-1), M.reshape(-1), L.reshape(-1), s, X


def test_stage_matches_numpy_restatement(orc):
    rng = np.random.default_rng(5)
    x = rng.standard_normal(4096).astype(np.float32) * np.repeat(rng.uniform(0.01, 30, 256), 16).astype(np.float32)
    x[:16] = 0.0
    x[16:32] = np.float32(2.0) ** np.arange(-8, 8)  # a group of exact powers of two
    h, m, l, s, t = orc.stage_activation(x)
    H, M, L, S, X = np_stage(x)
    np.testing.assert_array_equal(h, H)
    np.testing.assert_array_equal(m, M)
    np.testing.assert_array_equal(l, L)
    np.testing.assert_array_equal(s, S)
    np.testing.assert_array_equal(t, (s * X.sum(axis=1).astype(np.float32)).astype(np.float32))


def test_stage_properties(orc):
    rng = np.random.default_rng(6)
    x = rng.standard_normal(4096).astype(np.float32) * np.repeat(rng.uniform(1e-3, 1e3, 256), 16).astype(np.float32)
    h, m, l, s, _ = orc.stage_activation(x)
    assert h.min() >= -64 and h.max() <= 64
    assert m.min() >= -128 and m.max() <= 127 and l.min() >= -128 and l.max() <= 127
    X = 65536 * h.astype(np.int64) + 256 * m.astype(np.int64) + l.astype(np.int64)
    assert np.abs(X).max() <= LIM
    xs = np.repeat(s.astype(np.float64), 16)
    # the power-of-two scaling is exact, so X is x / s rounded once
    err = np.abs(x.astype(np.float64) - xs * X)
    assert np.all(err <= xs * 0.5)
    g = x.reshape(-1, 16)
    arg = np.abs(g).argmax(axis=1)
    top = np.abs(X.reshape(-1, 16)[np.arange(256), arg])
    assert np.all((top >= LIM // 2) & (top <= LIM))
    # s is a power of two and max|x| / s is in [2^21, 2^22)
    mant, _ = np.frexp(s)
    assert np.all(mant == 0.5)
    ratio = np.abs(g).max(axis=1).astype(np.float64) / s
    assert np.all((ratio >= LIM / 2) & (ratio < LIM))


def test_stage_weighted_zero_and_nonfinite_groups(orc):
    x = np.zeros(256, np.float32)
    x[16:32] = np.arange(16, dtype=np.float32) - 7.5
    x[32:48] = 1.0
    x[40] = np.nan
    x[48:64] = 1.0
    x[50] = np.inf
    w = np.full(256, 2.0, np.float32)
    h, m, l, s, t = orc.stage_activation(x, w)
    assert s[0] == 0.0 and t[0] == 0.0 and not h[:16].any() and not m[:16].any() and not l[:16].any()
    # group 1: v = 2 (j - 7.5), max |v| = 15 = 0.9375 * 2^4 -> s = 2^-18, X = v * 2^18
    X = 65536 * h[16:32].astype(int) + 256 * m[16:32].astype(int) + l[16:32].astype(int)
    assert s[1] == np.float32(2.0 ** -18)
    np.testing.assert_array_equal(X, (2 * (np.arange(16) - 7.5) * 2 ** 18).astype(int))
    assert X.sum() == 0 and t[1] == 0.0
    # a NaN poisons its group: s = NaN, digits zero; an infinite maximum: s = inf
    assert np.isnan(s[2]) and np.isnan(t[2]) and not h[32:48].any() and not l[32:48].any()
    assert np.isinf(s[3]) and s[3] > 0 and np.isnan(t[3]) and not m[48:64].any()


def test_stage_digits_hand_worked(orc):
    """Digits of hand-picked X through the oracle: a group whose maximum is
    2^22 - 1 has e = 22, s = 1, so X = v exactly. Balanced base-256 digits:
    X = 300 -> (0, 1, 44); 128 -> (0, 1, -128); 127 -> (0, 0, 127);
    -129 -> (0, -1, 127); 32767 -> (1, -128, -1); 32896 -> (1, -127, -128);
    2^22 - 1 -> (64, 0, -1)."""
    top = LIM - 1
    cases = [(300, 0, 1, 44), (-65, 0, 0, -65), (128, 0, 1, -128), (127, 0, 0, 127), (-128, 0, 0, -128),
             (-129, 0, -1, 127), (32767, 1, -128, -1), (32768, 1, -128, 0), (32896, 1, -127, -128),
             (-32897, -1, 127, 127), (top, 64, 0, -1), (-top, -64, 0, 1), (1, 0, 0, 1), (-1, 0, 0, -1)]
    x = np.zeros(16 * len(cases), np.float32)
    for i, (X, *_rest) in enumerate(cases):
        x[16 * i] = top  # group maximum: e = 22, scale exactly 1
        x[16 * i + 1] = X
    h, m, l, s, _ = orc.stage_activation(x)
    for i, (X, H, M, L) in enumerate(cases):
        assert s[i] == 1.0
        assert (h[16 * i + 1], m[16 * i + 1], l[16 * i + 1]) == (H, M, L), X
        assert 65536 * H + 256 * M + L == X


@pytest.mark.slow
def test_staged_f64_matvec_close_to_f64_oracle(orc):
    """The staging error (at most 2^-23 of each group's maximum per value)
    moves a 4096-column product by less than fp32 sequential accumulation
    does: compared with the float64 product on the raw x."""
    from rtxllm_amd import formats as F
    from rtxllm_amd import packs

    for fmt in (F.Q4K_SPLIT_NATIVE, F.Q5K, F.IQ2S, F.IQ3S):
        pack = packs.make_pack(fmt, 64, 4096, seed=99 + fmt)
        x = packs.normal_f32(1234, 4096)
        ref = orc.matvec_f64(fmt, pack.payload, pack.meta, x, 64, 4096, 4)
        got = orc.matvec_staged_f64(fmt, pack.payload, pack.meta, x, 64, 4096, 4)
        f32 = orc.matvec_f32(fmt, pack.payload, pack.meta, x, 64, 4096, 4)
        scale = np.max(np.abs(ref))
        e_staged = np.max(np.abs(got - ref)) / scale
        e_f32 = np.max(np.abs(f32 - ref)) / scale
        assert e_staged < 1e-6
        assert e_staged <= e_f32, (F.NAMES[fmt], e_staged, e_f32)
