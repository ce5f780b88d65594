"""GPU parity of the reference runner's RMSNorm / SiLU feedback family and the
greedy token kernels against the oracle (decode_kernels.cu:122-289, 2993-3073)."""

from __future__ import annotations

import numpy as np
import pytest

torch = pytest.importorskip("torch")

from rtxllm_amd import ops, packs  # noqa: E402
from rtxllm_amd._lib import lib  # noqa: E402

pytestmark = pytest.mark.gpu
EPS = 1e-6
TOL = 1e-5


def dev(a):
    return ops.to_dev(np.ascontiguousarray(a, np.float32))


def close(got, ref):
    scale = max(1.0, float(np.max(np.abs(ref))))
    assert float(np.max(np.abs(got - ref))) <= TOL * scale


@pytest.mark.parametrize("rows,cols", [(1, 5), (300, 1000), (4096, 14336), (14336, 4096)])
def test_rmsnorm_and_silu_feedback(orc, rows, cols):
    logits = packs.normal_f32(rows, rows) * np.float32(3.0)
    L, s, p = lib(), ops.stream(), ops.ptr
    lg = dev(logits)
    for name, oname in [("rtxllm_launch_rmsnorm_feedback", "orc_rmsnorm_feedback"),
                        ("rtxllm_launch_silu_rmsnorm_feedback", "orc_silu_rmsnorm_feedback")]:
        act = torch.zeros(cols, dtype=torch.float32, device="cuda:0")
        assert getattr(L, name)(p(lg), p(act), rows, cols, EPS, s) == 0
        ref = np.zeros(cols, np.float32)
        getattr(orc.lib(), oname)(orc.ptr(logits), rows, orc.ptr(ref), cols, EPS)
        close(act.cpu().numpy(), ref)

    act = torch.zeros(cols, dtype=torch.float32, device="cuda:0")
    cache = torch.zeros(cols, dtype=torch.float32, device="cuda:0")
    assert L.rtxllm_launch_rmsnorm_feedback_with_silu_cache(p(lg), p(act), p(cache), rows, cols, EPS, s) == 0
    ra, rc = np.zeros(cols, np.float32), np.zeros(cols, np.float32)
    orc.lib().orc_rmsnorm_feedback_with_silu_cache(orc.ptr(logits), rows, orc.ptr(ra), orc.ptr(rc), cols, EPS)
    close(act.cpu().numpy(), ra)
    close(cache.cpu().numpy(), rc)

    cache_cols = max(1, cols // 3)
    silu = packs.normal_f32(5, cache_cols)
    act = torch.zeros(cols, dtype=torch.float32, device="cuda:0")
    assert L.rtxllm_launch_gated_silu_rmsnorm_feedback(p(lg), p(dev(silu)), p(act), rows, cache_cols, cols, EPS,
                                                       s) == 0
    ref = np.zeros(cols, np.float32)
    orc.lib().orc_gated_silu_rmsnorm_feedback(orc.ptr(logits), rows, orc.ptr(silu), cache_cols, orc.ptr(ref), cols,
                                              EPS)
    close(act.cpu().numpy(), ref)


@pytest.mark.parametrize("accumulate", [0, 1])
def test_cache_kernels(orc, accumulate):
    rows, cols = 777, 2048
    logits = packs.normal_f32(11, rows)
    base = packs.normal_f32(12, cols)
    gate = packs.normal_f32(13, cols)
    L, s, p = lib(), ops.stream(), ops.ptr
    for name, silu in [("rtxllm_launch_rmsnorm_silu_cache", 1), ("rtxllm_launch_rmsnorm_cache", 0)]:
        cache = dev(base)
        assert getattr(L, name)(p(dev(logits)), p(cache), rows, cols, EPS, accumulate, s) == 0
        ref = base.copy()
        orc.lib().orc_rmsnorm_cache(orc.ptr(logits), rows, orc.ptr(ref), cols, EPS, silu, accumulate)
        close(cache.cpu().numpy(), ref)
    up = dev(base)
    act = torch.zeros(cols, dtype=torch.float32, device="cuda:0")
    assert L.rtxllm_launch_rmsnorm_cache_and_gated_product(p(dev(logits)), p(dev(gate)), p(up), p(act), rows, cols,
                                                           cols, EPS, accumulate, s) == 0
    ru, ra = base.copy(), np.zeros(cols, np.float32)
    orc.lib().orc_rmsnorm_cache_and_gated_product(orc.ptr(logits), rows, orc.ptr(gate), orc.ptr(ru), orc.ptr(ra),
                                                  cols, cols, EPS, accumulate)
    close(up.cpu().numpy(), ru)
    close(act.cpu().numpy(), ra)


@pytest.mark.parametrize("rows", [1, 255, 4097, 128256])
def test_output_token_sample(orc, rows):
    y = packs.normal_f32(rows, rows)
    y[rows // 2] = y.max() + 1.0  # unique max
    if rows > 10:
        y[rows // 3] = y[rows // 2]  # tie: lower index must win
    tok = torch.zeros(1, dtype=torch.int32, device="cuda:0")
    vocab, offset = 32000, 17
    assert lib().rtxllm_launch_output_token_sample(ops.ptr(dev(y)), ops.ptr(tok), rows, vocab, offset,
                                                   ops.stream()) == 0
    assert int(tok.cpu()[0]) == (orc.argmax(y) + offset) % vocab


def test_argmax_nan_and_all_negative_infinity(orc):
    tok = torch.zeros(1, dtype=torch.int32, device="cuda:0")
    y = np.array([np.nan, -1.0, 5.0, np.nan, 5.0], np.float32)
    assert lib().rtxllm_launch_output_token_sample(ops.ptr(dev(y)), ops.ptr(tok), 5, 100, 0, ops.stream()) == 0
    assert int(tok.cpu()[0]) == orc.argmax(y) == 2
    y = np.full(3000, -np.inf, np.float32)
    assert lib().rtxllm_launch_output_token_sample(ops.ptr(dev(y)), ops.ptr(tok), 3000, 100, 0, ops.stream()) == 0
    assert int(tok.cpu()[0]) == orc.argmax(y) == 0
