"""GPU parity of the standalone Llama-math entry points (weighted RMSNorm, RoPE
with a theta schedule, SiLU-gate multiply, Q5_K embedding gather, GQA decode
attention over a paged fp16 cache, greedy argmax) against the oracle's
functions, called through the C-ABI; plus the launchers' pointer-alignment
rules (any 4-byte aligned activation accepted, misaligned weight streams
refused)."""

from __future__ import annotations

import ctypes

import numpy as np
import pytest

torch = pytest.importorskip("torch")

from rtxllm_amd import formats as F  # noqa: E402
from rtxllm_amd import ops, packs  # noqa: E402
from rtxllm_amd._lib import lib  # noqa: E402

pytestmark = pytest.mark.gpu

HIP_INVALID_VALUE = 1
P = ops.ptr


def dev(a: np.ndarray) -> torch.Tensor:
    return ops.to_dev(a)


def test_rmsnorm_w_matches_oracle(orc):
    n, count = 4096, 5
    x = packs.normal_f32(11, n * count).reshape(count, n) * np.float32(3.0)
    x[3] *= np.float32(1e-3)
    w = packs.normal_f32(12, n, mean=1.0, std=0.02)
    out = torch.empty((count, n), dtype=torch.float32, device="cuda:0")
    xd, wd = dev(x), dev(w)  # device tensors stay referenced until the kernels ran
    for weight in (wd, None):
        assert lib().rtxllm_rmsnorm_w(P(xd), P(weight), n, count, 1e-6, P(out), ops.stream()) == 0
        got = out.cpu().numpy()
        for r in range(count):
            ref = np.empty(n, np.float32)
            wr = np.ones(n, np.float32) if weight is None else w
            xr = np.ascontiguousarray(x[r])  # kept alive across the call
            orc.lib().orc_rmsnorm_weighted(orc.ptr(xr), orc.ptr(wr), n, 1e-6, orc.ptr(ref))
            # only the order of the sum of squares differs (tree vs sequential)
            np.testing.assert_allclose(got[r], ref, rtol=2e-6, atol=0)
    # in place
    xd = dev(x)
    assert lib().rtxllm_rmsnorm_w(P(xd), P(wd), n, count, 1e-6, P(xd), ops.stream()) == 0
    torch.cuda.synchronize()
    ref0 = np.empty(n, np.float32)
    x0 = np.ascontiguousarray(x[0])
    orc.lib().orc_rmsnorm_weighted(orc.ptr(x0), orc.ptr(w), n, 1e-6, orc.ptr(ref0))
    np.testing.assert_allclose(xd.cpu().numpy()[0], ref0, rtol=2e-6)


@pytest.mark.parametrize("theta", [500000.0, 10000.0])
def test_rope_theta_matches_oracle(orc, theta):
    n_heads, hd = 32, 128
    positions = np.array([0, 1, 17, 2047, 4095, 131071], np.uint32)
    vec = packs.normal_f32(21, len(positions) * n_heads * hd).reshape(len(positions), -1)
    vd, pd = dev(vec), dev(positions)
    assert lib().rtxllm_rope_theta(P(vd), n_heads, hd, theta, P(pd), len(positions), ops.stream()) == 0
    got = vd.cpu().numpy()
    inv = np.empty(hd // 2, np.float32)
    orc.lib().orc_rope_inv_freq(hd, theta, orc.ptr(inv))
    for r, p in enumerate(positions):
        ref = vec[r].copy()
        orc.lib().orc_rope(orc.ptr(ref), n_heads, hd, orc.ptr(inv), int(p))
        # sin / cos of the same fp32 angle: double-rounded here, libm's sinf / cosf there
        np.testing.assert_allclose(got[r], ref, rtol=1e-6, atol=2e-6)
    assert np.array_equal(got[0], vec[0])  # position 0: the identity


def test_silu_mul_matches_oracle(orc):
    n = 14336 * 3 + 5
    g = packs.normal_f32(31, n) * np.float32(4.0)
    u = packs.normal_f32(32, n)
    g[:4] = [0.0, -100.0, 100.0, -0.0]
    out = torch.empty(n, dtype=torch.float32, device="cuda:0")
    gd, ud = dev(g), dev(u)
    assert lib().rtxllm_silu_mul(P(gd), P(ud), n, P(out), ops.stream()) == 0
    ref = np.empty(n, np.float32)
    orc.lib().orc_silu_mul(orc.ptr(g), orc.ptr(u), n, orc.ptr(ref))
    np.testing.assert_allclose(out.cpu().numpy(), ref, rtol=2e-6, atol=1e-30)


def test_embed_gather_q5k_bit_exact(orc):
    vocab, cols = 3000, 4096
    table = packs.synth_raw(F.Q5K, vocab, cols, seed=41)
    tokens = np.array([0, 1, 2999, 1234, 77, 3000, 2**31], np.uint32)  # the last two are out of range
    out = torch.empty((len(tokens), cols), dtype=torch.float32, device="cuda:0")
    td, kd = dev(table), dev(tokens)
    assert lib().rtxllm_embed_gather_q5k(P(td), vocab, cols, P(kd), len(tokens), P(out), ops.stream()) == 0
    got = out.cpu().numpy()
    for i, t in enumerate(tokens):
        if t >= vocab:
            assert np.all(np.isnan(got[i]))
            continue
        ref = np.empty(cols, np.float32)
        orc.lib().orc_embed_q5k(orc.ptr(table), cols, int(t), orc.ptr(ref))
        assert np.array_equal(got[i].view(np.uint32), ref.view(np.uint32)), t


@pytest.mark.parametrize("positions", [(0, 130, 2047, 4095), (3001,)], ids=["four-queries", "one-query"])
@pytest.mark.parametrize("heads", [(32, 8), (16, 16), (8, 2), (64, 8), (16, 8)],
                         ids=["gqa4", "mha", "gqa4-small", "gqa8", "gqa2"])
def test_attn_decode_gqa_f16_matches_oracle(orc, heads, positions):
    """Groups 1, 2, 4 and 8 (group 8 fills all 16 B-operand columns of the
    score MFMA: 8 heads x hi / lo); several queries run the batch kernels,
    one query the batch-1 kernels of the decode step."""
    n_heads, n_kv = heads
    hd, page, cap = 128, 64, 4096
    pps = cap // page
    positions = np.array(positions, np.uint32)
    count = len(positions)
    npages = count * pps
    # pages of all queries in one cache, interleaved by a permutation
    table = np.array([(37 * i + 11) % npages for i in range(npages)], np.int32)
    assert len(set(table.tolist())) == npages
    halves = npages * n_kv * page * hd
    k = packs.normal_f16_bits(51, halves)
    v = packs.normal_f16_bits(52, halves)
    q = packs.normal_f32(53, count * n_heads * hd) * np.float32(2.0)
    ws_bytes = int(lib().rtxllm_attn_decode_workspace(n_heads, n_kv, cap, count))
    assert ws_bytes > 0
    ws = torch.empty(ws_bytes, dtype=torch.uint8, device="cuda:0")
    out = torch.empty((count, n_heads * hd), dtype=torch.float32, device="cuda:0")
    qd, kd, vd, td, pd = dev(q), dev(k), dev(v), dev(table), dev(positions)
    rc = lib().rtxllm_attn_decode_gqa_f16(P(qd), P(kd), P(vd), P(td), pps, n_heads, n_kv, page, cap, P(pd), count,
                                          P(out), P(ws), ws_bytes, ops.stream())
    assert rc == 0
    got = out.cpu().numpy()
    for r, p in enumerate(positions):
        row = np.ascontiguousarray(table[r * pps:(r + 1) * pps])
        kv = orc.KvCache(orc.ptr(k), orc.ptr(v), orc.ptr(row), page, n_kv, hd)
        ref = np.empty(n_heads * hd, np.float32)
        qr = np.ascontiguousarray(q[r * n_heads * hd:(r + 1) * n_heads * hd])  # kept alive across the call
        orc.lib().orc_attention_decode(ctypes.byref(kv), orc.ptr(qr), n_heads, int(p), orc.ptr(ref))
        err = float(np.max(np.abs(got[r] - ref)) / np.max(np.abs(ref)))
        # the query enters the scores as an fp16 hi / lo pair (~22 bits)
        assert err <= 1e-5, (int(p), err)
    if positions[0] == 0:  # a single position returns its V row exactly (up to the 1 / l division)
        row0 = table[0]
        off = (int(row0) * n_kv) * page * hd
        v0 = v[off:off + hd].view(np.float16).astype(np.float32)
        np.testing.assert_allclose(got[0][:hd], v0, rtol=1e-6)


def test_attn_decode_rejects_bad_arguments():
    ws = torch.empty(1 << 20, dtype=torch.uint8, device="cuda:0")
    f = torch.zeros(4096, dtype=torch.float32, device="cuda:0")
    L, s = lib(), ops.stream()
    assert L.rtxllm_attn_decode_workspace(12, 8, 4096, 1) == 0  # group of 1.5
    assert L.rtxllm_attn_decode_workspace(24, 8, 4096, 1) == 0  # group 3
    need = int(L.rtxllm_attn_decode_workspace(32, 8, 256, 1))
    # workspace too small
    assert L.rtxllm_attn_decode_gqa_f16(P(f), P(f), P(f), P(f), 4, 32, 8, 64, 256, P(f), 1, P(f), P(ws), need - 1,
                                        s) == HIP_INVALID_VALUE
    # capacity not a multiple of the page size
    assert L.rtxllm_attn_decode_gqa_f16(P(f), P(f), P(f), P(f), 4, 32, 8, 64, 250, P(f), 1, P(f), P(ws), 1 << 20,
                                        s) == HIP_INVALID_VALUE


def test_argmax_rows_match_oracle(orc):
    n = 128256
    rows = [packs.normal_f32(61, n)]
    tie = packs.normal_f32(62, n)
    tie[[5000, 9, 70000]] = tie.max() + 1.0  # three equal maxima: the lowest index wins
    rows.append(tie)
    nan = packs.normal_f32(63, n)
    nan[::3] = np.nan  # NaN never wins
    rows.append(nan)
    rows.append(np.full(n, -np.inf, np.float32))  # nothing above -FLT_MAX: 0
    mix = np.full(n, -np.inf, np.float32)
    mix[0] = np.nan
    mix[7] = -np.float32(3.0e38)
    rows.append(mix)
    x = np.stack(rows)
    idx = torch.zeros(len(rows), dtype=torch.int32, device="cuda:0")
    xd = dev(x)
    assert lib().rtxllm_argmax(P(xd), n, len(rows), P(idx), ops.stream()) == 0
    got = idx.cpu().numpy().view(np.uint32)
    for r in range(len(rows)):
        assert int(got[r]) == orc.argmax(x[r]), r
    assert int(got[1]) == 9 and int(got[3]) == 0 and int(got[4]) == 7


# ---- pointer alignment ---------------------------------------------------------

@pytest.mark.parametrize("fmt", [F.Q4K_SPLIT_NATIVE, F.Q5K, F.IQ2S, F.IQ3S], ids=lambda f: F.NAMES[f])
def test_misaligned_activation_accepted(fmt):
    """x at a 4-byte (not 16-byte) aligned address: the same result, bit for
    bit, as the aligned copy, through rtxllm_matvec and rtxllm_stage_activation."""
    rows, cols = 300, 4096
    pack = packs.make_pack(fmt, rows, cols, seed=71 + fmt)
    d = ops.DevicePack(pack)
    x = packs.normal_f32(72, cols)
    big = torch.zeros(cols + 4, dtype=torch.float32, device="cuda:0")
    big[1:1 + cols] = ops.to_dev(x)
    xm = big[1:1 + cols]
    assert xm.data_ptr() % 16 == 4
    ya = ops.matvec(d, ops.to_dev(x)).cpu().numpy()
    ym = torch.empty(rows, dtype=torch.float32, device="cuda:0")
    assert lib().rtxllm_matvec(fmt, P(d.payload), P(d.meta), xm.data_ptr(), P(ym), rows, cols, ops.stream()) == 0
    assert np.array_equal(ym.cpu().numpy().view(np.uint32), ya.view(np.uint32))
    xq_a = ops.stage(ops.to_dev(x)).cpu().numpy()
    xq_m = torch.empty(ops.xq_bytes(cols), dtype=torch.uint8, device="cuda:0")
    assert lib().rtxllm_stage_activation(xm.data_ptr(), None, cols, P(xq_m), ops.stream()) == 0
    assert np.array_equal(xq_m.cpu().numpy(), xq_a)


def test_misaligned_activation_reference_launcher(orc):
    rows, cols = 256, 2048
    pack = packs.make_pack(F.IQ3S, rows, cols, seed=81)
    d = ops.DevicePack(pack)
    x = packs.normal_f32(82, cols)
    big = torch.zeros(cols + 4, dtype=torch.float32, device="cuda:0")
    big[3:3 + cols] = ops.to_dev(x)
    logits = torch.zeros(rows, dtype=torch.float32, device="cuda:0")
    kv = torch.zeros(64, dtype=torch.float32, device="cuda:0")
    tok = torch.zeros(1, dtype=torch.int32, device="cuda:0")
    rc = lib().rtxllm_launch_iq3s_matvec_decode_probe(P(d.payload), big[3:].data_ptr(), P(logits), P(kv), P(tok),
                                                      rows, cols, rows, 64, 16, 4, ops.stream())
    assert rc == 0
    ya = ops.matvec(d, ops.to_dev(x)).cpu().numpy()
    assert np.array_equal(logits.cpu().numpy().view(np.uint32), ya.view(np.uint32))


def test_misaligned_weight_streams_refused():
    """Weight streams below the kernels' load alignment are refused before any
    launch (hipErrorInvalidValue): Q4_K payload / native metadata 16 bytes,
    split-half metadata 8, split-compact 4, Q5_K 16, IQ2_S / IQ3_S 2."""
    buf = torch.zeros(1 << 16, dtype=torch.uint8, device="cuda:0")
    x = torch.zeros(512, dtype=torch.float32, device="cuda:0")
    y = torch.zeros(64, dtype=torch.float32, device="cuda:0")
    base = buf.data_ptr()
    L, s = lib(), ops.stream()
    cases = [(F.Q4K_SPLIT_NATIVE, 8, 0), (F.Q4K_SPLIT_NATIVE, 0, 8), (F.Q4K_RAW, 4, None), (F.Q5K, 8, None),
             (F.Q4K_SPLIT_HALF, 0, 4), (F.Q4K_SPLIT_COMPACT, 0, 2), (F.IQ2S, 1, None), (F.IQ3S, 1, None),
             (F.IQ2S_UNITS, 8, None)]
    for fmt, poff, moff in cases:
        meta = None if moff is None else base + 32768 + moff
        assert L.rtxllm_matvec(fmt, base + poff, meta, P(x), P(y), 4, 512, s) == HIP_INVALID_VALUE, (fmt, poff, moff)
        assert L.rtxllm_dequant_f32(fmt, base + poff, meta, 4, 512, P(x), s) == HIP_INVALID_VALUE, fmt
    # an activation below 4-byte alignment is refused too
    assert L.rtxllm_matvec(F.IQ2S, base, None, x.data_ptr() + 2, P(y), 4, 512, s) == HIP_INVALID_VALUE
    torch.cuda.synchronize()
