"""Pins of the oracle's Llama-layer math (oracle/rtxllm_oracle.c), which the
reference does not contain: closed forms and special cases that reduce to a
textbook value, invariants (rotation preserves norms, a zero residual branch is
the identity, GQA head mapping by distinct constants, paging is a relabelling),
and brute force in float64 on tiny inputs. Each check is chosen so that a
plausible mistake (a dropped term, a wrong sign or pair order, a transposed
head mapping, a norm weight applied on the wrong side) fails it."""

from __future__ import annotations

import ctypes
import math

import numpy as np
import pytest

from rtxllm_amd import formats as F
from rtxllm_amd import packs


def f32(*a):
    return np.ascontiguousarray(np.array(a, dtype=np.float32).ravel())


# ---- RMSNorm (weighted) ------------------------------------------------------------

def test_rmsnorm_weighted_closed_forms(orc):
    lib, P = orc.lib(), orc.ptr
    n, eps = 256, 1e-6
    out = np.empty(n, np.float32)
    # constant vector c: x / rms = sign(c) * |c| / sqrt(c^2 + eps)
    x = np.full(n, 3.0, np.float32)
    w = np.ones(n, np.float32)
    lib.orc_rmsnorm_weighted(P(x), P(w), n, eps, P(out))
    assert np.allclose(out, 3.0 / math.sqrt(9.0 + eps), rtol=1e-6)
    # the weight multiplies after normalisation (scaling w scales the output, not the rms)
    w2 = np.linspace(0.5, 2.0, n).astype(np.float32)
    lib.orc_rmsnorm_weighted(P(x), P(w2), n, eps, P(out))
    assert np.allclose(out, w2 * (3.0 / math.sqrt(9.0 + eps)), rtol=1e-6)
    # eps dominates a tiny vector
    x = np.full(n, 1e-4, np.float32)
    lib.orc_rmsnorm_weighted(P(x), P(w), n, 1e-2, P(out))
    assert np.allclose(out, 1e-4 / math.sqrt(1e-8 + 1e-2), rtol=1e-5)


def test_rmsnorm_weighted_matches_f64(orc):
    lib, P = orc.lib(), orc.ptr
    rng = np.random.default_rng(1)
    n, eps = 4096, 1e-6
    x = rng.standard_normal(n).astype(np.float32)
    w = (1.0 + 0.02 * rng.standard_normal(n)).astype(np.float32)
    out = np.empty(n, np.float32)
    lib.orc_rmsnorm_weighted(P(x), P(w), n, eps, P(out))
    xd = x.astype(np.float64)
    ref = xd / np.sqrt(np.mean(xd * xd) + eps) * w
    assert np.max(np.abs(out - ref)) / np.max(np.abs(ref)) < 2e-6


# ---- RoPE ----------------------------------------------------------------------------

def test_rope_inv_freq_schedule(orc):
    lib, P = orc.lib(), orc.ptr
    inv = np.empty(64, np.float32)
    lib.orc_rope_inv_freq(128, 500000.0, P(inv))
    assert inv[0] == 1.0
    want = np.array([np.float32(500000.0 ** (-2.0 * i / 128.0)) for i in range(64)], np.float32)
    assert np.array_equal(inv, want)  # rounded once from double
    assert np.all(np.diff(inv) < 0)
    assert abs(float(inv[32]) - 500000.0 ** -0.5) < 1e-9


def test_rope_rotate_pair_quarter_turns(orc):
    lib = orc.lib()
    e, o = ctypes.c_float(), ctypes.c_float()
    # (1, 0) by +90 degrees -> (0, 1): e' = e cos - o sin, o' = e sin + o cos
    lib.orc_rope_rotate_pair(1.0, 0.0, math.pi / 2, ctypes.byref(e), ctypes.byref(o))
    assert abs(e.value) < 1e-7 and abs(o.value - 1.0) < 1e-7
    lib.orc_rope_rotate_pair(0.0, 1.0, math.pi / 2, ctypes.byref(e), ctypes.byref(o))
    assert abs(e.value + 1.0) < 1e-7 and abs(o.value) < 1e-7


def test_rope_adjacent_pairs_and_invariants(orc):
    lib, P = orc.lib(), orc.ptr
    hd, heads = 128, 3
    inv = np.empty(hd // 2, np.float32)
    lib.orc_rope_inv_freq(hd, 10000.0, P(inv))
    rng = np.random.default_rng(2)
    v = rng.standard_normal(heads * hd).astype(np.float32)
    # position 0 is the identity
    w = v.copy()
    lib.orc_rope(P(w), heads, hd, P(inv), 0)
    assert np.array_equal(w, v)
    # pairs are adjacent (2i, 2i+1), each rotated by pos * inv_freq[i]; norms kept
    pos = 37
    w = v.copy()
    lib.orc_rope(P(w), heads, hd, P(inv), pos)
    a = v.reshape(heads, hd // 2, 2).astype(np.float64)
    b = w.reshape(heads, hd // 2, 2).astype(np.float64)
    assert np.allclose(np.hypot(a[..., 0], a[..., 1]), np.hypot(b[..., 0], b[..., 1]), rtol=1e-5)
    ang = np.float32(pos) * inv
    unit = np.zeros(hd, np.float32)
    unit[2 * 5] = 1.0  # pair 5, even element
    lib.orc_rope(P(unit), 1, hd, P(inv), pos)
    assert abs(unit[10] - math.cos(float(ang[5]))) < 1e-5 and abs(unit[11] - math.sin(float(ang[5]))) < 1e-5
    assert np.count_nonzero(unit) == 2  # nothing leaks into other pairs
    # composition: rotating by a then b equals rotating by a + b (up to fp32 angles)
    w1 = v.copy()
    lib.orc_rope(P(w1), heads, hd, P(inv), 5)
    lib.orc_rope(P(w1), heads, hd, P(inv), 7)
    w2 = v.copy()
    lib.orc_rope(P(w2), heads, hd, P(inv), 12)
    assert np.max(np.abs(w1 - w2)) < 1e-4


# ---- SiLU-gate -----------------------------------------------------------------------

def test_silu_mul_known_values(orc):
    lib, P = orc.lib(), orc.ptr
    g = f32(0.0, 1.0, -1.0, 20.0, -20.0, 2.0)
    u = f32(5.0, 1.0, 1.0, 1.0, 1.0, -3.0)
    out = np.empty(6, np.float32)
    lib.orc_silu_mul(P(g), P(u), 6, P(out))
    sig = lambda t: 1.0 / (1.0 + math.exp(-t))  # noqa: E731
    want = [0.0, 0.7310585786300049, -0.2689414213699951, 20.0 * sig(20.0), -20.0 * sig(-20.0), -3.0 * 2.0 * sig(2.0)]
    assert np.allclose(out, want, rtol=1e-6, atol=1e-12)


# ---- embedding gather ----------------------------------------------------------------

def test_embed_q5k_is_the_dequantised_row(orc):
    lib, P = orc.lib(), orc.ptr
    vocab, cols = 7, 512
    pack = packs.make_pack(F.Q5K, vocab, cols, 0x5EED1234)
    full = orc.dequant(F.Q5K, pack.payload, None, vocab, cols)
    out = np.empty(cols, np.float32)
    for token in (0, 3, 6):
        lib.orc_embed_q5k(P(pack.payload), cols, token, P(out))
        assert np.array_equal(out, full[token])


# ---- paged fp16 KV + GQA attention ------------------------------------------------------

def make_cache(orc, n_pages, n_kv, page, hd, table=None):
    k = np.zeros(n_pages * n_kv * page * hd, np.uint16)
    v = np.zeros_like(k)
    t = np.arange(n_pages, dtype=np.int32) if table is None else np.ascontiguousarray(table, np.int32)
    kv = orc.KvCache(orc.ptr(k), orc.ptr(v), orc.ptr(t), page, n_kv, hd)
    return kv, k, v, t


def append(orc, kv, pos, k, v):
    orc.lib().orc_kv_append(ctypes.byref(kv), pos, orc.ptr(k), orc.ptr(v))


def attention(orc, kv, q, n_heads, pos, hd):
    out = np.empty(n_heads * hd, np.float32)
    orc.lib().orc_attention_decode(ctypes.byref(kv), orc.ptr(q), n_heads, pos, orc.ptr(out))
    return out


def test_attention_single_position_returns_v(orc):
    hd, n_kv, n_heads = 8, 2, 4
    kv, *_ = make_cache(orc, 2, n_kv, 4, hd)
    rng = np.random.default_rng(3)
    k = rng.standard_normal(n_kv * hd).astype(np.float32)
    v = rng.standard_normal(n_kv * hd).astype(np.float32)
    append(orc, kv, 0, k, v)
    q = rng.standard_normal(n_heads * hd).astype(np.float32)
    out = attention(orc, kv, q, n_heads, 0, hd).reshape(n_heads, hd)
    v16 = v.astype(np.float16).astype(np.float32).reshape(n_kv, hd)
    # query heads 0,1 read kv head 0; heads 2,3 read kv head 1 (h / group)
    assert np.array_equal(out[0], v16[0]) and np.array_equal(out[1], v16[0])
    assert np.array_equal(out[2], v16[1]) and np.array_equal(out[3], v16[1])


def test_attention_equal_scores_average_v(orc):
    hd, n_kv, n_heads, npos = 8, 1, 2, 5
    kv, *_ = make_cache(orc, 2, n_kv, 4, hd)
    for p in range(npos):
        append(orc, kv, p, np.ones(hd, np.float32), np.full(hd, float(p + 1), np.float32))
    q = np.zeros(n_heads * hd, np.float32)  # all scores 0 -> uniform weights
    out = attention(orc, kv, q, n_heads, npos - 1, hd)
    assert np.allclose(out, 3.0, rtol=1e-6)  # mean of 1..5
    # only positions 0..pos count (causal): pos = 1 -> mean of 1, 2
    out = attention(orc, kv, q, n_heads, 1, hd)
    assert np.allclose(out, 1.5, rtol=1e-6)


def test_attention_matches_f64_and_paging_is_a_relabelling(orc):
    hd, n_kv, n_heads, page, npos = 16, 2, 6, 4, 11
    n_pages = 3
    rng = np.random.default_rng(4)
    ks = rng.standard_normal((npos, n_kv * hd)).astype(np.float32)
    vs = rng.standard_normal((npos, n_kv * hd)).astype(np.float32)
    q = rng.standard_normal(n_heads * hd).astype(np.float32)
    outs = []
    for table in (None, [2, 0, 1]):
        kv, *_ = make_cache(orc, n_pages, n_kv, page, hd, table)
        for p in range(npos):
            append(orc, kv, p, ks[p], vs[p])
        outs.append(attention(orc, kv, q, n_heads, npos - 1, hd))
    assert np.array_equal(outs[0], outs[1])
    k16 = ks.astype(np.float16).astype(np.float64).reshape(npos, n_kv, hd)
    v16 = vs.astype(np.float16).astype(np.float64).reshape(npos, n_kv, hd)
    group = n_heads // n_kv
    ref = np.empty((n_heads, hd))
    for h in range(n_heads):
        s = k16[:, h // group] @ q.reshape(n_heads, hd)[h].astype(np.float64) / math.sqrt(hd)
        p = np.exp(s - s.max())
        ref[h] = (p / p.sum()) @ v16[:, h // group]
    assert np.max(np.abs(outs[0] - ref.ravel())) / np.max(np.abs(ref)) < 1e-5


# ---- the layer: composition and residual structure ---------------------------------------

def tiny_layer(orc, seed, zero_o=False, zero_down=False):
    H, nh, nkv, hd, ff = 256, 2, 1, 128, 512
    fq = fo = F.IQ3S
    fgu, fdn = F.IQ2S, F.Q4K_SPLIT_NATIVE
    mk = lambda f, r, c, s: packs.make_pack(f, r, c, seed + s)  # noqa: E731
    wq, wk, wv, wo = mk(fq, nh * hd, H, 1), mk(fq, nkv * hd, H, 2), mk(fq, nkv * hd, H, 3), mk(fo, H, nh * hd, 4)
    wg, wu, wd = mk(fgu, ff, H, 5), mk(fgu, ff, H, 6), mk(fdn, H, ff, 7)
    if zero_o:
        wo.payload[:] = 0  # d = 0 in every block: W = 0
    if zero_down:
        wd.payload[:] = 0
        wd.meta[:] = 0
    an = packs.normal_f32(seed + 8, H, mean=1.0, std=0.02)
    fn = packs.normal_f32(seed + 9, H, mean=1.0, std=0.02)
    return dict(H=H, nh=nh, nkv=nkv, hd=hd, ff=ff, f=(fq, fo, fgu, fdn), w=(wq, wk, wv, wo, wg, wu, wd), an=an, fn=fn)


def run_layer(orc, L, h, pos, kvc, given_kv=False):
    P = orc.ptr
    wq, wk, wv, wo, wg, wu, wd = L["w"]
    fq, fo, fgu, fdn = L["f"]
    w = orc.LayerWeights(fq, fq, fq, fo, fgu, fgu, fdn,
                         P(wq.payload), None, P(wk.payload), None, P(wv.payload), None, P(wo.payload), None,
                         P(wg.payload), None, P(wu.payload), None, P(wd.payload), P(wd.meta), P(L["an"]), P(L["fn"]))
    inv = np.empty(L["hd"] // 2, np.float32)
    orc.lib().orc_rope_inv_freq(L["hd"], 500000.0, P(inv))
    shape = orc.LayerShape(L["H"], L["nh"], L["nkv"], L["hd"], L["ff"], 1e-6, P(inv))
    out = h.copy()
    fwd = orc.lib().orc_layer_forward_given_kv if given_kv else orc.lib().orc_layer_forward
    fwd(ctypes.byref(w), ctypes.byref(shape), ctypes.byref(kvc), pos, P(out), 1)
    return out


def test_layer_given_kv_equals_layer_on_the_same_cache(orc):
    """orc_layer_forward_given_kv on the cache state orc_layer_forward left
    (its own K / V of pos appended) gives the same h bit for bit; on a cache
    whose slot holds other values it differs (the slot is really read)."""
    L = tiny_layer(orc, 0x5EED2200)
    kvc, kpages, vpages, _ = make_cache(orc, 2, L["nkv"], 16, L["hd"])
    for p in range(5):
        append(orc, kvc, p, packs.normal_f32(0x5EED2300 + p, L["nkv"] * L["hd"]),
               packs.normal_f32(0x5EED2400 + p, L["nkv"] * L["hd"]))
    h = packs.normal_f32(0x5EED2500, L["H"])
    out = run_layer(orc, L, h, 5, kvc)  # appends its K / V of position 5
    again = run_layer(orc, L, h, 5, kvc, given_kv=True)
    assert np.array_equal(out.view(np.uint32), again.view(np.uint32))
    append(orc, kvc, 5, np.zeros(L["nkv"] * L["hd"], np.float32), np.zeros(L["nkv"] * L["hd"], np.float32))
    assert not np.array_equal(run_layer(orc, L, h, 5, kvc, given_kv=True), out)


def test_layer_zero_branches_are_identity(orc):
    L = tiny_layer(orc, 0x5EED2000, zero_o=True, zero_down=True)
    kvc, *_ = make_cache(orc, 2, L["nkv"], 16, L["hd"])
    h = packs.normal_f32(0x5EED2100, L["H"])
    out = run_layer(orc, L, h, 3, kvc)
    assert np.array_equal(out, h)  # h + 0 + 0


@pytest.mark.parametrize("pos", [0, 9])
def test_layer_matches_f64_composition(orc, pos):
    L = tiny_layer(orc, 0x5EED3000)
    H, nh, nkv, hd, ff = L["H"], L["nh"], L["nkv"], L["hd"], L["ff"]
    wq, wk, wv, wo, wg, wu, wd = L["w"]
    rng = np.random.default_rng(5)
    kvc, kpages, vpages, _ = make_cache(orc, 2, nkv, 16, hd)
    # positions before pos already hold K/V
    prev_k = rng.standard_normal((pos, nkv * hd)).astype(np.float32)
    prev_v = rng.standard_normal((pos, nkv * hd)).astype(np.float32)
    for p in range(pos):
        append(orc, kvc, p, prev_k[p], prev_v[p])
    h = packs.normal_f32(0x5EED3100, H)
    out = run_layer(orc, L, h, pos, kvc)

    # float64 restatement built from pinned pieces (dequant) and closed forms
    def W(pk, r, c):
        return orc.dequant(pk.fmt, pk.payload, pk.meta, r, c).astype(np.float64)

    def rms(x, w):
        return x / np.sqrt(np.mean(x * x) + 1e-6) * w

    inv = np.array([500000.0 ** (-2.0 * i / hd) for i in range(hd // 2)])

    def rope(x, n):
        x = x.reshape(n, hd // 2, 2).copy()
        ang = pos * inv
        c, s = np.cos(ang), np.sin(ang)
        e, o = x[..., 0].copy(), x[..., 1].copy()
        x[..., 0], x[..., 1] = e * c - o * s, e * s + o * c
        return x.ravel()

    hd64 = h.astype(np.float64)
    xn = rms(hd64, L["an"])
    q = rope(W(wq, nh * hd, H) @ xn, nh)
    k = rope(W(wk, nkv * hd, H) @ xn, nkv)
    v = W(wv, nkv * hd, H) @ xn
    K = np.vstack([prev_k, k[None, :]]).astype(np.float16).astype(np.float64).reshape(pos + 1, nkv, hd)
    V = np.vstack([prev_v, v[None, :]]).astype(np.float16).astype(np.float64).reshape(pos + 1, nkv, hd)
    att = np.empty(nh * hd)
    for hh in range(nh):
        s = K[:, hh // (nh // nkv)] @ q[hh * hd:(hh + 1) * hd] / math.sqrt(hd)
        p = np.exp(s - s.max())
        att[hh * hd:(hh + 1) * hd] = (p / p.sum()) @ V[:, hh // (nh // nkv)]
    h1 = hd64 + W(wo, H, nh * hd) @ att
    xn2 = rms(h1, L["fn"])
    g, u = W(wg, ff, H) @ xn2, W(wu, ff, H) @ xn2
    act = g / (1.0 + np.exp(-g)) * u
    ref = h1 + W(wd, H, ff) @ act
    err = np.max(np.abs(out - ref)) / np.max(np.abs(ref))
    assert err < 2e-4, err  # fp32 oracle vs float64, K/V rounded to fp16 in both


# ---- the reference runner's feedback family (unweighted RMSNorm over `rows` logits) ------

def test_feedback_family_closed_forms(orc):
    lib, P = orc.lib(), orc.ptr
    rows, cols, eps = 4, 10, 1e-6
    logits = f32(1.0, -2.0, 3.0, -4.0)
    inv = 1.0 / math.sqrt((1 + 4 + 9 + 16) / 4.0 + eps)  # rsqrt(mean(logits^2) + eps)
    n = np.array([logits[c % rows] * inv for c in range(cols)], np.float64)  # cyclic over rows
    silu = n / (1.0 + np.exp(-n))
    act = np.empty(cols, np.float32)
    cache = np.empty(cols, np.float32)
    lib.orc_rmsnorm_feedback(P(logits), rows, P(act), cols, eps)
    assert np.allclose(act, n, rtol=1e-6)
    lib.orc_silu_rmsnorm_feedback(P(logits), rows, P(act), cols, eps)
    assert np.allclose(act, silu, rtol=1e-6)
    lib.orc_rmsnorm_feedback_with_silu_cache(P(logits), rows, P(act), P(cache), cols, eps)
    assert np.allclose(act, n, rtol=1e-6) and np.allclose(cache, silu, rtol=1e-6)
    gate = f32(0.5, 2.0, -1.0)  # cache_cols = 3: act[c] = silu_cache[c % 3] * n[c]
    lib.orc_gated_silu_rmsnorm_feedback(P(logits), rows, P(gate), 3, P(act), cols, eps)
    assert np.allclose(act, [gate[c % 3] * n[c] for c in range(cols)], rtol=1e-6)
    # cache kernels: plain, SiLU, accumulate
    lib.orc_rmsnorm_cache(P(logits), rows, P(cache), cols, eps, 0, 0)
    assert np.allclose(cache, n, rtol=1e-6)
    lib.orc_rmsnorm_cache(P(logits), rows, P(cache), cols, eps, 1, 1)
    assert np.allclose(cache, n + silu, rtol=1e-6)
    up = np.ones(cols, np.float32)
    g2 = np.linspace(-1, 1, cols).astype(np.float32)
    lib.orc_rmsnorm_cache_and_gated_product(P(logits), rows, P(g2), P(up), P(act), cols, cols, eps, 1)
    assert np.allclose(up, 1.0 + n, rtol=1e-6) and np.allclose(act, g2 * (1.0 + n), rtol=1e-6, atol=1e-7)
