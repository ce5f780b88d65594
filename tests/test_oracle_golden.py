"""Pins the CPU oracle: the reference's own known answers for this path, closed
forms, exhaustive checks and an independent numpy decode. CPU only."""

from __future__ import annotations

import hashlib
import struct

import numpy as np
import pytest

import np_decode

Q4K_RAW, SPLIT_PRE, SPLIT_HALF, SPLIT_COMPACT, SPLIT_NATIVE, Q5K, IQ2S, IQ3S = range(8)


def half(v: float) -> bytes:
    return struct.pack("<e", v)


def sample_q4k_block() -> bytes:
    """runtime/tests/unit/test_q4k_resident_pack.py:20-27."""
    block = bytearray(144)
    block[0:2] = half(0.5)
    block[2:4] = half(0.25)
    block[4:16] = bytes([1, 2, 3, 4, 5, 6, 7, 8, 0x40, 0x80, 0xC0, 0x00])
    for i in range(128):
        block[16 + i] = i & 0xFF
    return bytes(block)


def u8(b: bytes) -> np.ndarray:
    return np.frombuffer(b, dtype=np.uint8).copy()


# ---- fp16 ------------------------------------------------------------------


def test_fp16_to_f32_exhaustive(orc):
    codes = np.arange(65536, dtype=np.uint16)
    ref = codes.view(np.float16).astype(np.float32)
    got = np.array([orc.lib().orc_fp16_to_f32(int(c)) for c in codes], dtype=np.float32)
    nan = np.isnan(ref)
    assert np.array_equal(got[~nan].view(np.uint32), ref[~nan].view(np.uint32))
    # main.cpp:1094-1096: any NaN code decodes to the canonical +quiet NaN.
    assert np.all(got[nan].view(np.uint32) == 0x7FC00000)


def test_f32_to_fp16_rne_matches_numpy(orc):
    rng = np.random.default_rng(7)
    vals = np.concatenate([
        rng.standard_normal(20000).astype(np.float32) * np.float32(3e-3),
        rng.uniform(-70000, 70000, 5000).astype(np.float32),
        (np.arange(1, 5000, dtype=np.float32) * np.float32(2.0 ** -25)),  # subnormal ties
        np.array([0.0, -0.0, 65504.0, 65519.99, 65520.0, np.inf, -np.inf, 2.0 ** -24, 2.0 ** -25, 3 * 2.0 ** -26],
                 np.float32),
    ])
    ref = vals.astype(np.float16).view(np.uint16)
    got = np.array([orc.lib().orc_f32_to_fp16_rne(float(v)) for v in vals], dtype=np.uint16)
    assert np.array_equal(got, ref)


# ---- get_scale_min_k4 ---------------------------------------------------------


def scale_min(orc, j: int, packed: bytes) -> tuple[int, int]:
    import ctypes

    buf = (ctypes.c_uint8 * 12).from_buffer_copy(packed)
    sc, m = ctypes.c_uint8(), ctypes.c_uint8()
    orc.lib().orc_scale_min_k4(j, ctypes.addressof(buf), ctypes.addressof(sc), ctypes.addressof(m))
    return sc.value, m.value


def test_scale_min_known_answers(orc):
    """test_q4k_resident_pack.py:31-37."""
    scales = sample_q4k_block()[4:16]
    assert scale_min(orc, 0, scales) == (1, 5)
    assert scale_min(orc, 3, scales) == (4, 8)
    assert scale_min(orc, 4, scales) == (0, 4)
    assert scale_min(orc, 5, scales) == (0, 8)
    assert scale_min(orc, 6, scales) == (0, 12)


def test_scale_min_bit_definition(orc):
    """Brute force against the 6-bit field packing: scales 0-3 are the low 6 bits
    of bytes 0-3, mins 0-3 the low 6 bits of bytes 4-7; scales/mins 4-7 take
    their low nibble from bytes 8-11 and their top two bits from the spare high
    bits of bytes 0-3 / 4-7."""
    rng = np.random.default_rng(1)
    for _ in range(300):
        p = rng.integers(0, 256, 12, dtype=np.uint8).tobytes()
        bits = int.from_bytes(p, "little")
        for j in range(8):
            if j < 4:
                sc = (bits >> (8 * j)) & 63
                m = (bits >> (8 * (j + 4))) & 63
            else:
                k = j - 4
                sc = ((bits >> (8 * (k + 8))) & 15) | (((bits >> (8 * k + 6)) & 3) << 4)
                m = ((bits >> (8 * (k + 8) + 4)) & 15) | (((bits >> (8 * (k + 4) + 6)) & 3) << 4)
            assert scale_min(orc, j, p) == (sc, m)


# ---- Q4_K resident split (test_q4k_resident_pack.py:39-66) ------------------


@pytest.mark.parametrize("fmt,mb", [(SPLIT_PRE, 64), (SPLIT_HALF, 32), (SPLIT_COMPACT, 20), (SPLIT_NATIVE, 16)])
def test_q4k_split_known_answers(orc, fmt, mb):
    block = sample_q4k_block()
    payload, meta = orc.q4k_split(fmt, u8(block), mb)
    assert payload.size == 128 and payload[:4].tolist() == [0, 1, 2, 3] and payload[-1] == 127
    assert meta.size == mb
    if fmt == SPLIT_PRE:
        assert struct.unpack("<ff", meta[:8].tobytes()) == (0.5, 1.25)
    elif fmt == SPLIT_COMPACT:
        assert meta[:4].tobytes() == block[:4]
        assert meta[4:8].tolist() == [1, 2, 3, 4]
        assert meta[12:16].tolist() == [5, 6, 7, 8]
    elif fmt == SPLIT_NATIVE:
        assert meta.tobytes() == block[:16]
    else:  # half: the same products rounded to fp16 (struct '<e')
        assert struct.unpack("<ee", meta[:4].tobytes()) == (0.5, 1.25)


def test_q4k_split_half_rounds_like_python_struct(orc):
    rng = np.random.default_rng(3)
    raw = rng.integers(0, 256, 144 * 64, dtype=np.uint8)
    raw.reshape(64, 144)[:, 0:2] = np.frombuffer(np.float16(rng.uniform(1e-4, 2e-3, 64)).tobytes(), np.uint8).reshape(64, 2)
    raw.reshape(64, 144)[:, 2:4] = np.frombuffer(np.float16(rng.uniform(1e-4, 2e-3, 64)).tobytes(), np.uint8).reshape(64, 2)
    _, pre = orc.q4k_split(SPLIT_PRE, raw, 64)
    _, hal = orc.q4k_split(SPLIT_HALF, raw, 32)
    products = np.frombuffer(pre.tobytes(), np.float32)
    expect = b"".join(struct.pack("<e", float(v)) for v in products)
    assert hal.tobytes() == expect


# ---- block sizes (test_gguf_block_formats.py:19-24, test_iq_resident_pack.py) --


def test_block_format_sizes(orc):
    blk = {0: 144, 5: 176, 6: 82, 7: 110}
    for f, b in blk.items():
        assert orc.lib().orc_payload_bytes(f) == b
    assert (2048 * 8192 // 256) * 144 == 9_437_184
    assert (2048 * 248320 // 256) * 176 == 349_634_560
    assert (2048 * 512 * 256 // 256) * 82 == 85_983_232
    assert (512 * 2048 * 256 // 256) * 110 == 115_343_360
    assert 2048 * 512 * 128 // 256 == 524_288
    assert [orc.lib().orc_meta_bytes(f) for f in (1, 2, 3, 4)] == [64, 32, 20, 16]


# ---- grid tables --------------------------------------------------------------


def test_grid_tables_pinned(orc):
    g2 = orc.iq2s_grid()
    g3 = orc.iq3s_grid()
    assert g2.size == 1024 and int(g2.sum()) == 16_519_059 and int(g2.max()) == 43_690
    assert np.all(np.diff(g2.astype(np.int64)) > 0)
    assert hashlib.sha256(g2.astype("<u2").tobytes()).hexdigest() == (
        "e6e75e121b65e8afa5c1f92b71463cfbe217b83893f438acde22fd5db06a43f7")
    assert g3.size == 512 and int(g3.astype(np.uint64).sum()) == 53_294_177_878
    assert np.all(np.diff(g3.astype(np.int64)) > 0)
    assert hashlib.sha256(g3.astype("<u4").tobytes()).hexdigest() == (
        "bd1af4945a1717c65610b0284e4628b9a1ba3b306fae3a06f6e5f597356e349f")
    b = g3.view(np.uint8)
    assert set(np.unique(b).tolist()) <= {1, 3, 5, 7, 9, 11, 13, 15}


# ---- dequant: hand-worked values -------------------------------------------------


def test_q4k_dequant_hand_values(orc):
    blk = u8(sample_q4k_block())
    out = orc.dequant(Q4K_RAW, blk, None, 1, 256)[0]
    # v=0: q=lo(0)=0, sc0=1, m0=5: 0.5*1*0 - 0.25*5
    assert out[0] == -1.25
    assert out[1] == -0.75  # q=1
    assert out[32] == -1.5  # pair 1: sc=2, m=6, q=hi(0)=0
    assert out[48] == -0.5  # q=hi(16)=1: 0.5*2*1 - 1.5
    assert out[128] == -1.0  # pair 4: sc=0, m=4
    assert out[129] == -1.0
    assert out[255] == 0.0  # pair 7: sc = 0, m = 0
    # split-native (payload + 16-byte head) decodes identically to the raw block
    payload, meta = orc.q4k_split(SPLIT_NATIVE, blk, 16)
    assert np.array_equal(orc.dequant(SPLIT_NATIVE, payload, meta, 1, 256)[0].view(np.uint32), out.view(np.uint32))


def test_iq3s_dequant_hand_values(orc):
    g3 = orc.iq3s_grid()
    blk = np.zeros(110, np.uint8)
    blk[0:2] = np.frombuffer(half(1.0), np.uint8)
    blk[106] = 0x21  # ib32 0 -> nibble 1 (scale 3), ib32 1 -> nibble 2 (scale 5)
    blk[2] = 1  # selector 0 -> grid[1] = 0x01010103
    blk[74] = 0x01  # sign of value 0
    out = orc.dequant(IQ3S, blk, None, 1, 256)[0]
    assert g3[1] == 0x01010103 and g3[0] == 0x01010101
    assert out[0] == -9.0 and out[1] == 3.0 and out[4] == 3.0
    assert out[32] == 5.0
    blk[66] = 0x01  # high bit of selector 0 -> grid[257]
    out = orc.dequant(IQ3S, blk, None, 1, 256)[0]
    assert out[0] == -3.0 * (int(g3[257]) & 0xFF)
    assert out[3] == 3.0 * ((int(g3[257]) >> 24) & 0xFF)


def test_iq2s_dequant_hand_values(orc):
    g2 = orc.iq2s_grid()
    blk = np.zeros(82, np.uint8)
    blk[0:2] = np.frombuffer(half(1.0), np.uint8)
    out = orc.dequant(IQ2S, blk, None, 1, 256)[0]
    assert np.all(out == 0.125)  # grid[0] = 0 -> magnitude 1, scale (0.5 + 0) * 0.25
    blk[2] = 2  # group 0 -> grid[2] = 0x0005: lanes 0, 1 have l=1 -> magnitude 3
    blk[74] = 0xF0  # ib32 0: low nibble 0 (groups 0, 1), high nibble 15 (groups 2, 3)
    blk[34] = 0x02  # sign of value 1
    out = orc.dequant(IQ2S, blk, None, 1, 256)[0]
    assert g2[2] == 0x0005
    assert out[0] == 0.375 and out[1] == -0.375 and out[2] == 0.125
    assert out[16] == 3.875  # group 2: (0.5 + 15) * 0.25, magnitude 1
    blk[66] = 0x01  # qh bits 0-1 -> group 0 index += 256
    out = orc.dequant(IQ2S, blk, None, 1, 256)[0]
    l0 = int(g2[256 + 2]) & 3
    assert out[0] == 0.125 * (2 * l0 + 1)


def test_q5k_dequant_hand_values(orc):
    blk = np.zeros(176, np.uint8)
    blk[0:2] = np.frombuffer(half(1.0), np.uint8)
    blk[2:4] = np.frombuffer(half(0.5), np.uint8)
    blk[4] = 1  # sc0 = 1
    blk[5] = 2  # sc1 = 2
    blk[8] = 3  # m0 = 3
    blk[48] = 0x2F  # qs[0]: lo 15 (value 0), hi 2 (value 32)
    blk[16] = 0x01  # qh[0] bit0: value 0 gets +16
    out = orc.dequant(Q5K, blk, None, 1, 256)[0]
    assert out[0] == 31.0 - 1.5
    assert out[32] == 2.0 * 2.0  # pair 1: sc 2, m 0, q 2
    blk[16] = 0x03
    out = orc.dequant(Q5K, blk, None, 1, 256)[0]
    assert out[32] == 2.0 * 18.0


# ---- dequant: independent numpy decode + exactness -------------------------------


def rand_blocks(fmt_bytes: int, n: int, seed: int, d_fields: int) -> np.ndarray:
    rng = np.random.default_rng(seed)
    b = rng.integers(0, 256, (n, fmt_bytes), dtype=np.uint8)
    for k in range(d_fields):
        d = np.float16(rng.uniform(1e-4, 2e-3, n))
        b[:, 2 * k : 2 * k + 2] = np.frombuffer(d.tobytes(), np.uint8).reshape(n, 2)
    return b.reshape(-1)


def test_dequant_matches_numpy_decode(orc):
    n = 96
    q4 = rand_blocks(144, n, 11, 2)
    ref = np_decode.q4k_raw(q4)
    assert np.array_equal(orc.dequant(Q4K_RAW, q4, None, n, 256).view(np.uint32), ref.view(np.uint32))
    for fmt, mb in [(SPLIT_PRE, 64), (SPLIT_HALF, 32), (SPLIT_COMPACT, 20), (SPLIT_NATIVE, 16)]:
        p, m = orc.q4k_split(fmt, q4, mb)
        got = orc.dequant(fmt, p, m, n, 256)
        if fmt == SPLIT_HALF:
            S = np.frombuffer(m.tobytes(), np.float16).reshape(n, 8, 2)[:, :, 0].astype(np.float32)
            M = np.frombuffer(m.tobytes(), np.float16).reshape(n, 8, 2)[:, :, 1].astype(np.float32)
            exp = np_decode.q4k_from_parts(S, M, p.reshape(n, 128))
        else:
            exp = ref
        assert np.array_equal(got.view(np.uint32), exp.view(np.uint32)), fmt
    q5 = rand_blocks(176, n, 12, 2)
    assert np.array_equal(orc.dequant(Q5K, q5, None, n, 256).view(np.uint32), np_decode.q5k(q5).view(np.uint32))
    i2 = rand_blocks(82, n, 13, 1)
    assert np.array_equal(orc.dequant(IQ2S, i2, None, n, 256).view(np.uint32),
                          np_decode.iq2s(i2, orc.iq2s_grid()).view(np.uint32))
    i3 = rand_blocks(110, n, 14, 1)
    assert np.array_equal(orc.dequant(IQ3S, i3, None, n, 256).view(np.uint32),
                          np_decode.iq3s(i3, orc.iq3s_grid()).view(np.uint32))


def test_dequant_products_are_exact(orc):
    """Every dequant product is exact in fp32, so the value equals the exact real
    number rounded once; computing it in float64 and rounding must agree."""
    n = 64
    q4 = rand_blocks(144, n, 21, 2).reshape(n, 144)
    got = orc.dequant(Q4K_RAW, q4.reshape(-1), None, n, 256)
    d = np_decode.f16(q4[:, 0], q4[:, 1]).astype(np.float64)
    dmin = np_decode.f16(q4[:, 2], q4[:, 3]).astype(np.float64)
    sc, m = np_decode.scale_min(q4[:, 4:16])
    qs = q4[:, 16:].reshape(n, 4, 32)
    q = np.empty((n, 8, 32))
    q[:, 0::2] = qs & 15
    q[:, 1::2] = qs >> 4
    exact = d[:, None, None] * sc[:, :, None] * q - dmin[:, None, None] * m[:, :, None]
    assert np.array_equal(got.reshape(n, 8, 32), exact.astype(np.float32))


# ---- matvec -------------------------------------------------------------------


def test_matvec_f32_threads_bit_identical_and_close_to_f64(orc):
    rows, cols = 64, 1024
    blocks = rand_blocks(110, rows * cols // 256, 31, 1)
    x = np.random.default_rng(5).standard_normal(cols).astype(np.float32)
    y1 = orc.matvec_f32(IQ3S, blocks, None, x, rows, cols, 1)
    y4 = orc.matvec_f32(IQ3S, blocks, None, x, rows, cols, 4)
    assert np.array_equal(y1.view(np.uint32), y4.view(np.uint32))
    y64 = orc.matvec_f64(IQ3S, blocks, None, x, rows, cols, 1)
    W = orc.dequant(IQ3S, blocks, None, rows, cols).astype(np.float64)
    assert np.allclose(y64, W @ x.astype(np.float64), rtol=1e-12, atol=1e-12)
    assert np.max(np.abs(y1 - y64)) / np.max(np.abs(y64)) < 1e-5


def test_matvec_sequential_order(orc):
    """main.cpp:1266-1289: acc += w*x over columns in order, in fp32."""
    rows, cols = 3, 512
    blocks = rand_blocks(144, rows * cols // 256, 41, 2)
    x = np.random.default_rng(6).standard_normal(cols).astype(np.float32)
    W = orc.dequant(Q4K_RAW, blocks, None, rows, cols)
    exp = np.zeros(rows, np.float32)
    for r in range(rows):
        acc = np.float32(0)
        for c in range(cols):
            acc = np.float32(acc + np.float32(W[r, c] * x[c]))
        exp[r] = acc
    got = orc.matvec_f32(Q4K_RAW, blocks, None, x, rows, cols, 1)
    assert np.array_equal(got.view(np.uint32), exp.view(np.uint32))


# ---- argmax / KV side-write ------------------------------------------------------


def test_argmax_rules(orc):
    assert orc.argmax(np.array([1, 3, 3, 2], np.float32)) == 1  # ties -> lowest index
    assert orc.argmax(np.array([np.nan, 0.5, np.nan], np.float32)) == 1  # NaN never wins
    assert orc.argmax(np.array([-np.inf, -np.inf], np.float32)) == 0
    y = np.random.default_rng(2).standard_normal(100_000).astype(np.float32)
    assert orc.argmax(y) == int(np.argmax(y))


def test_kv_side_write_closed_form(orc):
    rows, kv_words, page_words, active, token = 40, 97, 8, 30, 1234
    y = np.arange(rows, dtype=np.float32) + 0.5
    kv = np.zeros(kv_words, np.float32)
    orc.lib().orc_kv_side_write(orc.ptr(y), rows, orc.ptr(kv), kv_words, page_words, active, token)
    exp = np.zeros(kv_words, np.float32)
    for r in range(min(rows, active)):
        exp[(r * page_words + (token + r) % page_words) % kv_words] = y[r]
    assert np.array_equal(kv, exp)
