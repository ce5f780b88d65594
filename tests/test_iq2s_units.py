"""CPU checks of the unit layouts' host restatements (packs.iq2s_units,
packs.iq3s_units), which the GPU packers must match byte for byte: the
regrouping is a bijection of the tensor's bytes (IQ3_S: plus one copy of each
scale byte), it inverts, and hand-placed fields of a two-block tensor land
where the layout puts them."""

from __future__ import annotations

import numpy as np

from rtxllm_amd import formats as F
from rtxllm_amd import packs


def test_unit_order_is_a_permutation_and_inverts():
    for n in (1, 2, 7, 48):
        order = packs.iq2s_unit_order(n)
        assert np.array_equal(np.sort(order), np.arange(82 * n))
        raw = np.random.default_rng(n).integers(0, 256, 82 * n, dtype=np.uint8)
        assert np.array_equal(packs.iq2s_from_units(packs.iq2s_units(raw)), raw)


def test_two_block_fields_by_hand():
    # block b byte i = 100 b + i (i < 82) marks every source byte
    n = 2
    raw = np.array([(100 * b + i) % 256 for b in range(n) for i in range(82)], np.uint8)
    u = packs.iq2s_units(raw)
    # unit k = 3 of block 1: qs bytes 2 + 12 .. 2 + 15, sign bytes 34 + 12 .. 34 + 15
    assert list(u[64 * 1 + 8 * 3: 64 * 1 + 8 * 3 + 8]) == [100 + i for i in (14, 15, 16, 17, 46, 47, 48, 49)]
    # (qh[k], scales[k]) of unit 5 of block 0 at 64 N + 2 k, of block 1 at 64 N + 16 + 2 k
    assert list(u[64 * n + 10: 64 * n + 12]) == [66 + 5, 74 + 5]
    assert list(u[64 * n + 16 + 10: 64 * n + 16 + 12]) == [100 + 71, 100 + 79]
    # the two d fields at the end
    assert list(u[80 * n: 82 * n]) == [0, 1, 100, 101]


def test_unit_format_sizes():
    assert F.PAYLOAD_BYTES[F.IQ2S_UNITS] == F.PAYLOAD_BYTES[F.IQ2S] == 82
    assert F.meta_bytes(F.IQ2S_UNITS) == 0
    pack = packs.make_pack(F.IQ2S_UNITS, 3, 512, seed=5)
    assert np.array_equal(packs.iq2s_from_units(pack.payload), packs.make_pack(F.IQ2S, 3, 512, seed=5).payload)


def test_iq3s_unit_order_and_fields_by_hand():
    for n in (1, 3, 40):
        order = packs.iq3s_unit_order(n)
        assert len(set(order.tolist())) == 110 * n and order.max() < 114 * n
        raw = np.random.default_rng(n).integers(0, 256, 110 * n, dtype=np.uint8)
        u = packs.iq3s_units(raw)
        assert np.array_equal(packs.iq3s_from_units(u), raw)
        # every unit's (qh, scale) pair: the scale byte of its pair of units
        pairs = u[96 * n: 112 * n].reshape(n, 8, 2)
        assert np.array_equal(pairs[:, :, 0], raw.reshape(n, 110)[:, 66:74])
        assert np.array_equal(pairs[:, :, 1], np.repeat(raw.reshape(n, 110)[:, 106:110], 2, axis=1))
    n = 2
    raw = np.array([(100 * b + i) % 256 for b in range(n) for i in range(110)], np.uint8)
    u = packs.iq3s_units(raw)
    # unit 5 of block 1: qs bytes 2 + 40 .. 2 + 47, sign bytes 74 + 20 .. 74 + 23
    assert list(u[96 + 60: 96 + 72]) == [(100 + i) % 256 for i in list(range(42, 50)) + list(range(94, 98))]
    assert list(u[112 * n: 114 * n]) == [0, 1, 100, 101]
    assert F.PAYLOAD_BYTES[F.IQ3S_UNITS] == 114 and F.GGUF_BLOCK_BYTES[F.IQ3S_UNITS] == 110
