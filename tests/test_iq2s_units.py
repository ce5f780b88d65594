"""CPU checks of the IQ2S_UNITS layout's host restatement (packs.iq2s_units),
which the GPU packer must match byte for byte: the regrouping is a bijection
of the tensor's bytes, it inverts, and hand-placed fields of a two-block
tensor land where the layout puts them."""

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
