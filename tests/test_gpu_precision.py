"""GPU precision gates against the float64 oracle.

Every batch-1 matvec (the pure entry point, the staged-activation entry point
and the reference-named decode launchers) and the batched matvec must be at
least as close to the float64 product as the reference's own fp32 path: the
oracle's fp32 sequential accumulation (main.cpp:1261-1309). The bar is

    err(gpu) <= 2 * err(fp32 sequential),  err(y) = max|y - y64| / max|y64|,

and the same for the per-element relative error with a floor of 1e-3 of
max|y64| (tests/precision_ref.py), at the config shapes for every format, with N(0,1), outlier (one 1e3 value per
16-value group) and heavy-tailed activations. Every kernel rounds its activation
once on input (22 bits per 16-value group at batch 1, per 256-value block in the
batched matvec), so each is gated as gate_staged states: its arithmetic against
the float64 product of the rounded activation within the bar, and per element
against y64 within 2x the larger of the fp32 path's and the rounding's own
error (on heavy-tailed activations the rounding alone can exceed the bar). Also: a NaN activation poisons
the outputs as in fp32, and the device fp16 decode of d / dmin follows the
reference's rule (main.cpp:1086-1098) for subnormal, signed-zero, infinite and
NaN codes, bit for bit against the oracle's dequant."""

from __future__ import annotations

import numpy as np
import pytest

torch = pytest.importorskip("torch")

from rtxllm_amd import formats as F  # noqa: E402
from rtxllm_amd import ops, packs  # noqa: E402
from rtxllm_amd._lib import lib  # noqa: E402

pytestmark = pytest.mark.gpu

from precision_ref import (GATE, activation, batch_staged, elem64, err64, gate, gate_staged, oracle_args,  # noqa: E402,F401
                           references, references_staged)


CONFIG_CASES = (
    [(f, 4096, 4096) for f in (F.Q4K_SPLIT_NATIVE, F.Q4K_SPLIT_PREDECODED, F.Q4K_SPLIT_COMPACT,
                               F.Q4K_SPLIT_HALF, F.Q4K_RAW)]
    + [(f, r, c) for f in (F.Q4K_SPLIT_NATIVE, F.Q4K_RAW, F.Q5K) for (r, c) in ((14336, 4096), (4096, 14336))]
    + [(f, r, c) for f in (F.IQ2S, F.IQ3S, F.IQ2S_UNITS, F.IQ3S_UNITS)
       for (r, c) in ((14336, 4096), (4096, 14336))]
)


def case_id(c):
    return f"{F.NAMES[c[0]]}-{c[1]}x{c[2]}"


@pytest.mark.parametrize("case", CONFIG_CASES, ids=[case_id(c) for c in CONFIG_CASES])
def test_matvec_f64_gate_config_shapes(orc, case):
    fmt, rows, cols = case
    pack = packs.make_pack(fmt, rows, cols, seed=0x5EED0000 + fmt)
    dev = ops.DevicePack(pack)
    for kind in ("normal", "outlier", "heavy"):
        x = activation(kind, cols, 0x5EED0100 + cols + fmt)
        y32, y64, yst64 = references_staged(orc, pack, x)
        xd = ops.to_dev(x)
        y = ops.matvec(dev, xd).cpu().numpy()
        y_xq = ops.matvec_xq(dev, ops.stage(xd)).cpu().numpy()
        assert np.array_equal(y.view(np.uint32), y_xq.view(np.uint32))
        gate_staged(f"{case_id(case)} {kind}", y, y32, y64, yst64)


DECODE_NAMES = {
    F.Q4K_SPLIT_NATIVE: "rtxllm_launch_q4k_matvec_decode_split_native_vec4x4",
    F.Q4K_SPLIT_PREDECODED: "rtxllm_launch_q4k_matvec_decode_split_predecoded_vec4x4",
    F.Q4K_SPLIT_COMPACT: "rtxllm_launch_q4k_matvec_decode_split_compact_vec4x4",
    F.Q4K_RAW: "rtxllm_launch_q4k_matvec_decode",
    F.Q5K: "rtxllm_launch_q5k_matvec_decode_probe",
    F.IQ2S: "rtxllm_launch_iq2s_matvec_decode_probe",
    F.IQ3S: "rtxllm_launch_iq3s_matvec_decode_probe",
}


def run_decode_launcher(fmt, dev, x, rows, cols, kv_words=4096, page_words=16, active=64, token0=7):
    xd = ops.to_dev(x)
    logits = torch.zeros(rows, dtype=torch.float32, device="cuda:0")
    kv = torch.zeros(kv_words, dtype=torch.float32, device="cuda:0")
    tok = torch.tensor([token0], dtype=torch.int32, device="cuda:0")
    fn = getattr(lib(), DECODE_NAMES[fmt])
    p = ops.ptr
    if fmt in (F.Q5K, F.IQ2S, F.IQ3S):
        rc = fn(p(dev.payload), p(xd), p(logits), p(kv), p(tok), rows, cols, rows, kv_words, page_words, active,
                ops.stream())
    elif dev.meta is not None:
        rc = fn(p(dev.payload), p(dev.meta), p(xd), p(logits), p(kv), p(tok), rows, cols, kv_words, page_words,
                active, ops.stream())
    else:
        rc = fn(p(dev.payload), p(xd), p(logits), p(kv), p(tok), rows, cols, kv_words, page_words, active,
                ops.stream())
    assert rc == 0
    torch.cuda.synchronize()
    return logits.cpu().numpy(), kv.cpu().numpy(), int(tok.cpu().numpy()[0])


@pytest.mark.parametrize("fmt", list(DECODE_NAMES), ids=lambda f: F.NAMES[f])
def test_reference_named_launchers_f64_gate(orc, fmt):
    """The drop-in launchers take the reference's fp32 activation
    (decode_kernels.cu:2893-2991) and are held to the same bar."""
    rows, cols = (4096, 4096) if fmt in (F.Q4K_SPLIT_NATIVE, F.Q4K_SPLIT_PREDECODED, F.Q4K_SPLIT_COMPACT,
                                         F.Q4K_RAW) else (14336, 4096)
    pack = packs.make_pack(fmt, rows, cols, seed=0x5EED0200 + fmt)
    dev = ops.DevicePack(pack)
    for kind in ("normal", "outlier"):
        x = activation(kind, cols, 0x5EED0300 + fmt)
        y32, y64, yst64 = references_staged(orc, pack, x)
        logits, _, _ = run_decode_launcher(fmt, dev, x, rows, cols)
        gate_staged(f"{F.NAMES[fmt]} {kind}", logits, y32, y64, yst64)


@pytest.mark.parametrize("fmt", [F.Q4K_SPLIT_NATIVE, F.Q5K, F.IQ2S, F.IQ3S, F.IQ3S_UNITS],
                         ids=lambda f: F.NAMES[f])
def test_nan_activation_poisons_outputs(orc, fmt):
    """One NaN in x makes every fp32 output NaN (0 * NaN = NaN); the staged
    matvecs give the same."""
    rows, cols = 256, 4096
    pack = packs.make_pack(fmt, rows, cols, seed=0x5EED0400 + fmt)
    dev = ops.DevicePack(pack)
    x = packs.normal_f32(0x5EED0401, cols)
    x[1234] = np.nan
    y32, _ = references(orc, pack, x)
    assert np.all(np.isnan(y32))
    xd = ops.to_dev(x)
    assert np.all(np.isnan(ops.matvec(dev, xd).cpu().numpy()))
    assert np.all(np.isnan(ops.matvec_xq(dev, ops.stage(xd)).cpu().numpy()))


def test_nan_activation_reference_launcher(orc):
    """A NaN activation through a reference-named launcher: NaN logits, NaN in
    every side-written KV slot, and the token of the fp32 rule (no logit beats
    the -FLT_MAX start, so argmax = 0: token = (0 + token + 1) % 32000)."""
    rows, cols = 512, 2048
    pack = packs.make_pack(F.Q4K_SPLIT_NATIVE, rows, cols, seed=0x5EED0500)
    dev = ops.DevicePack(pack)
    x = packs.normal_f32(0x5EED0501, cols)
    x[7] = np.nan
    logits, kv, tok = run_decode_launcher(F.Q4K_SPLIT_NATIVE, dev, x, rows, cols, kv_words=1000, page_words=16,
                                          active=50, token0=31990)
    y32, _ = references(orc, pack, x)
    assert np.all(np.isnan(logits)) and np.all(np.isnan(y32))
    ref_kv = np.zeros(1000, np.float32)
    orc.lib().orc_kv_side_write(orc.ptr(y32), rows, orc.ptr(ref_kv), 1000, 16, 50, 31990)
    np.testing.assert_array_equal(np.isnan(kv), np.isnan(ref_kv))
    assert np.isnan(kv).sum() == 50
    assert tok == (orc.argmax(y32) + 31990 + 1) % 32000


def test_infinite_activation_non_finite_outputs(orc):
    rows, cols = 128, 1024
    pack = packs.make_pack(F.IQ2S, rows, cols, seed=0x5EED0600)
    dev = ops.DevicePack(pack)
    x = packs.normal_f32(0x5EED0601, cols)
    x[100] = np.inf
    y32, _ = references(orc, pack, x)
    y = ops.matvec(dev, ops.to_dev(x)).cpu().numpy()
    assert np.all(~np.isfinite(y32)) and np.all(~np.isfinite(y))


# ---- fp16 special codes in d / dmin, decoded on the device ---------------------

SPECIAL_F16 = np.array([0x0000, 0x8000, 0x0001, 0x8001, 0x03FF, 0x83FF, 0x0200, 0x7C00, 0xFC00, 0x7C01, 0x7E00,
                        0xFE00, 0x7FFF, 0xFFFF, 0x7D55, 0x3C00, 0x7BFF, 0x0400], dtype=np.uint16)

# (format, [(byte offset of an fp16 field within the record, record)]); record
# "payload" = the payload block, "meta" = the metadata block
SPECIAL_FIELDS = {
    F.Q4K_RAW: [(0, "payload"), (2, "payload")],
    F.Q4K_SPLIT_NATIVE: [(0, "meta"), (2, "meta")],
    F.Q4K_SPLIT_COMPACT: [(0, "meta"), (2, "meta")],
    F.Q4K_SPLIT_HALF: [(o, "meta") for o in range(0, 32, 2)],
    F.Q5K: [(0, "payload"), (2, "payload")],
    F.IQ2S: [(0, "payload")],
    F.IQ3S: [(0, "payload")],
}


def special_pack(fmt: int, rows: int, cols: int, seed: int) -> packs.Pack:
    pack = packs.make_pack(fmt, rows, cols, seed=seed)
    rng = np.random.default_rng(seed)
    for off, rec in SPECIAL_FIELDS[fmt]:
        buf = pack.payload if rec == "payload" else pack.meta
        size = F.PAYLOAD_BYTES[fmt] if rec == "payload" else F.META_BYTES[fmt]
        blocks = buf.reshape(-1, size)
        codes = SPECIAL_F16[rng.integers(0, SPECIAL_F16.size, blocks.shape[0])]
        blocks[:, off] = (codes & 0xFF).astype(np.uint8)
        blocks[:, off + 1] = (codes >> 8).astype(np.uint8)
    return pack


def same_or_both_nan(a: np.ndarray, b: np.ndarray) -> bool:
    """Bit-equal, except that any two NaNs match: the fp16 decode maps every
    NaN code to +qNaN (the oracle checks that value itself), but a product such
    as inf * 0 gives the host's default NaN (sign set on x86) and the GPU's
    canonical +qNaN."""
    na, nb = np.isnan(a), np.isnan(b)
    return bool(np.array_equal(na, nb) and np.array_equal(a[~na].view(np.uint32), b[~nb].view(np.uint32)))


@pytest.mark.parametrize("fmt", list(SPECIAL_FIELDS), ids=lambda f: F.NAMES[f])
def test_dequant_fp16_special_codes_bit_exact(orc, fmt):
    pack = special_pack(fmt, 32, 1024, seed=0x5EED0700 + fmt)
    got = ops.dequant(ops.DevicePack(pack)).cpu().numpy()
    ref = orc.dequant(fmt, pack.payload, pack.meta, pack.rows, pack.cols)
    assert np.isnan(ref).any() and np.isinf(ref).any()  # the special codes are reached
    assert same_or_both_nan(got, ref)


@pytest.mark.parametrize("fmt", [F.IQ2S, F.IQ3S], ids=lambda f: F.NAMES[f])
def test_dequant_fp16_special_codes_unit_layouts(orc, fmt):
    pack = special_pack(fmt, 16, 2048, seed=0x5EED0710 + fmt)
    units = packs.iq2s_units(pack.payload) if fmt == F.IQ2S else packs.iq3s_units(pack.payload)
    ufmt = F.IQ2S_UNITS if fmt == F.IQ2S else F.IQ3S_UNITS
    got = ops.dequant(ops.DevicePack(packs.Pack(ufmt, 16, 2048, units, None))).cpu().numpy()
    ref = orc.dequant(fmt, pack.payload, None, 16, 2048)
    assert same_or_both_nan(got, ref)


def test_fp16_nan_codes_decode_to_positive_qnan(orc):
    """d = a NaN code of either sign and any payload decodes to +qNaN
    0x7FC00000 (main.cpp:1086-1098); with d = NaN, sc = 1, q = 1 and
    dmin = +0 the Q4_K value is d itself, so the device shows the decoded bits."""
    for code in (0x7C01, 0x7E00, 0xFE00, 0x7FFF, 0xFFFF, 0x7D55):
        raw = packs.synth_raw(F.Q4K_RAW, 1, 256, seed=0x5EED0720).reshape(1, 144)
        raw[0, 0:2] = [code & 0xFF, code >> 8]
        raw[0, 2:4] = 0  # dmin = +0
        raw[0, 4:16] = [1, 1, 1, 1, 0, 0, 0, 0, 1, 1, 1, 1]  # sc = 1, m = 0 for every sub-block
        raw[0, 16:] = 0x11  # q = 1
        got = ops.dequant(ops.DevicePack(packs.Pack(F.Q4K_RAW, 1, 256, raw.reshape(-1), None))).cpu().numpy()
        ref = orc.dequant(F.Q4K_RAW, raw.reshape(-1), None, 1, 256)
        assert np.all(ref.view(np.uint32) == 0x7FC00000)
        assert np.array_equal(got.view(np.uint32), ref.view(np.uint32)), hex(code)


@pytest.mark.parametrize("fmt", [F.Q4K_SPLIT_NATIVE, F.Q4K_RAW, F.Q5K, F.IQ2S, F.IQ3S, F.IQ2S_UNITS],
                         ids=lambda f: F.NAMES[f])
def test_matvec_subnormal_scales(orc, fmt):
    """Every d (and dmin) an fp16 subnormal: the matvec's hardware fp16
    decode keeps them exact (within the fp32 gate as usual)."""
    base = F.IQ2S if fmt == F.IQ2S_UNITS else fmt
    rows, cols = 512, 4096
    pack = packs.make_pack(base, rows, cols, seed=0x5EED0800 + fmt)
    rng = np.random.default_rng(fmt)
    in_meta = base == F.Q4K_SPLIT_NATIVE  # d, dmin in the 16 B metadata head
    buf = pack.meta if in_meta else pack.payload
    blocks = buf.reshape(-1, F.META_BYTES[base] if in_meta else F.PAYLOAD_BYTES[base])
    for off in ((0,) if base in (F.IQ2S, F.IQ3S) else (0, 2)):
        codes = rng.integers(1, 0x400, blocks.shape[0]).astype(np.uint16)
        blocks[:, off] = (codes & 0xFF).astype(np.uint8)
        blocks[:, off + 1] = (codes >> 8).astype(np.uint8)
    if fmt == F.IQ2S_UNITS:
        pack = packs.Pack(fmt, rows, cols, packs.iq2s_units(pack.payload), None)
    x = packs.normal_f32(0x5EED0801, cols)
    y32, y64 = references(orc, pack, x)
    y = ops.matvec(ops.DevicePack(pack), ops.to_dev(x)).cpu().numpy()
    assert err64(y, y64) <= GATE * err64(y32, y64)


# ---- batched matvec at the config shapes ------------------------------------------

BATCH_FMTS = [F.Q4K_RAW, F.Q4K_SPLIT_NATIVE, F.Q5K, F.IQ2S, F.IQ3S]


@pytest.mark.parametrize("shape", [(14336, 4096), (4096, 14336)], ids=["14336x4096", "4096x14336"])
@pytest.mark.parametrize("fmt", BATCH_FMTS, ids=lambda f: F.NAMES[f])
def test_matvec_batch8_config_shapes(orc, fmt, shape):
    """rtxllm_matvec_batch for 8 vectors at the FFN shapes: every sequence
    within 1e-3 of the fp32 oracle and inside the float64 gate, and equal to
    rtxllm_matvec_batch_f32 (self-staging) bit for bit."""
    rows, cols = shape
    pack = packs.make_pack(fmt, rows, cols, seed=0x5EED0900 + fmt)
    dev = ops.DevicePack(pack)
    kinds = ["normal", "outlier", "heavy", "normal", "normal", "outlier", "normal", "heavy"]
    xs = np.stack([activation(k, cols, 0x5EED0A00 + 31 * s) for s, k in enumerate(kinds)])
    xd = ops.to_dev(xs)
    y = ops.matvec_batch(dev, ops.stage_batch(xd), 8).cpu().numpy()
    need = int(lib().rtxllm_matvec_batch_workspace(fmt, rows, cols))
    ws = torch.empty(max(need, 1), dtype=torch.uint8, device="cuda:0")
    y_self = torch.empty((8, rows), dtype=torch.float32, device="cuda:0")
    rc = lib().rtxllm_matvec_batch_f32(fmt, ops.ptr(dev.payload), ops.ptr(dev.meta), ops.ptr(xd), ops.ptr(y_self),
                                       rows, cols, 8, ops.ptr(ws) if need else None, need, ops.stream())
    assert rc == 0
    assert np.array_equal(y_self.cpu().numpy().view(np.uint32), y.view(np.uint32))
    of, pl, mt = oracle_args(pack)
    for s in range(8):
        y32, y64 = references(orc, pack, xs[s])
        yst64 = orc.matvec_f64(of, pl, mt, batch_staged(xs[s]), rows, cols, 16)
        assert float(np.max(np.abs(y[s] - y32)) / np.max(np.abs(y32))) <= 1e-3
        gate_staged(f"{F.NAMES[fmt]} {rows}x{cols} seq {s} {kinds[s]}", y[s], y32, y64, yst64)
