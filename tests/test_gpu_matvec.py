"""GPU parity: dequant bit-exact, matvec within 1e-3 normwise relative error of
the fp32 sequential oracle, reference-named decode launchers (logits, KV
side-write, token) and their argument errors. Calls go through the C-ABI."""

from __future__ import annotations

import ctypes

import numpy as np
import pytest

torch = pytest.importorskip("torch")

from rtxllm_amd import formats as F  # noqa: E402
from rtxllm_amd import ops, packs  # noqa: E402
from rtxllm_amd._lib import lib  # noqa: E402

from token_rule import check_token  # noqa: E402

pytestmark = pytest.mark.gpu

TOL = 1e-3  # max |y_gpu - y_ref| / max |y_ref|, fp32 accumulation
ALL_FMTS = list(F.PAYLOAD_BYTES)
HIP_INVALID_VALUE = 1


def rel_err(got: np.ndarray, ref: np.ndarray) -> float:
    return float(np.max(np.abs(got.astype(np.float64) - ref.astype(np.float64))) / np.max(np.abs(ref)))


def oracle_fmt(fmt: int) -> int:
    return F.Q4K_SPLIT_PREDECODED if fmt == F.Q4K_RAW_PREDECODED else fmt


def oracle_args(pack: packs.Pack):
    """The oracle has no raw+predecoded or unit layout; feed it the
    split-predecoded equivalent (same quants, same pairs) or the GGUF blocks."""
    if pack.fmt == F.Q4K_RAW_PREDECODED:
        pl = pack.payload.reshape(-1, 144)[:, 16:].copy().reshape(-1)
        return F.Q4K_SPLIT_PREDECODED, pl, pack.meta
    if pack.fmt == F.IQ2S_UNITS:  # the same bytes in GGUF block order
        return F.IQ2S, packs.iq2s_from_units(pack.payload), None
    if pack.fmt == F.IQ3S_UNITS:
        return F.IQ3S, packs.iq3s_from_units(pack.payload), None
    return pack.fmt, pack.payload, pack.meta


@pytest.mark.parametrize("fmt", ALL_FMTS, ids=[F.NAMES[f] for f in ALL_FMTS])
def test_dequant_bit_exact(orc, fmt):
    pack = packs.make_pack(fmt, 48, 1024, seed=1000 + fmt)
    dev = ops.DevicePack(pack)
    got = ops.dequant(dev).cpu().numpy()
    of, pl, mt = oracle_args(pack)
    ref = orc.dequant(of, pl, mt, pack.rows, pack.cols)
    assert np.array_equal(got.view(np.uint32), ref.view(np.uint32))


@pytest.mark.parametrize("shape", [(1, 256), (7, 512), (64, 1024), (133, 4096), (37, 2304), (2100, 4608)])
@pytest.mark.parametrize("fmt", ALL_FMTS, ids=[F.NAMES[f] for f in ALL_FMTS])
def test_matvec_small(orc, fmt, shape):
    rows, cols = shape
    pack = packs.make_pack(fmt, rows, cols, seed=2000 + 17 * fmt + rows)
    x = packs.normal_f32(3000 + cols, cols)
    y = ops.matvec(ops.DevicePack(pack), ops.to_dev(x)).cpu().numpy()
    of, pl, mt = oracle_args(pack)
    ref = orc.matvec_f32(of, pl, mt, x, rows, cols, 4)
    assert rel_err(y, ref) <= TOL


@pytest.mark.parametrize("shape", [(14336, 4096), (4096, 14336)], ids=["14336x4096", "4096x14336"])
@pytest.mark.parametrize("fmt", [F.Q4K_SPLIT_NATIVE, F.Q4K_RAW, F.Q5K, F.IQ2S, F.IQ3S],
                         ids=lambda f: F.NAMES[f])
def test_matvec_config_shapes(orc, fmt, shape):
    rows, cols = shape
    pack = packs.make_pack(fmt, rows, cols, seed=0x5EED0001)
    x = packs.normal_f32(0x5EED0101, cols)
    y = ops.matvec(ops.DevicePack(pack), ops.to_dev(x)).cpu().numpy()
    ref = orc.matvec_f32(pack.fmt, pack.payload, pack.meta, x, rows, cols, 8)
    assert rel_err(y, ref) <= TOL


@pytest.mark.parametrize("fmt", [F.IQ2S, F.IQ3S, F.IQ2S_UNITS, F.IQ3S_UNITS], ids=lambda f: F.NAMES[f])
def test_matvec_iq_one_wave_workgroups(orc, fmt):
    """2048 columns fit one wave per row (one column split), and past 16384 rows
    the IQ matvecs run a persistent grid of one-row-group workgroups: one-wave
    workgroups, whose codebook fill takes more pieces per thread than the
    two-wave layout it is sized for."""
    rows, cols = 32768, 2048
    pack = packs.make_pack(fmt, rows, cols, seed=0x1A0E + fmt)
    x = packs.normal_f32(0x1A0F + fmt, cols)
    y = ops.matvec(ops.DevicePack(pack), ops.to_dev(x)).cpu().numpy()
    of, pl, mt = oracle_args(pack)
    ref = orc.matvec_f32(of, pl, mt, x, rows, cols, 8)
    assert rel_err(y, ref) <= TOL


def test_matvec_q4k_4096_config0(orc):
    rows = cols = 4096
    for fmt in (F.Q4K_SPLIT_NATIVE, F.Q4K_SPLIT_PREDECODED, F.Q4K_SPLIT_COMPACT, F.Q4K_SPLIT_HALF):
        pack = packs.make_pack(fmt, rows, cols, seed=0x5EED0000)
        x = packs.normal_f32(0x5EED0100, cols)
        y = ops.matvec(ops.DevicePack(pack), ops.to_dev(x)).cpu().numpy()
        ref = orc.matvec_f32(fmt, pack.payload, pack.meta, x, rows, cols, 8)
        assert rel_err(y, ref) <= TOL, F.NAMES[fmt]


# ---- reference-named decode launchers ----------------------------------------

DECODE_Q4K = {
    F.Q4K_SPLIT_PREDECODED: "rtxllm_launch_q4k_matvec_decode_split_predecoded_vec4x4",
    F.Q4K_SPLIT_HALF: "rtxllm_launch_q4k_matvec_decode_split_half_vec4x4",
    F.Q4K_SPLIT_COMPACT: "rtxllm_launch_q4k_matvec_decode_split_compact_vec4x4",
    F.Q4K_SPLIT_NATIVE: "rtxllm_launch_q4k_matvec_decode_split_native_vec4x4",
    F.Q4K_RAW_PREDECODED: "rtxllm_launch_q4k_matvec_decode_predecoded_vec4x4",
}
RAW_ALIASES = [
    "rtxllm_launch_q4k_matvec_decode",
    "rtxllm_launch_q4k_matvec_decode_shared",
    "rtxllm_launch_q4k_matvec_decode_warp",
    "rtxllm_launch_q4k_matvec_decode_warp_broadcast",
    "rtxllm_launch_q4k_matvec_decode_warp_broadcast_vec4",
    "rtxllm_launch_q4k_matvec_decode_warp_broadcast_vec4x2",
    "rtxllm_launch_q4k_matvec_decode_warp_broadcast_vec4x4",
]
DECODE_PROBE = {
    F.Q5K: "rtxllm_launch_q5k_matvec_decode_probe",
    F.IQ2S: "rtxllm_launch_iq2s_matvec_decode_probe",
    F.IQ3S: "rtxllm_launch_iq3s_matvec_decode_probe",
}


def expected_decode(orc, pack, x, launched, kv_words, page_words, active, token0):
    of, pl, mt = oracle_args(pack)
    ref = orc.matvec_f32(of, pl, mt, x, pack.rows, pack.cols, 4)[:launched]
    kv = np.zeros(kv_words, np.float32)
    orc.lib().orc_kv_side_write(orc.ptr(ref), launched, orc.ptr(kv), kv_words, page_words, active, token0)
    token = (orc.argmax(ref) + token0 + 1) % 32000
    return ref, kv, token


def run_decode(name, pack, x, launched, rows_limit, kv_words, page_words, active, token0):
    dev = ops.DevicePack(pack)
    xd = ops.to_dev(x)
    logits = torch.zeros(pack.rows, dtype=torch.float32, device="cuda:0")
    kv = torch.zeros(kv_words, dtype=torch.float32, device="cuda:0")
    tok = torch.tensor([token0], dtype=torch.int32, device="cuda:0")
    fn = getattr(lib(), name)
    if rows_limit is None:
        rc = fn(ops.ptr(dev.payload), ops.ptr(dev.meta), ops.ptr(xd), ops.ptr(logits), ops.ptr(kv), ops.ptr(tok),
                pack.rows, pack.cols, kv_words, page_words, active, ops.stream()) if dev.meta is not None else \
            fn(ops.ptr(dev.payload), ops.ptr(xd), ops.ptr(logits), ops.ptr(kv), ops.ptr(tok),
               pack.rows, pack.cols, kv_words, page_words, active, ops.stream())
    else:
        rc = fn(ops.ptr(dev.payload), ops.ptr(xd), ops.ptr(logits), ops.ptr(kv), ops.ptr(tok), pack.rows,
                pack.cols, rows_limit, kv_words, page_words, active, ops.stream())
    assert rc == 0
    torch.cuda.synchronize()
    return logits.cpu().numpy()[:launched], kv.cpu().numpy(), int(tok.cpu().numpy()[0])


def check_decode(orc, name, pack, rows_limit=None):
    x = packs.normal_f32(77, pack.cols)
    launched = pack.rows if rows_limit is None else min(pack.rows, rows_limit)
    kv_words, page_words, active, token0 = 1000, 16, 50, 31990
    got_l, got_kv, got_t = run_decode(name, pack, x, launched, rows_limit, kv_words, page_words, active, token0)
    ref_l, ref_kv, ref_t = expected_decode(orc, pack, x, launched, kv_words, page_words, active, token0)
    assert rel_err(got_l, ref_l) <= TOL
    assert np.max(np.abs(got_kv - ref_kv)) <= TOL * np.max(np.abs(ref_l))
    assert (got_kv != 0).sum() == (ref_kv != 0).sum()
    # a different token only at a near-tie, inside the staging's error (~2e-5 of the maximum)
    assert ref_t == (int(np.argmax(ref_l)) + token0 + 1) % 32000
    check_token(f"{name} {pack.rows}x{pack.cols}", (got_t - token0 - 1) % 32000, ref_l, 1e-4)


@pytest.mark.parametrize("fmt", list(DECODE_Q4K), ids=lambda f: F.NAMES[f])
def test_q4k_decode_launchers(orc, fmt):
    check_decode(orc, DECODE_Q4K[fmt], packs.make_pack(fmt, 300, 2048, seed=4000 + fmt))


@pytest.mark.parametrize("name", RAW_ALIASES)
def test_q4k_raw_decode_aliases(orc, name):
    check_decode(orc, name, packs.make_pack(F.Q4K_RAW, 200, 1024, seed=4100))


@pytest.mark.parametrize("fmt", list(DECODE_PROBE), ids=lambda f: F.NAMES[f])
@pytest.mark.parametrize("rows_limit", [64, 10_000])
def test_probe_decode_launchers(orc, fmt, rows_limit):
    check_decode(orc, DECODE_PROBE[fmt], packs.make_pack(fmt, 160, 1536, seed=4200 + fmt), rows_limit=rows_limit)


def test_iq2s_matvec_probe_clips_rows(orc):
    pack = packs.make_pack(F.IQ2S, 100, 512, seed=4300)
    dev = ops.DevicePack(pack)
    x = packs.normal_f32(78, 512)
    logits = torch.full((100,), -7.0, dtype=torch.float32, device="cuda:0")
    xd = ops.to_dev(x)  # referenced until the kernel ran
    rc = lib().rtxllm_launch_iq2s_matvec_probe(ops.ptr(dev.payload), ops.ptr(xd), ops.ptr(logits), 100,
                                              512, 40, ops.stream())
    assert rc == 0
    got = logits.cpu().numpy()
    ref = orc.matvec_f32(F.IQ2S, pack.payload, None, x, 100, 512, 1)
    assert rel_err(got[:40], ref[:40]) <= TOL
    assert np.all(got[40:] == -7.0)


def test_invalid_arguments_rejected():
    dummy = torch.zeros(4096, dtype=torch.uint8, device="cuda:0")
    f = torch.zeros(1024, dtype=torch.float32, device="cuda:0")
    t = torch.zeros(1, dtype=torch.int32, device="cuda:0")
    L = lib()
    s = ops.stream()
    p = ops.ptr
    # cols % 256 != 0, zero rows, zero rows_limit (decode_kernels.cu:4046-4048)
    assert L.rtxllm_launch_iq3s_matvec_decode_probe(p(dummy), p(f), p(f), p(f), p(t), 4, 100, 4, 8, 4, 4, s) == 1
    assert L.rtxllm_launch_q5k_matvec_decode_probe(p(dummy), p(f), p(f), p(f), p(t), 0, 256, 4, 8, 4, 4, s) == 1
    assert L.rtxllm_launch_iq2s_matvec_probe(p(dummy), p(f), p(f), 4, 256, 0, s) == 1
    assert L.rtxllm_matvec(F.Q4K_SPLIT_NATIVE, p(dummy), None, p(f), p(f), 4, 256, s) == 1  # missing meta
    assert L.rtxllm_matvec(99, p(dummy), None, p(f), p(f), 4, 256, s) == 1  # unknown format
    assert L.rtxllm_launch_output_token_sample(None, p(t), 4, 10, 0, s) == 1
    assert L.rtxllm_launch_output_token_sample(p(f), p(t), 0, 10, 0, s) == 1
    assert L.rtxllm_launch_rmsnorm_cache(p(f), p(f), 4, 0, 1e-6, 0, s) == 1
    assert L.rtxllm_launch_rmsnorm_cache_and_gated_product(p(f), p(f), p(f), p(f), 4, 4, 0, 1e-6, 0, s) == 1
    torch.cuda.synchronize()


# ---- staged activation + matvec on staged x ------------------------------------

@pytest.mark.parametrize("cols", [256, 4096, 14336])
def test_stage_bit_exact(orc, cols):
    x = packs.normal_f32(cols + 5, cols) * np.float32(3.0)
    w = packs.normal_f32(cols + 6, cols, mean=1.0, std=0.02)
    for weight in (None, w):
        got = ops.stage(ops.to_dev(x), None if weight is None else ops.to_dev(weight)).cpu().numpy()
        ref = orc.stage_bytes(x, weight)
        assert np.array_equal(got, ref)


@pytest.mark.parametrize("shape", [(133, 4096), (512, 14336), (64, 1024)])
@pytest.mark.parametrize("fmt", ALL_FMTS, ids=[F.NAMES[f] for f in ALL_FMTS])
def test_matvec_xq_equals_self_staging_and_staged_oracle(orc, fmt, shape):
    rows, cols = shape
    pack = packs.make_pack(fmt, rows, cols, seed=5000 + fmt + rows)
    x = packs.normal_f32(6000 + cols, cols)
    dev = ops.DevicePack(pack)
    xd = ops.to_dev(x)
    y_self = ops.matvec(dev, xd).cpu().numpy()
    y_xq = ops.matvec_xq(dev, ops.stage(xd)).cpu().numpy()
    assert np.array_equal(y_self.view(np.uint32), y_xq.view(np.uint32))
    of, pl, mt = oracle_args(pack)
    ref = orc.matvec_staged_f64(of, pl, mt, x, rows, cols, 8)
    # same staged digits: only fp32 rounding of the per-group products separates them
    assert np.max(np.abs(y_xq - ref)) / np.max(np.abs(ref)) < 2e-6
    # and the 22-bit staging (an error of at most 2^-23 of each group's maximum)
    # keeps the product as close to the float64 oracle on the raw x
    ref64 = orc.matvec_f64(of, pl, mt, x, rows, cols, 8)
    assert np.max(np.abs(y_xq - ref64)) / np.max(np.abs(ref64)) < 2e-6


UNIT_CASES = [(F.IQ2S, F.IQ2S_UNITS, "rtxllm_iq2s_units_pack", packs.iq2s_units),
              (F.IQ3S, F.IQ3S_UNITS, "rtxllm_iq3s_units_pack", packs.iq3s_units)]


@pytest.mark.parametrize("case", UNIT_CASES, ids=["iq2s", "iq3s"])
@pytest.mark.parametrize("shape", [(1, 256), (133, 4096), (48, 14336)])
def test_units_pack_and_matvec_bit_identical(case, shape):
    """The unit-layout packers write the host restatement's bytes, and the unit
    layout's matvecs (fp32 x and staged x) equal the GGUF layout's bit for bit."""
    fmt, ufmt, packer, host = case
    rows, cols = shape
    raw = packs.synth_raw(fmt, rows, cols, seed=7100 + rows + fmt)
    d_raw = ops.to_dev(raw)
    d_units = torch.empty(F.PAYLOAD_BYTES[ufmt] * rows * (cols // 256), dtype=torch.uint8, device="cuda:0")
    assert getattr(lib(), packer)(ops.ptr(d_raw), rows, cols, ops.ptr(d_units), ops.stream()) == 0
    torch.cuda.synchronize()
    assert np.array_equal(d_units.cpu().numpy(), host(raw))
    x = ops.to_dev(packs.normal_f32(7200 + cols, cols))
    gguf = ops.DevicePack(packs.Pack(fmt, rows, cols, raw, None))
    units = ops.DevicePack(packs.Pack(ufmt, rows, cols, host(raw), None))
    y_raw = ops.matvec(gguf, x).cpu().numpy()
    assert np.array_equal(ops.matvec(units, x).cpu().numpy().view(np.uint32), y_raw.view(np.uint32))
    xq = ops.stage(x)
    y_raw_xq = ops.matvec_xq(gguf, xq).cpu().numpy()
    assert np.array_equal(ops.matvec_xq(units, xq).cpu().numpy().view(np.uint32), y_raw_xq.view(np.uint32))
