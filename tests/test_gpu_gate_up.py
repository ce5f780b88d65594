"""GPU parity of the batch-1 gate/up kernels against the float64 oracle.

The decode runner's gate/up stage has three kernels (rtxllm_gate_up_silu
picks the one the runner picks):
  * mvq_kernel: the IQ unit layouts on the int8 matrix cores (the 8B step's
    gate/up, its largest stage);
  * mv_kernel with one 16-wave workgroup per CU sharing the staged input and
    handing column-split partials over through bounded LDS waits (K-quant or
    GGUF IQ gate/up at hidden <= 4096);
  * mv_kernel with per-wave inputs (hidden > 4096).
Each is held to the staged float64 gate of tests/precision_ref.py
(gate_staged: the kernel's arithmetic against the float64 product of its
22-bit staged activation, and the result against the float64 product of x,
at most 2x the reference's own fp32 sequential path, main.cpp:1261-1309, or
2x the staging's own error where that is larger) at the 8B FFN shapes, for
N(0,1), outlier and heavy-tailed activations: the plain matvec on the matrix cores
(rtxllm_matvec_xq_mfma) on y = W x, and the fused stage on act = silu(g) u
with g, u from the float64 and fp32-sequential products. The bounded waits'
status bit is checked in both directions: 0 after every normal launch, and
set when a host-side test hook makes every wait run out (each wave still
finishes its rounds)."""

from __future__ import annotations

import numpy as np
import pytest

torch = pytest.importorskip("torch")

from rtxllm_amd import formats as F  # noqa: E402
from rtxllm_amd import ops, packs  # noqa: E402
from rtxllm_amd._lib import lib  # noqa: E402

from precision_ref import KINDS, activation, gate_staged, references_staged  # noqa: E402

pytestmark = pytest.mark.gpu

HIP_INVALID_VALUE = 1
WAIT_TIMEOUT = 2  # RTXLLM_STATUS_WAIT_TIMEOUT


def silu32(v: np.ndarray) -> np.ndarray:
    v = v.astype(np.float32)
    return (v / (np.float32(1.0) + np.exp(-v))).astype(np.float32)


def silu64(v: np.ndarray) -> np.ndarray:
    v = v.astype(np.float64)
    return v / (1.0 + np.exp(-v))


def mfma_matvec(dev: ops.DevicePack, xq: torch.Tensor) -> np.ndarray:
    y = torch.empty(dev.rows, dtype=torch.float32, device="cuda:0")
    rc = lib().rtxllm_matvec_xq_mfma(dev.fmt, ops.ptr(dev.payload), ops.ptr(xq), ops.ptr(y), dev.rows, dev.cols,
                                     ops.stream())
    assert rc == 0
    return y.cpu().numpy()


def unit_sumsq(cols: int) -> torch.Tensor:
    """One partial sum of squares equal to cols: with eps 0 the RMSNorm scale
    is 1 / sqrt(cols / cols + 0) = 1 exactly, so act = silu(g) u of W x."""
    return torch.tensor([float(cols)], dtype=torch.float32, device="cuda:0")


def gate_up(dev: ops.DevicePack, xq: torch.Tensor, hook: tuple[int, int] | None = None):
    act = torch.full((dev.rows // 2,), float("nan"), dtype=torch.float32, device="cuda:0")
    status = torch.zeros(1, dtype=torch.int32, device="cuda:0")
    sq = unit_sumsq(dev.cols)
    args = (dev.fmt, ops.ptr(dev.payload), ops.ptr(dev.meta), ops.ptr(xq), ops.ptr(sq), 1, 0.0, ops.ptr(act),
            dev.rows, dev.cols, ops.ptr(status))
    if hook is None:
        rc = lib().rtxllm_gate_up_silu(*args, ops.stream())
    else:
        rc = lib().rtxllm_test_gate_up_silu_waits(*args, hook[0], hook[1], ops.stream())
    assert rc == 0
    torch.cuda.synchronize()
    return act.cpu().numpy(), int(status.cpu().numpy()[0])


# (format, rows, cols): the runner's 8B gate/up (IQ2_S units, 2 x 14336 rows) and
# IQ2_S / IQ3_S unit tensors of 14336 rows (an IQ3_S gate/up of ffn 7168)
MFMA_CASES = [(F.IQ2S_UNITS, 28672, 4096), (F.IQ2S_UNITS, 14336, 4096), (F.IQ3S_UNITS, 14336, 4096),
              (F.IQ3S_UNITS, 28672, 4096)]


def cid(c):
    return f"{F.NAMES[c[0]]}-{c[1]}x{c[2]}"


@pytest.mark.parametrize("case", MFMA_CASES, ids=[cid(c) for c in MFMA_CASES])
def test_mfma_matvec_f64_gate(orc, case):
    """y = W x on the int8 matrix cores: within the float64 gate, and within
    fp32 rounding of the dot-product kernel on the same staged input (the
    same exact group dots, added in another order)."""
    fmt, rows, cols = case
    pack = packs.make_pack(fmt, rows, cols, seed=0x5EED0B00 + fmt + rows)
    dev = ops.DevicePack(pack)
    for kind in KINDS:
        x = activation(kind, cols, 0x5EED0B10 + cols + fmt)
        y32, y64, yst64 = references_staged(orc, pack, x)
        xq = ops.stage(ops.to_dev(x))
        y = mfma_matvec(dev, xq)
        gate_staged(f"mfma {cid(case)} {kind}", y, y32, y64, yst64)
        y_dot = ops.matvec_xq(dev, xq).cpu().numpy()
        d = float(np.max(np.abs(y.astype(np.float64) - y_dot)) / np.max(np.abs(y64)))
        print(f"  mfma vs v_dot4 kernel: {d:.3e}")
        assert d <= 1e-5, (kind, d)


# (format, rows, cols, kernel): rows interleave gate / up (2 x ffn)
GATE_UP_CASES = [
    (F.IQ2S_UNITS, 28672, 4096, "mfma"),
    (F.IQ3S_UNITS, 14336, 4096, "mfma"),
    (F.IQ2S_UNITS, 14336, 4096, "mfma"),
    (F.Q4K_SPLIT_NATIVE, 28672, 4096, "wide"),
    (F.Q5K, 28672, 4096, "wide"),
    (F.Q4K_RAW, 28672, 4096, "wide"),
    (F.IQ2S, 28672, 4096, "wide"),
    (F.Q4K_SPLIT_NATIVE, 4096, 1024, "wide"),
    (F.Q4K_SPLIT_NATIVE, 8192, 4608, "plain"),
    (F.IQ3S, 8192, 4608, "plain"),
]


@pytest.mark.parametrize("case", GATE_UP_CASES, ids=[f"{cid(c)}-{c[3]}" for c in GATE_UP_CASES])
def test_gate_up_silu_f64_gate(orc, case):
    """act = silu(g) u of the fused stage against silu(g64) u64 (float64
    products) with the fp32 sequential path's silu(g32) u32 as the bar; the
    wait status stays 0."""
    fmt, rows, cols, _ = case
    pack = packs.make_pack(fmt, rows, cols, seed=0x5EED0C00 + fmt + rows + cols)
    dev = ops.DevicePack(pack)
    for kind in KINDS:
        x = activation(kind, cols, 0x5EED0C10 + cols + fmt)
        y32, y64, yst64 = references_staged(orc, pack, x)
        act32 = silu32(y32[0::2]) * y32[1::2]
        act64 = silu64(y64[0::2]) * y64[1::2]
        actst64 = silu64(yst64[0::2]) * yst64[1::2]
        act, status = gate_up(dev, ops.stage(ops.to_dev(x)))
        assert status == 0
        assert np.all(np.isfinite(act))
        gate_staged(f"gate_up {cid(case)} {kind}", act, act32, act64, actst64)


def test_gate_up_wait_timeout_sets_status(orc):
    """The 16-wave gate/up workgroup (Q4_K at hidden 4096) with every LDS
    wait's target raised out of reach and one read per wait: each wait runs
    out, the launch still completes, and the status word carries the timeout
    bit. The same tensor and input then run normally: status 0, and act equal
    to the first normal launch's bit for bit."""
    rows, cols = 28672, 4096
    pack = packs.make_pack(F.Q4K_SPLIT_NATIVE, rows, cols, seed=0x5EED0D00)
    dev = ops.DevicePack(pack)
    xq = ops.stage(ops.to_dev(packs.normal_f32(0x5EED0D01, cols)))
    good, status = gate_up(dev, xq)
    assert status == 0
    _, status = gate_up(dev, xq, hook=(1, 1 << 30))
    assert status & WAIT_TIMEOUT
    again, status = gate_up(dev, xq)
    assert status == 0
    assert np.array_equal(again.view(np.uint32), good.view(np.uint32))


def test_gate_up_and_mfma_reject_bad_arguments():
    L, s, P = lib(), ops.stream(), ops.ptr
    buf = torch.zeros(1 << 20, dtype=torch.uint8, device="cuda:0")
    f = torch.zeros(1 << 16, dtype=torch.float32, device="cuda:0")
    # the matrix-core matvec takes the unit layouts on 16-row tiles and 512-column panels only
    assert L.rtxllm_matvec_xq_mfma(F.IQ2S, P(buf), P(buf), P(f), 64, 512, s) == HIP_INVALID_VALUE
    assert L.rtxllm_matvec_xq_mfma(F.IQ2S_UNITS, P(buf), P(buf), P(f), 40, 512, s) == HIP_INVALID_VALUE
    assert L.rtxllm_matvec_xq_mfma(F.IQ2S_UNITS, P(buf), P(buf), P(f), 64, 768, s) == HIP_INVALID_VALUE
    assert L.rtxllm_matvec_xq_mfma(F.IQ2S_UNITS, P(buf), P(buf), P(f), 64, 8704, s) == HIP_INVALID_VALUE
    # gate/up: rows % 4, no partial sums, a zero wait limit
    assert L.rtxllm_gate_up_silu(F.Q4K_RAW, P(buf), None, P(buf), P(f), 1, 0.0, P(f), 6, 256, None,
                                 s) == HIP_INVALID_VALUE
    assert L.rtxllm_gate_up_silu(F.Q4K_RAW, P(buf), None, P(buf), P(f), 0, 0.0, P(f), 8, 256, None,
                                 s) == HIP_INVALID_VALUE
    assert L.rtxllm_test_gate_up_silu_waits(F.Q4K_RAW, P(buf), None, P(buf), P(f), 1, 0.0, P(f), 8, 256, None, 0,
                                            0, s) == HIP_INVALID_VALUE
