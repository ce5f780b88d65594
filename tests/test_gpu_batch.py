"""GPU parity of the batched (up to 8 activation vectors) matvec on the matrix
cores against the oracle: every sequence of the batch within 1e-3 normwise of
the fp32 sequential oracle (the bar of the batch-1 path), at one panel group
(cols <= 4096) and at several (cols = 14336, the down projection: partial sums
through the workspace), ragged row counts, batch sizes 1..8, and activations
from 1e-3 to 1e3 in magnitude (the per-sequence power-of-two scaling). All
calls go through the C-ABI."""

from __future__ import annotations

import numpy as np
import pytest

torch = pytest.importorskip("torch")

from rtxllm_amd import formats as F  # noqa: E402
from rtxllm_amd import ops, packs  # noqa: E402
from rtxllm_amd._lib import HipError  # noqa: E402

pytestmark = pytest.mark.gpu

TOL = 1e-3
FORMATS = [F.IQ2S, F.IQ3S, F.Q5K, F.Q4K_RAW, F.Q4K_SPLIT_NATIVE]


def rel(a, b) -> float:
    a, b = np.asarray(a, np.float64), np.asarray(b, np.float64)
    return float(np.max(np.abs(a - b)) / np.max(np.abs(b)))


def run(orc, fmt, rows, cols, batch, seed, scales=None):
    pack = packs.make_pack(fmt, rows, cols, seed)
    w = ops.DevicePack(pack)
    xs = np.stack([packs.normal_f32(seed + 17 + s, cols) for s in range(batch)])
    if scales is not None:
        xs = (xs * np.asarray(scales, np.float32)[:batch, None]).astype(np.float32)
    x16 = ops.stage_batch(ops.to_dev(xs))
    y = ops.matvec_batch(w, x16, batch).cpu().numpy()
    for s in range(batch):
        ref = orc.matvec_f32(fmt, pack.payload, pack.meta, xs[s], rows, cols, 8)
        err = rel(y[s], ref)
        assert err <= TOL, (F.NAMES[fmt], rows, cols, batch, s, err)
    return y


@pytest.mark.parametrize("fmt", FORMATS)
@pytest.mark.parametrize("rows,cols,batch", [(256, 4096, 8), (300, 1024, 3), (48, 512, 1), (64, 14336, 8)])
def test_batch_matvec_matches_oracle(orc, fmt, rows, cols, batch):
    run(orc, fmt, rows, cols, batch, 0x5EED0B00 + fmt)


@pytest.mark.parametrize("fmt", [F.IQ2S, F.Q4K_SPLIT_NATIVE])
def test_batch_matvec_activation_range(orc, fmt):
    run(orc, fmt, 128, 2048, 8, 0x5EED0B40 + fmt, scales=[1e-3, 1e-2, 0.1, 1.0, 10.0, 100.0, 1e3, 3.0])


def test_batch_sequences_are_independent(orc):
    # sequence s of a batch of 8 equals the same vector run alone
    fmt, rows, cols = F.IQ3S, 64, 2048
    pack = packs.make_pack(fmt, rows, cols, 0x5EED0B60)
    w = ops.DevicePack(pack)
    xs = np.stack([packs.normal_f32(0x5EED0B61 + s, cols) for s in range(8)])
    y8 = ops.matvec_batch(w, ops.stage_batch(ops.to_dev(xs)), 8).cpu().numpy()
    for s in (0, 5):
        y1 = ops.matvec_batch(w, ops.stage_batch(ops.to_dev(xs[s:s + 1].copy())), 1).cpu().numpy()
        assert np.array_equal(y1[0], y8[s])


@pytest.mark.parametrize("fmt", FORMATS)
@pytest.mark.parametrize("rows,cols,batch", [(256, 4096, 8), (300, 1024, 3), (64, 14336, 8), (48, 512, 1)])
def test_batch_matvec_f32_equals_staged(fmt, rows, cols, batch):
    """rtxllm_matvec_batch_f32 (each wave stages its own columns) gives
    rtxllm_stage_batch + rtxllm_matvec_batch bit for bit, with activations
    from 1e-3 to 1e3 so that the block exponents differ."""
    from rtxllm_amd._lib import lib

    pack = packs.make_pack(fmt, rows, cols, 9100 + fmt)
    w = ops.DevicePack(pack)
    scales = np.array([1e-3, 1.0, 1e3, 0.5, 7.0, 1e-2, 30.0, 2.0], np.float32)[:batch, None]
    xs = (np.stack([packs.normal_f32(9200 + s, cols) for s in range(batch)]) * scales).astype(np.float32)
    xd = ops.to_dev(xs)
    y_staged = ops.matvec_batch(w, ops.stage_batch(xd), batch).cpu().numpy()
    need = int(lib().rtxllm_matvec_batch_workspace(fmt, rows, cols))
    ws = torch.empty(max(need, 1), dtype=torch.uint8, device="cuda:0")
    y = torch.empty((batch, rows), dtype=torch.float32, device="cuda:0")
    rc = lib().rtxllm_matvec_batch_f32(fmt, ops.ptr(w.payload), ops.ptr(w.meta), ops.ptr(xd), ops.ptr(y), rows, cols,
                                       batch, ops.ptr(ws) if need else None, need, ops.stream())
    assert rc == 0
    torch.cuda.synchronize()
    assert np.array_equal(y.cpu().numpy().view(np.uint32), y_staged.view(np.uint32))


def test_batch_invalid_arguments():
    pack = packs.make_pack(F.IQ2S, 16, 768, 1)
    w = ops.DevicePack(pack)
    x16 = ops.stage_batch(ops.to_dev(np.zeros((2, 768), np.float32)))
    with pytest.raises(HipError):
        ops.matvec_batch(w, x16, 2)  # cols % 512 != 0
    pack = packs.make_pack(F.Q4K_SPLIT_HALF, 16, 512, 1)
    with pytest.raises(HipError):
        ops.matvec_batch(ops.DevicePack(pack), ops.stage_batch(ops.to_dev(np.zeros((1, 512), np.float32))), 1)
    with pytest.raises((HipError, ValueError)):
        ops.stage_batch(ops.to_dev(np.zeros((9, 512), np.float32)))
