"""rtxllm_matvec_batch_noalloc (the allocation-free batched matvec) against
rtxllm_matvec_batch with a caller workspace: bit-identical on two calls in a
row, the second with a smaller input (fewer rows, columns and sequences), so
the second call reads none of the first call's partial sums; sizes beyond the
scratch array are refused before any launch. Through the C-ABI."""

from __future__ import annotations

import numpy as np
import pytest

torch = pytest.importorskip("torch")

from rtxllm_amd import formats as F  # noqa: E402
from rtxllm_amd import ops, packs  # noqa: E402
from rtxllm_amd._lib import lib  # noqa: E402

pytestmark = pytest.mark.gpu

HIP_INVALID_VALUE = 1
SCRATCH_BYTES = 8 << 20


def run_both(fmt, rows, cols, batch, seed):
    pack = packs.make_pack(fmt, rows, cols, seed=seed)
    d = ops.DevicePack(pack)
    xs = np.stack([packs.normal_f32(seed + 1 + i, cols) for i in range(batch)])
    xd = ops.to_dev(xs)
    x16 = ops.stage_batch(xd)
    y_ref = ops.matvec_batch(d, x16, batch).cpu().numpy()
    y = torch.full((batch, rows), np.nan, dtype=torch.float32, device="cuda:0")
    rc = lib().rtxllm_matvec_batch_noalloc(fmt, ops.ptr(d.payload), ops.ptr(d.meta), ops.ptr(x16), ops.ptr(y), rows,
                                           cols, batch, ops.stream())
    assert rc == 0
    torch.cuda.synchronize()
    return y.cpu().numpy(), y_ref


@pytest.mark.parametrize("fmt", [F.Q4K_SPLIT_NATIVE, F.IQ2S, F.Q5K], ids=lambda f: F.NAMES[f])
def test_noalloc_matches_workspace_entry_two_calls(fmt):
    groups = int(lib().rtxllm_matvec_batch_workspace(fmt, 4096, 14336)) // (4 * 8 * 4096)
    assert groups == 4  # the first call uses the scratch array
    y1, r1 = run_both(fmt, 4096, 14336, 8, 0x5EED0E00 + fmt)
    assert np.array_equal(y1.view(np.uint32), r1.view(np.uint32))
    y2, r2 = run_both(fmt, 1000, 6144, 3, 0x5EED0E10 + fmt)  # smaller: 2 panel groups, 3 sequences
    assert np.array_equal(y2.view(np.uint32), r2.view(np.uint32))
    y3, r3 = run_both(fmt, 512, 2048, 2, 0x5EED0E20 + fmt)  # one panel group: no scratch
    assert np.array_equal(y3.view(np.uint32), r3.view(np.uint32))


def test_noalloc_refuses_sizes_beyond_the_scratch_array():
    L, s = lib(), ops.stream()
    buf = torch.zeros(1024, dtype=torch.uint8, device="cuda:0")
    p = buf.data_ptr()
    # 131072 rows x 14336 columns (4 panel groups) x 8 sequences: 16 MiB of partial sums
    need = int(L.rtxllm_matvec_batch_workspace(F.IQ2S, 131072, 14336))
    assert need == 4 * 8 * 131072 * 4 and need > SCRATCH_BYTES
    assert L.rtxllm_matvec_batch_noalloc(F.IQ2S, p, None, p, p, 131072, 14336, 8, s) == HIP_INVALID_VALUE
    assert L.rtxllm_matvec_batch_noalloc(F.IQ2S, p, None, p, p, 4096, 14336, 9, s) == HIP_INVALID_VALUE
    torch.cuda.synchronize()
