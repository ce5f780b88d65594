"""Launch the C-ABI kernels on torch-allocated device memory.

torch supplies device memory and the current HIP stream only; every result is
computed by build/librtxllm.so. Shapes are checked on the host before any
launch so a kernel never sees buffers smaller than its grid assumes.
"""

from __future__ import annotations

import numpy as np
import torch

from . import formats as F
from ._lib import check, lib
from .packs import Pack


def stream() -> int:
    return torch.cuda.current_stream().cuda_stream


def ptr(t: torch.Tensor | None) -> int | None:
    if t is None:
        return None
    assert t.is_cuda and t.is_contiguous()
    return t.data_ptr()


def to_dev(a: np.ndarray, device: str = "cuda:0") -> torch.Tensor:
    return torch.from_numpy(np.ascontiguousarray(a)).to(device)


class DevicePack:
    """A resident pack uploaded to device memory."""

    def __init__(self, pack: Pack, device: str = "cuda:0"):
        self.fmt, self.rows, self.cols = pack.fmt, pack.rows, pack.cols
        self.payload = to_dev(pack.payload, device)
        self.meta = to_dev(pack.meta, device) if pack.meta is not None else None
        nb = self.rows * (self.cols // F.BLOCK_VALUES)
        if self.payload.numel() < nb * F.PAYLOAD_BYTES[self.fmt]:
            raise ValueError("payload smaller than rows x blocks x block bytes")
        if F.meta_bytes(self.fmt) and (self.meta is None or self.meta.numel() < nb * F.meta_bytes(self.fmt)):
            raise ValueError("metadata smaller than rows x blocks x meta bytes")


def _check_vec(t: torch.Tensor, n: int, dtype=torch.float32) -> None:
    if t.dtype != dtype or t.numel() < n or not t.is_cuda:
        raise ValueError(f"expected a device {dtype} tensor of >= {n} elements")


def matvec(w: DevicePack, x: torch.Tensor, y: torch.Tensor | None = None) -> torch.Tensor:
    _check_vec(x, w.cols)
    if y is None:
        y = torch.empty(w.rows, dtype=torch.float32, device=x.device)
    _check_vec(y, w.rows)
    check("rtxllm_matvec", lib().rtxllm_matvec(w.fmt, ptr(w.payload), ptr(w.meta), ptr(x), ptr(y), w.rows, w.cols,
                                                stream()))
    return y


def dequant(w: DevicePack) -> torch.Tensor:
    out = torch.empty((w.rows, w.cols), dtype=torch.float32, device=w.payload.device)
    check("rtxllm_dequant_f32", lib().rtxllm_dequant_f32(w.fmt, ptr(w.payload), ptr(w.meta), w.rows, w.cols,
                                                         ptr(out), stream()))
    return out


def xq_bytes(cols: int) -> int:
    return int(lib().rtxllm_xq_bytes(cols))


def stage(x: torch.Tensor, weight: torch.Tensor | None = None, out: torch.Tensor | None = None) -> torch.Tensor:
    """Staged activation buffer (uint8, rtxllm_xq_bytes(cols)) of x (* weight)."""
    cols = x.numel()
    _check_vec(x, cols)
    if weight is not None:
        _check_vec(weight, cols)
    if out is None:
        out = torch.empty(xq_bytes(cols), dtype=torch.uint8, device=x.device)
    if out.numel() < xq_bytes(cols):
        raise ValueError("staging buffer too small")
    check("rtxllm_stage_activation", lib().rtxllm_stage_activation(ptr(x), ptr(weight), cols, ptr(out), stream()))
    return out


def matvec_xq(w: DevicePack, xq: torch.Tensor, y: torch.Tensor | None = None) -> torch.Tensor:
    if xq.dtype != torch.uint8 or xq.numel() < xq_bytes(w.cols) or not xq.is_cuda:
        raise ValueError("expected a device staging buffer of rtxllm_xq_bytes(cols) bytes")
    if y is None:
        y = torch.empty(w.rows, dtype=torch.float32, device=xq.device)
    _check_vec(y, w.rows)
    check("rtxllm_matvec_xq", lib().rtxllm_matvec_xq(w.fmt, ptr(w.payload), ptr(w.meta), ptr(xq), ptr(y), w.rows,
                                                      w.cols, stream()))
    return y


# ---- batched matvec (1..8 activation vectors, matrix cores) -------------------------

BATCH_MAX = 8


def x16_bytes(cols: int) -> int:
    return int(lib().rtxllm_x16_bytes(cols))


def stage_batch(x: torch.Tensor, out: torch.Tensor | None = None) -> torch.Tensor:
    """x: device fp32 [batch, cols] -> the staged fp16 hi/lo buffer (uint8)."""
    if x.dim() != 2 or x.dtype != torch.float32 or not x.is_cuda or not x.is_contiguous():
        raise ValueError("expected a contiguous device fp32 [batch, cols] tensor")
    batch, cols = x.shape
    if out is None:
        out = torch.empty(x16_bytes(cols), dtype=torch.uint8, device=x.device)
    if out.numel() < x16_bytes(cols):
        raise ValueError("staging buffer smaller than rtxllm_x16_bytes(cols)")
    check("rtxllm_stage_batch", lib().rtxllm_stage_batch(ptr(x), batch, cols, ptr(out), stream()))
    return out


def matvec_batch(w: DevicePack, x16: torch.Tensor, batch: int, y: torch.Tensor | None = None,
                 workspace: torch.Tensor | None = None) -> torch.Tensor:
    """y [batch, rows] = W x_s for the staged activations."""
    if x16.dtype != torch.uint8 or x16.numel() < x16_bytes(w.cols) or not x16.is_cuda:
        raise ValueError("expected a device staging buffer of rtxllm_x16_bytes(cols) bytes")
    if y is None:
        y = torch.empty((batch, w.rows), dtype=torch.float32, device=x16.device)
    _check_vec(y, batch * w.rows)
    need = int(lib().rtxllm_matvec_batch_workspace(w.fmt, w.rows, w.cols))
    if need and (workspace is None or workspace.numel() < need):
        workspace = torch.empty(need, dtype=torch.uint8, device=x16.device)
    check("rtxllm_matvec_batch", lib().rtxllm_matvec_batch(w.fmt, ptr(w.payload), ptr(w.meta), ptr(x16), ptr(y),
                                                            w.rows, w.cols, batch,
                                                            ptr(workspace) if need else None, need, stream()))
    return y
