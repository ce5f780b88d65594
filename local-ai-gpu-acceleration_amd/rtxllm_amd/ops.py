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
