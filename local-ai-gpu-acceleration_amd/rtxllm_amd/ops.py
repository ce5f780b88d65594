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
