"""The C++ GGUF -> resident-pack producer (include/rtxllm/pack_producer.h),
called through the library's C-ABI.

pack_gguf() writes the packs of a GGUF file in the reference producers' output
form (tools/bench/q4k_resident_pack.py, iq_resident_pack.py,
q5k_resident_pack.py: one directory and manifest.json per producer, absolute
pack paths) plus the GGUF tensor plan; pack_tensor() is those producers'
pack_tensor for one tensor-plan row. The helpers below expose the producer's
shape, role and label rules. Every function raises ValueError with the
producer's message on a refused input.
"""

from __future__ import annotations

import ctypes
import json
from pathlib import Path

import numpy as np

from ._lib import PackOptions, lib


def _call(fn, *args, initial: int = 1 << 16) -> str:
    """Runs a C-ABI function that writes JSON text into (buf, len, err, err_len),
    growing the buffer when it reports -2."""
    size = initial
    while True:
        out = ctypes.create_string_buffer(size)
        err = ctypes.create_string_buffer(2048)
        rc = fn(*args, out, size, err, len(err))
        if rc == 0:
            return out.value.decode()
        msg = err.value.decode(errors="replace")
        if rc == -2 and "bytes needed" in msg:
            size = int(msg.split(":")[1].split()[0]) + 1
            continue
        raise ValueError(msg or f"{fn.__name__} failed ({rc})")


def _enc(s) -> bytes | None:
    return None if s is None else str(s).encode()


def pack_gguf(gguf_path, out_dir, policy: str = "auto", write_blocks: bool = False, types=None, names=None,
              layer: int = -1, limit: int = 0) -> dict[str, Path]:
    """Packs every selected Q4_K / Q5_K / IQ2_S / IQ3_S tensor of a GGUF file;
    returns the paths of "tensor_plan" and of each manifest written
    ("q4k_manifest", "iq_manifest", "q5k_manifest")."""
    opt = PackOptions(_enc(policy), 1 if write_blocks else 0, _enc(",".join(types)) if types else None,
                      _enc("\n".join(names)) if names else None, int(layer), int(limit))
    text = _call(lib().rtxllm_gguf_pack, _enc(gguf_path), _enc(out_dir), ctypes.byref(opt), initial=8192)
    return {k: Path(v) for k, v in json.loads(text).items() if v is not None}


def pack_tensor(model_path, tensor: dict, out_dir, policy: str = "auto", write_blocks: bool = False) -> dict:
    """One tensor-plan row (name, type, dimensions, absolute_offset,
    span_bytes) of the file at model_path -> its pack files in out_dir and
    its manifest record."""
    text = _call(lib().rtxllm_pack_tensor, _enc(model_path), _enc(json.dumps(tensor)), _enc(out_dir), _enc(policy),
                 1 if write_blocks else 0, initial=8192)
    return json.loads(text)


def tensor_plan(gguf_path) -> dict:
    """The GGUF tensor plan document (tensor_plan.json)."""
    return json.loads(_call(lib().rtxllm_gguf_tensor_plan, _enc(gguf_path)))


def tensor_shape(tensor_type: str, dims) -> tuple[int, int, int]:
    """(element count, block count, data bytes) of a tensor."""
    d = np.ascontiguousarray(np.asarray(list(dims), np.uint64))
    values, blocks, nbytes = ctypes.c_uint64(), ctypes.c_uint64(), ctypes.c_uint64()
    err = ctypes.create_string_buffer(1024)
    rc = lib().rtxllm_pack_tensor_shape(_enc(tensor_type), d.ctypes.data_as(ctypes.c_void_p), d.size,
                                        ctypes.byref(values), ctypes.byref(blocks), ctypes.byref(nbytes), err,
                                        len(err))
    if rc != 0:
        raise ValueError(err.value.decode(errors="replace"))
    return values.value, blocks.value, nbytes.value


def tensor_role(name: str) -> tuple[int | None, str]:
    """(layer or None, role) of a tensor name."""
    layer = ctypes.c_int()
    role = ctypes.create_string_buffer(len(name.encode()) + 1)
    if lib().rtxllm_pack_tensor_role(_enc(name), ctypes.byref(layer), role, len(role)) != 0:
        raise ValueError(f"tensor_role refused {name!r}")
    return (None if layer.value < 0 else layer.value), role.value.decode()


def sanitize_label(name: str) -> str:
    """The pack-file label of a tensor name."""
    out = ctypes.create_string_buffer(max(len(name.encode()), 6) + 1)
    if lib().rtxllm_pack_sanitize_label(_enc(name), out, len(out)) != 0:
        raise ValueError(f"sanitize_label refused {name!r}")
    return out.value.decode()
