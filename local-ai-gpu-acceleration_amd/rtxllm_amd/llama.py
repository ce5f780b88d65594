"""Python handle on the C-ABI Llama decode runner (include/rtxllm/llama.h).

The runner owns its VRAM arena; this wrapper only passes configuration,
host arrays to upload, and the HIP stream. Every computation runs in
build/librtxllm.so.
"""

from __future__ import annotations

import ctypes
from ctypes import c_float, c_int, c_uint32, c_uint64, c_void_p, c_size_t
from dataclasses import dataclass

import numpy as np

from . import formats as F
from ._lib import check, lib


class LlamaConfig(ctypes.Structure):
    _fields_ = [(n, c_uint32) for n in ("hidden", "n_heads", "n_kv_heads", "ffn", "vocab", "n_layers", "max_ctx",
                                         "page_size")] + [
        ("rope_theta", c_float),
        ("rms_eps", c_float),
    ] + [(n, c_int) for n in ("fmt_qkv", "fmt_o", "fmt_gate_up", "fmt_down", "fmt_lm_head")] + [
        ("batch", c_uint32),
    ]


EMBED, HEAD = 1, 2
HEAD_DIM = 128

# Formats of the 8B mixed-quant configuration: q/k/v/o IQ3_S, gate/up IQ2_S,
# down Q4_K (resident split-native pack), embedding and LM head Q5_K.
MIXED_8B_FORMATS = dict(fmt_qkv=F.IQ3S, fmt_o=F.IQ3S, fmt_gate_up=F.IQ2S, fmt_down=F.Q4K_SPLIT_NATIVE,
                        fmt_lm_head=F.Q5K)


@dataclass
class Shape:
    hidden: int
    n_heads: int
    n_kv_heads: int
    ffn: int
    vocab: int
    n_layers: int
    max_ctx: int
    page_size: int = 64
    rope_theta: float = 500000.0
    rms_eps: float = 1e-6
    batch: int = 1

    def config(self, formats: dict | None = None) -> LlamaConfig:
        f = dict(MIXED_8B_FORMATS)
        f.update(formats or {})
        return LlamaConfig(self.hidden, self.n_heads, self.n_kv_heads, self.ffn, self.vocab, self.n_layers,
                           self.max_ctx, self.page_size, self.rope_theta, self.rms_eps, f["fmt_qkv"], f["fmt_o"],
                           f["fmt_gate_up"], f["fmt_down"], f["fmt_lm_head"], self.batch)


LLAMA_8B = Shape(hidden=4096, n_heads=32, n_kv_heads=8, ffn=14336, vocab=128256, n_layers=32, max_ctx=4096)


def tensor_seed(seed: int, layer: int | None, role: str) -> int:
    """Seed of one synthetic weight tensor (rtxllm_llama_synth_weights)."""
    roles = {"qkv": 1, "o": 2, "gate_up": 3, "down": 4}
    if role == "embed":
        return seed + 5
    if role == "lm_head":
        return seed + 6
    return seed + 4096 * (layer + 1) + roles[role]


class Llama:
    def __init__(self, shape: Shape, formats: dict | None = None):
        self.shape = shape
        self.cfg = shape.config(formats)
        self.formats = {k: getattr(self.cfg, k) for k in MIXED_8B_FORMATS}
        handle = c_void_p()
        check("rtxllm_llama_create", lib().rtxllm_llama_create(ctypes.byref(self.cfg), ctypes.byref(handle)))
        self.h = handle.value

    def close(self) -> None:
        if self.h:
            lib().rtxllm_llama_destroy(self.h)
            self.h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    # -- regions -------------------------------------------------------------
    def region_bytes(self, name: str, layer: int = 0) -> int:
        n = c_size_t()
        p = lib().rtxllm_llama_region(self.h, name.encode(), layer, ctypes.byref(n))
        if not p:
            raise KeyError(name)
        return n.value

    def region_ptr(self, name: str, layer: int = 0) -> int:
        p = lib().rtxllm_llama_region(self.h, name.encode(), layer, None)
        if not p:
            raise KeyError(name)
        return p

    def upload(self, name: str, arr: np.ndarray, layer: int = 0, offset: int = 0) -> None:
        a = np.ascontiguousarray(arr)
        check("rtxllm_llama_upload", lib().rtxllm_llama_upload(self.h, name.encode(), layer, offset,
                                                                a.ctypes.data_as(c_void_p), a.nbytes))

    def download(self, name: str, dtype, count: int | None = None, layer: int = 0, offset: int = 0) -> np.ndarray:
        itemsize = np.dtype(dtype).itemsize
        if count is None:
            count = (self.region_bytes(name, layer) - offset) // itemsize
        out = np.empty(count, dtype=dtype)
        check("rtxllm_llama_download", lib().rtxllm_llama_download(self.h, name.encode(), layer, offset,
                                                                    out.ctypes.data_as(c_void_p), out.nbytes))
        return out

    # -- execution --------------------------------------------------------------
    def synth_weights(self, seed: int, stream: int = 0) -> None:
        check("rtxllm_llama_synth_weights", lib().rtxllm_llama_synth_weights(self.h, seed, stream))

    def forward(self, first: int, last: int, flags: int, stream: int = 0) -> None:
        check("rtxllm_llama_forward", lib().rtxllm_llama_forward(self.h, first, last, flags, stream))

    def step(self, stream: int = 0) -> None:
        check("rtxllm_llama_step", lib().rtxllm_llama_step(self.h, stream))

    def graph_capture(self, stream: int) -> None:
        check("rtxllm_llama_graph_capture", lib().rtxllm_llama_graph_capture(self.h, stream))

    def graph_replay(self, stream: int) -> None:
        check("rtxllm_llama_graph_replay", lib().rtxllm_llama_graph_replay(self.h, stream))

    def graph_capture_span(self, span: int, stream: int) -> None:
        """Capture a step whose attention covers only positions below `span`."""
        check("rtxllm_llama_graph_capture_span", lib().rtxllm_llama_graph_capture_span(self.h, span, stream))

    def graph_replay_span(self, span: int, stream: int) -> None:
        check("rtxllm_llama_graph_replay_span", lib().rtxllm_llama_graph_replay_span(self.h, span, stream))

    def graph_span_for(self, position: int) -> int:
        """Smallest captured span above `position` (0: none captured)."""
        return int(lib().rtxllm_llama_graph_span_for(self.h, position))

    def graph_bytes(self) -> int:
        return int(lib().rtxllm_llama_graph_bytes(self.h))

    STAGES = {"embed": 0, "qkv": 1, "attention": 2, "o": 3, "gate_up": 4, "down": 5, "lm_head": 6}

    def launch_stage(self, layer: int, stage: str, stream: int = 0) -> None:
        check("rtxllm_llama_launch_stage", lib().rtxllm_llama_launch_stage(self.h, layer, self.STAGES[stage], stream))

    def load_packs(self, q4k_manifest=None, iq_manifest=None, payload_root=None) -> None:
        """Fill the weights from resident-pack manifests (include/rtxllm/llama.h)."""
        err = ctypes.create_string_buffer(1024)
        enc = lambda p: None if p is None else str(p).encode()
        rc = lib().rtxllm_llama_load_packs(self.h, enc(q4k_manifest), enc(iq_manifest), enc(payload_root), err,
                                           len(err))
        if rc != 0:
            from ._lib import HipError
            raise HipError(f"rtxllm_llama_load_packs: {err.value.decode(errors='replace')}", rc)

    def load_pack_set(self, manifests, payload_root=None) -> None:
        """Fill the weights from any number of manifests, each read by the loader
        its producer needs (rtxllm_llama_load_pack_set)."""
        paths = [str(p).encode() for p in manifests]
        arr = (ctypes.c_char_p * max(1, len(paths)))(*paths)
        err = ctypes.create_string_buffer(1024)
        rc = lib().rtxllm_llama_load_pack_set(self.h, ctypes.cast(arr, c_void_p), len(paths),
                                              None if payload_root is None else str(payload_root).encode(), err,
                                              len(err))
        if rc != 0:
            from ._lib import HipError
            raise HipError(f"rtxllm_llama_load_pack_set: {err.value.decode(errors='replace')}", rc)

    def memory(self) -> dict:
        """The create-time admission figures: required, usable and arena bytes."""
        req, use, arena = c_size_t(), c_size_t(), c_size_t()
        check("rtxllm_llama_memory", lib().rtxllm_llama_memory(self.h, ctypes.byref(req), ctypes.byref(use),
                                                               ctypes.byref(arena)))
        return {"required_bytes": req.value, "usable_bytes": use.value, "arena_bytes": arena.value}

    def status(self, stream: int = 0) -> list[int]:
        """Per-sequence status words (RTXLLM_LLAMA_STATUS_*), read synchronously."""
        out = np.zeros(max(1, self.shape.batch), np.uint32)
        check("rtxllm_llama_status", lib().rtxllm_llama_status(self.h, out.ctypes.data_as(c_void_p), stream))
        return [int(v) for v in out]

    def clear_status(self, stream: int = 0) -> None:
        check("rtxllm_llama_clear_status", lib().rtxllm_llama_clear_status(self.h, stream))

    def launches_per_step(self) -> int:
        return int(lib().rtxllm_llama_launches_per_step(self.h))

    def set_token_pos(self, token, pos) -> None:
        """token / pos: ints (batch 1) or one per sequence."""
        self.upload("token", np.atleast_1d(np.asarray(token, np.uint32)))
        self.upload("pos", np.atleast_1d(np.asarray(pos, np.uint32)))
