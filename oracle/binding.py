"""ctypes binding of oracle/_build/liboracle.so (test infrastructure only)."""

from __future__ import annotations

import ctypes
import os
import subprocess
from ctypes import POINTER, Structure, c_double, c_float, c_int, c_int32, c_size_t, c_uint8, c_uint16, c_uint32, c_void_p
from pathlib import Path

import numpy as np

ROOT = Path(__file__).resolve().parent
LIB_PATH = ROOT / "_build" / "liboracle.so"

_P = c_void_p
_U = c_uint32


class KvCache(Structure):
    _fields_ = [
        ("k_pages", _P),
        ("v_pages", _P),
        ("block_table", _P),
        ("page_size", _U),
        ("n_kv_heads", _U),
        ("head_dim", _U),
    ]


class LayerWeights(Structure):
    _fields_ = [(n, c_int) for n in ("fmt_q", "fmt_k", "fmt_v", "fmt_o", "fmt_gate", "fmt_up", "fmt_down")] + [
        (n, _P)
        for n in (
            "wq", "wq_meta", "wk", "wk_meta", "wv", "wv_meta", "wo", "wo_meta",
            "wgate", "wgate_meta", "wup", "wup_meta", "wdown", "wdown_meta",
            "attn_norm", "ffn_norm",
        )
    ]


class LayerShape(Structure):
    _fields_ = [(n, _U) for n in ("hidden", "n_heads", "n_kv_heads", "head_dim", "ffn")] + [
        ("eps", c_float),
        ("inv_freq", _P),
    ]


_SIGS = {
    "orc_fp16_to_f32": (c_float, [c_uint16]),
    "orc_f32_to_fp16_rne": (c_uint16, [c_float]),
    "orc_scale_min_k4": (None, [c_int, _P, _P, _P]),
    "orc_iq2s_grid": (POINTER(c_uint16), []),
    "orc_iq3s_grid": (POINTER(c_uint32), []),
    "orc_payload_bytes": (_U, [c_int]),
    "orc_meta_bytes": (_U, [c_int]),
    "orc_dequant_value": (c_float, [c_int, _P, _P, _U]),
    "orc_dequant": (None, [c_int, _P, _P, _U, _U, _P]),
    "orc_matvec_f32": (None, [c_int, _P, _P, _P, _U, _U, _P, c_int]),
    "orc_matvec_f64": (None, [c_int, _P, _P, _P, _U, _U, _P, c_int]),
    "orc_q4k_split": (None, [c_int, _P, c_size_t, _P, _P]),
    "orc_argmax": (_U, [_P, _U]),
    "orc_stage_activation": (None, [_P, _P, _U, _P, _P, _P, _P, _P]),
    "orc_matvec_staged_f64": (None, [c_int, _P, _P, _P, _P, _P, _P, _U, _U, _P, c_int]),
    "orc_kv_side_write": (None, [_P, _U, _P, _U, _U, _U, _U]),
    "orc_rmsnorm_feedback": (None, [_P, _U, _P, _U, c_float]),
    "orc_silu_rmsnorm_feedback": (None, [_P, _U, _P, _U, c_float]),
    "orc_rmsnorm_feedback_with_silu_cache": (None, [_P, _U, _P, _P, _U, c_float]),
    "orc_gated_silu_rmsnorm_feedback": (None, [_P, _U, _P, _U, _P, _U, c_float]),
    "orc_rmsnorm_cache": (None, [_P, _U, _P, _U, c_float, c_int, c_int]),
    "orc_rmsnorm_cache_and_gated_product": (None, [_P, _U, _P, _P, _P, _U, _U, c_float, c_int]),
    "orc_rope_rotate_pair": (None, [c_float, c_float, c_float, _P, _P]),
    "orc_rmsnorm_weighted": (None, [_P, _P, _U, c_float, _P]),
    "orc_rope_inv_freq": (None, [_U, c_double, _P]),
    "orc_rope": (None, [_P, _U, _U, _P, _U]),
    "orc_silu_mul": (None, [_P, _P, _U, _P]),
    "orc_embed_q5k": (None, [_P, _U, _U, _P]),
    "orc_kv_append": (None, [POINTER(KvCache), _U, _P, _P]),
    "orc_attention_decode": (None, [POINTER(KvCache), _P, _U, _U, _P]),
    "orc_layer_forward": (None, [POINTER(LayerWeights), POINTER(LayerShape), POINTER(KvCache), _U, _P, c_int]),
    "orc_layer_forward_given_kv": (None, [POINTER(LayerWeights), POINTER(LayerShape), POINTER(KvCache), _U, _P,
                                          c_int]),
}

_lib = None


def build() -> None:
    subprocess.run(["make", "-s", "-C", os.fspath(ROOT)], check=True)


def lib() -> ctypes.CDLL:
    global _lib
    if _lib is None:
        if not LIB_PATH.is_file():
            build()
        h = ctypes.CDLL(os.fspath(LIB_PATH))
        for name, (res, args) in _SIGS.items():
            fn = getattr(h, name)
            fn.restype = res
            fn.argtypes = args
        _lib = h
    return _lib


def ptr(a: np.ndarray | None) -> int | None:
    if a is None:
        return None
    assert a.flags["C_CONTIGUOUS"]
    return a.ctypes.data_as(c_void_p).value


def dequant(fmt: int, payload: np.ndarray, meta: np.ndarray | None, rows: int, cols: int) -> np.ndarray:
    out = np.empty((rows, cols), dtype=np.float32)
    lib().orc_dequant(fmt, ptr(payload), ptr(meta), rows, cols, ptr(out))
    return out


def matvec_f32(fmt, payload, meta, x, rows, cols, threads=1) -> np.ndarray:
    y = np.empty(rows, dtype=np.float32)
    lib().orc_matvec_f32(fmt, ptr(payload), ptr(meta), ptr(np.ascontiguousarray(x, np.float32)), rows, cols, ptr(y), threads)
    return y


def matvec_f64(fmt, payload, meta, x, rows, cols, threads=1) -> np.ndarray:
    y = np.empty(rows, dtype=np.float64)
    lib().orc_matvec_f64(fmt, ptr(payload), ptr(meta), ptr(np.ascontiguousarray(x, np.float32)), rows, cols, ptr(y), threads)
    return y


def q4k_split(fmt: int, raw: np.ndarray, meta_bytes: int) -> tuple[np.ndarray, np.ndarray]:
    n = raw.size // 144
    payload = np.empty(n * 128, np.uint8)
    meta = np.empty(n * meta_bytes, np.uint8)
    lib().orc_q4k_split(fmt, ptr(raw), n, ptr(payload), ptr(meta))
    return payload, meta


def argmax(y: np.ndarray) -> int:
    y = np.ascontiguousarray(y, np.float32)
    return int(lib().orc_argmax(ptr(y), y.size))


def iq2s_grid() -> np.ndarray:
    return np.ctypeslib.as_array(lib().orc_iq2s_grid(), shape=(1024,)).copy()


def iq3s_grid() -> np.ndarray:
    return np.ctypeslib.as_array(lib().orc_iq3s_grid(), shape=(512,)).copy()


def stage_activation(x: np.ndarray, weight: np.ndarray | None = None):
    """(H, M, L int8[cols], scale f32[cols/16], sum f32[cols/16])."""
    x = np.ascontiguousarray(x, np.float32)
    cols = x.size
    h, m, l = (np.empty(cols, np.int8) for _ in range(3))
    s = np.empty(cols // 16, np.float32)
    t = np.empty(cols // 16, np.float32)
    w = None if weight is None else np.ascontiguousarray(weight, np.float32)
    lib().orc_stage_activation(ptr(x), ptr(w), cols, ptr(h), ptr(m), ptr(l), ptr(s), ptr(t))
    return h, m, l, s, t


def stage_bytes(x: np.ndarray, weight: np.ndarray | None = None) -> np.ndarray:
    """The staged activation in the product's one-buffer layout: H, M, L, scale, sum."""
    h, m, l, s, t = stage_activation(x, weight)
    return np.concatenate([h.view(np.uint8), m.view(np.uint8), l.view(np.uint8), s.view(np.uint8),
                           t.view(np.uint8)])


def matvec_staged_f64(fmt, payload, meta, x, rows, cols, threads=1, weight=None) -> np.ndarray:
    h, m, l, s, _ = stage_activation(x, weight)
    y = np.empty(rows, dtype=np.float64)
    lib().orc_matvec_staged_f64(fmt, ptr(payload), ptr(meta), ptr(h), ptr(m), ptr(l), ptr(s), rows, cols, ptr(y),
                                threads)
    return y
