"""ctypes binding of build/librtxllm.so, the gfx950 decode library's C-ABI.

The library is the product: nothing here falls back to another implementation.
If the shared object is missing or fails to load, ``lib()`` raises.
"""

from __future__ import annotations

import ctypes
import os
from ctypes import c_float, c_int, c_size_t, c_uint16, c_uint32, c_uint64, c_void_p
from pathlib import Path

PKG_ROOT = Path(__file__).resolve().parent.parent
LIB_PATH = PKG_ROOT / "build" / "librtxllm.so"
# The bench's measurement helper (a plain streaming read), not part of the library.
PROBE_LIB_PATH = PKG_ROOT / "build" / "librtxllm_probe.so"

_P = c_void_p  # device or host pointer
_U = c_uint32
_S = c_void_p  # hipStream_t

# name -> argtypes. Every launcher returns hipError_t (int).
_LAUNCH_SIGS: dict[str, list] = {
    "rtxllm_launch_rmsnorm_feedback": [_P, _P, _U, _U, c_float, _S],
    "rtxllm_launch_silu_rmsnorm_feedback": [_P, _P, _U, _U, c_float, _S],
    "rtxllm_launch_rmsnorm_feedback_with_silu_cache": [_P, _P, _P, _U, _U, c_float, _S],
    "rtxllm_launch_gated_silu_rmsnorm_feedback": [_P, _P, _P, _U, _U, _U, c_float, _S],
    "rtxllm_launch_rmsnorm_silu_cache": [_P, _P, _U, _U, c_float, _U, _S],
    "rtxllm_launch_rmsnorm_cache": [_P, _P, _U, _U, c_float, _U, _S],
    "rtxllm_launch_rmsnorm_cache_and_gated_product": [_P, _P, _P, _P, _U, _U, _U, c_float, _U, _S],
    "rtxllm_launch_output_token_sample": [_P, _P, _U, _U, _U, _S],
    "rtxllm_launch_q5k_matvec_decode_probe": [_P, _P, _P, _P, _P, _U, _U, _U, _U, _U, _U, _S],
    "rtxllm_launch_iq2s_matvec_probe": [_P, _P, _P, _U, _U, _U, _S],
    "rtxllm_launch_iq2s_matvec_decode_probe": [_P, _P, _P, _P, _P, _U, _U, _U, _U, _U, _U, _S],
    "rtxllm_launch_iq3s_matvec_decode_probe": [_P, _P, _P, _P, _P, _U, _U, _U, _U, _U, _U, _S],
    "rtxllm_dequant_f32": [c_int, _P, _P, _U, _U, _P, _S],
    "rtxllm_matvec": [c_int, _P, _P, _P, _P, _U, _U, _S],
    "rtxllm_stage_activation": [_P, _P, _U, _P, _S],
    "rtxllm_matvec_xq": [c_int, _P, _P, _P, _P, _U, _U, _S],
    "rtxllm_matvec_xq_mfma": [c_int, _P, _P, _P, _U, _U, _S],
    "rtxllm_gate_up_silu": [c_int, _P, _P, _P, _P, _U, c_float, _P, _U, _U, _P, _S],
    "rtxllm_test_gate_up_silu_waits": [c_int, _P, _P, _P, _P, _U, c_float, _P, _U, _U, _P, _U, _U, _S],
    "rtxllm_stage_batch": [_P, _U, _U, _P, _S],
    "rtxllm_matvec_batch": [c_int, _P, _P, _P, _P, _U, _U, _U, _P, c_size_t, _S],
    "rtxllm_matvec_batch_f32": [c_int, _P, _P, _P, _P, _U, _U, _U, _P, c_size_t, _S],
    "rtxllm_matvec_batch_noalloc": [c_int, _P, _P, _P, _P, _U, _U, _U, _S],
    "rtxllm_llama_create": [_P, _P],
    "rtxllm_llama_admission": [_P, c_size_t, _P, _P, _P, ctypes.c_char_p, c_size_t],
    "rtxllm_llama_upload": [_P, ctypes.c_char_p, _U, c_size_t, _P, c_size_t],
    "rtxllm_llama_download": [_P, ctypes.c_char_p, _U, c_size_t, _P, c_size_t],
    "rtxllm_llama_synth_weights": [_P, c_uint64, _S],
    "rtxllm_llama_forward": [_P, _U, _U, c_int, _S],
    "rtxllm_llama_step": [_P, _S],
    "rtxllm_llama_graph_capture": [_P, _S],
    "rtxllm_llama_graph_replay": [_P, _S],
    "rtxllm_llama_graph_capture_span": [_P, _U, _S],
    "rtxllm_llama_graph_replay_span": [_P, _U, _S],
    "rtxllm_llama_launch_stage": [_P, _U, c_int, _S],
    "rtxllm_llama_load_packs": [_P, ctypes.c_char_p, ctypes.c_char_p, ctypes.c_char_p, ctypes.c_char_p, c_size_t],
    "rtxllm_llama_load_pack_set": [_P, _P, _U, ctypes.c_char_p, ctypes.c_char_p, c_size_t],
    "rtxllm_llama_memory": [_P, _P, _P, _P],
    "rtxllm_llama_status": [_P, _P, _S],
    "rtxllm_llama_clear_status": [_P, _S],
    "rtxllm_rmsnorm_w": [_P, _P, _U, _U, c_float, _P, _S],
    "rtxllm_rope_theta": [_P, _U, _U, c_float, _P, _U, _S],
    "rtxllm_silu_mul": [_P, _P, c_size_t, _P, _S],
    "rtxllm_embed_gather_q5k": [_P, _U, _U, _P, _U, _P, _S],
    "rtxllm_attn_decode_gqa_f16": [_P, _P, _P, _P, _U, _U, _U, _U, _U, _P, _U, _P, _P, c_size_t, _S],
    "rtxllm_argmax": [_P, _U, _U, _P, _S],
    "rtxllm_iq2s_units_pack": [_P, _U, _U, _P, _S],
    "rtxllm_iq3s_units_pack": [_P, _U, _U, _P, _S],
}
for _name in (
    "rtxllm_launch_q4k_matvec_decode",
    "rtxllm_launch_q4k_matvec_decode_shared",
    "rtxllm_launch_q4k_matvec_decode_warp",
    "rtxllm_launch_q4k_matvec_decode_warp_broadcast",
    "rtxllm_launch_q4k_matvec_decode_warp_broadcast_vec4",
    "rtxllm_launch_q4k_matvec_decode_warp_broadcast_vec4x2",
    "rtxllm_launch_q4k_matvec_decode_warp_broadcast_vec4x4",
):
    _LAUNCH_SIGS[_name] = [_P, _P, _P, _P, _P, _U, _U, _U, _U, _U, _S]
for _name in (
    "rtxllm_launch_q4k_matvec_decode_predecoded_vec4x4",
    "rtxllm_launch_q4k_matvec_decode_split_predecoded_vec4x4",
    "rtxllm_launch_q4k_matvec_decode_split_half_vec4x4",
    "rtxllm_launch_q4k_matvec_decode_split_compact_vec4x4",
    "rtxllm_launch_q4k_matvec_decode_split_native_vec4x4",
):
    _LAUNCH_SIGS[_name] = [_P, _P, _P, _P, _P, _P, _U, _U, _U, _U, _U, _S]



class PackOptions(ctypes.Structure):
    """rtxllm_pack_options (include/rtxllm/pack_producer.h)."""
    _fields_ = [("q4k_policy", ctypes.c_char_p), ("write_blocks", c_int), ("types", ctypes.c_char_p),
                ("names", ctypes.c_char_p), ("layer", c_int), ("limit", c_uint64)]


_C = ctypes.c_char_p
# name -> (restype, argtypes) for host helpers.
_HOST_SIGS: dict[str, tuple] = {
    "rtxllm_gguf_pack": (c_int, [_C, _C, ctypes.POINTER(PackOptions), _C, c_size_t, _C, c_size_t]),
    "rtxllm_pack_tensor": (c_int, [_C, _C, _C, _C, c_int, _C, c_size_t, _C, c_size_t]),
    "rtxllm_gguf_tensor_plan": (c_int, [_C, _C, c_size_t, _C, c_size_t]),
    "rtxllm_pack_tensor_shape": (c_int, [_C, _P, c_uint32, _P, _P, _P, _C, c_size_t]),
    "rtxllm_pack_tensor_role": (c_int, [_C, _P, _C, c_size_t]),
    "rtxllm_pack_sanitize_label": (c_int, [_C, _C, c_size_t]),
    "rtxllm_format_payload_block_bytes": (c_uint32, [c_int]),
    "rtxllm_format_meta_block_bytes": (c_uint32, [c_int]),
    "rtxllm_xq_bytes": (c_size_t, [c_uint32]),
    "rtxllm_x16_bytes": (c_size_t, [c_uint32]),
    "rtxllm_matvec_batch_workspace": (c_size_t, [c_int, c_uint32, c_uint32]),
    "rtxllm_attn_decode_workspace": (c_size_t, [c_uint32, c_uint32, c_uint32, c_uint32]),
    "rtxllm_llama_destroy": (None, [_P]),
    "rtxllm_llama_weights_changed": (None, [_P]),
    "rtxllm_llama_region": (_P, [_P, ctypes.c_char_p, _U, _P]),
    "rtxllm_llama_launches_per_step": (c_uint32, [_P]),
    "rtxllm_llama_graph_span_for": (c_uint32, [_P, _U]),
    "rtxllm_llama_graph_bytes": (c_size_t, [_P]),
    "rtxllm_q4k_split_pack": (c_int, [c_int, _P, c_size_t, _P, _P]),
    "rtxllm_synth_raw_blocks": (c_int, [c_int, c_uint64, c_size_t, c_float, c_float, _P, c_int]),
    "rtxllm_synth_normal_f32": (c_int, [c_uint64, c_size_t, c_float, c_float, _P, c_int]),
    "rtxllm_synth_normal_f16": (c_int, [c_uint64, c_size_t, c_float, c_float, _P, c_int]),
}

_lib: ctypes.CDLL | None = None


def lib() -> ctypes.CDLL:
    """Load build/librtxllm.so (once) and declare every exported signature."""
    global _lib
    if _lib is None:
        if not LIB_PATH.is_file():
            raise RuntimeError(
                f"{LIB_PATH} is missing: build it with `make -C {PKG_ROOT}` "
                "(or __graft_entry__.build()); there is no fallback path"
            )
        handle = ctypes.CDLL(os.fspath(LIB_PATH), mode=ctypes.RTLD_GLOBAL)
        for name, argtypes in _LAUNCH_SIGS.items():
            fn = getattr(handle, name)
            fn.restype = c_int
            fn.argtypes = argtypes
        for name, (restype, argtypes) in _HOST_SIGS.items():
            fn = getattr(handle, name)
            fn.restype = restype
            fn.argtypes = argtypes
        _lib = handle
    return _lib


_probe: ctypes.CDLL | None = None


def probe_lib() -> ctypes.CDLL:
    """Load build/librtxllm_probe.so, the bench's streaming-read helper."""
    global _probe
    if _probe is None:
        if not PROBE_LIB_PATH.is_file():
            raise RuntimeError(f"{PROBE_LIB_PATH} is missing: build it with `make -C {PKG_ROOT}`")
        handle = ctypes.CDLL(os.fspath(PROBE_LIB_PATH))
        handle.rtxllm_stream_read.restype = c_int
        handle.rtxllm_stream_read.argtypes = [_P, c_size_t, _P, _U, _U, _S]
        _probe = handle
    return _probe


def exported_names() -> list[str]:
    return sorted(list(_LAUNCH_SIGS) + list(_HOST_SIGS))


class HipError(RuntimeError):
    def __init__(self, name: str, code: int):
        super().__init__(f"{name} returned hipError_t {code}")
        self.code = code


def check(name: str, code: int) -> None:
    if code != 0:
        raise HipError(name, code)


__all__ = ["lib", "probe_lib", "check", "HipError", "exported_names", "LIB_PATH", "PROBE_LIB_PATH", "PackOptions",
           "c_uint16"]
