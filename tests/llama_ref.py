"""Oracle-side decode step for the runner tests: builds the oracle's layer
structs from the runner's own regions (weights downloaded after the device
generator filled them) and runs embed -> layers -> final norm -> LM head ->
argmax on the CPU (oracle/rtxllm_oracle.c)."""

from __future__ import annotations

import ctypes

import numpy as np

from rtxllm_amd import formats as F
from rtxllm_amd.llama import HEAD_DIM, Llama

ORC_FMT = {F.Q4K_SPLIT_NATIVE: F.Q4K_SPLIT_NATIVE, F.Q4K_RAW: F.Q4K_RAW, F.Q5K: F.Q5K, F.IQ2S: F.IQ2S,
           F.IQ3S: F.IQ3S, F.Q4K_SPLIT_PREDECODED: F.Q4K_SPLIT_PREDECODED, F.Q4K_SPLIT_HALF: F.Q4K_SPLIT_HALF,
           F.Q4K_SPLIT_COMPACT: F.Q4K_SPLIT_COMPACT}


def row_bytes(fmt: int, cols: int) -> int:
    return (cols // 256) * F.PAYLOAD_BYTES[fmt]


def meta_row_bytes(fmt: int, cols: int) -> int:
    return (cols // 256) * F.META_BYTES.get(fmt, 0)


class HostModel:
    """Host copies of every region the oracle reads."""

    def __init__(self, m: Llama, layers: range):
        s, f = m.shape, m.formats
        self.m, self.layers = m, layers
        self.q_rows, self.kv_rows = s.n_heads * HEAD_DIM, s.n_kv_heads * HEAD_DIM
        self.L = {}
        for l in layers:
            d = {}
            for role in ("qkv", "o", "gate_up", "down"):
                d[role] = m.download(role, np.uint8, layer=l)
                try:
                    d[role + "_meta"] = m.download(role + "_meta", np.uint8, layer=l)
                except KeyError:
                    d[role + "_meta"] = None
            for nm in ("attn_norm", "ffn_norm"):
                d[nm] = m.download(nm, np.float32, layer=l)
            d["k_cache"] = m.download("k_cache", np.uint16, layer=l)
            d["v_cache"] = m.download("v_cache", np.uint16, layer=l)
            d["block_table"] = m.download("block_table", np.int32, layer=l)
            # stacked q | k | v rows
            fq, H = f["fmt_qkv"], s.hidden
            rb, mb = row_bytes(fq, H), meta_row_bytes(fq, H)
            qkv, qm = d["qkv"], d["qkv_meta"]
            cuts = [0, self.q_rows, self.q_rows + self.kv_rows, self.q_rows + 2 * self.kv_rows]
            for i, nm in enumerate(("wq", "wk", "wv")):
                d[nm] = np.ascontiguousarray(qkv[cuts[i] * rb:cuts[i + 1] * rb])
                d[nm + "_meta"] = None if qm is None else np.ascontiguousarray(qm[cuts[i] * mb:cuts[i + 1] * mb])
            # interleaved gate / up rows
            fg = f["fmt_gate_up"]
            rb, mb = row_bytes(fg, H), meta_row_bytes(fg, H)
            gu = d["gate_up"].reshape(s.ffn, 2, rb)
            d["wgate"], d["wup"] = np.ascontiguousarray(gu[:, 0]).ravel(), np.ascontiguousarray(gu[:, 1]).ravel()
            if d["gate_up_meta"] is not None:
                gm = d["gate_up_meta"].reshape(s.ffn, 2, mb)
                d["wgate_meta"], d["wup_meta"] = (np.ascontiguousarray(gm[:, 0]).ravel(),
                                                  np.ascontiguousarray(gm[:, 1]).ravel())
            else:
                d["wgate_meta"] = d["wup_meta"] = None
            self.L[l] = d
        self.embed = m.download("embed", np.uint8)
        self.lm_head = m.download("lm_head", np.uint8)
        try:
            self.lm_meta = m.download("lm_head_meta", np.uint8)
        except KeyError:
            self.lm_meta = None
        self.out_norm = m.download("out_norm", np.float32)

    def run(self, orc, h: np.ndarray, pos: int, threads: int = 8, head: bool = True, layers=None, seq: int = 0,
            given_kv: bool = False):
        """Layers (all of this model's, or the given subset) in place on h
        (float32) for sequence `seq` (its block-table row and KV pages);
        returns (h, logits or None). given_kv: the host caches already hold the
        K / V of `pos` (no append; orc_layer_forward_given_kv)."""
        s, f, P = self.m.shape, self.m.formats, orc.ptr
        lib = orc.lib()
        inv_freq = np.empty(HEAD_DIM // 2, np.float32)
        lib.orc_rope_inv_freq(HEAD_DIM, s.rope_theta, P(inv_freq))
        shape = orc.LayerShape(s.hidden, s.n_heads, s.n_kv_heads, HEAD_DIM, s.ffn, s.rms_eps, P(inv_freq))
        for l in (self.layers if layers is None else layers):
            d = self.L[l]
            w = orc.LayerWeights(
                f["fmt_qkv"], f["fmt_qkv"], f["fmt_qkv"], f["fmt_o"], f["fmt_gate_up"], f["fmt_gate_up"],
                f["fmt_down"],
                P(d["wq"]), P(d["wq_meta"]), P(d["wk"]), P(d["wk_meta"]), P(d["wv"]), P(d["wv_meta"]),
                P(d["o"]), P(d["o_meta"]), P(d["wgate"]), P(d["wgate_meta"]), P(d["wup"]), P(d["wup_meta"]),
                P(d["down"]), P(d["down_meta"]), P(d["attn_norm"]), P(d["ffn_norm"]))
            pps = s.max_ctx // s.page_size
            table = np.ascontiguousarray(d["block_table"][seq * pps:(seq + 1) * pps])
            kv = orc.KvCache(P(d["k_cache"]), P(d["v_cache"]), P(table), s.page_size, s.n_kv_heads, HEAD_DIM)
            fwd = lib.orc_layer_forward_given_kv if given_kv else lib.orc_layer_forward
            fwd(ctypes.byref(w), ctypes.byref(shape), ctypes.byref(kv), pos, P(h), threads)
        if not head:
            return h, None
        xn = np.empty_like(h)
        lib.orc_rmsnorm_weighted(P(h), P(self.out_norm), s.hidden, s.rms_eps, P(xn))
        logits = orc.matvec_f32(f["fmt_lm_head"], self.lm_head, self.lm_meta, xn, s.vocab, s.hidden, threads)
        return h, logits

    def kv_of(self, orc, h: np.ndarray, pos: int, layer: int) -> tuple[np.ndarray, np.ndarray]:
        """The oracle's fp32 k (rotated) and v of layer `layer` for input h at pos."""
        s, f, P = self.m.shape, self.m.formats, orc.ptr
        lib = orc.lib()
        d = self.L[layer]
        xn = np.empty(s.hidden, np.float32)
        hh = np.ascontiguousarray(h, np.float32)
        lib.orc_rmsnorm_weighted(P(hh), P(d["attn_norm"]), s.hidden, s.rms_eps, P(xn))
        k = orc.matvec_f32(f["fmt_qkv"], d["wk"], d["wk_meta"], xn, self.kv_rows, s.hidden, 8)
        v = orc.matvec_f32(f["fmt_qkv"], d["wv"], d["wv_meta"], xn, self.kv_rows, s.hidden, 8)
        inv_freq = np.empty(HEAD_DIM // 2, np.float32)
        lib.orc_rope_inv_freq(HEAD_DIM, s.rope_theta, P(inv_freq))
        lib.orc_rope(P(k), s.n_kv_heads, HEAD_DIM, P(inv_freq), pos)
        return k, v

    def embed_row(self, orc, token: int) -> np.ndarray:
        out = np.empty(self.m.shape.hidden, np.float32)
        orc.lib().orc_embed_q5k(orc.ptr(self.embed), self.m.shape.hidden, token, orc.ptr(out))
        return out


def kv_slot(m: Llama, pos: int, head: int, table: np.ndarray) -> int:
    s = m.shape
    page = int(table[pos // s.page_size])
    return (((page * s.n_kv_heads + head) * s.page_size) + pos % s.page_size) * HEAD_DIM
