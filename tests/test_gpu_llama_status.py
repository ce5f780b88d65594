"""The decode runner at the end of the context: a step at the last position
(max_ctx - 1) is an ordinary step; a step at max_ctx has no KV slot for its
token, so it leaves the sequence's token and position as they were and sets
the sequence's RTXLLM_LLAMA_STATUS_CONTEXT_FULL bit (eagerly and in a graph
replay, batch 1 and per sequence of a batch). Positions at or past max_ctx and
tokens past the vocabulary are refused on upload."""

from __future__ import annotations

import ctypes

import numpy as np
import pytest

torch = pytest.importorskip("torch")

from rtxllm_amd import packs  # noqa: E402
from rtxllm_amd._lib import HipError, lib  # noqa: E402
from rtxllm_amd.llama import Llama, Shape  # noqa: E402

pytestmark = pytest.mark.gpu

CONTEXT_FULL = 1


def build(shape: Shape, seed: int) -> Llama:
    m = Llama(shape)
    m.synth_weights(seed)
    torch.cuda.synchronize()
    H = shape.hidden
    for l in range(shape.n_layers):
        m.upload("attn_norm", packs.normal_f32(seed + 100 + 2 * l, H, mean=1.0, std=0.02), layer=l)
        m.upload("ffn_norm", packs.normal_f32(seed + 101 + 2 * l, H, mean=1.0, std=0.02), layer=l)
        n = m.region_bytes("k_cache", l) // 2
        m.upload("k_cache", packs.normal_f16_bits(seed + 300 + 2 * l, n), layer=l)
        m.upload("v_cache", packs.normal_f16_bits(seed + 301 + 2 * l, n), layer=l)
    m.upload("out_norm", packs.normal_f32(seed + 99, H, mean=1.0, std=0.02))
    return m


def status(m: Llama, stream: int) -> list[int]:
    out = np.zeros(m.shape.batch, np.uint32)
    assert lib().rtxllm_llama_status(m.h, out.ctypes.data_as(ctypes.c_void_p), stream) == 0
    return [int(v) for v in out]


@pytest.mark.parametrize("use_graph", [False, True], ids=["eager", "graph"])
def test_context_end_batch1(use_graph):
    s = Shape(hidden=512, n_heads=4, n_kv_heads=2, ffn=1024, vocab=1000, n_layers=2, max_ctx=256, page_size=16)
    m = build(s, 0x5EED0C01)
    sp = torch.cuda.Stream().cuda_stream
    step = (lambda: m.graph_replay(sp)) if use_graph else (lambda: m.step(sp))
    if use_graph:
        m.graph_capture(sp)
    m.set_token_pos(5, s.max_ctx - 1)
    step()
    torch.cuda.synchronize()
    assert status(m, sp) == [0]
    assert int(m.download("pos", np.uint32)[0]) == s.max_ctx
    tok = int(m.download("token", np.uint32)[0])
    k_before = [m.download("k_cache", np.uint16, layer=l) for l in range(s.n_layers)]
    for _ in range(2):  # steps past the end: no KV write, token and position frozen
        step()
        torch.cuda.synchronize()
        assert status(m, sp) == [CONTEXT_FULL]
        assert int(m.download("pos", np.uint32)[0]) == s.max_ctx
        assert int(m.download("token", np.uint32)[0]) == tok
        for l in range(s.n_layers):
            assert np.array_equal(m.download("k_cache", np.uint16, layer=l), k_before[l])
    assert lib().rtxllm_llama_clear_status(m.h, sp) == 0
    assert status(m, sp) == [0]
    with pytest.raises(HipError):
        m.set_token_pos(5, s.max_ctx)
    with pytest.raises(HipError):
        m.set_token_pos(s.vocab, 0)
    m.close()


def test_context_end_per_sequence_of_a_batch():
    s = Shape(hidden=512, n_heads=4, n_kv_heads=2, ffn=1024, vocab=1000, n_layers=2, max_ctx=256, page_size=16,
              batch=4)
    m = build(s, 0x5EED0C02)
    sp = torch.cuda.Stream().cuda_stream
    positions = [s.max_ctx - 1, 10, s.max_ctx - 2, 0]
    m.set_token_pos([1, 2, 3, 4], positions)
    m.step(sp)
    torch.cuda.synchronize()
    assert status(m, sp) == [0, 0, 0, 0]
    tok1 = m.download("token", np.uint32).copy()
    m.step(sp)  # sequence 0 is at max_ctx now
    torch.cuda.synchronize()
    assert status(m, sp) == [CONTEXT_FULL, 0, 0, 0]
    pos = m.download("pos", np.uint32)
    assert list(pos) == [s.max_ctx, 12, s.max_ctx, 2]
    assert int(m.download("token", np.uint32)[0]) == int(tok1[0])
    m.step(sp)  # and sequence 2 as well
    torch.cuda.synchronize()
    assert status(m, sp) == [CONTEXT_FULL, 0, CONTEXT_FULL, 0]
    assert list(m.download("pos", np.uint32)) == [s.max_ctx, 13, s.max_ctx, 3]
    m.close()
