"""GPU parity of the decode runner against the oracle at a small Llama shape:
device-generated packs equal the host generator's bytes; one full decode step
(Q5_K embedding gather, two mixed-quant layers with fused RMSNorm / RoPE / KV
append / GQA attention / SiLU-gate / residuals, Q5_K LM head, greedy argmax)
matches the oracle's step within 1e-3 normwise on logits and hidden state, with
the same token and the same KV-cache writes; a hipGraph replay of the step,
and of a step captured over a shorter attention span that still holds the
position, is bit-identical to the eager step. All calls go through the C-ABI."""

from __future__ import annotations

import numpy as np
import pytest

torch = pytest.importorskip("torch")

from rtxllm_amd import formats as F  # noqa: E402
from rtxllm_amd import packs  # noqa: E402
from rtxllm_amd.llama import HEAD_DIM, Llama, Shape, tensor_seed  # noqa: E402

from llama_ref import HostModel, kv_slot  # noqa: E402
from token_rule import argmax_lowest, check_token  # noqa: E402

pytestmark = pytest.mark.gpu

TOL = 1e-3
SMALL = Shape(hidden=512, n_heads=4, n_kv_heads=2, ffn=1024, vocab=1000, n_layers=2, max_ctx=256, page_size=16)
SEED = 0x5EED0004


def rel(a, b) -> float:
    a, b = np.asarray(a, np.float64), np.asarray(b, np.float64)
    return float(np.max(np.abs(a - b)) / np.max(np.abs(b)))


def build(shape: Shape, pos: int, seed: int = SEED, permute_pages: bool = True, formats: dict | None = None) -> Llama:
    m = Llama(shape, formats=formats)
    m.synth_weights(seed)
    torch.cuda.synchronize()
    H = shape.hidden
    for l in range(shape.n_layers):
        m.upload("attn_norm", packs.normal_f32(seed + 100 + 2 * l, H, mean=1.0, std=0.02), layer=l)
        m.upload("ffn_norm", packs.normal_f32(seed + 101 + 2 * l, H, mean=1.0, std=0.02), layer=l)
        n = m.region_bytes("k_cache", l) // 2
        m.upload("k_cache", packs.normal_f16_bits(seed + 300 + 2 * l, n), layer=l)
        m.upload("v_cache", packs.normal_f16_bits(seed + 301 + 2 * l, n), layer=l)
        if permute_pages:
            npages = shape.max_ctx // shape.page_size
            table = np.array([(7 * i + 3) % npages for i in range(npages)], np.int32)
            assert len(set(table.tolist())) == npages
            m.upload("block_table", table, layer=l)
    m.upload("out_norm", packs.normal_f32(seed + 99, H, mean=1.0, std=0.02))
    return m


def test_device_synth_matches_host_generator():
    s = SMALL
    m = Llama(s)
    m.synth_weights(SEED)
    torch.cuda.synchronize()
    qkv_rows = (s.n_heads + 2 * s.n_kv_heads) * HEAD_DIM
    cases = [("qkv", 1, F.IQ3S, qkv_rows, s.hidden), ("o", 0, F.IQ3S, s.hidden, s.n_heads * HEAD_DIM),
             ("gate_up", 1, F.IQ2S, 2 * s.ffn, s.hidden), ("down", 0, F.Q4K_SPLIT_NATIVE, s.hidden, s.ffn)]
    for role, layer, fmt, rows, cols in cases:
        host = packs.make_pack(fmt, rows, cols, tensor_seed(SEED, layer, role))
        assert np.array_equal(m.download(role, np.uint8, layer=layer), host.payload), role
        if host.meta is not None:
            assert np.array_equal(m.download(role + "_meta", np.uint8, layer=layer), host.meta), role
    for role in ("embed", "lm_head"):
        host = packs.make_pack(F.Q5K, s.vocab, s.hidden, tensor_seed(SEED, None, role))
        assert np.array_equal(m.download(role, np.uint8), host.payload), role
    m.close()


# hidden above 4096: qkv / o read their input per wave rather than from one
# shared LDS copy per workgroup (kShareXCols); gate_up runs on the matrix cores
# with 9 panel waves per workgroup (8 at 4096, 1 at the small shape)
HIDDEN_4608 = Shape(hidden=4608, n_heads=4, n_kv_heads=2, ffn=1024, vocab=1000, n_layers=1, max_ctx=256,
                    page_size=16)


# gate_up of 65536 rows x 4096 columns: 8 rounds per workgroup of the
# matrix-core matvec, reusing each double-buffered partials slot three times
FFN_32768 = Shape(hidden=4096, n_heads=4, n_kv_heads=2, ffn=32768, vocab=1000, n_layers=1, max_ctx=256,
                  page_size=16)


# gate_up in IQ3_S: the runner's IQ3S_UNITS copy on the matrix cores
IQ3S_GATE_UP = dict(fmt_gate_up=F.IQ3S)

# K-quant gate_up at hidden <= 4096: one 16-wave workgroup per CU sharing the
# staged input, its column-split waves handing partials over through bounded
# LDS waits (at hidden 4608: per-wave inputs)
Q4K_GATE_UP = dict(fmt_gate_up=F.Q4K_SPLIT_NATIVE)
Q5K_GATE_UP = dict(fmt_gate_up=F.Q5K)
HIDDEN_4096 = Shape(hidden=4096, n_heads=32, n_kv_heads=8, ffn=14336, vocab=1000, n_layers=1, max_ctx=256,
                    page_size=16)


@pytest.mark.parametrize("s,pos,formats", [(SMALL, 0, None), (SMALL, 37, None), (SMALL, 200, None),
                                           (HIDDEN_4608, 37, None), (FFN_32768, 37, None), (SMALL, 37, IQ3S_GATE_UP),
                                           (HIDDEN_4608, 37, IQ3S_GATE_UP), (SMALL, 37, Q4K_GATE_UP),
                                           (SMALL, 37, Q5K_GATE_UP), (HIDDEN_4096, 100, Q4K_GATE_UP),
                                           (HIDDEN_4608, 37, Q4K_GATE_UP)],
                         ids=["small-0", "small-37", "small-200", "hidden4608-37", "ffn32768-37", "small-37-iq3s-ffn",
                              "hidden4608-37-iq3s-ffn", "small-37-q4k-ffn", "small-37-q5k-ffn",
                              "hidden4096-100-q4k-ffn", "hidden4608-37-q4k-ffn"])
def test_decode_step_matches_oracle(orc, s, pos, formats):
    m = build(s, pos, formats=formats)
    token = 123
    m.set_token_pos(token, pos)
    ref = HostModel(m, range(s.n_layers))
    m.step()
    torch.cuda.synchronize()

    h0 = ref.embed_row(orc, token)
    h_ref, logits_ref = ref.run(orc, h0.copy(), pos)
    logits = m.download("logits", np.float32)
    h = m.download("h", np.float32)
    assert rel(h, h_ref) <= TOL
    assert rel(logits, logits_ref) <= TOL
    tok = int(m.download("token", np.uint32)[0])
    assert orc.argmax(logits_ref) == argmax_lowest(logits_ref)
    assert tok == int(np.argmax(logits))  # the GPU's own argmax of its logits (lowest index on ties)
    check_token(f"runner {s.hidden}x{s.ffn} pos {pos} {formats}", tok, logits_ref, 1e-3)
    assert int(m.download("pos", np.uint32)[0]) == pos + 1
    assert m.status() == [0]  # no context end, no in-kernel wait ran out
    # KV written at pos in every layer: the oracle's layer pass wrote the same slots
    for l in range(s.n_layers):
        table = ref.L[l]["block_table"]
        kc = m.download("k_cache", np.uint16, layer=l).view(np.float16).astype(np.float32)
        vc = m.download("v_cache", np.uint16, layer=l).view(np.float16).astype(np.float32)
        rk = ref.L[l]["k_cache"].view(np.float16).astype(np.float32)
        rv = ref.L[l]["v_cache"].view(np.float16).astype(np.float32)
        for g in range(s.n_kv_heads):
            o = kv_slot(m, pos, g, table)
            assert rel(kc[o:o + HEAD_DIM], rk[o:o + HEAD_DIM]) <= 4e-3
            assert rel(vc[o:o + HEAD_DIM], rv[o:o + HEAD_DIM]) <= 4e-3
        # nothing else in the cache changed
        mask = np.ones(kc.size, bool)
        for g in range(s.n_kv_heads):
            o = kv_slot(m, pos, g, table)
            mask[o:o + HEAD_DIM] = False
        assert np.array_equal(kc[mask], rk[mask]) and np.array_equal(vc[mask], rv[mask])
    m.close()


def test_graph_replay_bit_identical_to_eager():
    s = SMALL
    pos, token = 150, 7
    m = build(s, pos)
    k0 = [m.download("k_cache", np.uint16, layer=l) for l in range(s.n_layers)]
    stream = torch.cuda.Stream()
    sp = stream.cuda_stream
    m.set_token_pos(token, pos)
    m.step(sp)
    torch.cuda.synchronize()
    eager_logits = m.download("logits", np.float32)
    eager_tok = m.download("token", np.uint32)[0]
    m.graph_capture(sp)
    for _ in range(3):  # every replay from the same state gives the same result
        for l in range(s.n_layers):
            m.upload("k_cache", k0[l], layer=l)
        m.set_token_pos(token, pos)
        m.graph_replay(sp)
        torch.cuda.synchronize()
        assert np.array_equal(m.download("logits", np.float32).view(np.uint32), eager_logits.view(np.uint32))
        assert m.download("token", np.uint32)[0] == eager_tok
        assert m.download("pos", np.uint32)[0] == pos + 1
    m.close()


LONG = Shape(hidden=512, n_heads=4, n_kv_heads=2, ffn=1024, vocab=1000, n_layers=2, max_ctx=1024, page_size=16)


@pytest.mark.parametrize("pos", [0, 100, 127, 300, 511])
def test_span_graph_bit_identical_to_full_step(pos):
    """A step graph captured over a 128- or 512-position span (1 or 4 of the
    8 attention chunks) gives the full-span eager step's logits, token and KV
    writes bit for bit while the position is below the span: the chunks it
    leaves out hold no position of the context."""
    s, token = LONG, 11
    m = build(s, pos)
    k0 = [m.download("k_cache", np.uint16, layer=l) for l in range(s.n_layers)]
    stream = torch.cuda.Stream()
    sp = stream.cuda_stream
    m.set_token_pos(token, pos)
    m.step(sp)
    torch.cuda.synchronize()
    eager_logits = m.download("logits", np.float32)
    eager_tok = m.download("token", np.uint32)[0]
    eager_k = [m.download("k_cache", np.uint16, layer=l) for l in range(s.n_layers)]
    assert m.graph_span_for(pos) == 0 and m.graph_bytes() == 0
    for span in (512, 128):
        m.graph_capture_span(span, sp)
    m.graph_capture(sp)
    span = m.graph_span_for(pos)
    assert span == (128 if pos < 128 else 512)
    assert m.graph_span_for(512) == 0 and m.graph_bytes() > 0
    for _ in range(2):
        for l in range(s.n_layers):
            m.upload("k_cache", k0[l], layer=l)
        m.set_token_pos(token, pos)
        m.graph_replay_span(span, sp)
        torch.cuda.synchronize()
        assert np.array_equal(m.download("logits", np.float32).view(np.uint32), eager_logits.view(np.uint32))
        assert m.download("token", np.uint32)[0] == eager_tok
        assert m.download("pos", np.uint32)[0] == pos + 1
        for l in range(s.n_layers):
            assert np.array_equal(m.download("k_cache", np.uint16, layer=l), eager_k[l])
    m.close()


def test_span_graph_rejects_bad_spans():
    from rtxllm_amd._lib import HipError

    m = build(SMALL, 0)
    sp = torch.cuda.Stream().cuda_stream
    for bad in (0, SMALL.max_ctx + 1):
        with pytest.raises(HipError):
            m.graph_capture_span(bad, sp)
    with pytest.raises(HipError):  # never captured
        m.graph_replay_span(128, sp)
    m.close()


def test_unit_copies_follow_weight_changes():
    """Batch 1 with IQ3_S q/k/v/o and IQ2_S gate/up: the matvecs' unit-layout
    copies equal the host regrouping of their tensors after capture, and after
    an upload of new gate/up weights a graph replay rebuilds that copy first,
    giving the eager step's result on the new weights."""
    s, pos, token = SMALL, 40, 3
    m = build(s, pos)
    sp = torch.cuda.Stream().cuda_stream
    k0 = [m.download("k_cache", np.uint16, layer=l) for l in range(s.n_layers)]
    m.graph_capture(sp)  # rebuilds the copies before capturing
    torch.cuda.synchronize()
    for l in range(s.n_layers):
        assert np.array_equal(m.download("gate_up_units", np.uint8, layer=l),
                              packs.iq2s_units(m.download("gate_up", np.uint8, layer=l)))
        for role in ("qkv", "o"):
            assert np.array_equal(m.download(role + "_units", np.uint8, layer=l),
                                  packs.iq3s_units(m.download(role, np.uint8, layer=l)))
    new = packs.synth_raw(F.IQ2S, 2 * s.ffn, s.hidden, seed=SEED + 777)
    m.upload("gate_up", new, layer=1)

    def run(step):
        for l in range(s.n_layers):
            m.upload("k_cache", k0[l], layer=l)
        m.set_token_pos(token, pos)
        step()
        torch.cuda.synchronize()
        return m.download("logits", np.float32)

    replayed = run(lambda: m.graph_replay(sp))
    assert np.array_equal(m.download("gate_up_units", np.uint8, layer=1), packs.iq2s_units(new))
    eager = run(lambda: m.step(sp))
    assert np.array_equal(replayed.view(np.uint32), eager.view(np.uint32))
    m.close()


def test_create_rejects_bad_configs():
    from rtxllm_amd._lib import HipError

    for bad in (dict(hidden=500), dict(n_kv_heads=3), dict(ffn=1000), dict(max_ctx=250), dict(n_heads=32)):
        kw = dict(SMALL.__dict__)
        kw.update(bad)
        with pytest.raises(HipError):
            Llama(Shape(**kw))
    # the unit layouts are the runner's own copies, not configurable formats
    for fmt in (F.IQ2S_UNITS, F.IQ3S_UNITS):
        with pytest.raises(HipError):
            Llama(SMALL, formats=dict(fmt_gate_up=fmt))
