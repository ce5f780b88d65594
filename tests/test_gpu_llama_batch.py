"""GPU parity of the batch decode step (8 sequences through the same weights
on the matrix cores; 2, 3, 5 and 7 as well) against the oracle at a small Llama shape: every
sequence, with its own token, position and KV pages (one permutation of all
the batch's pages, so sequences interleave in the cache), matches the
oracle's batch-1 step for that sequence within 1e-3 normwise on logits and
hidden state, gets the same token, and writes exactly its own KV slots.
Sequences are independent (changing one leaves the others bit-identical) and a
hipGraph replay is bit-identical to the eager step. All calls go through the
C-ABI."""

from __future__ import annotations

import numpy as np
import pytest

torch = pytest.importorskip("torch")

from rtxllm_amd import packs  # noqa: E402
from rtxllm_amd._lib import HipError  # noqa: E402
from rtxllm_amd.llama import HEAD_DIM, Llama, Shape  # noqa: E402

from llama_ref import HostModel, kv_slot  # noqa: E402
from token_rule import check_token  # noqa: E402

pytestmark = pytest.mark.gpu

TOL = 1e-3
B = 8
SMALL_B = Shape(hidden=512, n_heads=4, n_kv_heads=2, ffn=1024, vocab=1000, n_layers=2, max_ctx=256, page_size=16,
                batch=B)
SEED = 0x5EED0B80
TOKENS = [123, 7, 999, 0, 500, 42, 777, 311]
POSITIONS = [0, 37, 200, 255, 16, 15, 100, 128]


def rel(a, b) -> float:
    a, b = np.asarray(a, np.float64), np.asarray(b, np.float64)
    return float(np.max(np.abs(a - b)) / np.max(np.abs(b)))


def build(shape: Shape, seed: int = SEED) -> Llama:
    m = Llama(shape)
    m.synth_weights(seed)
    torch.cuda.synchronize()
    H, pps = shape.hidden, shape.max_ctx // shape.page_size
    npages = shape.batch * pps
    for l in range(shape.n_layers):
        m.upload("attn_norm", packs.normal_f32(seed + 100 + 2 * l, H, mean=1.0, std=0.02), layer=l)
        m.upload("ffn_norm", packs.normal_f32(seed + 101 + 2 * l, H, mean=1.0, std=0.02), layer=l)
        n = m.region_bytes("k_cache", l) // 2
        m.upload("k_cache", packs.normal_f16_bits(seed + 300 + 2 * l, n), layer=l)
        m.upload("v_cache", packs.normal_f16_bits(seed + 301 + 2 * l, n), layer=l)
        # one permutation of every page of the batch: sequence s owns row s
        table = np.array([(11 * i + 5 + l) % npages for i in range(npages)], np.int32)
        assert len(set(table.tolist())) == npages
        m.upload("block_table", table, layer=l)
    m.upload("out_norm", packs.normal_f32(seed + 99, H, mean=1.0, std=0.02))
    return m


@pytest.fixture(scope="module")
def model():
    m = build(SMALL_B)
    yield m
    m.close()


def test_batch_step_matches_oracle_per_sequence(orc, model):
    check_step(orc, model, SMALL_B)


@pytest.mark.parametrize("batch", [2, 3, 5, 7])
def test_batch_step_matches_oracle_at_smaller_batches(orc, batch):
    """2-7 sequences: the matrix-core operands' unused columns (sequences past
    the batch) stay zero, the attention grid, the staging and the argmax keys
    follow the batch, and every sequence still matches the oracle."""
    s = Shape(**{**SMALL_B.__dict__, "batch": batch})
    m = build(s, SEED + batch)
    try:
        check_step(orc, m, s)
    finally:
        m.close()


def test_batch_step_wide_ffn_panel_groups(orc):
    """ffn 4608 > 4096 columns: the down projection splits into two panel
    groups, whose partial sums the residual staging adds per sequence."""
    s = Shape(hidden=512, n_heads=4, n_kv_heads=2, ffn=4608, vocab=1000, n_layers=2, max_ctx=256, page_size=16,
              batch=B)
    m = build(s, SEED + 7)
    try:
        check_step(orc, m, s)
    finally:
        m.close()


def check_step(orc, m, s):
    b = s.batch
    tok, pos = TOKENS[:b], POSITIONS[:b]
    m.set_token_pos(tok, pos)
    ref = HostModel(m, range(s.n_layers))
    k_before = {l: ref.L[l]["k_cache"].copy() for l in range(s.n_layers)}
    v_before = {l: ref.L[l]["v_cache"].copy() for l in range(s.n_layers)}
    m.step()
    torch.cuda.synchronize()
    h = m.download("h", np.float32).reshape(b, s.hidden)
    logits = m.download("logits", np.float32).reshape(b, s.vocab)
    tokens = m.download("token", np.uint32)
    assert list(m.download("pos", np.uint32)) == [p + 1 for p in pos]
    for q in range(b):
        h_ref, logits_ref = ref.run(orc, ref.embed_row(orc, tok[q]), pos[q], seq=q)
        assert rel(h[q], h_ref) <= TOL, (q, rel(h[q], h_ref))
        assert rel(logits[q], logits_ref) <= TOL, (q, rel(logits[q], logits_ref))
        assert int(tokens[q]) == int(np.argmax(logits[q]))  # the GPU's argmax of its own logits
        check_token(f"batch runner sequence {q}", int(tokens[q]), logits_ref, 1e-3)
    # every layer: each sequence's slot at its position holds the oracle's K / V;
    # every other cache entry is unchanged
    pps = s.max_ctx // s.page_size
    for l in range(s.n_layers):
        table = ref.L[l]["block_table"]
        kc = m.download("k_cache", np.uint16, layer=l)
        vc = m.download("v_cache", np.uint16, layer=l)
        kf, vf = kc.view(np.float16).astype(np.float32), vc.view(np.float16).astype(np.float32)
        rk = ref.L[l]["k_cache"].view(np.float16).astype(np.float32)
        rv = ref.L[l]["v_cache"].view(np.float16).astype(np.float32)
        mask = np.ones(kc.size, bool)
        for q in range(b):
            row = table[q * pps:(q + 1) * pps]
            for g in range(s.n_kv_heads):
                o = kv_slot(m, pos[q], g, row)
                assert rel(kf[o:o + HEAD_DIM], rk[o:o + HEAD_DIM]) <= 4e-3, (l, q, g)
                assert rel(vf[o:o + HEAD_DIM], rv[o:o + HEAD_DIM]) <= 4e-3, (l, q, g)
                mask[o:o + HEAD_DIM] = False
        assert np.array_equal(kc[mask], k_before[l][mask]) and np.array_equal(vc[mask], v_before[l][mask])


def test_batch_sequences_are_independent(model):
    m, s = model, SMALL_B
    m.set_token_pos(TOKENS, POSITIONS)
    m.step()
    torch.cuda.synchronize()
    l1 = m.download("logits", np.float32).reshape(B, s.vocab)
    h1 = m.download("h", np.float32).reshape(B, s.hidden)
    other = list(TOKENS)
    other[5] = 901
    m.set_token_pos(other, POSITIONS)
    m.step()
    torch.cuda.synchronize()
    l2 = m.download("logits", np.float32).reshape(B, s.vocab)
    h2 = m.download("h", np.float32).reshape(B, s.hidden)
    for q in range(B):
        if q == 5:
            assert not np.array_equal(l1[q], l2[q])
        else:
            assert np.array_equal(l1[q].view(np.uint32), l2[q].view(np.uint32)), q
            assert np.array_equal(h1[q].view(np.uint32), h2[q].view(np.uint32)), q


def test_batch_graph_replay_bit_identical_to_eager():
    s = SMALL_B
    m = build(s, SEED + 1)
    k0 = [m.download("k_cache", np.uint16, layer=l) for l in range(s.n_layers)]
    stream = torch.cuda.Stream()
    sp = stream.cuda_stream
    m.set_token_pos(TOKENS, POSITIONS)
    m.step(sp)
    torch.cuda.synchronize()
    eager_logits = m.download("logits", np.float32)
    eager_tok = m.download("token", np.uint32)
    m.graph_capture(sp)
    for _ in range(3):  # every replay from the same state gives the same result
        for l in range(s.n_layers):
            m.upload("k_cache", k0[l], layer=l)
        m.set_token_pos(TOKENS, POSITIONS)
        m.graph_replay(sp)
        torch.cuda.synchronize()
        assert np.array_equal(m.download("logits", np.float32).view(np.uint32), eager_logits.view(np.uint32))
        assert np.array_equal(m.download("token", np.uint32), eager_tok)
        assert list(m.download("pos", np.uint32)) == [p + 1 for p in POSITIONS]
    m.close()


def test_batch_span_graph_bit_identical_to_full_step():
    """Batch 8 over a 1024-position cache, positions below 512: the 512-span
    step graph gives the eager full-span step's logits and tokens bit for bit."""
    s = Shape(hidden=512, n_heads=4, n_kv_heads=2, ffn=1024, vocab=1000, n_layers=2, max_ctx=1024, page_size=16,
              batch=B)
    positions = [0, 37, 200, 255, 16, 15, 100, 511]
    m = build(s)
    k0 = [m.download("k_cache", np.uint16, layer=l) for l in range(s.n_layers)]
    sp = torch.cuda.Stream().cuda_stream
    m.set_token_pos(TOKENS, positions)
    m.step(sp)
    torch.cuda.synchronize()
    eager_logits = m.download("logits", np.float32)
    eager_tok = m.download("token", np.uint32)
    m.graph_capture_span(512, sp)
    assert m.graph_span_for(max(positions)) == 512
    for _ in range(2):
        for l in range(s.n_layers):
            m.upload("k_cache", k0[l], layer=l)
        m.set_token_pos(TOKENS, positions)
        m.graph_replay_span(512, sp)
        torch.cuda.synchronize()
        assert np.array_equal(m.download("logits", np.float32).view(np.uint32), eager_logits.view(np.uint32))
        assert np.array_equal(m.download("token", np.uint32), eager_tok)
    m.close()


def test_batch_regions_and_launch_count(model):
    m, s = model, SMALL_B
    pps = s.max_ctx // s.page_size
    assert m.region_bytes("h") == 4 * B * s.hidden
    assert m.region_bytes("logits") == 4 * B * s.vocab
    assert m.region_bytes("block_table", 0) == 4 * B * pps
    assert m.region_bytes("k_cache", 0) == 2 * B * pps * s.n_kv_heads * s.page_size * HEAD_DIM
    assert m.launches_per_step() == 1 + 8 * s.n_layers + 2


def test_batch_create_rejects_bad_configs():
    for bad in (dict(batch=9), dict(hidden=768), dict(ffn=768), dict(n_heads=2, n_kv_heads=2)):
        kw = dict(SMALL_B.__dict__)
        kw.update(bad)
        with pytest.raises(HipError):
            Llama(Shape(**kw))
