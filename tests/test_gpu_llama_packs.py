"""GPU: the decode runner loads its weights from resident packs through the
tensor-pack loaders (rtxllm_llama_load_packs). Packs written from a model's
own synthetic weights (q / k / v split out of the stacked rows, gate / up out
of the interleaved rows, Q4_K down re-joined into raw blocks and packed
split-native) load back bit-identically into a second model, whose decode
step then matches the first bit for bit; a missing tensor, a pack layout
other than the configured one and a corrupted file are refused. A GGUF file
goes through the library's C++ producer (one manifest per producer, in the
reference producers' form) and rtxllm_llama_load_pack_set, which also refuses
a tensor named twice and an unknown producer. All calls go through the
C-ABI."""

from __future__ import annotations

import numpy as np
import pytest

torch = pytest.importorskip("torch")

from rtxllm_amd import formats as F  # noqa: E402
from rtxllm_amd import manifest as M  # noqa: E402
from rtxllm_amd import packs  # noqa: E402
from rtxllm_amd._lib import HipError  # noqa: E402
from rtxllm_amd.llama import HEAD_DIM, Llama, Shape  # noqa: E402

pytestmark = pytest.mark.gpu

SMALL = Shape(hidden=512, n_heads=4, n_kv_heads=2, ffn=1024, vocab=1000, n_layers=2, max_ctx=256, page_size=16)
SEED = 0x5EED0C00
WEIGHT_REGIONS = ("qkv", "o", "gate_up", "down", "down_meta")


def gguf_tensors(m: Llama) -> list[M.Tensor]:
    s = m.shape
    H, Q, KV, FF = s.hidden, s.n_heads * HEAD_DIM, s.n_kv_heads * HEAD_DIM, s.ffn
    out = []
    for l in range(s.n_layers):
        b = f"blk.{l}."
        qkv = m.download("qkv", np.uint8, layer=l).reshape(Q + 2 * KV, -1)
        out += [M.Tensor(b + "attn_q.weight", F.IQ3S, Q, H, qkv[:Q].ravel()),
                M.Tensor(b + "attn_k.weight", F.IQ3S, KV, H, qkv[Q:Q + KV].ravel()),
                M.Tensor(b + "attn_v.weight", F.IQ3S, KV, H, qkv[Q + KV:].ravel()),
                M.Tensor(b + "attn_output.weight", F.IQ3S, H, Q, m.download("o", np.uint8, layer=l))]
        gu = m.download("gate_up", np.uint8, layer=l).reshape(FF, 2, -1)
        out += [M.Tensor(b + "ffn_gate.weight", F.IQ2S, FF, H, gu[:, 0].ravel()),
                M.Tensor(b + "ffn_up.weight", F.IQ2S, FF, H, gu[:, 1].ravel())]
        # split-native = the raw block's 16 B head + its 128 B of quants
        pay = m.download("down", np.uint8, layer=l).reshape(-1, 128)
        meta = m.download("down_meta", np.uint8, layer=l).reshape(-1, 16)
        out.append(M.Tensor(b + "ffn_down.weight", F.Q4K_RAW, H, FF, np.concatenate([meta, pay], axis=1).ravel()))
    out.append(M.Tensor("token_embd.weight", F.Q5K, s.vocab, H, m.download("embed", np.uint8)))
    out.append(M.Tensor("output.weight", F.Q5K, s.vocab, H, m.download("lm_head", np.uint8)))
    return out


def prepare(m: Llama, seed: int) -> None:
    H = m.shape.hidden
    for l in range(m.shape.n_layers):
        m.upload("attn_norm", packs.normal_f32(seed + 100 + 2 * l, H, mean=1.0, std=0.02), layer=l)
        m.upload("ffn_norm", packs.normal_f32(seed + 101 + 2 * l, H, mean=1.0, std=0.02), layer=l)
        n = m.region_bytes("k_cache", l) // 2
        m.upload("k_cache", packs.normal_f16_bits(seed + 300 + 2 * l, n), layer=l)
        m.upload("v_cache", packs.normal_f16_bits(seed + 301 + 2 * l, n), layer=l)
    m.upload("out_norm", packs.normal_f32(seed + 99, H, mean=1.0, std=0.02))


@pytest.fixture(scope="module")
def source():
    m = Llama(SMALL)
    m.synth_weights(SEED)
    torch.cuda.synchronize()
    yield m
    m.close()


def test_packs_load_bit_identical_and_step_matches(source, tmp_path):
    paths = M.write_packs(tmp_path, gguf_tensors(source), policy="split-native")
    m = Llama(SMALL)
    m.load_packs(paths["q4k_manifest"], paths["iq_manifest"], tmp_path)
    for l in range(SMALL.n_layers):
        for r in WEIGHT_REGIONS:
            assert np.array_equal(m.download(r, np.uint8, layer=l), source.download(r, np.uint8, layer=l)), (l, r)
    for r in ("embed", "lm_head"):
        assert np.array_equal(m.download(r, np.uint8), source.download(r, np.uint8)), r
    for x in (source, m):
        prepare(x, SEED)
        x.set_token_pos(321, 77)
        x.step()
    torch.cuda.synchronize()
    assert np.array_equal(m.download("logits", np.float32).view(np.uint32),
                          source.download("logits", np.float32).view(np.uint32))
    assert m.download("token", np.uint32)[0] == source.download("token", np.uint32)[0]
    mem = m.memory()
    assert 0 < mem["arena_bytes"] <= mem["required_bytes"] <= mem["usable_bytes"]
    m.close()


def test_packs_refused_when_incomplete_mislaid_or_corrupt(source, tmp_path):
    tensors = gguf_tensors(source)
    m = Llama(SMALL)
    paths = M.write_packs(tmp_path / "a", [t for t in tensors if t.name != "blk.1.ffn_up.weight"])
    with pytest.raises(HipError, match="tensor missing from the packs: blk.1.ffn_up.weight"):
        m.load_packs(paths["q4k_manifest"], paths["iq_manifest"], tmp_path / "a")
    paths = M.write_packs(tmp_path / "b", tensors, policy="split-compact")
    with pytest.raises(HipError, match="not the configured one"):
        m.load_packs(paths["q4k_manifest"], paths["iq_manifest"], tmp_path / "b")
    paths = M.write_packs(tmp_path / "c", tensors)
    f = next((tmp_path / "c").glob("output.weight.q5_k_raw_blocks.bin"))
    b = bytearray(f.read_bytes())
    b[100] ^= 1
    f.write_bytes(bytes(b))
    with pytest.raises(HipError, match="checksum mismatch: output.weight"):
        m.load_packs(paths["q4k_manifest"], paths["iq_manifest"], tmp_path / "c")
    m.close()


def test_gguf_file_loads_bit_identical_and_step_matches(source, tmp_path):
    """The same model as a GGUF file (quantized tensors + F32 norms + llama.*
    keys): rtxllm_amd.gguf reads its shape and formats, writes the packs and
    loads them with the norms into a new model, which matches the source."""
    from rtxllm_amd import gguf as G

    s = SMALL
    prepare(source, SEED)
    meta = [("general.architecture", 8, "llama"), ("llama.embedding_length", 4, s.hidden),
            ("llama.block_count", 4, s.n_layers), ("llama.attention.head_count", 4, s.n_heads),
            ("llama.attention.head_count_kv", 4, s.n_kv_heads), ("llama.feed_forward_length", 4, s.ffn),
            ("llama.rope.freq_base", 6, s.rope_theta), ("llama.attention.layer_norm_rms_epsilon", 6, s.rms_eps)]
    gtype = {F.IQ3S: "IQ3_S", F.IQ2S: "IQ2_S", F.Q4K_RAW: "Q4_K", F.Q5K: "Q5_K"}
    tensors = [(t.name, gtype[t.fmt], [t.cols, t.rows], t.blocks) for t in gguf_tensors(source)]
    H = s.hidden
    for l in range(s.n_layers):
        tensors.append((f"blk.{l}.attn_norm.weight", "F32", [H], source.download("attn_norm", np.float32, layer=l)))
        tensors.append((f"blk.{l}.ffn_norm.weight", "F32", [H], source.download("ffn_norm", np.float32, layer=l)))
    tensors.append(("output_norm.weight", "F32", [H], source.download("out_norm", np.float32)))
    path = tmp_path / "small.gguf"
    G.write(path, meta, tensors)
    g = G.read(path)
    fields = G.llama_shape(g)
    assert np.float32(fields.pop("rms_eps")) == np.float32(s.rms_eps)
    shape = Shape(**fields, max_ctx=s.max_ctx, page_size=s.page_size)
    m = Llama(shape, formats=G.model_formats(g))
    G.load_into(m, g, tmp_path / "packs")
    for l in range(s.n_layers):
        for r in WEIGHT_REGIONS + ("attn_norm", "ffn_norm"):
            assert np.array_equal(m.download(r, np.uint8, layer=l), source.download(r, np.uint8, layer=l)), (l, r)
        for r in ("k_cache", "v_cache"):
            m.upload(r, source.download(r, np.uint16, layer=l), layer=l)
    for r in ("embed", "lm_head", "out_norm"):
        assert np.array_equal(m.download(r, np.uint8), source.download(r, np.uint8)), r
    for x in (source, m):
        x.set_token_pos(99, 120)
        x.step()
    torch.cuda.synchronize()
    assert np.array_equal(m.download("logits", np.float32).view(np.uint32),
                          source.download("logits", np.float32).view(np.uint32))
    m.close()


def test_pack_set_refuses_duplicates_and_unknown_producers(source, tmp_path):
    """rtxllm_llama_load_pack_set: a tensor named by two manifests and a
    manifest of an unknown producer are refused, and the weights stay as they
    were; the same manifests without the duplicate load bit-identically."""
    import json

    tensors = gguf_tensors(source)
    paths = M.write_packs(tmp_path / "a", tensors, absolute_paths=True)
    extra = M.write_packs(tmp_path / "b", [t for t in tensors if t.name == "output.weight"], absolute_paths=True)
    m = Llama(SMALL)
    m.synth_weights(SEED + 1)
    torch.cuda.synchronize()
    before = m.download("lm_head", np.uint8)
    with pytest.raises(HipError, match="tensor in two manifests: output.weight"):
        m.load_pack_set([paths["q4k_manifest"], paths["iq_manifest"], extra["iq_manifest"]])
    doc = json.loads(paths["iq_manifest"].read_text())
    doc["path"] = "q6k_resident_pack"
    odd = tmp_path / "odd.json"
    odd.write_text(json.dumps(doc))
    with pytest.raises(HipError, match="unknown pack producer q6k_resident_pack"):
        m.load_pack_set([paths["q4k_manifest"], odd])
    assert np.array_equal(m.download("lm_head", np.uint8), before)
    m.load_pack_set([paths["q4k_manifest"], paths["iq_manifest"]])
    for l in range(SMALL.n_layers):
        for r in WEIGHT_REGIONS:
            assert np.array_equal(m.download(r, np.uint8, layer=l), source.download(r, np.uint8, layer=l)), (l, r)
    m.close()
