"""GGUF container and the GGUF -> resident-pack step (rtxllm_amd.gguf), on the
CPU: the reference inspector's self-test blob parses to its known layout
(tools/bench/gguf_inspect.py:200-214: version 3, two metadata keys, tensor
blk.0.weight [16, 32] F32 at offset 0; tensor infos end at byte 158, data at
160 = align_up(158, 32), both counted by hand from the format), a written model
round-trips (metadata of every value type, arrays, tensors of five types at a
non-default alignment, padding), spans that overrun or over-pad are refused,
and the packs of a GGUF Llama model pass the C++ manifest loaders with the
tensors' true file offsets in the tensor plan."""

from __future__ import annotations

import io
import json
import struct
import subprocess

import numpy as np
import pytest

from rtxllm_amd import formats as F
from rtxllm_amd import gguf as G
from rtxllm_amd import packs


def _s(v: str) -> bytes:
    b = v.encode()
    return struct.pack("<Q", len(b)) + b


def reference_self_test_blob() -> bytes:
    """The byte layout gguf_inspect.build_self_test_blob describes (written here
    from the format: magic, header, two metadata entries, one tensor info)."""
    out = b"GGUF" + struct.pack("<IQQ", 3, 1, 2)
    out += _s("general.architecture") + struct.pack("<I", 8) + _s("test")
    out += _s("general.context_length") + struct.pack("<I", 4) + struct.pack("<I", 2048)
    out += _s("blk.0.weight") + struct.pack("<I", 2) + struct.pack("<QQ", 16, 32) + struct.pack("<IQ", 0, 0)
    return out


def test_reference_self_test_blob_layout():
    g = G.read(io.BytesIO(reference_self_test_blob()), check_spans=False)
    assert g.version == 3 and len(g.tensors) == 1
    assert g.metadata == {"general.architecture": "test", "general.context_length": 2048}
    assert g.value_types == {"general.architecture": "string", "general.context_length": "uint32"}
    t = g.tensors[0]
    assert (t.name, t.dims, t.type, t.offset) == ("blk.0.weight", [16, 32], "F32", 0)
    assert (t.cols, t.rows, t.nbytes) == (16, 32, 16 * 32 * 4)
    assert g.tensor_info_end == 158 and g.data_offset == 160 and g.alignment == 32
    # the blob carries no tensor data: the span check refuses it
    with pytest.raises(ValueError, match="does not hold"):
        G.read(io.BytesIO(reference_self_test_blob()))


def _tensor_set(seed=5):
    rows, cols = 32, 512
    return [("token_embd.weight", "Q5_K", [cols, rows], packs.synth_raw(F.Q5K, rows, cols, seed)),
            ("blk.0.attn_norm.weight", "F32", [cols], packs.normal_f32(seed, cols, mean=1.0, std=0.02).view(np.uint8)),
            ("blk.0.ffn_down.weight", "Q4_K", [cols, rows], packs.synth_raw(F.Q4K_RAW, rows, cols, seed + 1)),
            ("blk.0.ffn_gate.weight", "IQ2_S", [cols, rows], packs.synth_raw(F.IQ2S, rows, cols, seed + 2)),
            ("blk.0.attn_q.weight", "IQ3_S", [cols, rows], packs.synth_raw(F.IQ3S, rows, cols, seed + 3))]


@pytest.mark.parametrize("alignment", [32, 64])
def test_round_trip(tmp_path, alignment):
    meta = [("general.architecture", 8, "llama"), ("general.alignment", 4, alignment),
            ("llama.block_count", 4, 1), ("llama.rope.freq_base", 6, 500000.0), ("flag", 7, True),
            ("i64", 11, -5), ("f64", 12, 0.25), ("u8", 0, 7), ("i16", 3, -300),
            ("tokenizer.ggml.tokens", 9, (8, ["a", "bb", ""])), ("scores", 9, (6, [0.5, -1.0]))]
    tensors = _tensor_set()
    path = tmp_path / "m.gguf"
    G.write(path, meta, tensors, alignment=alignment)
    g = G.read(path)
    assert g.alignment == alignment and g.data_offset % alignment == 0
    assert g.metadata["tokenizer.ggml.tokens"] == ["a", "bb", ""] and g.metadata["scores"] == [0.5, -1.0]
    assert g.metadata["flag"] is True and g.metadata["i64"] == -5 and g.metadata["i16"] == -300
    assert [t.name for t in g.tensors] == [t[0] for t in tensors]
    for (name, tname, dims, data), t in zip(tensors, g.tensors):
        assert t.type == tname and t.dims == dims and t.offset % alignment == 0
        assert np.array_equal(np.asarray(g.data(t)), np.asarray(data).view(np.uint8).reshape(-1))
        assert 0 <= t.span - t.nbytes < alignment
    plan = g.plan()
    assert all(r["absolute_offset"] == g.data_offset + t.offset for r, t in zip(plan, g.tensors))


def test_span_errors(tmp_path):
    path = tmp_path / "m.gguf"
    G.write(path, [], _tensor_set())
    blob = bytearray(path.read_bytes())
    with pytest.raises(ValueError, match="does not hold"):  # last tensor cut short
        G.read(io.BytesIO(bytes(blob[:-10])))
    with pytest.raises(ValueError, match="does not hold"):  # 64 bytes of padding at alignment 32
        G.read(io.BytesIO(bytes(blob) + bytes(64)))
    with pytest.raises(ValueError, match="not a GGUF"):
        G.read(io.BytesIO(b"GGUG" + bytes(blob[4:])))


def tiny_llama(tmp_path, down_type="Q4_K"):
    H, FF, V, NL = 512, 1024, 300, 2
    rng_seed = 21
    meta = [("general.architecture", 8, "llama"), ("llama.embedding_length", 4, H), ("llama.block_count", 4, NL),
            ("llama.attention.head_count", 4, 4), ("llama.attention.head_count_kv", 4, 2),
            ("llama.feed_forward_length", 4, FF), ("llama.rope.freq_base", 6, 10000.0),
            ("llama.attention.layer_norm_rms_epsilon", 6, 1e-5)]
    fmt = {"Q4_K": F.Q4K_RAW, "Q5_K": F.Q5K, "IQ2_S": F.IQ2S, "IQ3_S": F.IQ3S}
    tensors, i = [], 0

    def add(name, tname, rows, cols):
        nonlocal i
        i += 1
        if tname == "F32":
            data = packs.normal_f32(rng_seed + i, cols, mean=1.0, std=0.02).view(np.uint8)
            tensors.append((name, tname, [cols], data))
        else:
            tensors.append((name, tname, [cols, rows], packs.synth_raw(fmt[tname], rows, cols, rng_seed + i)))

    add("token_embd.weight", "Q5_K", V, H)
    for l in range(NL):
        b = f"blk.{l}."
        add(b + "attn_norm.weight", "F32", 1, H)
        add(b + "attn_q.weight", "IQ3_S", H, H)
        add(b + "attn_k.weight", "IQ3_S", 256, H)
        add(b + "attn_v.weight", "IQ3_S", 256, H)
        add(b + "attn_output.weight", "IQ3_S", H, H)
        add(b + "ffn_norm.weight", "F32", 1, H)
        add(b + "ffn_gate.weight", "IQ2_S", FF, H)
        add(b + "ffn_up.weight", "IQ2_S", FF, H)
        add(b + "ffn_down.weight", down_type, H, FF)
    add("output_norm.weight", "F32", 1, H)
    add("output.weight", "Q5_K", V, H)
    path = tmp_path / "tiny.gguf"
    G.write(path, meta, tensors)
    return path, tensors


def test_llama_shape_formats_and_norms(tmp_path):
    path, tensors = tiny_llama(tmp_path)
    g = G.read(path)
    assert G.llama_shape(g) == {"hidden": 512, "n_layers": 2, "n_heads": 4, "ffn": 1024, "vocab": 300,
                                "n_kv_heads": 2, "rope_theta": 10000.0, "rms_eps": pytest.approx(1e-5)}
    assert G.model_formats(g, "split-compact") == {"fmt_qkv": F.IQ3S, "fmt_o": F.IQ3S, "fmt_gate_up": F.IQ2S,
                                                   "fmt_down": F.Q4K_SPLIT_COMPACT, "fmt_lm_head": F.Q5K}
    n = G.norms(g)
    assert sorted(n) == [("attn_norm", 0), ("attn_norm", 1), ("ffn_norm", 0), ("ffn_norm", 1), ("out_norm", 0)]
    src = {t[0]: t[3] for t in tensors}
    assert np.array_equal(n[("ffn_norm", 1)].view(np.uint8), src["blk.1.ffn_norm.weight"])
    bad = G.read(path)
    bad.tensors[[t.name for t in bad.tensors].index("blk.0.attn_k.weight")].type_id = G.GGML_TYPE_IDS["IQ2_S"]
    with pytest.raises(ValueError, match="differ in type"):
        G.model_formats(bad)


@pytest.mark.parametrize("policy", ["split-native", "split-predecoded"])
def test_packs_from_gguf_pass_the_loaders(selftest, tmp_path, policy):
    (tmp_path / "m").mkdir()
    path, _ = tiny_llama(tmp_path / "m")
    g = G.read(path)
    out = tmp_path / "packs"
    paths = G.to_packs(g, out, policy=policy)
    plan = {r["name"]: r for r in json.loads(paths["tensor_plan"].read_text())["tensors"]}
    for t in g.tensors:
        if t.type in G.PACK_FORMATS:
            assert plan[t.name]["absolute_offset"] == g.data_offset + t.offset
    manifests = [str(paths[k]) for k in ("q4k_manifest", "iq_manifest", "q5k_manifest")]
    r = subprocess.run([str(selftest), "--load-set", str(paths["tensor_plan"]), str(out)] + manifests,
                       capture_output=True, text=True, timeout=120)
    assert r.returncode == 0, r.stdout + r.stderr
    assert len(r.stdout.splitlines()) == 16


def test_cli_inspect(tmp_path, capsys):
    path, _ = tiny_llama(tmp_path)
    assert G.main(["inspect", str(path)]) == 0
    info = json.loads(capsys.readouterr().out)
    assert info["tensor_count"] == 21 and info["tensor_data_offset"] % 32 == 0


def test_auto_policy(selftest, tmp_path):
    from rtxllm_amd import manifest as M

    assert M.auto_policy(4096, 4096) == "split-native" and M.auto_policy(14336, 4096) == "split-native"
    assert M.auto_policy(4096, 4096, lossy=True) == "split-native"  # 65536 blocks: not above
    assert M.auto_policy(4096, 14336, lossy=True) == "split-half"
    small = M.Tensor("blk.0.ffn_down.weight", F.Q4K_RAW, 64, 1024, packs.synth_raw(F.Q4K_RAW, 64, 1024, 3))
    big = M.Tensor("blk.1.ffn_down.weight", F.Q4K_RAW, 4352, 4096, packs.synth_raw(F.Q4K_RAW, 4352, 4096, 4))
    for policy, want in (("auto", ["split-native", "split-native"]), ("auto-lossy", ["split-native", "split-half"])):
        out = tmp_path / policy
        paths = M.write_packs(out, [small, big], policy=policy)
        rec = json.loads(paths["q4k_manifest"].read_text())
        assert rec["policy"] == policy and [t["policy"] for t in rec["tensors"]] == want
        r = subprocess.run([str(selftest), "--load", str(paths["q4k_manifest"]), "-", str(paths["tensor_plan"]),
                            str(out)], capture_output=True, text=True, timeout=120)
        assert r.returncode == 0, r.stdout + r.stderr
    with pytest.raises(ValueError, match="unknown Q4_K policy"):
        M.write_packs(tmp_path / "x", [small], policy="fastest")
