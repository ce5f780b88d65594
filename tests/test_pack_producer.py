"""The C++ GGUF -> resident-pack producer (include/rtxllm/pack_producer.h,
through the library's C-ABI: rtxllm_amd/producer.py, and the rtxllm_gguf_pack
command), on the CPU.

* The reference producers' own unit tests, restated against it:
  runtime/tests/unit/test_q5k_resident_pack.py:22-61 (the index % 251 payload
  behind a 6-byte prefix, its byte-sum checksums, runtime_kernel
  "q5_k_raw_pending"), test_iq_resident_pack.py:8-87 (IQ shapes, the role
  parser, the layer filter before the limit, requested names, the IQ3_S
  runtime_kernel), test_q4k_resident_pack.py:16-81 (the sample block's
  scale / min unpacking, payload extraction, predecoded / compact / native
  metadata) and test_gguf_block_formats.py:19-24 (data bytes per type).
* A GGUF model packed by it: one manifest per producer in the reference form
  (absolute paths, "path" producer names, *.q4k_meta.<format>.bin files,
  compression_ratio_vs_fp16), pack bytes equal to the GGUF tensors and to the
  split restatement, the tensor plan's offsets and spans, the C++ loaders
  accepting every manifest, and the command writing the same packs.
* Manifests written by hand in the reference producers' record form (as they
  would come from tools/bench/*_resident_pack.py) load through the C++ loaders.
* Refusals: malformed shapes, short spans and reads, unknown policies, fp16
  overflow of split-half products, non-GGUF and truncated files.
"""

from __future__ import annotations

import json
import struct
import subprocess
from pathlib import Path

import numpy as np
import pytest

from rtxllm_amd import formats as F
from rtxllm_amd import gguf as G
from rtxllm_amd import packs
from rtxllm_amd import producer as P
from rtxllm_amd._lib import PKG_ROOT

from test_gguf import reference_self_test_blob, tiny_llama

CLI = PKG_ROOT / "build" / "rtxllm_gguf_pack"

RAW_KEYS = ["name", "type", "layer", "role", "dimensions", "element_count", "block_size", "block_type_size",
            "block_count", "source_offset", "source_bytes", "source_checksum", "payload_path", "payload_bytes",
            "payload_checksum", "resident_bytes", "policy", "runtime_kernel"]
Q4K_KEYS = ["name", "dimensions", "rows", "cols", "block_count", "source_offset", "source_bytes", "source_checksum",
            "policy", "metadata_format", "payload_path", "payload_bytes", "payload_checksum", "metadata_path",
            "metadata_bytes", "metadata_checksum", "blocks_path", "resident_bytes", "compression_ratio_vs_fp16",
            "runtime_kernel"]


# ---- test_q5k_resident_pack.py ---------------------------------------------------------

def test_q5k_shape_uses_256_value_blocks():
    values, blocks, _ = P.tensor_shape("Q5_K", [2048, 248320])
    assert (values, blocks) == (508_559_360, 1_986_560)


def test_role_parser_handles_output_weight():
    assert P.tensor_role("output.weight") == (None, "output")
    assert P.tensor_role("blk.1.some.weight") == (1, "some.weight")


def test_q5k_pack_tensor_writes_raw_blocks_and_manifest_row(tmp_path):
    model = tmp_path / "tiny.gguf"
    payload = bytes(index % 251 for index in range(176 * 2))
    prefix = b"header"
    model.write_bytes(prefix + payload)
    out = tmp_path / "pack"
    out.mkdir()
    row = P.pack_tensor(model, {"name": "output.weight", "type": "Q5_K", "dimensions": [256, 2],
                                "absolute_offset": len(prefix), "span_bytes": len(payload)}, out)
    path = Path(row["payload_path"])
    assert path.read_bytes() == payload
    assert row["block_count"] == 2 and row["block_type_size"] == 176
    assert row["payload_checksum"] == sum(payload) and row["source_checksum"] == sum(payload)
    assert row["runtime_kernel"] == "q5_k_raw_pending"
    json.dumps(row)
    # the reference record's form: its keys in order, an absolute path, the file label
    assert list(row) == RAW_KEYS
    assert path.is_absolute() and path.name == "output.weight.q5_k_raw_blocks.bin"
    assert (row["layer"], row["role"], row["policy"], row["element_count"]) == (None, "output", "raw-blocks", 512)
    assert row["source_offset"] == 6 and row["resident_bytes"] == row["payload_bytes"] == 352


# ---- test_iq_resident_pack.py ----------------------------------------------------------

def test_iq2s_shape_uses_256_value_blocks():
    assert P.tensor_shape("IQ2_S", [2048, 512, 128])[:2] == (134217728, 524288)


def test_iq3s_shape_uses_same_block_width():
    assert P.tensor_shape("IQ3_S", [2048, 512])[:2] == (1048576, 4096)


def test_role_parser_preserves_layer_and_weight_suffix():
    assert P.tensor_role("blk.12.ffn_gate_exps.weight") == (12, "ffn_gate_exps.weight")
    assert P.tensor_role("output.weight") == (None, "output")
    # names the regex does not take keep the whole name, less a ".weight"
    assert P.tensor_role("blk.x.a.weight") == (None, "blk.x.a")
    assert P.tensor_role("blk.3.") == (None, "blk.3.")
    assert P.tensor_role("rope_freqs") == (None, "rope_freqs")


def _iq_gguf(tmp_path, names) -> Path:
    """A GGUF holding one 256-value IQ2_S tensor per name, in that order."""
    tensors = [(n, "IQ2_S", [256], packs.synth_raw(F.IQ2S, 1, 256, 40 + i)) for i, n in enumerate(names)]
    path = tmp_path / "iq.gguf"
    G.write(path, [("general.architecture", 8, "test")], tensors)
    return path


def test_select_tensors_filters_layer_before_limit(tmp_path):
    names = ["blk.0.attn_gate.weight", "blk.0.ffn_gate_exps.weight", "blk.1.attn_gate.weight", "output.weight"]
    paths = P.pack_gguf(_iq_gguf(tmp_path, names), tmp_path / "out", layer=0, limit=1)
    man = json.loads(paths["iq_manifest"].read_text())
    assert [t["name"] for t in man["tensors"]] == ["blk.0.attn_gate.weight"]
    assert "q4k_manifest" not in paths and "q5k_manifest" not in paths


def test_select_tensors_respects_requested_names(tmp_path):
    names = ["blk.0.attn_gate.weight", "blk.0.ffn_gate_exps.weight"]
    paths = P.pack_gguf(_iq_gguf(tmp_path, names), tmp_path / "out", names=["blk.0.ffn_gate_exps.weight"])
    man = json.loads(paths["iq_manifest"].read_text())
    assert [t["name"] for t in man["tensors"]] == ["blk.0.ffn_gate_exps.weight"]


def test_pack_tensor_marks_iq3s_runtime_probe_kernel(tmp_path):
    model = tmp_path / "model.gguf"
    model.write_bytes(bytes(range(110)))
    out = tmp_path / "pack"
    out.mkdir()
    row = P.pack_tensor(model, {"name": "blk.0.ffn_down_shexp.weight", "type": "IQ3_S", "dimensions": [256],
                                "absolute_offset": 0, "span_bytes": 110}, out)
    assert row["runtime_kernel"] == "iq3s_raw_block_probe"
    assert row["block_type_size"] == 110
    assert (row["layer"], row["role"]) == (0, "ffn_down_shexp.weight")
    assert Path(row["payload_path"]).read_bytes() == bytes(range(110))


# ---- test_q4k_resident_pack.py ---------------------------------------------------------

def _half(value: float) -> bytes:
    return struct.pack("<e", value)


def sample_block() -> bytes:
    block = bytearray(144)
    block[0:2] = _half(0.5)
    block[2:4] = _half(0.25)
    block[4:16] = bytes([1, 2, 3, 4, 5, 6, 7, 8, 0x40, 0x80, 0xC0, 0x00])
    for index in range(128):
        block[16 + index] = index & 0xFF
    return bytes(block)


def _pack_sample(tmp_path, policy: str) -> tuple[dict, bytes, bytes]:
    model = tmp_path / f"q4k_{policy}.bin"
    model.write_bytes(b"\0" * 32 + sample_block())
    out = tmp_path / f"pack_{policy}"
    out.mkdir()
    row = P.pack_tensor(model, {"name": "blk.0.ffn_down.weight", "type": "Q4_K", "dimensions": [256, 1],
                                "absolute_offset": 32, "span_bytes": 144}, out, policy=policy)
    return row, Path(row["payload_path"]).read_bytes(), Path(row["metadata_path"]).read_bytes()


def test_scale_min_unpacking_matches_ggml_k4_layout(tmp_path):
    # the compact metadata holds the 8 unpacked scales then the 8 unpacked mins
    _, _, meta = _pack_sample(tmp_path, "split-compact")
    scales, mins = meta[4:12], meta[12:20]
    for j, want in ((0, (1, 5)), (3, (4, 8)), (4, (0, 4)), (5, (0, 8)), (6, (0, 12))):
        assert (scales[j], mins[j]) == want, j


def test_payload_extraction_strips_q4k_metadata(tmp_path):
    _, payload, _ = _pack_sample(tmp_path, "split-native")
    assert len(payload) == 128
    assert payload[:4] == bytes([0, 1, 2, 3]) and payload[-1] == 127


def test_split_predecoded_metadata_products_are_fp32(tmp_path):
    row, _, meta = _pack_sample(tmp_path, "split-predecoded")
    assert len(meta) == 64 and row["metadata_format"] == "fp32-products"
    assert struct.unpack("<ff", meta[:8]) == (0.5, 1.25)


def test_compact_metadata_preserves_raw_d_and_unpacked_scales(tmp_path):
    row, _, meta = _pack_sample(tmp_path, "split-compact")
    block = sample_block()
    assert len(meta) == 20 and row["metadata_format"] == "compact-u8"
    assert meta[:4] == block[:4]
    assert meta[4:8] == bytes([1, 2, 3, 4])
    assert meta[12:16] == bytes([5, 6, 7, 8])


def test_native_metadata_preserves_original_sixteen_bytes(tmp_path):
    row, _, meta = _pack_sample(tmp_path, "split-native")
    assert meta == sample_block()[:16] and row["metadata_format"] == "native16"
    assert Path(row["metadata_path"]).name == "blk.0.ffn_down.weight.q4k_meta.native16.bin"


def test_split_half_metadata_products_are_fp16(tmp_path):
    row, _, meta = _pack_sample(tmp_path, "split-half")
    assert len(meta) == 32 and row["metadata_format"] == "fp16-products"
    assert struct.unpack("<ee", meta[:4]) == (0.5, 1.25)


def test_q4k_record_form(tmp_path):
    row, payload, meta = _pack_sample(tmp_path, "split-native")
    assert list(row) == Q4K_KEYS
    assert (row["rows"], row["cols"], row["block_count"], row["source_offset"]) == (1, 256, 1, 32)
    assert row["source_checksum"] == sum(sample_block())
    assert row["payload_checksum"] == sum(payload) and row["metadata_checksum"] == sum(meta)
    assert row["blocks_path"] == "" and row["runtime_kernel"] == "split-native"
    assert row["compression_ratio_vs_fp16"] == 256 * 2 / 144.0
    row_b = P.pack_tensor(tmp_path / "q4k_split-native.bin",
                          {"name": "blk.0.ffn_down.weight", "type": "Q4_K", "dimensions": [256, 1],
                           "absolute_offset": 32, "span_bytes": 144}, tmp_path / "pack_split-native",
                          write_blocks=True)
    assert Path(row_b["blocks_path"]).read_bytes() == sample_block()


def test_auto_policy_is_the_mi355x_choice(tmp_path):
    """The reference's auto rule (q4k_resident_pack.py:75-79: compact up to 4096
    blocks, else predecoded) is an RTX 3060 measurement; this producer's auto
    is split-native at every shape and auto-lossy adds split-half above 65536
    blocks (the MI355X layout sweep). The named policies are the reference's."""
    blocks = [("blk.0.ffn_down.weight", 4, 512), ("blk.1.ffn_down.weight", 257, 65536)]
    tensors = [(n, "Q4_K", [c, r], packs.synth_raw(F.Q4K_RAW, r, c, 60 + i)) for i, (n, r, c) in enumerate(blocks)]
    path = tmp_path / "q.gguf"
    G.write(path, [("general.architecture", 8, "test")], tensors)
    for policy, want in (("auto", ["split-native", "split-native"]),
                         ("auto-lossy", ["split-native", "split-half"])):
        man = json.loads(P.pack_gguf(path, tmp_path / policy, policy=policy)["q4k_manifest"].read_text())
        assert man["policy"] == policy and [t["policy"] for t in man["tensors"]] == want


# ---- test_gguf_block_formats.py --------------------------------------------------------

def test_expected_data_bytes_for_target_formats():
    assert P.tensor_shape("Q4_K", [2048, 8192])[2] == 9_437_184
    assert P.tensor_shape("Q5_K", [2048, 248320])[2] == 349_634_560
    assert P.tensor_shape("IQ2_S", [2048, 512, 256])[2] == 85_983_232
    assert P.tensor_shape("IQ3_S", [512, 2048, 256])[2] == 115_343_360
    assert P.tensor_shape("F32", [2048])[2] == 8192
    with pytest.raises(ValueError, match="not divisible by block size"):
        P.tensor_shape("IQ2_S", [100])
    with pytest.raises(ValueError, match="unsupported tensor type"):
        P.tensor_shape("Q6_K", [256])
    with pytest.raises(ValueError, match="non-empty"):
        P.tensor_shape("F32", [])


def test_sanitize_label_matches_the_reference_rule():
    assert P.sanitize_label("blk.0.attn_q.weight") == "blk.0.attn_q.weight"
    assert P.sanitize_label("a b/c") == "a_b_c"
    assert P.sanitize_label("  x y  ") == "x_y"
    assert P.sanitize_label("-._a.b_-.") == "a.b"
    assert P.sanitize_label("...") == "native" and P.sanitize_label("") == "native"
    assert P.sanitize_label("café.w") == "caf_.w"


# ---- GGUF header and tensor plan ---------------------------------------------------------

def test_tensor_plan_of_the_reference_self_test_blob(tmp_path):
    path = tmp_path / "blob.gguf"
    path.write_bytes(reference_self_test_blob() + bytes(2 + 16 * 32 * 4))  # padding to 160, then the data
    plan = P.tensor_plan(path)
    assert plan["path"] == "gguf_tensor_plan" and plan["model_size_bytes"] == 160 + 2048
    assert plan["metadata"] == {"architecture": "test", "name": None, "tensor_count": 1, "metadata_count": 2,
                                "tensor_data_offset": 160, "tensor_data_alignment": 32}
    (row,) = plan["tensors"]
    assert row == {"name": "blk.0.weight", "layer": 0, "span_bytes": 2048, "span_mib": 2048 / 2 ** 20, "offset": 0,
                   "absolute_offset": 160, "type": "F32", "type_id": 0, "dimensions": [16, 32]}


def test_tensor_plan_matches_the_python_reader(tmp_path):
    path, _ = tiny_llama(tmp_path)
    g = G.read(path)
    plan = P.tensor_plan(path)
    rows = {r["name"]: r for r in plan["tensors"]}
    assert [r["offset"] for r in plan["tensors"]] == sorted(r["offset"] for r in plan["tensors"])
    assert plan["metadata"]["tensor_data_offset"] == g.data_offset and plan["layer_count"] == 2
    for t in g.tensors:
        r = rows[t.name]
        assert (r["type"], r["dimensions"], r["span_bytes"], r["absolute_offset"]) == (
            t.type, [int(d) for d in t.dims], t.span, g.data_offset + t.offset)
        assert r["layer"] == (int(t.name.split(".")[1]) if t.name.startswith("blk.") else None)


def test_refuses_non_gguf_and_truncated_files(tmp_path):
    bad = tmp_path / "bad.gguf"
    bad.write_bytes(b"GGML" + bytes(60))
    with pytest.raises(ValueError, match="not a GGUF file"):
        P.tensor_plan(bad)
    bad.write_bytes(reference_self_test_blob()[:100])
    with pytest.raises(ValueError, match="unexpected end"):
        P.tensor_plan(bad)
    blob = bytearray(reference_self_test_blob())
    blob[24:32] = struct.pack("<Q", 1 << 40)  # first key's length beyond the file
    bad.write_bytes(bytes(blob))
    with pytest.raises(ValueError, match="longer than the file"):
        P.tensor_plan(bad)


# ---- a GGUF model ------------------------------------------------------------------------

def _load_set(selftest, plan, root, manifests):
    return subprocess.run([str(selftest), "--load-set", str(plan), str(root)] + [str(m) for m in manifests],
                          capture_output=True, text=True, timeout=120)


@pytest.mark.parametrize("policy", ["split-native", "split-compact", "split-predecoded"])
def test_gguf_model_packs_in_the_reference_form(selftest, tmp_path, policy):
    (tmp_path / "m").mkdir()
    path, _ = tiny_llama(tmp_path / "m")
    g = G.read(path)
    out = tmp_path / "packs"
    paths = P.pack_gguf(path, out, policy=policy, write_blocks=True)
    assert set(paths) == {"tensor_plan", "q4k_manifest", "iq_manifest", "q5k_manifest"}
    q4k, iq, q5k = (json.loads(paths[k].read_text()) for k in ("q4k_manifest", "iq_manifest", "q5k_manifest"))
    # one directory and manifest per producer, the producers' top-level fields in order
    assert paths["q4k_manifest"] == out / "q4k" / "manifest.json" and (out / "q4k" / "manifest.md").is_file()
    assert list(q4k) == ["path", "generated_at", "model", "tensor_plan", "output_dir", "policy", "write_blocks",
                         "tensor_count", "source_bytes", "payload_bytes", "metadata_bytes", "resident_bytes",
                         "tensors"]
    assert list(iq) == ["path", "generated_at", "model", "tensor_plan", "output_dir", "types", "tensor_count",
                        "source_bytes", "payload_bytes", "resident_bytes", "tensors"]
    assert (q4k["path"], iq["path"], q5k["path"]) == ("q4k_resident_pack", "iq_resident_pack", "q5k_resident_pack")
    assert iq["types"] == ["IQ2_S", "IQ3_S"] and q5k["types"] == ["Q5_K"]
    assert q4k["policy"] == policy and q4k["write_blocks"] is True and q4k["model"] == str(path.resolve())
    assert q4k["tensor_count"] == 2 and iq["tensor_count"] == 12 and q5k["tensor_count"] == 2
    assert q4k["resident_bytes"] == q4k["payload_bytes"] + q4k["metadata_bytes"]
    fmt = {"split-native": F.Q4K_SPLIT_NATIVE, "split-compact": F.Q4K_SPLIT_COMPACT,
           "split-predecoded": F.Q4K_SPLIT_PREDECODED}[policy]
    for rec in q4k["tensors"]:
        assert list(rec) == Q4K_KEYS and Path(rec["payload_path"]).is_absolute()
        t = g.tensor(rec["name"])
        payload, meta = packs.q4k_split(fmt, np.asarray(g.data(t)))
        assert Path(rec["payload_path"]).read_bytes() == payload.tobytes()
        assert Path(rec["metadata_path"]).read_bytes() == meta.tobytes()
        assert Path(rec["blocks_path"]).read_bytes() == np.asarray(g.data(t)).tobytes()
        assert rec["source_offset"] == g.data_offset + t.offset
        assert rec["compression_ratio_vs_fp16"] == t.rows * t.cols * 2 / float(payload.size + meta.size)
    for man, kernels in ((iq, {"IQ2_S": "iq2s_raw_block_probe", "IQ3_S": "iq3s_raw_block_probe"}),
                         (q5k, {"Q5_K": "q5_k_raw_pending"})):
        for rec in man["tensors"]:
            t = g.tensor(rec["name"])
            assert list(rec) == RAW_KEYS and rec["runtime_kernel"] == kernels[rec["type"]]
            assert Path(rec["payload_path"]).read_bytes() == np.asarray(g.data(t)).tobytes()
            assert rec["source_offset"] == g.data_offset + t.offset
    # the C++ loaders take every manifest (paths absolute: any root works)
    r = _load_set(selftest, paths["tensor_plan"], "/nonexistent",
                  [paths["q4k_manifest"], paths["iq_manifest"], paths["q5k_manifest"]])
    assert r.returncode == 0, r.stdout + r.stderr
    lines = r.stdout.splitlines()
    assert len(lines) == 16 and all(line.endswith("ok=1") for line in lines)
    assert "raw output.weight type=Q5_K layer=-1 blocks=600 kernel=q5_k_raw_pending ok=1" in lines


def test_command_writes_the_same_packs(tmp_path):
    (tmp_path / "m").mkdir()
    path, _ = tiny_llama(tmp_path / "m")
    a = P.pack_gguf(path, tmp_path / "a", policy="split-half")
    r = subprocess.run([str(CLI), "--model", str(path), "--output-dir", str(tmp_path / "b"), "--policy", "split-half"],
                       capture_output=True, text=True, timeout=120)
    assert r.returncode == 0, r.stderr
    lines = r.stdout.splitlines()
    assert lines[0] == f"tensor_plan={tmp_path / 'b' / 'tensor_plan.json'}"
    assert f"json={tmp_path / 'b' / 'q4k' / 'manifest.json'}" in lines and "tensors=12" in lines
    for kind in ("q4k", "iq", "q5k"):
        ma = json.loads((tmp_path / "a" / kind / "manifest.json").read_text())
        mb = json.loads((tmp_path / "b" / kind / "manifest.json").read_text())
        for ra, rb in zip(ma["tensors"], mb["tensors"]):
            for key in ra:
                if key.endswith("_path") and ra[key]:
                    assert Path(ra[key]).read_bytes() == Path(rb[key]).read_bytes()
                elif not key.endswith("_path"):
                    assert ra[key] == rb[key], key
    # selection options and refusals of the command
    r = subprocess.run([str(CLI), "--model", str(path), "--output-dir", str(tmp_path / "c"), "--type", "Q5_K",
                        "--tensor", "output.weight"], capture_output=True, text=True, timeout=120)
    assert r.returncode == 0 and "tensors=1" in r.stdout and not (tmp_path / "c" / "iq").exists()
    r = subprocess.run([str(CLI), "--model", str(path), "--output-dir", str(tmp_path / "d"), "--type", "Q6_K"],
                       capture_output=True, text=True, timeout=120)
    assert r.returncode == 1 and "unsupported pack type" in r.stderr
    r = subprocess.run([str(CLI), "--model", str(path)], capture_output=True, text=True, timeout=120)
    assert r.returncode == 1 and "usage" in r.stderr


def test_gguf_to_packs_goes_through_the_cxx_producer(selftest, tmp_path):
    (tmp_path / "m").mkdir()
    path, _ = tiny_llama(tmp_path / "m")
    paths = G.to_packs(G.read(path), tmp_path / "p", policy="split-native")
    assert json.loads(paths["q5k_manifest"].read_text())["path"] == "q5k_resident_pack"
    r = _load_set(selftest, paths["tensor_plan"], tmp_path, [p for k, p in paths.items() if k.endswith("manifest")])
    assert r.returncode == 0, r.stdout + r.stderr


# ---- manifests in the reference producers' form, written by hand -------------------------

def _ref_raw_record(name, tname, dims, blocks: np.ndarray, offset, out_dir: Path, kernel) -> dict:
    """A record as iq_resident_pack.py / q5k_resident_pack.py pack_tensor returns it."""
    label = name  # already a clean label
    p = out_dir / f"{label}.{tname.lower()}_raw_blocks.bin"
    p.write_bytes(blocks.tobytes())
    layer = int(name.split(".")[1]) if name.startswith("blk.") else None
    role = ".".join(name.split(".")[2:]) if layer is not None else name.removesuffix(".weight")
    n = int(np.prod(dims))
    size = {"IQ2_S": 82, "IQ3_S": 110, "Q5_K": 176}[tname]
    s = int(blocks.sum(dtype=np.uint64))
    return {"name": name, "type": tname, "layer": layer, "role": role, "dimensions": dims, "element_count": n,
            "block_size": 256, "block_type_size": size, "block_count": n // 256, "source_offset": offset,
            "source_bytes": int(blocks.size), "source_checksum": s, "payload_path": str(p),
            "payload_bytes": int(blocks.size), "payload_checksum": s, "resident_bytes": int(blocks.size),
            "policy": "raw-blocks", "runtime_kernel": kernel}


def test_reference_form_manifests_load(selftest, tmp_path):
    """Packs laid out as the reference producers write them by default
    (packs/<kind>/<model>/<stamp>/manifest.json, absolute paths) load through
    the C++ loaders and match what this producer writes for the same tensors."""
    rows, cols = 8, 512
    q4 = packs.synth_raw(F.Q4K_RAW, rows, cols, 71)
    iq = packs.synth_raw(F.IQ3S, rows, cols, 72)
    q5 = packs.synth_raw(F.Q5K, rows, cols, 73)
    tensors = [("blk.0.ffn_down.weight", "Q4_K", [cols, rows], q4), ("blk.0.attn_q.weight", "IQ3_S", [cols, rows], iq),
               ("output.weight", "Q5_K", [cols, rows], q5)]
    model = tmp_path / "ref.gguf"
    G.write(model, [("general.architecture", 8, "llama")], tensors)
    g = G.read(model)
    off = {t.name: g.data_offset + t.offset for t in g.tensors}
    plan = tmp_path / "gguf_tensor_plan_ref.json"
    plan.write_text(json.dumps({"path": "gguf_tensor_plan", "tensors": [
        {"name": n, "layer": 0 if n.startswith("blk.") else None, "span_bytes": int(d.size), "offset": 0,
         "absolute_offset": off[n], "type": t, "dimensions": dims} for n, t, dims, d in tensors]}, indent=2))
    stamp = "1764644400"
    dirs = {k: tmp_path / "packs" / k / "ref" / stamp for k in ("q4k", "iq", "q5k")}
    for d in dirs.values():
        d.mkdir(parents=True)
    payload, meta = packs.q4k_split(F.Q4K_SPLIT_PREDECODED, q4)
    pp, mp = dirs["q4k"] / "blk.0.ffn_down.weight.q4k_payload.bin", dirs["q4k"] / "blk.0.ffn_down.weight.q4k_meta.fp32-products.bin"
    pp.write_bytes(payload.tobytes())
    mp.write_bytes(meta.tobytes())
    q4k_rec = {"name": "blk.0.ffn_down.weight", "dimensions": [cols, rows], "rows": rows, "cols": cols,
               "block_count": rows * cols // 256, "source_offset": off["blk.0.ffn_down.weight"],
               "source_bytes": int(q4.size), "source_checksum": int(q4.sum(dtype=np.uint64)),
               "policy": "split-predecoded", "metadata_format": "fp32-products", "payload_path": str(pp),
               "payload_bytes": int(payload.size), "payload_checksum": int(payload.sum(dtype=np.uint64)),
               "metadata_path": str(mp), "metadata_bytes": int(meta.size),
               "metadata_checksum": int(meta.sum(dtype=np.uint64)), "blocks_path": "",
               "resident_bytes": int(payload.size + meta.size),
               "compression_ratio_vs_fp16": rows * cols * 2 / float(payload.size + meta.size),
               "runtime_kernel": "split-predecoded"}
    manifests = {
        "q4k": {"path": "q4k_resident_pack", "generated_at": "2025-12-02T03:00:00.000000+00:00", "model": str(model),
                "tensor_plan": str(plan), "output_dir": str(dirs["q4k"]), "policy": "auto", "write_blocks": False,
                "tensor_count": 1, "source_bytes": q4k_rec["source_bytes"], "payload_bytes": q4k_rec["payload_bytes"],
                "metadata_bytes": q4k_rec["metadata_bytes"], "resident_bytes": q4k_rec["resident_bytes"],
                "tensors": [q4k_rec]},
        "iq": {"path": "iq_resident_pack", "generated_at": "2025-12-02T03:00:00.000000+00:00", "model": str(model),
               "tensor_plan": str(plan), "output_dir": str(dirs["iq"]), "types": ["IQ3_S"], "tensor_count": 1,
               "tensors": [_ref_raw_record("blk.0.attn_q.weight", "IQ3_S", [cols, rows], iq,
                                           off["blk.0.attn_q.weight"], dirs["iq"], "iq3s_raw_block_probe")]},
        "q5k": {"path": "q5k_resident_pack", "generated_at": "2025-12-02T03:00:00.000000+00:00", "model": str(model),
                "tensor_plan": str(plan), "output_dir": str(dirs["q5k"]), "types": ["Q5_K"], "tensor_count": 1,
                "tensors": [_ref_raw_record("output.weight", "Q5_K", [cols, rows], q5, off["output.weight"],
                                            dirs["q5k"], "q5_k_raw_pending")]},
    }
    for k in ("iq", "q5k"):
        t = manifests[k]["tensors"]
        for f in ("source_bytes", "payload_bytes", "resident_bytes"):
            manifests[k][f] = sum(r[f] for r in t)
    files = []
    for k, m in manifests.items():
        files.append(dirs[k] / "manifest.json")
        files[-1].write_text(json.dumps(m, indent=2))
    r = _load_set(selftest, plan, tmp_path / "elsewhere", files)
    assert r.returncode == 0, r.stdout + r.stderr
    assert r.stdout.splitlines() == [
        f"q4k blk.0.ffn_down.weight layer=0 role=ffn_down.weight rows={rows} cols={cols} policy=split-predecoded ok=1",
        f"raw blk.0.attn_q.weight type=IQ3_S layer=0 blocks=16 kernel=iq3s_raw_block_probe ok=1",
        f"raw output.weight type=Q5_K layer=-1 blocks=16 kernel=q5_k_raw_pending ok=1"]
    # this producer writes the same records for the same tensors, paths aside
    ours = P.pack_gguf(model, tmp_path / "ours", policy="split-predecoded")
    for k, key in (("q4k", "q4k_manifest"), ("iq", "iq_manifest"), ("q5k", "q5k_manifest")):
        mine = json.loads(ours[key].read_text())["tensors"][0]
        theirs = manifests[k]["tensors"][0]
        assert list(mine) == list(theirs)
        for f in theirs:
            if f.endswith("_path") and theirs[f]:
                assert Path(mine[f]).name == Path(theirs[f]).name
                assert Path(mine[f]).read_bytes() == Path(theirs[f]).read_bytes()
            else:
                assert mine[f] == theirs[f], (k, f)


# ---- refusals ----------------------------------------------------------------------------

def test_pack_tensor_refusals(tmp_path):
    model = tmp_path / "m.bin"
    model.write_bytes(sample_block() * 2)
    out = tmp_path / "o"
    out.mkdir()

    def pack(row, policy="split-native"):
        return P.pack_tensor(model, dict({"name": "w", "absolute_offset": 0, "span_bytes": 288}, **row), out,
                             policy=policy)

    with pytest.raises(ValueError, match="is not a 2D Q4_K tensor"):
        pack({"type": "Q4_K", "dimensions": [256, 1, 2]})
    with pytest.raises(ValueError, match="unsupported Q4_K dimensions"):
        pack({"type": "Q4_K", "dimensions": [128, 2]})
    with pytest.raises(ValueError, match="span is smaller than expected Q4_K bytes"):
        pack({"type": "Q4_K", "dimensions": [256, 2], "span_bytes": 200})
    with pytest.raises(ValueError, match="short read"):
        pack({"type": "Q4_K", "dimensions": [256, 2], "absolute_offset": 100})
    with pytest.raises(ValueError, match="unknown Q4_K metadata policy"):
        pack({"type": "Q4_K", "dimensions": [256, 2]}, policy="fastest")
    with pytest.raises(ValueError, match="unsupported raw-block type"):
        pack({"type": "Q6_K", "dimensions": [256]})
    with pytest.raises(ValueError, match="span is smaller than expected IQ bytes"):
        pack({"type": "IQ2_S", "dimensions": [256], "span_bytes": 10})
    with pytest.raises(ValueError, match="absolute_offset"):
        P.pack_tensor(model, {"name": "w", "type": "IQ2_S", "dimensions": [256]}, out)
    # split-half products beyond the fp16 range are refused (the reference's
    # struct.pack("<e") raises on them): d = 65504, scale 63
    big = bytearray(sample_block())
    big[0:2] = _half(65504.0)
    big[4] = 63
    model.write_bytes(bytes(big))
    with pytest.raises(ValueError, match="beyond the fp16 range"):
        pack({"type": "Q4_K", "dimensions": [256, 1], "span_bytes": 144}, policy="split-half")
    pack({"type": "Q4_K", "dimensions": [256, 1], "span_bytes": 144}, policy="split-predecoded")


def test_pack_gguf_refusals(tmp_path):
    path = _iq_gguf(tmp_path, ["blk.0.a.weight"])
    with pytest.raises(ValueError, match="no Q4_K / Q5_K / IQ2_S / IQ3_S tensors selected"):
        P.pack_gguf(path, tmp_path / "o", layer=3)
    with pytest.raises(ValueError, match="unsupported pack type"):
        P.pack_gguf(path, tmp_path / "o", types=["F32"])
    with pytest.raises(ValueError, match="unknown Q4_K metadata policy"):
        P.pack_gguf(path, tmp_path / "o", policy="fastest")
    with pytest.raises(ValueError, match="failed to stat"):
        P.pack_gguf(tmp_path / "missing.gguf", tmp_path / "o")


def test_huge_rows_are_refused_before_allocating(tmp_path):
    """A row whose dimensions claim far more data than the file holds is
    refused from the file size, without reading or allocating that much."""
    model = tmp_path / "m.bin"
    model.write_bytes(bytes(1024))
    out = tmp_path / "o"
    out.mkdir()
    huge = {"name": "w", "type": "Q4_K", "dimensions": [1 << 31, 1 << 20], "absolute_offset": 0,
            "span_bytes": (1 << 63)}
    with pytest.raises(ValueError, match="short read"):
        P.pack_tensor(model, huge, out)
    with pytest.raises(ValueError, match="short read"):
        P.pack_tensor(model, dict(huge, type="IQ2_S", dimensions=[256, 1 << 40]), out)
