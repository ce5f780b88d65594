"""Host contracts of the runner, on the CPU: the native self-test of the layer
role plan, layer executor, admission and tensor-pack manifest loaders
(tests/native/runtime_selftest.cpp, built here with g++), and a round trip
of the Python pack producer (rtxllm_amd.manifest) through the C++ loaders:
every record accepted, validated against the tensor plan, every file's size
and byte-sum checksum confirmed."""

from __future__ import annotations

import json
import subprocess
from pathlib import Path

import numpy as np
import pytest

from rtxllm_amd import formats as F
from rtxllm_amd import manifest as M
from rtxllm_amd import packs

REPO = Path(__file__).resolve().parent.parent


def test_native_runtime_selftest(selftest):
    r = subprocess.run([str(selftest)], capture_output=True, text=True, timeout=120)
    assert r.returncode == 0, r.stderr
    assert "cases passed" in r.stdout and int(r.stdout.split()[2]) >= 19


def small_model_tensors(seed: int = 11) -> list[M.Tensor]:
    H, Q, KV, FF, V = 512, 512, 256, 1024, 300
    shapes = [("blk.0.attn_q.weight", F.IQ3S, Q, H), ("blk.0.attn_k.weight", F.IQ3S, KV, H),
              ("blk.0.attn_v.weight", F.IQ3S, KV, H), ("blk.0.attn_output.weight", F.IQ3S, H, Q),
              ("blk.0.ffn_gate.weight", F.IQ2S, FF, H), ("blk.0.ffn_up.weight", F.IQ2S, FF, H),
              ("blk.0.ffn_down.weight", F.Q4K_RAW, H, FF), ("token_embd.weight", F.Q5K, V, H),
              ("output.weight", F.Q5K, V, H)]
    return [M.Tensor(n, f, r, c, packs.synth_raw(f, r, c, seed + i)) for i, (n, f, r, c) in enumerate(shapes)]


@pytest.mark.parametrize("policy", ["split-native", "split-compact"])
def test_pack_producer_round_trip_through_loaders(selftest, tmp_path, policy):
    tensors = small_model_tensors()
    paths = M.write_packs(tmp_path, tensors, policy=policy)
    r = subprocess.run([str(selftest), "--load", str(paths["q4k_manifest"]), str(paths["iq_manifest"]),
                        str(paths["tensor_plan"]), str(tmp_path)], capture_output=True, text=True, timeout=120)
    assert r.returncode == 0, r.stdout + r.stderr
    lines = r.stdout.splitlines()
    assert len(lines) == len(tensors) and all(l.endswith("ok=1") for l in lines), lines
    assert f"q4k blk.0.ffn_down.weight layer=0 role=ffn_down.weight rows=512 cols=1024 policy={policy} ok=1" in lines
    assert "raw token_embd.weight type=Q5_K layer=-1 blocks=600 ok=1" in lines
    # the producer wrote the split streams of its policy
    q = json.loads(paths["q4k_manifest"].read_text())["tensors"][0]
    fmt = M.Q4K_POLICIES[policy][0]
    payload, meta = packs.q4k_split(fmt, tensors[6].blocks)
    assert np.array_equal(np.fromfile(tmp_path / q["payload_path"], np.uint8), payload)
    assert np.array_equal(np.fromfile(tmp_path / q["metadata_path"], np.uint8), meta)


def test_loaders_reject_a_corrupted_pack(selftest, tmp_path):
    paths = M.write_packs(tmp_path, small_model_tensors())
    raw = json.loads(paths["iq_manifest"].read_text())
    f = tmp_path / raw["tensors"][0]["payload_path"]
    b = bytearray(f.read_bytes())
    b[5] ^= 0x40
    f.write_bytes(bytes(b))
    r = subprocess.run([str(selftest), "--load", str(paths["q4k_manifest"]), str(paths["iq_manifest"]),
                        str(paths["tensor_plan"]), str(tmp_path)], capture_output=True, text=True, timeout=120)
    assert r.returncode == 1  # a checksum mismatch fails the load
    assert any(l.startswith("raw blk.0.attn_q.weight") and l.endswith("ok=0") for l in r.stdout.splitlines())
    (tmp_path / raw["tensors"][1]["payload_path"]).write_bytes(b"short")
    r = subprocess.run([str(selftest), "--load", str(paths["q4k_manifest"]), str(paths["iq_manifest"]),
                        str(paths["tensor_plan"]), str(tmp_path)], capture_output=True, text=True, timeout=120)
    assert r.returncode == 1 and "size mismatch" in r.stdout
