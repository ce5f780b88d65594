"""GPU: the decode-step command (build/rtxllm_decode_runner) and its pass /
fail contract, the reference runner's (mixed_sequence_benchmark_runner/
main.cpp:3736-3762, 5813): exit 0 with every gate passed, 2 when strict
admission refuses the model, 3 when a gate fails; one JSON object on stdout.

* A small synthetic model passes its own gates (finite logits, token =
  argmax, context not exhausted, graph replay = eager step) at batch 1 and 8.
* Given the oracle's logits for the same seeded model, token and position
  (written by this test from rtxllm_amd's own copy of the model and the
  oracle), the runner's reference gate passes within 1e-3; given logits moved
  by 5 % of their range at one entry it fails with exit 3.
* A GGUF model goes through the command's C++ path (producer, pack loader,
  F32 norms from the file) and gives the Python loader path's logits bit for
  bit (tolerance 0).
* A guard larger than the GPU's memory makes admission refuse: exit 2,
  "admitted": false, nothing allocated.
* At the 32-layer 8B shapes (synthetic weights) every gate passes at batch
  1 and 8.
"""

from __future__ import annotations

import json
import subprocess

import numpy as np
import pytest

torch = pytest.importorskip("torch")

from rtxllm_amd import gguf as G  # noqa: E402
from rtxllm_amd import packs  # noqa: E402
from rtxllm_amd._lib import PKG_ROOT  # noqa: E402
from rtxllm_amd.llama import Llama, Shape  # noqa: E402

from llama_ref import HostModel  # noqa: E402
from test_gguf import tiny_llama  # noqa: E402

pytestmark = pytest.mark.gpu

RUNNER = PKG_ROOT / "build" / "rtxllm_decode_runner"
SMALL = Shape(hidden=512, n_heads=4, n_kv_heads=2, ffn=1024, vocab=1000, n_layers=2, max_ctx=256, page_size=16)
SEED = 0x5EED0D00
SMALL_ARGS = ["--shape", "small", "--max-ctx", "256", "--page-size", "16", "--seed", str(SEED)]


def run(args, timeout=300):
    print("runner:", " ".join(str(a) for a in args), flush=True)
    r = subprocess.run([str(RUNNER)] + [str(a) for a in args], capture_output=True, text=True, timeout=timeout)
    out = json.loads(r.stdout) if r.stdout.strip().startswith("{") else None
    return r.returncode, out, r.stderr


def seeded(m: Llama, seed: int, norms: bool = True) -> None:
    """The runner's seeded norms and KV cache (batch 1)."""
    s = m.shape
    for l in range(s.n_layers):
        if norms:
            m.upload("attn_norm", packs.normal_f32(seed + 100 + 2 * l, s.hidden, mean=1.0, std=0.02), layer=l)
            m.upload("ffn_norm", packs.normal_f32(seed + 101 + 2 * l, s.hidden, mean=1.0, std=0.02), layer=l)
        n = m.region_bytes("k_cache", l) // 2
        m.upload("k_cache", packs.normal_f16_bits(seed + 300 + 2 * l, n), layer=l)
        m.upload("v_cache", packs.normal_f16_bits(seed + 301 + 2 * l, n), layer=l)
    if norms:
        m.upload("out_norm", packs.normal_f32(seed + 99, s.hidden, mean=1.0, std=0.02))


@pytest.mark.parametrize("batch", [1, 8])
def test_runner_small_model_passes_its_gates(batch):
    rc, out, err = run(SMALL_ARGS + ["--batch", batch, "--steps", 5, "--warmup", 1, "--position", 100])
    assert rc == 0, (out, err)
    assert out["path"] == "rtxllm_decode_runner" and out["admitted"] is True and out["gates_passed"] is True
    assert all(out["gates"].values()), out["gates"]
    assert out["reference_checked"] is False
    assert out["config"]["batch"] == batch and len(out["token_observed"]) == batch
    assert out["tok_s"] > 0 and out["latency_ms"]["p50"] > 0 and out["steps"] == 5
    assert out["launches_per_step"] == (1 + 6 * 2 + 2 if batch == 1 else 1 + 8 * 2 + 2)


def test_runner_reference_gate_against_the_oracle(orc, tmp_path):
    token, pos = 123, 100
    m = Llama(SMALL)
    m.synth_weights(SEED)
    torch.cuda.synchronize()
    seeded(m, SEED)
    ref = HostModel(m, range(SMALL.n_layers))
    _, logits = ref.run(orc, ref.embed_row(orc, token), pos)
    m.close()
    want = tmp_path / "oracle_logits.f32"
    np.asarray(logits, np.float32).tofile(want)
    rc, out, err = run(SMALL_ARGS + ["--token", token, "--position", pos, "--steps", 2, "--warmup", 0,
                                     "--expect-logits", want])
    assert rc == 0, (out, err)
    assert out["reference_checked"] is True and out["reference_passed"] is True
    assert out["max_logit_rel_error"] <= 1e-3
    assert out["token_observed"] == [int(np.argmax(logits))] or out["token_expected"] == out["token_observed"]
    # logits moved by 5 % of their range at one entry: the gate fails, exit 3
    bad = np.asarray(logits, np.float32).copy()
    bad[7] += 0.05 * float(np.max(np.abs(bad)))
    bad.tofile(tmp_path / "moved.f32")
    rc, out, err = run(SMALL_ARGS + ["--token", token, "--position", pos, "--steps", 2, "--warmup", 0,
                                     "--expect-logits", tmp_path / "moved.f32"])
    assert rc == 3, (out, err)
    assert out["reference_passed"] is False and out["gates_passed"] is True and out["max_logit_rel_error"] > 1e-3
    # a file of the wrong size is an error, exit 1
    bad[:10].tofile(tmp_path / "short.f32")
    rc, out, err = run(SMALL_ARGS + ["--expect-logits", tmp_path / "short.f32", "--steps", 1])
    assert rc == 1 and "batch x vocab" in err


def test_runner_gguf_model_matches_the_python_loader(tmp_path):
    (tmp_path / "m").mkdir()
    path, _ = tiny_llama(tmp_path / "m")
    g = G.read(path)
    fields = G.llama_shape(g)
    shape = Shape(**fields, max_ctx=256, page_size=16)
    m = Llama(shape, formats=G.model_formats(g, "split-native"))
    G.load_into(m, g, tmp_path / "py_packs")
    seeded(m, SEED, norms=False)
    m.set_token_pos(42, 77)
    m.step()
    torch.cuda.synchronize()
    logits = m.download("logits", np.float32)
    token = int(m.download("token", np.uint32)[0])
    m.close()
    logits.tofile(tmp_path / "py.f32")
    rc, out, err = run(["--gguf", path, "--pack-dir", tmp_path / "cli_packs", "--max-ctx", 256, "--page-size", 16,
                        "--seed", SEED, "--token", 42, "--position", 77, "--steps", 3, "--warmup", 1,
                        "--expect-logits", tmp_path / "py.f32", "--tolerance", 0])
    assert rc == 0, (out, err)
    assert out["reference_passed"] is True and out["max_logit_rel_error"] == 0.0
    assert out["token_observed"] == [token] and out["source"] == str(path)
    assert (tmp_path / "cli_packs" / "q5k" / "manifest.json").is_file()


def test_runner_admission_refusal_exits_2():
    rc, out, err = run(SMALL_ARGS + ["--guard-mib", 1 << 40])
    assert rc == 2, (out, err)
    assert out["admitted"] is False and out["admission_reason"] and out["required_bytes"] > 0
    assert "gates" not in out and "tok_s" not in out


@pytest.mark.parametrize("batch", [1, 8])
def test_runner_8b_shapes_pass_their_gates(batch):
    """The decode-step command at the 32-layer 8B shapes (synthetic weights,
    4096-position caches): every gate passes, 195 / 259 launches per step."""
    rc, out, err = run(["--batch", batch, "--steps", 10, "--warmup", 2], timeout=600)
    assert rc == 0, (out, err)
    assert out["gates_passed"] is True and all(out["gates"].values())
    assert out["config"]["n_layers"] == 32 and out["config"]["vocab"] == 128256
    assert out["launches_per_step"] == (195 if batch == 1 else 259)
    assert out["tok_s"] > 0
