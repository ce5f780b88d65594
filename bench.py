"""Decode hot-path benchmark on one MI355X.

Headline workload (one "step"): one batch-1 greedy decode step of a 32-layer
Llama-8B-shaped model in the mixed GGUF formats (q/k/v/o IQ3_S, gate/up IQ2_S,
down Q4_K split-native, Q5_K embedding and LM head), fp16 paged KV cache of
4096 positions ~ N(0,1), random-init synthetic weights, replayed as one
hipGraph with the token and position advanced on the device. value = tokens/s.

Also reported: per-stage kernel times of the step (the roofline entry is the
stage with the largest share of the step), the same step for a batch of 8
sequences (one pass over the weights on the matrix cores; tok/s counts all 8),
the batch-1 matvec set at the 8B FFN shapes (cold weights, GB/s), and the CPU
reference path (the oracle's scalar restatement of the reference gate) timed
on this host on a bounded sample.

Prints one JSON line (the driver's contract).
"""

from __future__ import annotations

import argparse
import json
import os
import sys
import time
from pathlib import Path

REPO = Path(__file__).resolve().parent
sys.path.insert(0, str(REPO / "local-ai-gpu-acceleration_amd"))
sys.path.insert(0, str(REPO))

HBM_PEAK_GBS = 8000.0
MALL_BYTES = 256 << 20
SEED = 0x5EED0004


def parse() -> argparse.Namespace:
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=200)
    ap.add_argument("--warmup", type=int, default=5)
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--no-matvec-set", action="store_true")
    ap.add_argument("--no-batch8", action="store_true", help="skip the batch-8 decode step")
    ap.add_argument("--no-read-ceiling", action="store_true", help="skip the streaming-read ceiling per stage size")
    ap.add_argument("--no-context-buckets", action="store_true",
                    help="skip the short-context decode with a span-bucketed step graph")
    ap.add_argument("--traffic-probe", action="store_true",
                    help="run a 256 MiB device copy and each decode stage of layer 0 a few times (for "
                         "rocprofv3 --pmc FETCH_SIZE / WRITE_SIZE passes), print nothing else")
    ap.add_argument("--q4k-sweep", action="store_true",
                    help="time every Q4_K resident layout at the config shapes (HBM-cold, rotating copies) and "
                         "print the fastest per shape as JSON, nothing else")
    ap.add_argument("--read-ceiling", action="store_true",
                    help="time a plain streaming read (rtxllm_stream_read) of each stage's byte count over "
                         "rotating HBM-cold buffers and print it as JSON, nothing else")
    ap.add_argument("--units-sweep", action="store_true",
                    help="time the IQ decode matvecs in the GGUF and the unit layouts (batch 1, HBM-cold)")
    ap.add_argument("--mfma-probe", action="store_true",
                    help="run the batch-1 gate_up and attention and the batch-8 matvec stages of one layer (the "
                         "matrix-core counter workload)")
    ap.add_argument("--mfma-summary", nargs=2, metavar=("PMC_DIR", "TRACE_DIR"),
                    help="matrix-core work, rate and busy share per matrix-core kernel from the counter and trace runs")
    ap.add_argument("--trace-summary", metavar="TRACE_DIR",
                    help="per-kernel launch statistics of a rocprofv3 --kernel-trace run as a markdown table, "
                         "with the kernels both decode paths launch split by grid size")
    ap.add_argument("--counter-summary", nargs="+", metavar="PMC_DIR",
                    help="instruction accounting per decode stage kernel from rocprofv3 --pmc runs of "
                         "--traffic-probe (SQ_* counters, any split over passes), with the VALU issue floor "
                         "against the time budget at 70%% of the HBM peak")
    ap.add_argument("--timeline", action="store_true",
                    help="run the batch-1 and batch-8 steps on the profiling build (build/librtxllm_timeline.so) and "
                         "print the per-wave timeline of their last layer and LM head as markdown, nothing else")
    ap.add_argument("--traffic-summary", nargs=2, metavar=("FETCH_DIR", "WRITE_DIR"),
                    help="summarise two rocprofv3 --pmc runs of --traffic-probe (FETCH_SIZE, WRITE_SIZE) as "
                         "HBM bytes per launch, calibrated on the copy kernel")
    return ap.parse_args()


MATVECS = [
    # (name, format, rows, cols, seed)
    ("q4k_native_4096x4096", 4, 4096, 4096, 0x5EED0000),
    ("q4k_native_14336x4096", 4, 14336, 4096, 0x5EED0001),
    ("q4k_native_4096x14336", 4, 4096, 14336, 0x5EED0001),
    ("q5k_14336x4096", 5, 14336, 4096, 0x5EED0001),
    ("q5k_4096x14336", 5, 4096, 14336, 0x5EED0001),
    ("iq2s_14336x4096", 6, 14336, 4096, 0x5EED0002),
    ("iq2s_4096x14336", 6, 4096, 14336, 0x5EED0002),
    ("iq3s_14336x4096", 7, 14336, 4096, 0x5EED0002),
    ("iq3s_4096x14336", 7, 4096, 14336, 0x5EED0002),
]


def _cpu_model() -> str:
    try:
        for line in Path("/proc/cpuinfo").read_text().splitlines():
            if line.startswith("model name"):
                return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return "unknown"


def time_graph(torch, stream, fn, reps: int = 10) -> float:
    """Capture fn() into a graph, replay it `reps` times; mean ms per replay
    from HIP events recorded on the replay stream."""
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g, stream=stream):
        fn()
    torch.cuda.synchronize()
    with torch.cuda.stream(stream):
        g.replay()
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record(stream)
        for _ in range(reps):
            g.replay()
        e1.record(stream)
    torch.cuda.synchronize()
    return e0.elapsed_time(e1) / reps


# ---- the decode step ------------------------------------------------------------

def layer_weight_bytes(shape) -> dict:
    """Algorithmic bytes of each matvec stage: rows * (cols / 256) * GGUF block
    bytes + fp32 x (4 cols) + fp32 y (4 rows), the matvec figure of the
    roofline (formats.algorithmic_bytes)."""
    from rtxllm_amd import formats as F

    H, q, kv, ff = shape.hidden, shape.n_heads * 128, shape.n_kv_heads * 128, shape.ffn
    return {
        "qkv": F.algorithmic_bytes(F.IQ3S, q + 2 * kv, H),
        "o": F.algorithmic_bytes(F.IQ3S, H, q),
        "gate_up": F.algorithmic_bytes(F.IQ2S, 2 * ff, H),
        "down": F.algorithmic_bytes(F.Q4K_SPLIT_NATIVE, H, ff),
        "lm_head": F.algorithmic_bytes(F.Q5K, shape.vocab, H),
    }


def build_model(torch, shape):
    """The 8B-shape model with its weights, norms and fp16 KV ~ N(0,1); a batch
    model's sequences share one seeded cache image per layer role (k, v) of
    all their pages, generated once."""
    import numpy as np

    from rtxllm_amd import packs
    from rtxllm_amd.llama import Llama

    m = Llama(shape)
    m.synth_weights(SEED)
    torch.cuda.synchronize()
    H = shape.hidden
    threads = min(16, os.cpu_count() or 1)
    shared = None
    if shape.batch > 1:
        n = m.region_bytes("k_cache", 0) // 2
        shared = (packs.normal_f16_bits(SEED + 300, n, threads=threads),
                  packs.normal_f16_bits(SEED + 301, n, threads=threads))
    for l in range(shape.n_layers):
        m.upload("attn_norm", packs.normal_f32(SEED + 100 + 2 * l, H, mean=1.0, std=0.02), layer=l)
        m.upload("ffn_norm", packs.normal_f32(SEED + 101 + 2 * l, H, mean=1.0, std=0.02), layer=l)
        if shared is None:
            n = m.region_bytes("k_cache", l) // 2
            m.upload("k_cache", packs.normal_f16_bits(SEED + 300 + 2 * l, n, threads=threads), layer=l)
            m.upload("v_cache", packs.normal_f16_bits(SEED + 301 + 2 * l, n, threads=threads), layer=l)
        else:
            m.upload("k_cache", shared[0], layer=l)
            m.upload("v_cache", shared[1], layer=l)
    m.upload("out_norm", packs.normal_f32(SEED + 99, H, mean=1.0, std=0.02))
    rng = np.random.default_rng(SEED)
    tokens = [int(t) for t in rng.integers(0, shape.vocab, size=shape.batch)]
    return m, (tokens[0] if shape.batch == 1 else tokens)


def decode_bench(torch, args, batch: int = 1) -> dict:
    """One decode step of `batch` sequences (every one at the same ~4096
    context) replayed as a hipGraph, plus per-stage kernel times."""
    import dataclasses

    import numpy as np

    from rtxllm_amd.llama import LLAMA_8B

    shape = dataclasses.replace(LLAMA_8B, batch=batch)
    m, token = build_model(torch, shape)
    stream = torch.cuda.Stream()
    sp = stream.cuda_stream
    total = args.warmup + args.steps
    if total + 1 > shape.max_ctx:
        raise SystemExit(f"warmup + steps must be < {shape.max_ctx} (KV capacity)")
    pos0 = shape.max_ctx - total - 1  # every timed step attends over ~4096 positions
    m.set_token_pos(token, [pos0] * batch if batch > 1 else pos0)
    m.graph_capture(sp)
    with torch.cuda.stream(stream):
        for _ in range(args.warmup):
            m.graph_replay(sp)
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        e0.record(stream)
        for _ in range(args.steps):
            m.graph_replay(sp)
        e1.record(stream)
    torch.cuda.synchronize()
    wall = time.perf_counter() - t0
    ms = e0.elapsed_time(e1) / args.steps
    pos_end = m.download("pos", np.uint32)
    assert all(int(p) == pos0 + total for p in pos_end), (pos_end, pos0, total)
    tokens = [int(t) for t in m.download("token", np.uint32)]
    assert m.status(sp) == [0] * batch  # no sequence reached the end of its context

    # latency distribution (the reference reports p50 / p95 / p99 of its replays,
    # main.cpp:4838-4913): the same replays from the same positions, one event
    # after each, so each step's device time is the gap between two events
    m.set_token_pos(token, [pos0] * batch if batch > 1 else pos0)
    torch.cuda.synchronize()
    with torch.cuda.stream(stream):
        for _ in range(args.warmup):
            m.graph_replay(sp)
        evs = [torch.cuda.Event(enable_timing=True) for _ in range(args.steps + 1)]
        evs[0].record(stream)
        for i in range(args.steps):
            m.graph_replay(sp)
            evs[i + 1].record(stream)
    torch.cuda.synchronize()
    per_step = np.array([evs[i].elapsed_time(evs[i + 1]) for i in range(args.steps)])
    latency = {f"p{q}": round(float(np.percentile(per_step, q)), 5) for q in (50, 95, 99)}
    latency.update({"mean": round(float(per_step.mean()), 5), "max": round(float(per_step.max()), 5),
                    "unit": "ms per step", "steps": args.steps})

    wb = layer_weight_bytes(shape)
    mean_ctx = pos0 + args.warmup + (args.steps + 1) / 2.0
    kv_layer = batch * 2 * shape.n_kv_heads * 128 * 2 * mean_ctx  # every sequence's K and V
    # weights once per step, KV, embedding rows and logits per sequence
    step_bytes = shape.n_layers * (wb["qkv"] + wb["o"] + wb["gate_up"] + wb["down"] + kv_layer) + wb["lm_head"] + \
        batch * ((shape.hidden // 256) * 176 + 4 * shape.vocab)

    # per-stage kernel time: one graph per stage with one launch per layer
    m.set_token_pos(token, [pos0 + args.warmup] * batch if batch > 1 else pos0 + args.warmup)
    stages = {}
    for st in ("qkv", "attention", "o", "gate_up", "down"):
        ms_g = time_graph(torch, stream, lambda st=st: [m.launch_stage(l, st, sp) for l in range(shape.n_layers)])
        us = ms_g * 1e3 / shape.n_layers
        b = kv_layer if st == "attention" else wb[st]
        stages[st] = {"us": round(us, 3), "launches_per_step": shape.n_layers, "bytes": int(b),
                      "GB/s": round(b / us / 1e3, 1)}
    reps = 8
    ms_g = time_graph(torch, stream, lambda: [m.launch_stage(0, "lm_head", sp) for _ in range(reps)])
    us = ms_g * 1e3 / reps
    stages["lm_head"] = {"us": round(us, 3), "launches_per_step": 1, "bytes": wb["lm_head"],
                         "GB/s": round(wb["lm_head"] / us / 1e3, 1)}
    for v in stages.values():
        v["frac"] = round(v["GB/s"] / HBM_PEAK_GBS, 4)
        v["share_of_step"] = round(v["us"] * v["launches_per_step"] / (ms * 1e3), 4)
    for st, dist in phase_latency(torch, m, stream, shape.n_layers, min(args.steps, 50)).items():
        stages[st]["launch_latency"] = dist
    dom = max(stages, key=lambda k: stages[k]["us"] * stages[k]["launches_per_step"])
    launches = m.launches_per_step()
    buckets = None if args.no_context_buckets else context_buckets(torch, m, stream, token, batch, args.steps)
    m.close()
    return {
        "ms_per_step": ms, "tok_s": batch * 1e3 / ms, "wall_s": wall, "step_bytes": step_bytes, "latency": latency,
        "GB/s": step_bytes / (ms * 1e-3) / 1e9, "stages": stages, "dominant": dom, "launches": launches,
        "mean_context": mean_ctx, "tokens_after": tokens, "context_buckets": buckets,
    }


def phase_latency(torch, m, stream, n_layers: int, steps: int) -> dict:
    """Per-launch latency distribution of each stage, as the reference times
    its phases (main.cpp:4838-4907: an event before and after each launch,
    every launch issued on its own, percentiles over the samples): `steps`
    passes over the step's stages in order (every layer's qkv, attention, o,
    gate_up, down, then the LM head), each launch between two events on the
    launch stream. Launches are issued from the host one by one, so each runs
    on an otherwise idle GPU: these figures include the launch's own ramp and
    drain, unlike the graph-replay means."""
    import numpy as np

    sp = stream.cuda_stream
    order = [(l, st) for l in range(n_layers) for st in ("qkv", "attention", "o", "gate_up", "down")]
    order.append((0, "lm_head"))
    evs = [(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)) for _ in order]
    samples: dict = {}
    with torch.cuda.stream(stream):
        for _ in range(steps):
            for (l, st), (e0, e1) in zip(order, evs):
                e0.record(stream)
                m.launch_stage(l, st, sp)
                e1.record(stream)
            evs[-1][1].synchronize()
            for (l, st), (e0, e1) in zip(order, evs):
                samples.setdefault(st, []).append(e0.elapsed_time(e1) * 1e3)
    out = {}
    for st, v in samples.items():
        a = np.array(v)
        out[st] = {f"p{q}": round(float(np.percentile(a, q)), 3) for q in (50, 95, 99)}
        out[st].update({"mean": round(float(a.mean()), 3), "samples": int(a.size), "unit": "us per launch"})
    return out


SHORT_POS = 64  # a short context: the first step's position


def context_buckets(torch, m, stream, token, batch: int, steps: int) -> dict:
    """Short-context decode: `steps` replays from position SHORT_POS of the
    full-span step graph against the smallest 128-multiple span graph that
    holds the last position (its attention launches cover only that span)."""
    import numpy as np

    sp = stream.cuda_stream
    span = -(-(SHORT_POS + steps + 1) // 128) * 128
    m.graph_capture_span(span, sp)
    assert m.graph_span_for(SHORT_POS + steps - 1) == span
    out = {"first_pos": SHORT_POS, "steps": steps, "span_positions": span}
    for name, replay in (("full", lambda: m.graph_replay(sp)), ("span", lambda: m.graph_replay_span(span, sp))):
        m.set_token_pos(token, [SHORT_POS] * batch if batch > 1 else SHORT_POS)
        with torch.cuda.stream(stream):
            replay()  # warm
            torch.cuda.synchronize()  # the upload below must not race the replay's position update
            m.set_token_pos(token, [SHORT_POS] * batch if batch > 1 else SHORT_POS)
            torch.cuda.synchronize()
            e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            e0.record(stream)
            for _ in range(steps):
                replay()
            e1.record(stream)
        torch.cuda.synchronize()
        ms = e0.elapsed_time(e1) / steps
        assert all(int(p) == SHORT_POS + steps for p in m.download("pos", np.uint32))
        out[name] = {"ms_per_step": round(ms, 4), "tok_s": round(batch * 1e3 / ms, 1),
                     "tokens_after": [int(t) for t in m.download("token", np.uint32)]}
    out["same_tokens"] = out["full"]["tokens_after"] == out["span"]["tokens_after"]
    out["graph_bytes"] = m.graph_bytes()
    return out


# ---- HBM traffic from counters ------------------------------------------------------

COPY_BYTES = 256 << 20
TRAFFIC_FILE = REPO / "profiles" / "decode_8b_hbm_traffic.txt"
STAGE_KERNELS = {  # decode stage -> substring of its kernel's name
    "qkv": "EpiQkv", "attention": "attn_partial_kernel", "o": "mv_kernel<10, 1, 4, false, rtxllm::(anonymous "
    "namespace)::EpiResidual", "gate_up": "EpiGateUp", "down": "mv_kernel<4, 1, 4, true", "lm_head": "EpiLogits",
}
BATCH8_STAGE_KERNELS = {  # batch-8 decode stage -> substring of its matrix-core kernel's name
    "qkv": "mm_kernel<7, rtxllm::(anonymous namespace)::MmQkv", "o": "mm_kernel<7, rtxllm::MmStore",
    "gate_up": "MmGateUp", "down": "mm_kernel<4, rtxllm::MmStore, true", "lm_head": "MmLogits",
}


def traffic_probe(torch) -> None:
    """The workload of the two counter passes: a plain fill and a plain sum of
    COPY_BYTES (the calibration: kernels whose HBM bytes are known) and each
    decode stage of layer 0, three times each."""
    from rtxllm_amd.llama import LLAMA_8B

    m, token = build_model(torch, LLAMA_8B)
    m.set_token_pos(token, LLAMA_8B.max_ctx - 64)
    buf = torch.empty(COPY_BYTES // 4, dtype=torch.float32, device="cuda:0")
    for _ in range(3):
        buf.fill_(1.0)         # writes COPY_BYTES
        float(buf.sum())       # reads COPY_BYTES
        for st in ("qkv", "attention", "o", "gate_up", "down", "lm_head"):
            m.launch_stage(0, st, torch.cuda.current_stream().cuda_stream)
    torch.cuda.synchronize()
    m.close()


MFMA_PEAK_TFLOPS = 2500.0  # MI355X dense fp16 / bf16 matrix-core peak
MFMA_STAGES = ("qkv", "o", "gate_up", "down", "lm_head")


def mfma_probe(torch) -> None:
    """The workload of the matrix-core counter pass: the batch-1 decode step's
    gate_up (int8 matrix cores) and attention (fp16 score MFMAs) and the
    batch-8 step's matvec stages, layer 0 at ~4030 positions, three times each."""
    import dataclasses

    from rtxllm_amd.llama import LLAMA_8B

    sp = torch.cuda.current_stream().cuda_stream
    for batch, stages in ((1, ("gate_up", "attention")), (8, MFMA_STAGES)):
        shape = dataclasses.replace(LLAMA_8B, batch=batch)
        m, token = build_model(torch, shape)
        m.set_token_pos(token, [shape.max_ctx - 64] * batch if batch > 1 else shape.max_ctx - 64)
        for _ in range(3):
            for st in stages:
                m.launch_stage(0, st, sp)
        torch.cuda.synchronize()
        m.close()


MFMA_KERNELS = ("mm_kernel", "mvq_kernel", "attn_partial_kernel")
MFMA_COUNTERS = ("SQ_INSTS_VALU_MFMA_MOPS_F16", "SQ_INSTS_VALU_MFMA_MOPS_I8", "SQ_VALU_MFMA_BUSY_CYCLES",
                 "SQ_BUSY_CU_CYCLES", "GRBM_GUI_ACTIVE")
INT8_PEAK_TOPS = 5000.0  # MI355X dense int8 matrix-core peak


def mfma_summary(pmc_dir: str, trace_dir: str) -> str:
    """Per matrix-core kernel (batch matvecs, the batch-1 gate_up, attention
    partials): matrix-core work per dispatch from SQ_INSTS_VALU_MFMA_MOPS_F16 /
    _I8 (units of 512 FLOP or OP), the mean dispatch time from the kernel trace
    of the same workload, the achieved rate against the dense fp16 / int8 peak,
    and the matrix-core busy share: SQ_VALU_MFMA_BUSY_CYCLES (summed over the
    1024 SIMDs) / (1024 * the kernel's busy cycles), where GRBM_GUI_ACTIVE sums
    the 8 XCDs' busy cycles (busy = GRBM_GUI_ACTIVE / 8)."""
    import csv
    import glob

    vals: dict = {}
    for f in glob.glob(str(Path(pmc_dir) / "**" / "*counter_collection.csv"), recursive=True):
        for r in csv.DictReader(open(f)):
            if r["Counter_Name"] in MFMA_COUNTERS and any(k in r["Kernel_Name"] for k in MFMA_KERNELS):
                key = (r["Kernel_Name"], r["Grid_Size"])
                vals.setdefault(key, {}).setdefault(r["Counter_Name"], []).append(float(r["Counter_Value"]))
    dur: dict = {}
    for f in glob.glob(str(Path(trace_dir) / "**" / "*kernel_trace.csv"), recursive=True):
        for r in csv.DictReader(open(f)):
            if any(k in r["Kernel_Name"] for k in MFMA_KERNELS):
                g = str(int(r["Grid_Size_X"]) * int(r["Grid_Size_Y"]) * int(r["Grid_Size_Z"]))
                us = (int(r["End_Timestamp"]) - int(r["Start_Timestamp"])) / 1e3
                dur.setdefault((r["Kernel_Name"], g), []).append(us)
    mean = lambda v: sum(v) / len(v) if v else float("nan")
    lines = []
    for (name, grid), c in sorted(vals.items(), key=lambda kv: kv[0]):
        f16 = 512.0 * mean(c.get("SQ_INSTS_VALU_MFMA_MOPS_F16", []))
        i8 = 512.0 * mean(c.get("SQ_INSTS_VALU_MFMA_MOPS_I8", []))
        busy, gui = mean(c.get("SQ_VALU_MFMA_BUSY_CYCLES", [])), mean(c.get("GRBM_GUI_ACTIVE", []))
        us = mean(dur.get((name, grid), []))
        short = _short_kernel(name)
        line = f"{short} grid {grid}: us {us:.2f}"
        if f16 > 0:
            line += f" f16_flop {f16:.4g} TFLOP/s {f16 / us / 1e6:.2f} frac_of_fp16_peak {f16 / us / 1e6 / MFMA_PEAK_TFLOPS:.5f}"
        if i8 > 0:
            line += f" i8_op {i8:.4g} TOP/s {i8 / us / 1e6:.2f} frac_of_int8_peak {i8 / us / 1e6 / INT8_PEAK_TOPS:.5f}"
        if busy == busy and gui == gui and gui > 0:
            line += f" mfma_busy_cycles {busy:.4g} gui_active {gui:.4g} mfma_busy_share {busy * 8 / (gui * 1024):.4f}"
        lines.append(line)
    return "\n".join(lines) + "\n"


def traffic_summary(fetch_dir: str, write_dir: str) -> str:
    """Per-kernel mean FETCH_SIZE / WRITE_SIZE (KiB per dispatch), each scaled by
    true bytes / counter bytes of a calibration kernel: the sum (reads
    COPY_BYTES) for FETCH_SIZE, the fill (writes COPY_BYTES) for WRITE_SIZE."""
    import csv
    import glob

    def read(d: str, counter: str) -> dict:
        vals: dict = {}
        for f in glob.glob(str(Path(d) / "**" / "*counter_collection.csv"), recursive=True):
            for r in csv.DictReader(open(f)):
                if r["Counter_Name"] == counter:
                    vals.setdefault(r["Kernel_Name"], []).append(float(r["Counter_Value"]))
        return {k: sum(v) / len(v) for k, v in vals.items()}

    fetch, write = read(fetch_dir, "FETCH_SIZE"), read(write_dir, "WRITE_SIZE")
    fk = [k for k in fetch if "reduce_kernel" in k]
    wk = [k for k in write if "FillFunctor" in k]
    if not fk or not wk:
        raise SystemExit("calibration kernels (sum, fill) missing from the counter runs")
    fk, wk = max(fk, key=lambda k: fetch[k]), max(wk, key=lambda k: write[k])
    f_scale = COPY_BYTES / (fetch[fk] * 1024.0)
    w_scale = COPY_BYTES / (write[wk] * 1024.0)
    lines = [f"calibration_read {COPY_BYTES} bytes: FETCH_SIZE {fetch[fk]:.0f} KiB -> fetch_scale {f_scale:.4f}",
             f"calibration_write {COPY_BYTES} bytes: WRITE_SIZE {write[wk]:.0f} KiB -> write_scale {w_scale:.4f}"]
    for st, key in STAGE_KERNELS.items():
        ks = [k for k in fetch if key in k]
        if not ks:
            continue
        k = ks[0]
        fb = fetch[k] * 1024.0 * f_scale
        wb = write.get(k, 0.0) * 1024.0 * w_scale
        lines.append(f"{st} fetch_bytes {fb:.0f} write_bytes {wb:.0f} traffic_bytes {fb + wb:.0f}")
    return "\n".join(lines) + "\n"


TL_REGION = 65536  # slots per timeline region (csrc/timeline.h)
TL_REGIONS = 32    # 16 per instrumented translation unit (layer.hip, batch.hip)
TL_US = 0.01       # s_memrealtime counts (100 MHz)


def _timeline_step(torch, L, batch: int):
    """Builds the 8B-shape model at `batch`, replays its step graph and yields
    (instrumented step ms, [record of each of three further replays])."""
    import dataclasses

    import numpy as np

    from rtxllm_amd.llama import LLAMA_8B

    shape = dataclasses.replace(LLAMA_8B, batch=batch)
    m, token = build_model(torch, shape)
    stream = torch.cuda.Stream()
    sp = stream.cuda_stream
    p0 = shape.max_ctx - 40
    m.set_token_pos(token, [p0] * batch if batch > 1 else p0)
    m.graph_capture(sp)
    for _ in range(10):
        m.graph_replay(sp)
    torch.cuda.synchronize()
    with torch.cuda.stream(stream):
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record(stream)
        for _ in range(20):
            m.graph_replay(sp)
        e1.record(stream)
    torch.cuda.synchronize()
    step_ms = e0.elapsed_time(e1) / 20
    records = []
    for _ in range(3):
        assert L.rtxllm_timeline_clear() == 0
        torch.cuda.synchronize()
        m.graph_replay(sp)
        torch.cuda.synchronize()
        b = np.zeros(TL_REGIONS * TL_REGION, np.uint64)
        assert L.rtxllm_timeline_read(b.ctypes.data, b.size) == 0
        records.append(b.astype(np.int64))
    m.close()
    return step_ms, records


def _timeline_table(records, roles) -> list:
    """Rows of the kernel-span table: roles = [(name, region, points per wave,
    entry point, end point)]."""
    import numpy as np

    out = ["| replay | stage | waves | first entry | last entry | first end | median end | last end | gap before |",
           "|---|---|---:|---:|---:|---:|---:|---:|---:|"]
    for rep, b in enumerate(records):
        t0 = None
        prev_end = None
        for name, r, k, pe, pd in roles:
            a = b[r * TL_REGION:(r + 1) * TL_REGION].reshape(-1, k)
            a = a[(a[:, pe] > 0) & (a[:, pd] > 0)]
            if t0 is None:
                t0 = a[:, pe].min()
            ent, end = (a[:, pe] - t0) * TL_US, (a[:, pd] - t0) * TL_US
            gap = "" if prev_end is None else f"{ent.min() - prev_end:.2f}"
            out.append(f"| {rep} | {name} | {a.shape[0]} | {ent.min():.2f} | {ent.max():.2f} | {end.min():.2f} | "
                       f"{np.median(end):.2f} | {end.max():.2f} | {gap} |")
            prev_end = end.max()
    return out


def timeline(torch) -> str:
    """Per-wave timeline of one decode step (8B shapes, context ~4050) at
    batch 1 and batch 8, from the profiling build: each kernel role's stamps
    describe its last launch in the step (layer 31, then the LM head). Three
    replays each; times in us from the first wave of the layer's first kernel."""
    import ctypes

    import numpy as np

    from rtxllm_amd import _lib

    _lib.LIB_PATH = _lib.LIB_PATH.with_name("librtxllm_timeline.so")
    L = _lib.lib()
    L.rtxllm_timeline_read.argtypes = [ctypes.c_void_p, ctypes.c_size_t]
    med = lambda v: float(np.median(v)) * TL_US
    reg = lambda b, r, k: b[r * TL_REGION:(r + 1) * TL_REGION].reshape(-1, k)

    step_ms, records = _timeline_step(torch, L, 1)
    out = ["## Batch 1", "", f"instrumented step: {step_ms:.4f} ms (mean of 20 graph replays)", ""]
    out += _timeline_table(records, [("qkv", 3, 2, 0, 1), ("attention partial", 0, 4, 0, 3),
                                     ("attention combine", 1, 4, 0, 2), ("o", 4, 2, 0, 1), ("gate_up", 2, 8, 0, 7),
                                     ("down", 5, 2, 0, 1), ("LM head", 6, 2, 0, 1)])
    out.append("")
    for rep, b in enumerate(records):
        p = reg(b, 0, 4)
        p = p[(p[:, 0] > 0) & (p[:, 1] > 0)]
        c = reg(b, 1, 4)
        c = c[c[:, 0] > 0]
        g = reg(b, 2, 8)
        g = g[g[:, 0] > 0]
        out.append(f"- replay {rep}: attention partial per wave: entry to scores {med(p[:, 1] - p[:, 0]):.2f} "
                   f"(p90 {np.percentile(p[:, 1] - p[:, 0], 90) * TL_US:.2f}), scores to weighted V sum "
                   f"{med(p[:, 2] - p[:, 1]):.2f}, to end (record merge, store) {med(p[:, 3] - p[:, 2]):.2f}; "
                   f"combine per wave: entry to merged {med(c[:, 1] - c[:, 0]):.2f}, staging {med(c[:, 2] - c[:, 1]):.2f}; "
                   f"gate_up per wave: entry to codebook barrier {med(g[:, 1] - g[:, 0]):.2f}, rounds "
                   + ", ".join(f"{med(g[g[:, k + 1] > 0, k + 1] - g[g[:, k + 1] > 0, k]):.2f}" for k in range(1, 5)
                               if (g[:, k + 1] > 0).any()))
        # down: entry / end in region 5, the self-staging point in region 9, same slot
        d = reg(b, 5, 2)
        st = b[9 * TL_REGION:9 * TL_REGION + d.shape[0]]
        ok = (d[:, 0] > 0) & (st > 0)
        if ok.any():
            out.append(f"  down per wave: entry to activation staged {med(st[ok] - d[ok, 0]):.2f} "
                       f"(p90 {np.percentile(st[ok] - d[ok, 0], 90) * TL_US:.2f}), staged to end "
                       f"{med(d[ok, 1] - st[ok]):.2f}")
        lm = reg(b, 6, 2)
        slots = np.nonzero(lm[:, 0] > 0)[0]
        t0 = reg(b, 3, 2)[:, 0]
        t0 = t0[t0 > 0].min()
        wg = slots // 8  # the logits epilogue's slot stride: 8 waves per workgroup
        end = (lm[slots, 1] - t0) * TL_US
        rank = wg // 8   # dispatch rank of the workgroup on its XCD (workgroups go round-robin over 8 XCDs)
        per = max(1, (int(rank.max()) + 1) // 3)
        out.append("  LM head wave ends by dispatch rank within the XCD: " + ", ".join(
            f"ranks {lo}-{lo + per - 1} median {float(np.median(end[(rank >= lo) & (rank < lo + per)])):.2f}"
            for lo in range(0, int(rank.max()) + 1, per)))

    step_ms, records = _timeline_step(torch, L, 8)
    out += ["", "## Batch 8", "", f"instrumented step: {step_ms:.4f} ms (mean of 20 graph replays)", ""]
    out += _timeline_table(records, [("qkv", 16, 16, 0, 15), ("attention partial", 7, 4, 0, 3),
                                     ("attention combine + staging", 8, 2, 0, 1), ("o", 17, 16, 0, 15),
                                     ("residual + norm staging", 21, 2, 0, 1), ("gate_up", 18, 16, 0, 15),
                                     ("down", 19, 16, 0, 15), ("residual + norm staging", 22, 2, 0, 1),
                                     ("LM head", 20, 16, 0, 15)])
    out.append("")
    for rep, b in enumerate(records):
        parts = []
        for name, r in (("qkv", 16), ("o", 17), ("gate_up", 18), ("down", 19), ("LM head", 20)):
            a = reg(b, r, 16)
            a = a[(a[:, 0] > 0) & (a[:, 1] > 0) & (a[:, 2] > 0)]
            tiles = [f"{med(a[a[:, k + 1] > 0, k + 1] - a[a[:, k + 1] > 0, k]):.2f}" for k in range(2, 14)
                     if (a[:, k + 1] > 0).any()]
            parts.append(f"{name}: entry to codebook barrier {med(a[:, 1] - a[:, 0]):.2f}, to RMSNorm scale "
                         f"{med(a[:, 2] - a[:, 1]):.2f}, tiles " + ", ".join(tiles))
        p = reg(b, 7, 4)
        p = p[(p[:, 0] > 0) & (p[:, 1] > 0)]
        parts.append(f"attention partial: entry to scores {med(p[:, 1] - p[:, 0]):.2f}, to weighted V sum "
                     f"{med(p[:, 2] - p[:, 1]):.2f}, to end {med(p[:, 3] - p[:, 2]):.2f}")
        out.append(f"- replay {rep} per wave (medians): " + "; ".join(parts))
    return "\n".join(out) + "\n"


def _short_kernel(name: str) -> str:
    """Readable kernel name: namespaces and parameter lists dropped. Names the
    profiler left mangled (those with _Float16 parameters) are read as
    _ZN <len><id>... [I Li<n>E... E]: the last identifier plus its integer
    template arguments."""
    import re

    if name.startswith("_ZN"):
        i, ident = 3, ""
        while i < len(name) and name[i].isdigit():
            m = re.match(r"\d+", name[i:])
            n = int(m.group(0))
            i += len(m.group(0))
            ident = name[i:i + n]
            i += n
        targs = re.match(r"I((?:Li\d+E)+)E", name[i:])
        if targs:
            ident += "<" + ", ".join(re.findall(r"Li(\d+)E", targs.group(1))) + ">"
        return ident
    n = re.sub(r"rtxllm::\(anonymous namespace\)::|rtxllm::", "", name).replace("void ", "")
    return n.split("(")[0] if "(" in n else n


def trace_summary(trace_dir: str) -> str:
    """Per-kernel count / mean / min / max launch time (us) and share of GPU time
    from the kernel trace of one run. The batch-1 and batch-8 steps launch the
    same attention and argmax kernels; their launches are told apart by the grid
    dimension that counts sequences (attention partials: z, combine: y,
    argmax finalize: x / 256)."""
    import csv
    import glob
    import statistics

    rows: dict = {}
    for f in glob.glob(str(Path(trace_dir) / "**" / "*kernel_trace.csv"), recursive=True):
        for r in csv.DictReader(open(f)):
            name = _short_kernel(r["Kernel_Name"])
            gx, gy, gz = int(r["Grid_Size_X"]), int(r["Grid_Size_Y"]), int(r["Grid_Size_Z"])
            seqs = None
            if name.startswith("attn_partial"):
                seqs = gz
            elif name.startswith("attn_combine"):
                seqs = gy
            elif name.startswith("argmax_finalize"):
                seqs = max(1, gx // 256)
            if seqs is not None:
                name += f" (batch {seqs})"
            rows.setdefault(name, []).append((int(r["End_Timestamp"]) - int(r["Start_Timestamp"])) / 1e3)
    if not rows:
        raise SystemExit(f"no kernel trace under {trace_dir}")
    total = sum(sum(v) for v in rows.values())
    lines = ["| kernel | calls | avg us | min us | max us | % of GPU time |", "|---|---:|---:|---:|---:|---:|"]
    for k, v in sorted(rows.items(), key=lambda kv: -sum(kv[1])):
        if sum(v) / total < 0.002:
            continue
        lines.append(f"| `{k}` | {len(v)} | {statistics.mean(v):.2f} | {min(v):.2f} | {max(v):.2f} | "
                     f"{100 * sum(v) / total:.2f} |")
    return "\n".join(lines) + "\n"


ENGINE_CLOCK_GHZ = 2.4     # MI355X peak engine clock
SIMDS = 256 * 4            # 256 CUs x 4 SIMDs
VALU_CYCLES_PER_OP = 4     # a wave64 VALU instruction on a 16-lane SIMD
STAGE_UNITS = {  # 32-value weight units per launch at the 8B shapes (rows x cols / 32)
    "qkv": 6144 * 4096 // 32, "o": 4096 * 4096 // 32, "gate_up": 28672 * 4096 // 32,
    "down": 4096 * 14336 // 32, "lm_head": 128256 * 4096 // 32,
}
STAGE_BYTES = {"qkv": 10854400, "attention": 16672768, "o": 7241728, "gate_up": 37748736, "down": 33103872,
               "lm_head": 361698304}  # layer_weight_bytes at the 8B shapes; attention: K + V at ~4070 positions


def counter_summary(pmc_dirs) -> str:
    """Per decode-stage kernel, the mean per dispatch of every SQ counter found
    in the given --pmc runs of --traffic-probe (batch-1 stages) or --mfma-probe
    (also the batch-8 matrix-core stages, rows "<stage>_b8"), and derived
    figures: instructions per wave; per 64 weight units (one unit per lane: a
    wave's pass over 64 units), which is the cost per pass of the batch-1
    matvecs; wait / VALU-active shares of wave cycles; LDS bank conflicts per
    LDS-active cycle. The VALU floor is the time the SIMDs need to issue the
    launch's VALU instructions (4 cycles each on 1024 SIMDs at 2.4 GHz; the
    count includes the MFMA instructions, which occupy their pipe longer); the
    budget is the time of the launch's algorithmic bytes at 70 % of 8 TB/s."""
    import csv
    import glob

    kernels = {**STAGE_KERNELS, **{st + "_b8": k for st, k in BATCH8_STAGE_KERNELS.items()}}
    vals: dict = {}
    for d in pmc_dirs:
        for f in glob.glob(str(Path(d) / "**" / "*counter_collection.csv"), recursive=True):
            for r in csv.DictReader(open(f)):
                for st, key in kernels.items():
                    if key in r["Kernel_Name"]:
                        vals.setdefault(st, {}).setdefault(r["Counter_Name"], []).append(float(r["Counter_Value"]))
    if not vals:
        raise SystemExit("no decode stage kernel in the counter runs")
    lines = []
    for st in kernels:
        if st not in vals:
            continue
        c = {k: sum(v) / len(v) for k, v in vals[st].items()}
        base = st[:-3] if st.endswith("_b8") else st
        parts = [st] + [f"{k} {c[k]:.0f}" for k in sorted(c)]
        waves = c.get("SQ_WAVES")
        if waves:
            for k in ("SQ_INSTS_VALU", "SQ_INSTS_LDS", "SQ_INSTS_SALU", "SQ_INSTS_VMEM_RD", "SQ_INSTS_SMEM"):
                if k in c:
                    parts.append(f"{k.replace('SQ_INSTS_', '').lower()}_per_wave {c[k] / waves:.1f}")
        if st in STAGE_UNITS:  # batch 1 only
            passes = STAGE_UNITS[st] / 64.0
            for k in ("SQ_INSTS_VALU", "SQ_INSTS_LDS", "SQ_INSTS_SALU", "SQ_INSTS_VMEM_RD"):
                if k in c:
                    parts.append(f"{k.replace('SQ_INSTS_', '').lower()}_per_64_units {c[k] / passes:.1f}")
        if "SQ_WAVE_CYCLES" in c and c["SQ_WAVE_CYCLES"] > 0:
            for k in ("SQ_WAIT_ANY", "SQ_WAIT_INST_ANY", "SQ_ACTIVE_INST_ANY", "SQ_ACTIVE_INST_VALU",
                      "SQ_ACTIVE_INST_VMEM", "SQ_WAIT_INST_LDS", "SQ_ACTIVE_INST_LDS"):
                if k in c:
                    parts.append(f"{k.replace('SQ_', '').lower()}_share {c[k] / c['SQ_WAVE_CYCLES']:.3f}")
        if c.get("SQ_ACTIVE_INST_LDS"):
            if "SQ_LDS_BANK_CONFLICT" in c:
                parts.append(f"lds_conflict_per_active {c['SQ_LDS_BANK_CONFLICT'] / c['SQ_ACTIVE_INST_LDS']:.3f}")
        if "SQ_INSTS_VALU" in c:
            floor = c["SQ_INSTS_VALU"] * VALU_CYCLES_PER_OP / (ENGINE_CLOCK_GHZ * 1e3 * SIMDS)
            budget = STAGE_BYTES[base] / (0.7 * HBM_PEAK_GBS * 1e3)
            parts.append(f"valu_floor_us {floor:.2f} budget_us_at_70pct {budget:.2f}")
        lines.append(" ".join(parts))
    return "\n".join(lines) + "\n"


def traffic_of(stage: str):
    """HBM bytes per launch of a stage from the committed counter summary, or None."""
    try:
        for line in TRAFFIC_FILE.read_text().splitlines():
            parts = line.split()
            if parts and parts[0] == stage and "traffic_bytes" in parts:
                return int(parts[parts.index("traffic_bytes") + 1])
    except OSError:
        pass
    return None


# ---- matvec set -----------------------------------------------------------------

def time_matvec(torch, stream, fmt: int, rows: int, cols: int, seed: int) -> tuple[float, int, int]:
    """Mean us of one batch-1 matvec (staged x) over rotating weight copies
    spanning more than twice the MALL, so every launch reads HBM; also the
    copy count and the layout's resident bytes."""
    from rtxllm_amd import ops, packs

    dev = "cuda:0"
    pack = packs.make_pack(fmt, rows, cols, seed)
    base = ops.DevicePack(pack, dev)
    nbytes = pack.payload.nbytes + (pack.meta.nbytes if pack.meta is not None else 0)
    copies = [base]
    while len(copies) * nbytes < 2 * MALL_BYTES + nbytes:
        c = ops.DevicePack.__new__(ops.DevicePack)
        c.fmt, c.rows, c.cols = base.fmt, base.rows, base.cols
        c.payload = base.payload.clone()
        c.meta = base.meta.clone() if base.meta is not None else None
        copies.append(c)
    xq = ops.stage(ops.to_dev(packs.normal_f32(seed + 0x100, cols), dev))
    y = torch.empty(rows, dtype=torch.float32, device=dev)
    ms = time_graph(torch, stream, lambda: [ops.matvec_xq(c, xq, y) for c in copies], reps=5)
    n = len(copies)
    del copies, base
    torch.cuda.empty_cache()
    return ms * 1e3 / n, n, nbytes


def matvec_set_bench(torch) -> dict:
    from rtxllm_amd import formats as F

    stream = torch.cuda.Stream()
    per = {}
    for name, fmt, rows, cols, seed in MATVECS:
        us, n, _ = time_matvec(torch, stream, fmt, rows, cols, seed)
        ab = F.algorithmic_bytes(fmt, rows, cols)
        per[name] = {"us": round(us, 3), "GB/s": round(ab / us / 1e3, 1),
                     "frac": round(ab / us / 1e3 / HBM_PEAK_GBS, 4), "copies": n}
    tot_b = sum(F.algorithmic_bytes(f, r, c) for _, f, r, c, _ in MATVECS)
    tot_us = sum(v["us"] for v in per.values())
    return {"per_matvec": per, "GB/s": round(tot_b / tot_us / 1e3, 1),
            "frac": round(tot_b / tot_us / 1e3 / HBM_PEAK_GBS, 4)}


Q4K_LAYOUTS = {"raw": 0, "split-predecoded": 1, "split-half": 2, "split-compact": 3, "split-native": 4,
               "raw-predecoded": 8}
Q4K_SWEEP_SHAPES = [(4096, 4096), (14336, 4096), (4096, 14336)]


def q4k_sweep(torch) -> dict:
    """Every Q4_K resident layout at the config shapes: us, algorithmic GB/s
    (144 B per block) and resident bytes; the fastest layout per shape is the
    MI355X pack policy (rtxllm_amd.manifest.auto_policy)."""
    from rtxllm_amd import formats as F

    stream = torch.cuda.Stream()
    out = {}
    for rows, cols in Q4K_SWEEP_SHAPES:
        ab = F.algorithmic_bytes(F.Q4K_RAW, rows, cols)
        row = {}
        for name, fmt in Q4K_LAYOUTS.items():
            us, _, nbytes = time_matvec(torch, stream, fmt, rows, cols, 0x5EED0001)
            row[name] = {"us": round(us, 3), "GB/s": round(ab / us / 1e3, 1), "resident_bytes": int(nbytes)}
        best = min(row, key=lambda k: row[k]["us"])
        out[f"{rows}x{cols}"] = {"blocks": rows * cols // 256, "layouts": row, "fastest": best}
    return out


UNIT_SWEEP = [("gate_up", 6, 9, 28672, 4096), ("iq2s_14336x4096", 6, 9, 14336, 4096),
              ("qkv", 7, 10, 6144, 4096), ("o", 7, 10, 4096, 4096)]


def units_sweep(torch) -> dict:
    """Batch-1 matvec (staged x, HBM-cold) of each IQ decode shape in the GGUF
    layout and in its unit layout (IQ2S_UNITS / IQ3S_UNITS): us and GB/s of the
    GGUF bytes, and the unit layout's resident bytes."""
    from rtxllm_amd import formats as F

    stream = torch.cuda.Stream()
    out = {}
    for name, fmt, ufmt, rows, cols in UNIT_SWEEP:
        ab = F.algorithmic_bytes(fmt, rows, cols)
        us, _, _ = time_matvec(torch, stream, fmt, rows, cols, 0x5EED0001)
        uus, _, ubytes = time_matvec(torch, stream, ufmt, rows, cols, 0x5EED0001)
        out[name] = {"shape": f"{rows}x{cols}", "gguf_us": round(us, 3), "gguf_GBps": round(ab / us / 1e3, 1),
                     "units_us": round(uus, 3), "units_GBps": round(ab / uus / 1e3, 1),
                     "units_resident_bytes": int(ubytes), "gguf_bytes": int(ab), "speedup": round(us / uus, 3)}
    return out


READ_MODES = {0: "grid-stride x4", 1: "grid-stride x8", 2: "chunk per workgroup x4"}
READ_SIZES = {"o": 7241728, "qkv": 10854400, "attention": 16777216, "iq2s_14336x4096": 18882560,
              "down": 33103872, "gate_up": 37748736, "lm_head": 361698304}


def read_ceiling(torch) -> dict:
    """What a plain streaming read of the same bytes takes on this GPU
    (rtxllm_stream_read: 16-byte nontemporal loads; the best of three access
    patterns, grid-stride with four or eight loads in flight per lane or one
    contiguous chunk per workgroup, at five grid sizes), one launch per buffer
    over rotating buffers spanning more than twice the MALL (HBM-cold), in a
    hipGraph like the stages."""
    from rtxllm_amd._lib import check, probe_lib

    stream = torch.cuda.Stream()
    sp = stream.cuda_stream
    out = {}
    for name, nbytes in READ_SIZES.items():
        k = max(2, (2 * MALL_BYTES) // nbytes + 1)
        bufs = [torch.ones(nbytes // 4, dtype=torch.int32, device="cuda:0") for _ in range(k)]
        res = torch.empty(16384, dtype=torch.int32, device="cuda:0")
        best = None
        for mode in READ_MODES:
            for grid in (512, 1024, 2048, 4096, 8192):
                def run(grid=grid, mode=mode):
                    for b in bufs:
                        check("rtxllm_stream_read", probe_lib().rtxllm_stream_read(b.data_ptr(), nbytes, res.data_ptr(),
                                                                              grid, mode, sp))

                us = time_graph(torch, stream, run, reps=5) * 1e3 / k
                best = (us, grid, mode) if best is None or us < best[0] else best
        us, grid, mode = best
        out[name] = {"bytes": nbytes, "us": round(us, 3), "GB/s": round(nbytes / us / 1e3, 1),
                     "frac": round(nbytes / us / 1e3 / HBM_PEAK_GBS, 4), "workgroups": grid,
                     "pattern": READ_MODES[mode]}
        del bufs, res
        torch.cuda.empty_cache()
    return out


# ---- CPU baseline -------------------------------------------------------------

def cpu_info() -> dict:
    """Host CPU model, sockets, cores and threads (lscpu when present), and the
    CPUs this process may run on."""
    import subprocess

    info = {"model": _cpu_model(), "online_cpus": os.cpu_count()}
    try:
        info["usable_cpus"] = len(os.sched_getaffinity(0))
    except (AttributeError, OSError):
        pass
    try:
        out = subprocess.run(["lscpu"], capture_output=True, text=True, timeout=20).stdout
        for line in out.splitlines():
            k, _, v = line.partition(":")
            k = k.strip()
            if k in ("Model name", "Socket(s)", "Core(s) per socket", "Thread(s) per core", "CPU(s)", "CPU max MHz",
                     "L3 cache"):
                info["lscpu " + k] = v.strip()
    except (OSError, subprocess.SubprocessError):
        pass
    return info


def cpu_baseline() -> dict:
    """The oracle (scalar fp32 per-element dequant, sequential accumulation: the
    reference gate's algorithm) on the host: one full decode step of the
    32-layer 8B-shape model (embedding row, 32 layers at 4096 context, final
    norm, Q5_K LM head, argmax) row-parallel on every usable host thread (each
    row keeps its sequential order, so the outputs equal the 1-thread ones), and
    one full layer on one thread. Distinct seeded weights per layer, so no
    layer's 88 MB of packs is cache-resident when the next starts."""
    import ctypes

    import numpy as np

    from oracle import binding as orc
    from rtxllm_amd import formats as F
    from rtxllm_amd import packs
    from rtxllm_amd.llama import HEAD_DIM, LLAMA_8B, tensor_seed

    s = LLAMA_8B
    lib, P = orc.lib(), orc.ptr
    H, q, kv, ff = s.hidden, s.n_heads * HEAD_DIM, s.n_kv_heads * HEAD_DIM, s.ffn
    try:
        threads = len(os.sched_getaffinity(0))
    except (AttributeError, OSError):
        threads = os.cpu_count() or 1
    threads = max(1, min(64, threads))
    rb = (H // 256) * 110
    inv_freq = np.empty(HEAD_DIM // 2, np.float32)
    lib.orc_rope_inv_freq(HEAD_DIM, s.rope_theta, P(inv_freq))
    shape = orc.LayerShape(H, s.n_heads, s.n_kv_heads, HEAD_DIM, ff, s.rms_eps, P(inv_freq))
    n = (s.max_ctx // s.page_size) * s.n_kv_heads * s.page_size * HEAD_DIM
    table = np.arange(s.max_ctx // s.page_size, dtype=np.int32)
    layers = []
    for l in range(s.n_layers):
        qkv = packs.make_pack(F.IQ3S, q + 2 * kv, H, tensor_seed(SEED, l, "qkv")).payload
        gu = packs.make_pack(F.IQ2S, 2 * ff, H, tensor_seed(SEED, l, "gate_up")).payload.reshape(ff, 2, -1)
        d = {"wq": qkv[:q * rb], "wk": qkv[q * rb:(q + kv) * rb], "wv": qkv[(q + kv) * rb:],
             "wo": packs.make_pack(F.IQ3S, H, q, tensor_seed(SEED, l, "o")).payload,
             "wg": np.ascontiguousarray(gu[:, 0]).ravel(), "wu": np.ascontiguousarray(gu[:, 1]).ravel(),
             "dn": packs.make_pack(F.Q4K_SPLIT_NATIVE, H, ff, tensor_seed(SEED, l, "down")),
             "an": packs.normal_f32(SEED + 100 + 2 * l, H, mean=1.0, std=0.02),
             "fn": packs.normal_f32(SEED + 101 + 2 * l, H, mean=1.0, std=0.02),
             "kc": packs.normal_f16_bits(SEED + 300 + 2 * l, n), "vc": packs.normal_f16_bits(SEED + 301 + 2 * l, n)}
        d["w"] = orc.LayerWeights(F.IQ3S, F.IQ3S, F.IQ3S, F.IQ3S, F.IQ2S, F.IQ2S, F.Q4K_SPLIT_NATIVE,
                                  P(d["wq"]), None, P(d["wk"]), None, P(d["wv"]), None, P(d["wo"]), None, P(d["wg"]),
                                  None, P(d["wu"]), None, P(d["dn"].payload), P(d["dn"].meta), P(d["an"]), P(d["fn"]))
        d["cache"] = orc.KvCache(P(d["kc"]), P(d["vc"]), P(table), s.page_size, s.n_kv_heads, HEAD_DIM)
        layers.append(d)
    embed = packs.make_pack(F.Q5K, s.vocab, H, tensor_seed(SEED, None, "embed")).payload
    lm = packs.make_pack(F.Q5K, s.vocab, H, tensor_seed(SEED, None, "lm_head")).payload
    out_norm = packs.normal_f32(SEED + 99, H, mean=1.0, std=0.02)
    pos = s.max_ctx - 1

    def layer(l: int, h: np.ndarray, nthreads: int) -> None:
        d = layers[l]
        lib.orc_layer_forward(ctypes.byref(d["w"]), ctypes.byref(shape), ctypes.byref(d["cache"]), pos, P(h),
                              nthreads)

    # one full layer on one thread (the reference gate's own mode)
    h1 = packs.normal_f32(SEED + 7, H)
    t0 = time.perf_counter()
    layer(0, h1, 1)
    t_layer1 = time.perf_counter() - t0
    # the full step on every usable thread
    t0 = time.perf_counter()
    h = np.empty(H, np.float32)
    lib.orc_embed_q5k(P(embed), H, 1234, P(h))
    t_layers = []
    for l in range(s.n_layers):
        tl = time.perf_counter()
        layer(l, h, threads)
        t_layers.append(time.perf_counter() - tl)
    xn = np.empty(H, np.float32)
    lib.orc_rmsnorm_weighted(P(h), P(out_norm), H, s.rms_eps, P(xn))
    th = time.perf_counter()
    logits = orc.matvec_f32(F.Q5K, lm, None, xn, s.vocab, H, threads)
    t_head = time.perf_counter() - th
    token = orc.argmax(logits)
    t_step = time.perf_counter() - t0
    est1 = s.n_layers * t_layer1 + t_head * threads  # 1-thread step, from the measured layer (head scaled)
    return {
        "value": round(1.0 / t_step, 5),
        "unit": "tok/s",
        "cores": threads,
        "kind": "port",
        "sample": (f"oracle (scalar restatement of the reference CPU gate: per-element dequant, sequential fp32 "
                   f"accumulation) on one full decode step of the 32-layer 8B-shape model at context {pos + 1}: "
                   f"embedding row, 32 layers (distinct weights), final norm, Q5_K LM head, argmax (token {token}); "
                   f"{threads} threads row-parallel, {t_step:.1f} s (layers {sum(t_layers):.1f} s, "
                   f"head {t_head:.2f} s)"),
        "single_thread": {"layer_s": round(t_layer1, 3), "unit": "s per layer (one full 8B layer, 1 thread)",
                          "step_estimate_tok_s": round(1.0 / est1, 5)},
        "host": cpu_info(),
    }


def main() -> int:
    args = parse()
    if args.gpus != 1:
        print(json.dumps({"error": "bench.py measures one GPU only; run with --gpus 1 (multi-GPU is design-only)"}))
        return 2
    if args.traffic_summary:
        sys.stdout.write(traffic_summary(*args.traffic_summary))
        return 0
    if args.mfma_summary:
        sys.stdout.write(mfma_summary(*args.mfma_summary))
        return 0
    if args.counter_summary:
        sys.stdout.write(counter_summary(args.counter_summary))
        return 0
    if args.trace_summary:
        sys.stdout.write(trace_summary(args.trace_summary))
        return 0
    import torch

    torch.cuda.set_device(0)
    if args.traffic_probe:
        traffic_probe(torch)
        return 0
    if args.mfma_probe:
        mfma_probe(torch)
        return 0
    if args.timeline:
        sys.stdout.write(timeline(torch))
        return 0
    if args.read_ceiling:
        print(json.dumps({"read_ceiling": read_ceiling(torch)}), flush=True)
        return 0
    if args.q4k_sweep:
        print(json.dumps({"q4k_sweep": q4k_sweep(torch)}), flush=True)
        return 0
    if args.units_sweep:
        print(json.dumps({"units_sweep": units_sweep(torch)}), flush=True)
        return 0
    dec = decode_bench(torch, args)
    dom = dec["stages"][dec["dominant"]]
    out = {
        "metric": "batch-1 decode tok/s, 32-layer mixed-quant 8B shapes (matvec HBM GB/s, % of peak)",
        "value": round(dec["tok_s"], 2),
        "unit": "tok/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(dec["ms_per_step"], 5),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f32 activations staged to 22-bit block fixed point per 16 values (3 int8 digits), exact int32 "
                 "dot4 with the weight codes, f32 scales and accumulation",
        "data": "synthetic: random-init seeded GGUF packs (splitmix64), norms 1+N(0,0.02), fp16 KV ~ N(0,1)",
        "config": {"workload": "llama-8B-shape decode step: 32 layers (q/k/v/o IQ3_S, gate/up IQ2_S, down Q4_K "
                               "split-native), Q5_K embed + LM head (vocab 128256), GQA 32/8 x 128, "
                               f"paged fp16 KV, context ~{int(dec['mean_context'])}, greedy argmax, one hipGraph",
                   "batch": 1, "launches_per_step": dec["launches"], "wall_s": round(dec["wall_s"], 4)},
        "latency": dec["latency"],
        "step_hbm_GBps": round(dec["GB/s"], 1),
        "step_frac_of_hbm_peak": round(dec["GB/s"] / HBM_PEAK_GBS, 4),
        "step_algorithmic_bytes": int(dec["step_bytes"]),
        "stages": dec["stages"],
        "roofline": {"bound": "hbm", "kernel": dec["dominant"], "achieved": dom["GB/s"], "peak": HBM_PEAK_GBS,
                     "unit": "GB/s", "frac": dom["frac"], "traffic": traffic_of(dec["dominant"]),
                     "algorithmic_bytes": dom["bytes"], "us_per_launch": dom["us"]},
    }
    if dec["context_buckets"] is not None:
        out["context_buckets"] = dec["context_buckets"]
    if not args.no_batch8:
        b8 = decode_bench(torch, args, batch=8)
        out["batch8"] = {
            "workload": "the same decode step for 8 sequences at once (one pass over the weights on the matrix "
                        "cores, every sequence with its own token, position and KV pages, context ~"
                        f"{int(b8['mean_context'])} each), one hipGraph",
            "tok_s": round(b8["tok_s"], 2), "ms_per_step": round(b8["ms_per_step"], 5), "latency": b8["latency"],
            "step_hbm_GBps": round(b8["GB/s"], 1), "step_frac_of_hbm_peak": round(b8["GB/s"] / HBM_PEAK_GBS, 4),
            "step_algorithmic_bytes": int(b8["step_bytes"]), "launches_per_step": b8["launches"],
            "dtype": "fp16 weight codes x sub-block scale (exact) times hi+lo fp16 activations on the matrix "
                     "cores, f32 accumulate",
            "stages": b8["stages"],
        }
        if b8["context_buckets"] is not None:
            out["batch8"]["context_buckets"] = b8["context_buckets"]
    if not args.no_read_ceiling:
        ceil = read_ceiling(torch)
        out["read_ceiling"] = ceil
        for st, v in out["stages"].items():
            if st in ceil and abs(ceil[st]["bytes"] - v["bytes"]) <= 0.02 * v["bytes"]:  # attention: 4096 positions
                v["read_ceiling_us"] = ceil[st]["us"]
                v["frac_of_read_ceiling"] = round(ceil[st]["us"] / v["us"], 4)
        dom_c = ceil.get(dec["dominant"])
        if dom_c is not None:
            out["roofline"]["read_ceiling_GBps"] = dom_c["GB/s"]
    if not args.no_matvec_set:
        out["matvec_set"] = matvec_set_bench(torch)
    if not args.no_cpu_baseline:
        out["cpu_baseline"] = cpu_baseline()
    print(json.dumps(out), flush=True)
    return 0


if __name__ == "__main__":
    raise SystemExit(main())
