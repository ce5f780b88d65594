"""Decode hot-path benchmark on one MI355X.

Workload (one "step"): the batch-1 mixed-quant matvec set at the 8B FFN
shapes -- Q4_K (split-native) and Q5_K at 14336x4096 and 4096x14336, IQ2_S and
IQ3_S at both shapes, plus the Q4_K 4096x4096 matvec -- each read from HBM
(weights rotate over >= 2x the 256 MB Infinity Cache so no launch hits a warm
copy), replayed as one hipGraph. value = algorithmic bytes / kernel time.

Prints one JSON line (the driver's contract). The cpu_baseline leg times the
oracle (the reference gate's scalar restatement) on a bounded sample.
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


def parse() -> argparse.Namespace:
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=50)
    ap.add_argument("--warmup", type=int, default=5)
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--cpu-seconds", type=float, default=10.0)
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


def cpu_baseline(seconds: float) -> dict:
    """Oracle (scalar fp32, per-element dequant, sequential accumulation -- the
    reference gate's algorithm) on the same packs, one thread, for ~`seconds`."""
    import numpy as np

    from oracle import binding as orc
    from rtxllm_amd import formats as F
    from rtxllm_amd import packs

    orc.lib()
    total_bytes, total_t, done = 0, 0.0, []
    rows_sample = 1024
    for name, fmt, rows, cols, seed in MATVECS:
        if total_t >= seconds:
            break
        pack = packs.make_pack(fmt, rows_sample, cols, seed)
        x = packs.normal_f32(seed + 0x100, cols)
        t0 = time.perf_counter()
        orc.matvec_f32(fmt, pack.payload, pack.meta, x, rows_sample, cols, 1)
        dt = time.perf_counter() - t0
        total_t += dt
        total_bytes += F.algorithmic_bytes(fmt, rows_sample, cols)
        done.append(f"{name}[:{rows_sample}]")
    nthreads = min(os.cpu_count() or 1, 16)
    pack = packs.make_pack(4, 4096, 4096, 0x5EED0000)
    x = packs.normal_f32(0x5EED0100, 4096)
    t0 = time.perf_counter()
    orc.matvec_f32(4, pack.payload, pack.meta, x, 4096, 4096, nthreads)
    mt = time.perf_counter() - t0
    return {
        "value": round(total_bytes / total_t / 1e9, 4),
        "unit": "GB/s",
        "cores": 1,
        "kind": "port",
        "sample": "oracle fp32 scalar matvec, first 1024 rows of each of: " + ", ".join(done),
        "multithread": {"threads": nthreads, "GB/s": round(F.algorithmic_bytes(4, 4096, 4096) / mt / 1e9, 4),
                        "sample": "q4k_native_4096x4096 full"},
        "cpu_model": _cpu_model(),
    }


def _cpu_model() -> str:
    try:
        for line in Path("/proc/cpuinfo").read_text().splitlines():
            if line.startswith("model name"):
                return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return "unknown"


def main() -> int:
    args = parse()
    if args.gpus != 1:
        print(json.dumps({"error": "this build measures one GPU only; run with --gpus 1"}))
        return 2
    import torch

    from rtxllm_amd import formats as F
    from rtxllm_amd import ops, packs

    torch.cuda.set_device(0)
    dev = "cuda:0"
    runs = []  # (name, fmt, rows, cols, [DevicePack copies], x, y)
    for name, fmt, rows, cols, seed in MATVECS:
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
        x = ops.to_dev(packs.normal_f32(seed + 0x100, cols), dev)
        xq = ops.stage(x)
        y = torch.empty(rows, dtype=torch.float32, device=dev)
        runs.append((name, fmt, rows, cols, copies, (x, xq), y))

    # One step = every matvec once; successive steps rotate the weight copies.
    n_rot = max(len(r[4]) for r in runs)

    def launch_step(k: int) -> None:
        # every activation is staged once per step, then each matvec reads it
        for _, _, _, _, _, (x, xq), _ in runs:
            ops.stage(x, out=xq)
        for _, _, _, _, copies, (x, xq), y in runs:
            ops.matvec_xq(copies[k % len(copies)], xq, y)

    stream = torch.cuda.Stream()
    with torch.cuda.stream(stream):
        for k in range(n_rot):
            launch_step(k)
    torch.cuda.synchronize()

    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph, stream=stream):
        for k in range(n_rot):
            launch_step(k)
    torch.cuda.synchronize()

    # Per-matvec kernel time: one graph per matvec over its copies.
    per = {}
    for name, fmt, rows, cols, copies, (x, xq), y in runs:
        g = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g, stream=stream):
            for c in copies:
                ops.matvec_xq(c, xq, y)
        torch.cuda.synchronize()
        for _ in range(2):
            g.replay()
        torch.cuda.synchronize()
        reps = 20
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        with torch.cuda.stream(stream):
            e0.record(stream)
            for _ in range(reps):
                g.replay()
            e1.record(stream)
        torch.cuda.synchronize()
        us = e0.elapsed_time(e1) * 1e3 / (reps * len(copies))
        ab = F.algorithmic_bytes(fmt, rows, cols)
        per[name] = {"us": round(us, 3), "GB/s": round(ab / us / 1e3, 1), "frac": round(ab / us / 1e3 / HBM_PEAK_GBS, 4),
                     "algorithmic_bytes": ab, "copies": len(copies)}

    for _ in range(args.warmup):
        graph.replay()
    torch.cuda.synchronize()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    replays = max(1, args.steps // n_rot)
    steps = replays * n_rot
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    with torch.cuda.stream(stream):
        e0.record(stream)
        for _ in range(replays):
            graph.replay()
        e1.record(stream)
    torch.cuda.synchronize()
    wall = time.perf_counter() - t0
    ms_step = e0.elapsed_time(e1) / steps
    step_bytes = sum(F.algorithmic_bytes(r[1], r[2], r[3]) for r in runs)
    value = step_bytes / (ms_step * 1e-3) / 1e9

    dom = max(per, key=lambda n: per[n]["us"])
    out = {
        "metric": "mixed-quant matvec HBM GB/s (batch 1, 8B FFN shapes)",
        "value": round(value, 2),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms_step, 5),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "int8 dot4 (weight codes x 2-digit int8 activation) + f32 scales",
        "data": "synthetic seeded packs (splitmix64), x ~ N(0,1)",
        "config": {"workload": "matvec set: " + ", ".join(r[0] for r in runs), "batch": 1,
                   "wall_s": round(wall, 3)},
        "frac_of_hbm_peak": round(value / HBM_PEAK_GBS, 4),
        "per_matvec": per,
        "roofline": {"bound": "hbm", "kernel": dom, "achieved": per[dom]["GB/s"], "peak": HBM_PEAK_GBS,
                     "unit": "GB/s", "frac": per[dom]["frac"], "traffic": None},
    }
    if not args.no_cpu_baseline:
        out["cpu_baseline"] = cpu_baseline(args.cpu_seconds)
    print(json.dumps(out), flush=True)
    return 0


if __name__ == "__main__":
    raise SystemExit(main())
