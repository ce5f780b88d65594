"""Pack writer for tensors held in memory (a model's own weights, synthetic
blocks): the pack files and manifest.json records of the reference's pack
producers (tools/bench/q4k_resident_pack.py:170-222 for Q4_K,
iq_resident_pack.py:115-147 for IQ2_S / IQ3_S, q5k_resident_pack.py:93-120 for
Q5_K, with their runtime_kernel labels and file labels), plus a GGUF tensor
plan (tools/bench/gguf_tensor_plan.py: name, type, dimensions, span_bytes,
absolute_offset). GGUF files are packed by the library's C++ producer
(producer.pack_gguf); this writer serves callers without a file. It writes
two manifests, Q4_K and raw blocks (IQ2_S / IQ3_S / Q5_K together, which the
raw-block loader accepts), read back through rtxllm_llama_load_packs
(include/rtxllm/pack_manifest.h loaders).

Q4_K tensors get the payload + metadata streams of one split layout (the
policy) and, with write_blocks, the raw blocks file. Checksums are byte sums;
pack paths are written relative to out_dir (the runner takes out_dir as the
payload root) unless absolute_paths.
"""

from __future__ import annotations

import json
import re
from dataclasses import dataclass
from pathlib import Path

import numpy as np

from . import formats as F
from . import packs

# Q4_K pack policy -> (split format, metadata_format label) (q4k_resident_pack.py:82-97)
Q4K_POLICIES = {
    "split-predecoded": (F.Q4K_SPLIT_PREDECODED, "fp32-products"),
    "split-half": (F.Q4K_SPLIT_HALF, "fp16-products"),
    "split-compact": (F.Q4K_SPLIT_COMPACT, "compact-u8"),
    "split-native": (F.Q4K_SPLIT_NATIVE, "native16"),
}
RAW_TYPES = {F.IQ2S: "IQ2_S", F.IQ3S: "IQ3_S", F.Q5K: "Q5_K"}


def auto_policy(rows: int, cols: int, lossy: bool = False) -> str:
    """The Q4_K pack layout for a rows x cols tensor on MI355X, from the layout
    sweep (bench.py --q4k-sweep, HBM-cold, at 4096x4096, 14336x4096 and
    4096x14336): split-native (the raw 16-byte head beside the quants) is the
    fastest exact layout at every shape; split-half (fp16 products, lossy) is
    4-7 % faster above 65536 blocks and is chosen only when lossy layouts are
    allowed. The reference's auto policy (q4k_resident_pack.py:75-79: compact
    up to 4096 blocks, else predecoded) is an RTX 3060 measurement; on MI355X
    both are slower than split-native."""
    return "split-half" if lossy and rows * cols // F.BLOCK_VALUES > 65536 else "split-native"
# runtime_kernel of the raw-block producers (iq_resident_pack.py:124-127, q5k_resident_pack.py:119)
KERNEL_LABELS = {"IQ2_S": "iq2s_raw_block_probe", "IQ3_S": "iq3s_raw_block_probe", "Q5_K": "q5_k_raw_pending"}


@dataclass
class Tensor:
    """One GGUF tensor: W[rows][cols] as raw GGUF blocks of format fmt (Q4K_RAW,
    IQ2S, IQ3S or Q5K)."""
    name: str
    fmt: int
    rows: int
    cols: int
    blocks: np.ndarray  # uint8, rows * cols / 256 blocks
    offset: int | None = None  # absolute offset in the source GGUF (else synthetic, in tensor order)


def _label(name: str) -> str:
    """File label of a tensor name (tools/bench/native_harness.py:126-128)."""
    return re.sub(r"[^A-Za-z0-9_.-]+", "_", name.strip()).strip("._-") or "native"


def _checksum(a: np.ndarray) -> int:
    return int(np.asarray(a, np.uint8).sum(dtype=np.uint64))


def _layer_role(name: str) -> tuple[int | None, str]:
    m = re.match(r"blk\.(\d+)\.(.+)$", name)
    if m:
        return int(m.group(1)), m.group(2)
    return None, name[:-len(".weight")] if name.endswith(".weight") else name


def write_packs(out_dir: Path, tensors: list[Tensor], policy: str = "split-native", write_blocks: bool = True,
                absolute_paths: bool = False, model: str = "synthetic.gguf") -> dict[str, Path]:
    """Writes the packs; returns the paths of "q4k_manifest", "iq_manifest" and
    "tensor_plan" (a manifest only when it has tensors). policy: a Q4_K split
    layout, or "auto" / "auto-lossy" for auto_policy() per tensor."""
    out_dir = Path(out_dir)
    out_dir.mkdir(parents=True, exist_ok=True)
    if policy not in Q4K_POLICIES and policy not in ("auto", "auto-lossy"):
        raise ValueError(f"unknown Q4_K policy {policy!r}")

    def rel(p: Path) -> str:
        return str(p.resolve() if absolute_paths else p.relative_to(out_dir))

    next_offset = 4096  # synthetic GGUF data offsets, in tensor order
    plan, q4k, raw = [], [], []
    for t in tensors:
        offset = t.offset if t.offset is not None else next_offset
        n_blocks = t.rows * (t.cols // F.BLOCK_VALUES)
        block_bytes = F.GGUF_BLOCK_BYTES[F.Q4K_RAW if t.fmt == F.Q4K_RAW else t.fmt]
        blocks = np.ascontiguousarray(t.blocks, dtype=np.uint8)
        if blocks.size != n_blocks * block_bytes:
            raise ValueError(f"{t.name}: {blocks.size} bytes for {n_blocks} blocks of {block_bytes}")
        gguf_type = "Q4_K" if t.fmt == F.Q4K_RAW else RAW_TYPES[t.fmt]
        plan.append({"name": t.name, "type": gguf_type, "dimensions": [t.cols, t.rows], "span_bytes": int(blocks.size),
                     "absolute_offset": offset})
        label = _label(t.name)
        if t.fmt == F.Q4K_RAW:
            tpolicy = policy if policy in Q4K_POLICIES else auto_policy(t.rows, t.cols, policy == "auto-lossy")
            split_fmt, meta_label = Q4K_POLICIES[tpolicy]
            payload, meta = packs.q4k_split(split_fmt, blocks)
            pp = out_dir / f"{label}.q4k_payload.bin"
            mp = out_dir / f"{label}.q4k_meta.{meta_label}.bin"
            payload.tofile(pp)
            meta.tofile(mp)
            bp = ""
            if write_blocks:
                bpath = out_dir / f"{label}.q4k_blocks.bin"
                blocks.tofile(bpath)
                bp = rel(bpath)
            q4k.append({
                "name": t.name, "dimensions": [t.cols, t.rows], "rows": t.rows, "cols": t.cols,
                "block_count": n_blocks, "source_offset": offset, "source_bytes": int(blocks.size),
                "source_checksum": _checksum(blocks), "policy": tpolicy, "metadata_format": meta_label,
                "payload_path": rel(pp), "payload_bytes": int(payload.size), "payload_checksum": _checksum(payload),
                "metadata_path": rel(mp), "metadata_bytes": int(meta.size), "metadata_checksum": _checksum(meta),
                "blocks_path": bp, "resident_bytes": int(payload.size + meta.size),
                "compression_ratio_vs_fp16": (t.rows * t.cols * 2) / float(payload.size + meta.size),
                "runtime_kernel": tpolicy,
            })
        else:
            pp = out_dir / f"{label}.{gguf_type.lower()}_raw_blocks.bin"
            blocks.tofile(pp)
            layer, role = _layer_role(t.name)
            raw.append({
                "name": t.name, "type": gguf_type, "layer": layer, "role": role, "dimensions": [t.cols, t.rows],
                "element_count": t.rows * t.cols, "block_size": F.BLOCK_VALUES, "block_type_size": block_bytes,
                "block_count": n_blocks, "source_offset": offset, "source_bytes": int(blocks.size),
                "source_checksum": _checksum(blocks), "payload_path": rel(pp), "payload_bytes": int(blocks.size),
                "payload_checksum": _checksum(blocks), "resident_bytes": int(blocks.size), "policy": "raw-blocks",
                "runtime_kernel": KERNEL_LABELS[gguf_type],
            })
        next_offset = offset + int(blocks.size)

    paths = {"tensor_plan": out_dir / "tensor_plan.json"}
    paths["tensor_plan"].write_text(json.dumps({"model": model, "tensors": plan}, indent=1))
    stamp = "1970-01-01T00:00:00Z"
    if q4k:
        paths["q4k_manifest"] = out_dir / "q4k_manifest.json"
        paths["q4k_manifest"].write_text(json.dumps({
            "path": "q4k_resident_pack", "generated_at": stamp, "model": model, "tensor_plan": str(paths["tensor_plan"]), "output_dir": str(out_dir),
            "policy": policy, "tensor_count": len(q4k),
            "resident_bytes": sum(t["resident_bytes"] for t in q4k),
            "payload_bytes": sum(t["payload_bytes"] for t in q4k),
            "metadata_bytes": sum(t["metadata_bytes"] for t in q4k), "tensors": q4k}, indent=1))
    if raw:
        paths["iq_manifest"] = out_dir / "iq_manifest.json"
        paths["iq_manifest"].write_text(json.dumps({
            "path": "iq_resident_pack", "generated_at": stamp, "model": model, "tensor_plan": str(paths["tensor_plan"]),
            "types": sorted({t["type"] for t in raw}), "tensor_count": len(raw),
            "source_bytes": sum(t["source_bytes"] for t in raw), "payload_bytes": sum(t["payload_bytes"] for t in raw),
            "resident_bytes": sum(t["resident_bytes"] for t in raw), "tensors": raw}, indent=1))
    return paths
