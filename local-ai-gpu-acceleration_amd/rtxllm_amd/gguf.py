"""GGUF container reader / writer and the GGUF -> resident-pack step.

The container is the public GGUF v3 layout, read the way the reference's
inspector reads it (tools/bench/gguf_inspect.py:13-200): "GGUF", u32 version,
u64 tensor count, u64 metadata count, typed key / value metadata (value types
0..12, arrays as item type + u64 length + items), tensor infos (name, u32
n_dims, u64 dims, u32 ggml type, u64 offset into the data section), and the
data section at align_up(end of tensor infos, general.alignment) (default
32). A tensor's span runs to the next tensor's offset (or the end of the
file) and may carry alignment padding (tools/bench/gguf_tensor_plan.py:53-80,
gguf_block_formats.py:47-80): padding >= alignment is refused.

to_packs() turns the quantized tensors of a GGUF Llama model into the resident
packs and manifests the decode runner loads (rtxllm_llama_load_pack_set),
through the library's C++ producer (rtxllm_gguf_pack, producer.py): Q4_K
tensors into the chosen split layout, IQ2_S / IQ3_S / Q5_K as raw blocks, one
manifest per producer in the reference producers' form, with the tensors'
absolute file offsets in the tensor plan. The fp32 norm vectors are returned
by norms() for upload; llama_shape() reads the model shape from the llama.*
metadata keys.
"""

from __future__ import annotations

import io
import struct
from dataclasses import dataclass, field
from pathlib import Path
from typing import BinaryIO

import numpy as np

from . import formats as F
from . import manifest as M

# gguf_inspect.py:13-27
VALUE_TYPES = {0: "uint8", 1: "int8", 2: "uint16", 3: "int16", 4: "uint32", 5: "int32", 6: "float32", 7: "bool",
               8: "string", 9: "array", 10: "uint64", 11: "int64", 12: "float64"}
_SCALAR = {0: "<B", 1: "<b", 2: "<H", 3: "<h", 4: "<I", 5: "<i", 6: "<f", 10: "<Q", 11: "<q", 12: "<d"}

# ggml type ids (gguf_inspect.py:29-65), the ones this runtime stores or reads
GGML_TYPES = {0: "F32", 1: "F16", 8: "Q8_0", 12: "Q4_K", 13: "Q5_K", 14: "Q6_K", 21: "IQ3_S", 22: "IQ2_S", 30: "BF16"}
GGML_TYPE_IDS = {v: k for k, v in GGML_TYPES.items()}
# (values per block, bytes per block): gguf_block_formats.py:14-22
BLOCKS = {"F32": (1, 4), "F16": (1, 2), "BF16": (1, 2), "Q8_0": (32, 34), "Q4_K": (256, 144), "Q5_K": (256, 176),
          "Q6_K": (256, 210), "IQ2_S": (256, 82), "IQ3_S": (256, 110)}
# GGUF type -> pack format of the decode kernels (Q4_K: the split layout is the policy's)
PACK_FORMATS = {"Q4_K": F.Q4K_RAW, "Q5_K": F.Q5K, "IQ2_S": F.IQ2S, "IQ3_S": F.IQ3S}

DEFAULT_ALIGNMENT = 32


def align_up(value: int, alignment: int) -> int:
    return (value + alignment - 1) // alignment * alignment


@dataclass
class GGUFTensor:
    name: str
    dims: list[int]       # GGUF order: dims[0] = values per row (cols), then rows
    type_id: int
    offset: int           # into the data section
    span: int = 0         # bytes to the next tensor (set by read())

    @property
    def type(self) -> str:
        return GGML_TYPES.get(self.type_id, f"unknown:{self.type_id}")

    @property
    def cols(self) -> int:
        return int(self.dims[0])

    @property
    def rows(self) -> int:
        n = 1
        for d in self.dims[1:]:
            n *= int(d)
        return n

    @property
    def nbytes(self) -> int:
        """Data bytes implied by type and dims (no padding)."""
        if self.type not in BLOCKS:
            raise ValueError(f"{self.name}: tensor type {self.type} has no known block size")
        per, size = BLOCKS[self.type]
        elements = self.rows * self.cols
        if elements % per:
            raise ValueError(f"{self.name}: {elements} values are not whole {self.type} blocks")
        return elements // per * size


@dataclass
class GGUF:
    version: int
    metadata: dict
    value_types: dict
    tensors: list[GGUFTensor]
    tensor_info_end: int
    data_offset: int
    alignment: int
    path: Path | None = None
    size: int | None = None
    _map: np.ndarray | None = field(default=None, repr=False)

    def tensor(self, name: str) -> GGUFTensor:
        for t in self.tensors:
            if t.name == name:
                return t
        raise KeyError(name)

    def data(self, t: GGUFTensor) -> np.ndarray:
        """The tensor's bytes (uint8, memory-mapped, no padding)."""
        if self._map is None:
            if self.path is None:
                raise ValueError("tensor data needs a file-backed GGUF")
            self._map = np.memmap(self.path, dtype=np.uint8, mode="r")
        start = self.data_offset + t.offset
        n = t.nbytes
        if start + n > self._map.size:
            raise ValueError(f"{t.name}: data past the end of the file")
        return self._map[start:start + n]

    def plan(self) -> list[dict]:
        """The tensor plan rows (gguf_tensor_plan.py:53-80): name, type, dimensions,
        span_bytes, absolute_offset."""
        return [{"name": t.name, "type": t.type, "dimensions": [int(d) for d in t.dims], "span_bytes": t.span,
                 "absolute_offset": self.data_offset + t.offset} for t in self.tensors]


class _Reader:
    def __init__(self, fh: BinaryIO):
        self.fh = fh

    def exact(self, n: int) -> bytes:
        b = self.fh.read(n)
        if len(b) != n:
            raise EOFError("unexpected end of GGUF data")
        return b

    def scalar(self, fmt: str):
        return struct.unpack(fmt, self.exact(struct.calcsize(fmt)))[0]

    def string(self) -> str:
        return self.exact(self.scalar("<Q")).decode("utf-8", errors="replace")

    def value(self, vtype: int):
        if vtype in _SCALAR:
            return self.scalar(_SCALAR[vtype])
        if vtype == 7:
            return bool(self.scalar("<B"))
        if vtype == 8:
            return self.string()
        if vtype == 9:
            item = self.scalar("<I")
            n = self.scalar("<Q")
            return [self.value(item) for _ in range(n)]
        raise ValueError(f"unsupported GGUF metadata value type {vtype}")


def read(source, check_spans: bool = True) -> GGUF:
    """Parse a GGUF file (path) or stream: header, metadata, tensor infos and
    each tensor's span; tensor data stays on disk (GGUF.data maps it). With
    check_spans, every tensor of a known type must fit its span with less than
    one alignment of padding."""
    path = None
    if isinstance(source, (str, Path)):
        path = Path(source)
        fh = path.open("rb")
    else:
        fh = source
    try:
        r = _Reader(fh)
        if r.exact(4) != b"GGUF":
            raise ValueError("not a GGUF file")
        version = r.scalar("<I")
        n_tensors = r.scalar("<Q")
        n_meta = r.scalar("<Q")
        metadata, vtypes = {}, {}
        for _ in range(n_meta):
            key = r.string()
            vt = r.scalar("<I")
            vtypes[key] = VALUE_TYPES.get(vt, f"unknown:{vt}")
            metadata[key] = r.value(vt)
        tensors = []
        for _ in range(n_tensors):
            name = r.string()
            nd = r.scalar("<I")
            dims = [r.scalar("<Q") for _ in range(nd)]
            tensors.append(GGUFTensor(name, dims, r.scalar("<I"), r.scalar("<Q")))
        end = fh.tell()
        if path is not None:
            size = path.stat().st_size
        else:
            fh.seek(0, io.SEEK_END)
            size = fh.tell()
    finally:
        if path is not None:
            fh.close()
    alignment = metadata.get("general.alignment", DEFAULT_ALIGNMENT)
    if not isinstance(alignment, int) or isinstance(alignment, bool) or alignment <= 0:
        alignment = DEFAULT_ALIGNMENT
    data_offset = align_up(end, alignment)
    order = sorted(tensors, key=lambda t: t.offset)
    for i, t in enumerate(order):
        nxt = order[i + 1].offset if i + 1 < len(order) else size - data_offset
        t.span = max(0, nxt - t.offset)
    g = GGUF(version, metadata, vtypes, tensors, end, data_offset, alignment, path, size)
    for t in tensors if check_spans else []:
        if t.type in BLOCKS:
            pad = t.span - t.nbytes
            if pad < 0 or pad >= alignment:
                raise ValueError(f"{t.name}: span {t.span} B does not hold {t.nbytes} B of {t.type} data "
                                 f"(alignment {alignment})")
    return g


# ---- writer ------------------------------------------------------------------------

def _pack_value(vtype: int, value) -> bytes:
    if vtype in _SCALAR:
        return struct.pack(_SCALAR[vtype], value)
    if vtype == 7:
        return struct.pack("<B", 1 if value else 0)
    if vtype == 8:
        b = value.encode("utf-8")
        return struct.pack("<Q", len(b)) + b
    raise ValueError(f"value type {vtype} is not a scalar")


def write(path, metadata: list[tuple], tensors: list[tuple], version: int = 3,
          alignment: int = DEFAULT_ALIGNMENT) -> None:
    """Write a GGUF file. metadata: (key, value_type_id, value) or, for arrays,
    (key, 9, (item_type_id, [values])); tensors: (name, ggml type name, dims,
    bytes) in file order, each tensor's data aligned to `alignment` (set
    general.alignment in metadata when it is not 32)."""
    out = bytearray(b"GGUF")
    out += struct.pack("<IQQ", version, len(tensors), len(metadata))
    for key, vt, value in metadata:
        out += _pack_value(8, key) + struct.pack("<I", vt)
        if vt == 9:
            item, values = value
            out += struct.pack("<IQ", item, len(values))
            for v in values:
                out += _pack_value(item, v)
        else:
            out += _pack_value(vt, value)
    offset = 0
    datas = []
    for name, tname, dims, data in tensors:
        data = np.ascontiguousarray(np.frombuffer(bytes(data), np.uint8) if not isinstance(data, np.ndarray)
                                    else data).view(np.uint8).reshape(-1)
        t = GGUFTensor(name, list(dims), GGML_TYPE_IDS[tname], offset)
        if data.size != t.nbytes:
            raise ValueError(f"{name}: {data.size} bytes for {t.nbytes} of {tname} data")
        out += _pack_value(8, name) + struct.pack("<I", len(dims))
        out += b"".join(struct.pack("<Q", int(d)) for d in dims)
        out += struct.pack("<IQ", t.type_id, offset)
        datas.append((offset, data))
        offset = align_up(offset + data.size, alignment)
    start = align_up(len(out), alignment)
    out += bytes(start - len(out))
    with Path(path).open("wb") as fh:
        fh.write(out)
        pos = 0
        for off, data in datas:
            fh.write(bytes(off - pos))
            fh.write(data.tobytes())
            pos = off + data.size


# ---- Llama models --------------------------------------------------------------------

def llama_shape(g: GGUF) -> dict:
    """Shape fields of a GGUF Llama model (llama.* keys; vocab from token_embd)."""
    m = g.metadata
    arch = m.get("general.architecture", "llama")
    if arch != "llama":
        raise ValueError(f"architecture {arch!r} is not llama")

    def key(k, default=None):
        v = m.get(f"llama.{k}", default)
        if v is None:
            raise KeyError(f"llama.{k}")
        return v

    shape = {"hidden": int(key("embedding_length")), "n_layers": int(key("block_count")),
             "n_heads": int(key("attention.head_count")), "ffn": int(key("feed_forward_length")),
             "vocab": g.tensor("token_embd.weight").rows}
    shape["n_kv_heads"] = int(m.get("llama.attention.head_count_kv", shape["n_heads"]))
    if "llama.rope.freq_base" in m:
        shape["rope_theta"] = float(m["llama.rope.freq_base"])
    if "llama.attention.layer_norm_rms_epsilon" in m:
        shape["rms_eps"] = float(m["llama.attention.layer_norm_rms_epsilon"])
    if shape["hidden"] != 128 * shape["n_heads"]:
        raise ValueError(f"head_dim {shape['hidden'] / shape['n_heads']} is not 128")
    return shape


def model_formats(g: GGUF, policy: str = "split-native") -> dict:
    """Per-role pack formats of the model (the runner's qkv / o / gate_up / down
    / lm_head), from the block-0 and output tensor types; q, k, v (and gate,
    up) must share a type since the runner stacks them."""
    def fmt(*names):
        types = {g.tensor(n).type for n in names}
        if len(types) != 1:
            raise ValueError(f"{names} differ in type: {sorted(types)}")
        t = types.pop()
        if t not in PACK_FORMATS:
            raise ValueError(f"{names[0]}: type {t} has no decode kernel (Q4_K, Q5_K, IQ2_S, IQ3_S)")
        if t != "Q4_K":
            return PACK_FORMATS[t]
        p = policy
        if p in ("auto", "auto-lossy"):
            p = M.auto_policy(g.tensor(names[0]).rows, g.tensor(names[0]).cols, p == "auto-lossy")
        return M.Q4K_POLICIES[p][0]

    b = "blk.0."
    return {"fmt_qkv": fmt(b + "attn_q.weight", b + "attn_k.weight", b + "attn_v.weight"),
            "fmt_o": fmt(b + "attn_output.weight"), "fmt_gate_up": fmt(b + "ffn_gate.weight", b + "ffn_up.weight"),
            "fmt_down": fmt(b + "ffn_down.weight"), "fmt_lm_head": fmt("output.weight")}


def to_packs(g: GGUF, out_dir, policy: str = "split-native", write_blocks: bool = True) -> dict[str, Path]:
    """Resident packs + manifests of every Q4_K / Q5_K / IQ2_S / IQ3_S tensor of
    a file-backed GGUF, written by the C++ producer (producer.pack_gguf):
    returns the paths of "tensor_plan" and of the "q4k_manifest",
    "iq_manifest" and "q5k_manifest" written."""
    if g.path is None:
        raise ValueError("to_packs needs a file-backed GGUF")
    from . import producer

    return producer.pack_gguf(g.path, out_dir, policy=policy, write_blocks=write_blocks)


def norms(g: GGUF) -> dict[tuple[str, int], np.ndarray]:
    """fp32 norm weights: (region, layer) -> vector for the runner's attn_norm /
    ffn_norm (per layer) and out_norm."""
    out = {}
    for t in g.tensors:
        role = None
        if t.name == "output_norm.weight":
            role, layer = "out_norm", 0
        elif t.name.startswith("blk.") and t.name.endswith((".attn_norm.weight", ".ffn_norm.weight")):
            layer = int(t.name.split(".")[1])
            role = "attn_norm" if t.name.endswith(".attn_norm.weight") else "ffn_norm"
        if role is None:
            continue
        if t.type != "F32":
            raise ValueError(f"{t.name}: norm weights must be F32, not {t.type}")
        out[(role, layer)] = np.asarray(g.data(t)).view(np.float32).copy()
    return out


def load_into(model, g: GGUF, work_dir, policy: str = "split-native") -> dict[str, Path]:
    """Fill a rtxllm_amd.llama.Llama created with llama_shape(g) and
    model_formats(g, policy): packs written to work_dir and loaded through
    rtxllm_llama_load_pack_set, norm vectors uploaded. Returns the pack paths."""
    paths = to_packs(g, work_dir, policy=policy)
    model.load_pack_set([p for k, p in paths.items() if k.endswith("_manifest")])
    for (role, layer), v in norms(g).items():
        model.upload(role, v, layer=layer)
    return paths


def main(argv=None) -> int:
    import argparse
    import json

    ap = argparse.ArgumentParser(description="GGUF inspection and GGUF -> resident packs")
    sub = ap.add_subparsers(dest="cmd", required=True)
    ins = sub.add_parser("inspect", help="print header, metadata keys and tensor plan as JSON")
    ins.add_argument("path")
    pk = sub.add_parser("pack", help="write the resident packs and manifests of a GGUF Llama model")
    pk.add_argument("path")
    pk.add_argument("out_dir")
    pk.add_argument("--policy", default="auto", choices=sorted(M.Q4K_POLICIES) + ["auto", "auto-lossy"])
    a = ap.parse_args(argv)
    g = read(a.path)
    if a.cmd == "inspect":
        def short(v):
            return {"array_length": len(v)} if isinstance(v, list) else v
        print(json.dumps({"version": g.version, "tensor_count": len(g.tensors), "alignment": g.alignment,
                          "tensor_info_end_offset": g.tensor_info_end, "tensor_data_offset": g.data_offset,
                          "metadata": {k: short(v) for k, v in g.metadata.items()}, "tensors": g.plan()},
                         indent=1))
    else:
        paths = to_packs(g, a.out_dir, policy=a.policy)
        print(json.dumps({k: str(v) for k, v in paths.items()}, indent=1))
    return 0


if __name__ == "__main__":
    raise SystemExit(main())
