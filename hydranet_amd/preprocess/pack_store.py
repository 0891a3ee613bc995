"""Packed INT4 expert files: experts.bin / experts.idx writers and the legacy
per-expert format.

Formats (kept byte-compatible with the reference):

* **experts.bin** — one blob per expert (BlobLayout order, no padding), blobs
  back to back in the order written; **experts.idx** — JSON
  ``{"format_version": "2.0", ["model_type"], "quant_config": {bits,
  group_size, symmetric}, "model_config": {num_layers, num_experts,
  hidden_dim, intermediate_dim}, "experts": [{layer_idx, expert_idx, offset,
  size}]}`` (reference preprocess/pack_glm4.py:72-141,
  cache/packed_expert_store.py:627-739).
* **legacy per-expert file** ``expert_L{ll}_E{ee}.bin`` — a 20-byte header of
  five little-endian u32 (layer, expert, hidden_dim, intermediate_dim,
  group_size) followed by the same six tensors in blob order, indexed by
  ``metadata.json`` format "1.0" with per-expert keys layer / expert / file /
  size_bytes / checksum and a total_size_bytes (reference
  preprocess/pack_weights.py:271-449).  After the header a legacy file holds
  exactly the expert's blob, so conversion to experts.bin is a byte copy.

Writers stream one expert at a time (a Mixtral store is 23.25 GB, GLM-4.5-Air
51.38 GB).  Quantisation from fp16 runs on the GPU (``quantize_int4``, the
ExpertWeightPacker.quantize_tensor rule); tensors already packed are written
as they are.  Reading is ``cache.packed_expert_store.PackedExpertStore``.
"""
from __future__ import annotations

import json
import struct
from dataclasses import dataclass
from pathlib import Path
from typing import Dict, Iterable, Iterator, Optional, Tuple

import numpy as np
import torch

from ..cache.blob_layout import TENSORS, BlobLayout

__all__ = ["QuantConfig", "PackedExpert", "compute_expert_checksum", "verify_expert_checksum",
           "pack_expert", "expert_blob", "blob_tensors", "ExpertStoreWriter", "write_packed_store",
           "pack_experts", "pack_glm4_experts", "save_packed_expert", "load_packed_expert",
           "write_legacy_store", "pack_to_single_blob", "legacy_expert_filename",
           "iter_store_experts"]

_HEADER = struct.Struct("<IIIII")
# reference field name of each blob tensor in PackedExpert (pack_weights.py:59-80)
_LEGACY_NAMES = {"gate_packed": "gate_proj_packed", "gate_scales": "gate_proj_scales",
                 "up_packed": "up_proj_packed", "up_scales": "up_proj_scales",
                 "down_packed": "down_proj_packed", "down_scales": "down_proj_scales"}


@dataclass
class QuantConfig:
    """bits=4, group_size, symmetric -> zero_point 8 (reference pack_weights.py:23-33)."""
    bits: int = 4
    group_size: int = 128
    symmetric: bool = True

    @property
    def zero_point(self) -> int:
        return 2 ** (self.bits - 1) if self.symmetric else 0

    def to_json(self) -> dict:
        return {"bits": self.bits, "group_size": self.group_size, "symmetric": self.symmetric}


def compute_expert_checksum(weights: Dict[str, torch.Tensor]) -> str:
    """Hex of the little-endian float64 bits of sum(|w|) over gate, up, down
    (each summed in fp32 by torch on the host; reference pack_weights.py:36-50)."""
    total = 0.0
    for name in ("gate_proj", "up_proj", "down_proj"):
        if name in weights:
            total += weights[name].detach().float().abs().sum().item()
    return struct.pack("<d", total).hex()


def verify_expert_checksum(weights: Dict[str, torch.Tensor], expected: str) -> bool:
    return compute_expert_checksum(weights) == expected


@dataclass
class PackedExpert:
    """One expert's six INT4 tensors plus dims (reference pack_weights.py:56-110)."""
    layer_idx: int
    expert_idx: int
    gate_proj_packed: torch.Tensor
    up_proj_packed: torch.Tensor
    down_proj_packed: torch.Tensor
    gate_proj_scales: torch.Tensor
    up_proj_scales: torch.Tensor
    down_proj_scales: torch.Tensor
    hidden_dim: int
    intermediate_dim: int
    group_size: int
    checksum: str = ""

    def size_bytes(self) -> int:
        return sum(t.numel() * t.element_size() for t in self.blob_tensors().values())

    def blob_tensors(self) -> Dict[str, torch.Tensor]:
        """Blob-order name -> tensor (gate_packed, gate_scales, ...)."""
        return {n: getattr(self, _LEGACY_NAMES[n]) for n in TENSORS}

    def to_pinned(self) -> "PackedExpert":
        pinned = {_LEGACY_NAMES[n]: t.pin_memory() for n, t in self.blob_tensors().items()}
        return PackedExpert(self.layer_idx, self.expert_idx, hidden_dim=self.hidden_dim,
                            intermediate_dim=self.intermediate_dim, group_size=self.group_size,
                            checksum=self.checksum, **pinned)

    @classmethod
    def from_blob_tensors(cls, layer_idx: int, expert_idx: int, tensors: Dict[str, torch.Tensor],
                          group_size: int, checksum: str = "") -> "PackedExpert":
        I, half_h = tensors["gate_packed"].shape
        return cls(layer_idx, expert_idx, hidden_dim=2 * half_h, intermediate_dim=I,
                   group_size=group_size, checksum=checksum,
                   **{_LEGACY_NAMES[n]: tensors[n] for n in TENSORS})


def pack_expert(layer_idx: int, expert_idx: int, weights: Dict[str, torch.Tensor],
                group_size: int = 128, device="cuda") -> PackedExpert:
    """Quantise gate_proj [I, H], up_proj [I, H], down_proj [H, I] (fp16) on the
    GPU with the ExpertWeightPacker rule; tensors are returned on the host
    (reference pack_weights.py:183-228, checksum taken before quantising)."""
    from ..kernels.int4_gemm import quantize_int4
    checksum = compute_expert_checksum(weights)
    out = {}
    for proj, pre in (("gate_proj", "gate"), ("up_proj", "up"), ("down_proj", "down")):
        w = weights[proj].to(device=device, dtype=torch.float16)
        p, s = quantize_int4(w, group_size, mode=0)
        out[f"{pre}_packed"], out[f"{pre}_scales"] = p.cpu(), s.cpu()
    return PackedExpert.from_blob_tensors(layer_idx, expert_idx, out, group_size, checksum)


def _tensor_bytes(t: torch.Tensor) -> np.ndarray:
    t = t.detach().contiguous().cpu()
    return t.view(torch.uint8).reshape(-1).numpy() if t.dtype != torch.uint8 else \
        t.reshape(-1).numpy()


def expert_blob(tensors, layout: Optional[BlobLayout] = None, group_size: Optional[int] = None
                ) -> np.ndarray:
    """The expert's blob (uint8 array of layout.total_size bytes) from six
    blob-order tensors (dict) or a PackedExpert; every tensor's shape and
    dtype is checked against the layout."""
    if isinstance(tensors, PackedExpert):
        group_size = tensors.group_size
        tensors = tensors.blob_tensors()
    I, half_h = tensors["gate_packed"].shape
    H = 2 * half_h
    if group_size is None:
        group_size = H // tensors["gate_scales"].shape[1]
    shapes = BlobLayout.shapes(H, I, group_size)
    if layout is None:
        layout = BlobLayout.from_dims(H, I, group_size)
    blob = np.empty(layout.total_size, dtype=np.uint8)
    for name, off, size in layout.spans():
        t = tensors[name]
        shape, dt = shapes[name]
        want = torch.uint8 if dt == "uint8" else torch.float16
        if tuple(t.shape) != tuple(shape) or t.dtype != want:
            raise ValueError(f"{name}: {tuple(t.shape)} {t.dtype}, expected {shape} {want}")
        b = _tensor_bytes(t)
        if b.size != size:
            raise ValueError(f"{name}: {b.size} bytes, layout says {size}")
        blob[off:off + size] = b
    return blob


def blob_tensors(blob, hidden_dim: int, intermediate_dim: int, group_size: int
                 ) -> Dict[str, torch.Tensor]:
    """Six host tensors viewing a blob (bytes-like or uint8 array)."""
    layout = BlobLayout.from_dims(hidden_dim, intermediate_dim, group_size)
    raw = torch.frombuffer(bytearray(blob), dtype=torch.uint8)
    if raw.numel() != layout.total_size:
        raise ValueError(f"blob of {raw.numel()} bytes, layout needs {layout.total_size}")
    out = {}
    for name, (shape, dt) in BlobLayout.shapes(hidden_dim, intermediate_dim, group_size).items():
        off, size = getattr(layout, f"{name}_offset"), getattr(layout, f"{name}_size")
        v = raw[off:off + size]
        out[name] = (v.view(torch.float16) if dt == "float16" else v).view(*shape)
    return out


class ExpertStoreWriter:
    """Streams blobs into experts.bin and writes experts.idx on close."""

    def __init__(self, output_dir, num_layers: int, num_experts: int, hidden_dim: int,
                 intermediate_dim: int, group_size: int = 128, model_type: Optional[str] = None,
                 quant_config: Optional[QuantConfig] = None):
        self.output_dir = Path(output_dir)
        self.output_dir.mkdir(parents=True, exist_ok=True)
        qc = quant_config or QuantConfig(group_size=group_size)
        if qc.group_size != group_size:
            raise ValueError("quant_config.group_size != group_size")
        self.layout = BlobLayout.from_dims(hidden_dim, intermediate_dim, group_size)
        self.dims = (hidden_dim, intermediate_dim, group_size)
        self.index = {"format_version": "2.0"}
        if model_type is not None:
            self.index["model_type"] = model_type
        self.index["quant_config"] = qc.to_json()
        self.index["model_config"] = {"num_layers": num_layers, "num_experts": num_experts,
                                      "hidden_dim": hidden_dim,
                                      "intermediate_dim": intermediate_dim}
        self.index["experts"] = []
        self.bin_path = self.output_dir / "experts.bin"
        self.index_path = self.output_dir / "experts.idx"
        self._f = open(self.bin_path, "wb")
        self._offset = 0
        self._seen = set()

    def add(self, layer_idx: int, expert_idx: int, tensors) -> int:
        """Append one expert (six blob-order tensors, a PackedExpert, or a
        ready blob); returns its offset in experts.bin."""
        key = (int(layer_idx), int(expert_idx))
        if key in self._seen:
            raise ValueError(f"expert {key} written twice")
        if isinstance(tensors, (bytes, bytearray, memoryview, np.ndarray)):
            blob = np.frombuffer(tensors, dtype=np.uint8) if not isinstance(tensors, np.ndarray) \
                else tensors.view(np.uint8).reshape(-1)
            if blob.size != self.layout.total_size:
                raise ValueError(f"blob of {blob.size} bytes, layout needs "
                                 f"{self.layout.total_size}")
        else:
            blob = expert_blob(tensors, self.layout, self.dims[2])
        self._f.write(memoryview(blob))
        off = self._offset
        self.index["experts"].append({"layer_idx": key[0], "expert_idx": key[1], "offset": off,
                                      "size": self.layout.total_size})
        self._offset += self.layout.total_size
        self._seen.add(key)
        return off

    def close(self) -> dict:
        if self._f is not None:
            self._f.close()
            self._f = None
            with open(self.index_path, "w") as f:
                json.dump(self.index, f, indent=2)
        return self.index

    def __enter__(self):
        return self

    def __exit__(self, *exc):
        self.close()


def write_packed_store(output_dir, experts: Iterable[Tuple[int, int, object]], num_layers: int,
                       num_experts: int, hidden_dim: int, intermediate_dim: int,
                       group_size: int = 128, model_type: Optional[str] = None) -> dict:
    """experts.bin + experts.idx from already-packed experts, in iteration order."""
    with ExpertStoreWriter(output_dir, num_layers, num_experts, hidden_dim, intermediate_dim,
                           group_size, model_type) as w:
        for layer_idx, expert_idx, t in experts:
            w.add(layer_idx, expert_idx, t)
    return w.index


def pack_experts(iter_experts: Iterable[Tuple[int, int, Dict[str, torch.Tensor]]], output_dir,
                 num_layers: int, num_experts: int, hidden_dim: int, intermediate_dim: int,
                 group_size: int = 128, model_type: Optional[str] = None, device="cuda") -> dict:
    """Quantise fp16 experts on the GPU and stream them into experts.bin/.idx.
    ``iter_experts`` yields (layer_idx, expert_idx, {gate_proj, up_proj,
    down_proj}) like the reference loaders' iter_experts (model/loader.py:176-185)."""
    with ExpertStoreWriter(output_dir, num_layers, num_experts, hidden_dim, intermediate_dim,
                           group_size, model_type) as w:
        for layer_idx, expert_idx, weights in iter_experts:
            w.add(layer_idx, expert_idx,
                  pack_expert(layer_idx, expert_idx, weights, group_size, device))
    return w.index


def pack_glm4_experts(iter_experts, output_dir, group_size: int = 128, num_layers: int = 45,
                      num_experts: int = 128, hidden_dim: int = 4096,
                      moe_intermediate_dim: int = 1408, device="cuda") -> dict:
    """GLM-4.5-Air routed experts -> experts.bin/.idx with model_type
    "glm4_air" (reference preprocess/pack_glm4.py:33-149); layers are MoE-layer
    indices counted from the first MoE layer."""
    return pack_experts(iter_experts, output_dir, num_layers, num_experts, hidden_dim,
                        moe_intermediate_dim, group_size, "glm4_air", device)


# ---------------------------------------------------------------- legacy format
def legacy_expert_filename(layer_idx: int, expert_idx: int) -> str:
    return f"expert_L{layer_idx:02d}_E{expert_idx:02d}.bin"


def save_packed_expert(packed: PackedExpert, path) -> int:
    """Write one legacy per-expert file (20-byte header + blob); returns the
    payload size (reference pack_weights.py:336-353)."""
    blob = expert_blob(packed)
    with open(path, "wb") as f:
        f.write(_HEADER.pack(packed.layer_idx, packed.expert_idx, packed.hidden_dim,
                             packed.intermediate_dim, packed.group_size))
        f.write(memoryview(blob))
    return blob.size


def _read_legacy(path) -> Tuple[Tuple[int, int, int, int, int], bytes]:
    with open(path, "rb") as f:
        head = f.read(_HEADER.size)
        if len(head) != _HEADER.size:
            raise ValueError(f"{path}: truncated header")
        hdr = _HEADER.unpack(head)
        payload = f.read()
    _, _, H, I, g = hdr
    if g == 0 or H % g or I % g or H % 2 or I % 2:
        raise ValueError(f"{path}: bad dims H={H} I={I} group={g}")
    need = BlobLayout.from_dims(H, I, g).total_size
    if len(payload) != need:
        raise ValueError(f"{path}: {len(payload)} payload bytes, dims need {need}")
    return hdr, payload


def load_packed_expert(path) -> PackedExpert:
    """Read a legacy per-expert file (reference pack_weights.py:392-449); the
    size is checked against the header dims."""
    (layer, expert, H, I, g), payload = _read_legacy(path)
    t = {n: v.clone() for n, v in blob_tensors(payload, H, I, g).items()}
    return PackedExpert.from_blob_tensors(layer, expert, t, g)


def write_legacy_store(experts: Iterable[PackedExpert], output_dir, num_layers: int,
                       num_experts: int, quant_config: Optional[QuantConfig] = None) -> dict:
    """Legacy layout: one file per expert + metadata.json format "1.0"
    (reference pack_weights.py:271-389)."""
    out = Path(output_dir)
    out.mkdir(parents=True, exist_ok=True)
    meta = {"format_version": "1.0", "quant_config": None, "model_config": None, "experts": []}
    total = 0
    for p in experts:
        if meta["model_config"] is None:
            qc = quant_config or QuantConfig(group_size=p.group_size)
            meta["quant_config"] = qc.to_json()
            meta["model_config"] = {"num_layers": num_layers, "num_experts": num_experts,
                                    "hidden_dim": p.hidden_dim,
                                    "intermediate_dim": p.intermediate_dim}
        name = legacy_expert_filename(p.layer_idx, p.expert_idx)
        size = save_packed_expert(p, out / name)
        total += size
        meta["experts"].append({"layer": p.layer_idx, "expert": p.expert_idx, "file": name,
                                "size_bytes": size, "checksum": p.checksum})
    meta["total_size_bytes"] = total
    with open(out / "metadata.json", "w") as f:
        json.dump(meta, f, indent=2)
    return meta


def pack_to_single_blob(input_dir, output_dir, num_layers: int, num_experts: int,
                        hidden_dim: int, intermediate_dim: int, group_size: int = 128,
                        model_type: Optional[str] = None) -> dict:
    """Convert legacy per-expert files (every layer x expert, in that order)
    to experts.bin/.idx (reference cache/packed_expert_store.py:627-739).  A
    missing file raises FileNotFoundError; a header that disagrees with the
    target dims raises ValueError."""
    input_dir = Path(input_dir)
    with ExpertStoreWriter(output_dir, num_layers, num_experts, hidden_dim, intermediate_dim,
                           group_size, model_type) as w:
        for layer in range(num_layers):
            for expert in range(num_experts):
                path = input_dir / legacy_expert_filename(layer, expert)
                if not path.exists():
                    raise FileNotFoundError(f"Missing expert file: {path}")
                (l, e, H, I, g), payload = _read_legacy(path)
                if (l, e, H, I, g) != (layer, expert, hidden_dim, intermediate_dim, group_size):
                    raise ValueError(f"{path}: header {(l, e, H, I, g)} does not match "
                                     f"{(layer, expert, hidden_dim, intermediate_dim, group_size)}")
                w.add(layer, expert, payload)
    return w.index


def iter_store_experts(store) -> Iterator[Tuple[int, int, Dict[str, torch.Tensor]]]:
    """(layer, expert, six host tensors) for every entry of an open
    PackedExpertStore, in index order."""
    for (layer, expert) in sorted(store.index, key=lambda k: store.index[k].offset):
        blob, layout = store.get_expert_blob(layer, expert)
        yield layer, expert, blob_tensors(blob, store.hidden_dim, store.intermediate_dim,
                                          store.group_size)
