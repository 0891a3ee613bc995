"""Packed INT4 expert storage: GPU slots, pinned staging, experts.bin/.idx reader.

Counterpart of the reference's cache/packed_expert_store.py, re-laid for a
288 GB HBM part:

* ``GpuExpertSlot`` (reference :111-331) keeps the reference attributes
  (``gate_packed``, ``gate_scales``, ... , ``group_size``, ``ready_event``,
  ``dequantize``, ``_cached_fp16``, ``wait_ready``) but backs all six tensors
  with ONE contiguous HBM slab in BlobLayout order, so a load is one
  hipMemcpyAsync of the whole blob instead of six, and the slab address table
  for the grouped kernels is one pointer per expert.
* ``PinnedStagingRing`` (reference :334-395): pinned host slots reused only
  after the event of the copy that read them has completed.
* ``PackedExpertStore`` (reference :398-624): experts.idx JSON (format 2.0) +
  experts.bin, mmap'd (MADV_SEQUENTIAL) or read into RAM; loads go mmap ->
  pinned staging (host memcpy) -> one async H2D on a dedicated copy stream,
  then ``ready_event`` is recorded on that stream.

Copy streams are created at default priority.
"""
from __future__ import annotations

import json
import mmap
import os
import threading
import warnings
from collections import deque
from concurrent.futures import ThreadPoolExecutor
from dataclasses import dataclass
from pathlib import Path
from typing import Dict, Optional, Tuple

import torch

from .blob_layout import BlobLayout

__all__ = ["BlobLayout", "ExpertIndex", "GpuExpertSlot", "PinnedStagingRing", "PackedExpertStore"]


@dataclass
class ExpertIndex:
    layer_idx: int
    expert_idx: int
    offset: int
    size: int
    hidden_dim: int
    intermediate_dim: int
    group_size: int


def _slab_views(slab: torch.Tensor, layout: BlobLayout, H: int, I: int, g: int) -> dict:
    views = {}
    for name, (shape, dtype) in BlobLayout.shapes(H, I, g).items():
        off = getattr(layout, f"{name}_offset")
        size = getattr(layout, f"{name}_size")
        v = slab[off:off + size]
        if dtype == "float16":
            v = v.view(torch.float16)
        views[name] = v.view(*shape)
    return views


class GpuExpertSlot:
    """One expert's INT4 weights resident on the GPU (one slab, six views)."""

    def __init__(self, slot_idx: int, hidden_dim: int, intermediate_dim: int, group_size: int,
                 device: torch.device, slab: Optional[torch.Tensor] = None):
        self.slot_idx = slot_idx
        self.hidden_dim = hidden_dim
        self.intermediate_dim = intermediate_dim
        self.group_size = group_size
        self.device = torch.device(device)
        self.layer_idx: Optional[int] = None
        self.expert_idx: Optional[int] = None
        self.layout = BlobLayout.from_dims(hidden_dim, intermediate_dim, group_size)
        if slab is None:
            slab = torch.empty(self.layout.total_size, dtype=torch.uint8, device=self.device)
        elif (slab.dtype != torch.uint8 or slab.numel() != self.layout.total_size
              or not slab.is_contiguous() or slab.device != self.device):
            raise ValueError("slab must be a contiguous uint8 tensor of the blob size on "
                             f"{self.device} ({self.layout.total_size} bytes)")
        # a caller-provided slab is a window of a larger arena (one allocation per layer)
        self.slab = slab
        for name, view in _slab_views(self.slab, self.layout, hidden_dim, intermediate_dim,
                                      group_size).items():
            setattr(self, name, view)
        self._cached_fp16: Optional[Dict[str, torch.Tensor]] = None
        self.ready_event = torch.cuda.Event() if self.device.type == "cuda" else None

    def load_from_pinned(self, pinned_buffer: torch.Tensor, layout: BlobLayout, layer_idx: int,
                         expert_idx: int, stream: Optional[torch.cuda.Stream] = None):
        """Async copy of a whole blob (pinned host, BlobLayout order) into the slab."""
        assert layout.total_size == self.layout.total_size, "blob layout mismatch"
        self.layer_idx = layer_idx
        self.expert_idx = expert_idx
        self._cached_fp16 = None
        src = pinned_buffer.view(torch.uint8).view(-1)[: self.layout.total_size]
        if self.device.type == "cuda" and stream is not None:
            with torch.cuda.stream(stream):
                self.slab.copy_(src, non_blocking=True)
        else:
            self.slab.copy_(src, non_blocking=self.device.type == "cuda")

    def load_from_tensors(self, tensors: dict, layer_idx: int = 0, expert_idx: int = 0):
        """Fill from six tensors (already on any device), e.g. from the GPU packer."""
        self.layer_idx, self.expert_idx = layer_idx, expert_idx
        self._cached_fp16 = None
        for name in ("gate_packed", "gate_scales", "up_packed", "up_scales", "down_packed",
                     "down_scales"):
            getattr(self, name).copy_(tensors[name])

    def dequantize(self) -> Dict[str, torch.Tensor]:
        """fp16 gate/up/down weights (bit-exact dequant), cached until the next load."""
        if self._cached_fp16 is not None:
            return self._cached_fp16
        H, I = self.hidden_dim, self.intermediate_dim
        self._cached_fp16 = {
            "gate_proj": self._dequant_tensor(self.gate_packed, self.gate_scales, I, H),
            "up_proj": self._dequant_tensor(self.up_packed, self.up_scales, I, H),
            "down_proj": self._dequant_tensor(self.down_packed, self.down_scales, H, I),
        }
        return self._cached_fp16

    def _dequant_tensor(self, packed, scales, out_features: int, in_features: int):
        from ..kernels.int4_gemm import dequantize_int4
        assert packed.shape == (out_features, in_features // 2)
        return dequantize_int4(packed, scales, self.group_size)

    def size_bytes(self) -> int:
        return self.layout.total_size

    def wait_ready(self):
        """Make the current stream wait for this slot's last load (no host block)."""
        if self.ready_event is not None:
            torch.cuda.current_stream(self.device).wait_event(self.ready_event)

    def data_ptrs(self) -> Tuple[int, int, int, int, int, int]:
        return (self.gate_packed.data_ptr(), self.gate_scales.data_ptr(),
                self.up_packed.data_ptr(), self.up_scales.data_ptr(),
                self.down_packed.data_ptr(), self.down_scales.data_ptr())


class PinnedStagingRing:
    """Pinned host staging slots; a slot is reused only after its copy completed."""

    def __init__(self, num_slots: int, slot_size: int, device: torch.device):
        self.num_slots = num_slots
        self.slot_size = slot_size
        self.device = torch.device(device)
        pin = self.device.type == "cuda" and torch.cuda.is_available()
        self.slots = [torch.empty(slot_size, dtype=torch.uint8, pin_memory=pin)
                      for _ in range(num_slots)]
        self._lock = threading.Lock()
        self._free = deque(range(num_slots))
        self._inflight: deque = deque()  # (event, idx), oldest first

    def _reclaim_completed(self):
        keep = deque()
        for ev, idx in self._inflight:
            if ev is None or ev.query():
                self._free.append(idx)
            else:
                keep.append((ev, idx))
        self._inflight = keep

    def acquire(self) -> Tuple[int, torch.Tensor]:
        """Next free slot; if none, wait for the oldest in-flight copy."""
        with self._lock:
            self._reclaim_completed()
            if not self._free:
                if not self._inflight:
                    raise RuntimeError("PinnedStagingRing: every slot is acquired and none is "
                                       "in flight (release() each acquired slot)")
                ev, idx = self._inflight.popleft()
                if ev is not None:
                    ev.synchronize()
                self._free.append(idx)
            idx = self._free.popleft()
            return idx, self.slots[idx]

    def release(self, idx: int, ev: Optional[torch.cuda.Event]):
        """Slot idx may be reused once ev (the copy reading it) has completed."""
        with self._lock:
            self._inflight.append((ev, idx))


# Blob reads: pieces of 8 MiB on up to eight threads (one Mixtral expert is
# twelve pieces).
_READ_CHUNK = 8 << 20
_READ_THREADS = 8


class PackedExpertStore:
    """experts.idx + experts.bin reader feeding GPU slots through pinned staging."""

    def __init__(self, index_path, bin_path=None, device: torch.device = torch.device("cuda"),
                 use_mmap: bool = True, num_staging_slots: int = 4):
        index_path = Path(index_path)
        self.device = torch.device(device)
        self.use_mmap = use_mmap
        with open(index_path) as f:
            index_data = json.load(f)
        self.format_version = index_data["format_version"]
        self.quant_config = index_data["quant_config"]
        self.model_config = index_data["model_config"]
        self.model_type = index_data.get("model_type")
        H = self.model_config["hidden_dim"]
        I = self.model_config["intermediate_dim"]
        g = self.quant_config["group_size"]
        self.index: Dict[Tuple[int, int], ExpertIndex] = {}
        for e in index_data["experts"]:
            key = (e["layer_idx"], e["expert_idx"])
            self.index[key] = ExpertIndex(e["layer_idx"], e["expert_idx"], e["offset"], e["size"],
                                          H, I, g)
        self.layout = BlobLayout.from_dims(H, I, g)
        self.bin_path = Path(bin_path) if bin_path is not None else index_path.parent / "experts.bin"
        self._file = None
        self._mmap = None
        self._data = None
        if use_mmap:
            self._file = open(self.bin_path, "rb")
            self._mmap = mmap.mmap(self._file.fileno(), 0, access=mmap.ACCESS_READ)
            try:
                self._mmap.madvise(mmap.MADV_SEQUENTIAL)
            except (AttributeError, OSError):
                pass
        else:
            with open(self.bin_path, "rb") as f:
                self._data = memoryview(f.read())
        for ent in self.index.values():
            if ent.size != self.layout.total_size:
                raise ValueError(f"expert ({ent.layer_idx}, {ent.expert_idx}) size {ent.size} "
                                 f"!= blob layout {self.layout.total_size}")
        self.staging = PinnedStagingRing(num_staging_slots, self.layout.total_size, self.device)
        self.memcpy_stream = (torch.cuda.Stream(device=self.device)
                              if self.device.type == "cuda" and torch.cuda.is_available() else None)
        self.load_count = 0
        self.total_bytes_loaded = 0
        # the compute thread (misses) and the cache manager's prefetch thread
        # both load: one reader pool, made under the lock, and the counters
        # updated under it
        self._lock = threading.Lock()
        self._readers: Optional[ThreadPoolExecutor] = None

    @property
    def hidden_dim(self) -> int:
        return self.model_config["hidden_dim"]

    @property
    def intermediate_dim(self) -> int:
        return self.model_config["intermediate_dim"]

    @property
    def group_size(self) -> int:
        return self.quant_config["group_size"]

    def prefault_expert(self, layer_idx: int, expert_idx: int):
        key = (layer_idx, expert_idx)
        if key not in self.index or not self.use_mmap:
            return
        ent = self.index[key]
        try:
            page = mmap.PAGESIZE
            start = ent.offset - ent.offset % page
            self._mmap.madvise(mmap.MADV_WILLNEED, start, ent.size + ent.offset - start)
        except (AttributeError, OSError, ValueError):
            pass

    def get_expert_blob(self, layer_idx: int, expert_idx: int):
        key = (layer_idx, expert_idx)
        if key not in self.index:
            raise ValueError(f"Expert ({layer_idx}, {expert_idx}) not in index")
        ent = self.index[key]
        self._count(ent.size)
        src = self._mmap if self.use_mmap else self._data
        return src[ent.offset:ent.offset + ent.size], self.layout

    def load_to_staging(self, layer_idx: int, expert_idx: int):
        if self._file is None:
            blob, layout = self.get_expert_blob(layer_idx, expert_idx)
            slot_idx, staging = self.staging.acquire()
            with warnings.catch_warnings():  # a read-only window, only copied from
                warnings.simplefilter("ignore", UserWarning)
                t = torch.frombuffer(blob, dtype=torch.uint8)
            staging[: t.numel()].copy_(t)
            return slot_idx, staging, layout
        # read the blob from the file straight into the pinned slot, in
        # _READ_CHUNK pieces on a few threads (the read releases the GIL):
        # kernel copies out of the page cache (slicing the mmap would first
        # copy it into a bytes object, then into the slot)
        key = (layer_idx, expert_idx)
        if key not in self.index:
            raise ValueError(f"Expert ({layer_idx}, {expert_idx}) not in index")
        ent = self.index[key]
        slot_idx, staging = self.staging.acquire()
        dst = memoryview(staging.numpy())[: ent.size]
        fd = self._file.fileno()

        def read_piece(lo: int) -> bool:
            hi = min(lo + _READ_CHUNK, ent.size)
            while lo < hi:
                k = os.preadv(fd, [dst[lo:hi]], ent.offset + lo)
                if k <= 0:
                    return False
                lo += k
            return True

        starts = range(0, ent.size, _READ_CHUNK)
        with self._lock:
            if self._readers is None:
                self._readers = ThreadPoolExecutor(max_workers=_READ_THREADS)
            readers = self._readers
        if not all(readers.map(read_piece, starts)):
            self.staging.release(slot_idx, None)
            raise IOError(f"experts.bin ended inside expert ({layer_idx}, {expert_idx})")
        self._count(ent.size)
        return slot_idx, staging, self.layout

    def load_to_gpu_slot(self, layer_idx: int, expert_idx: int, gpu_slot: GpuExpertSlot,
                         stream: Optional[torch.cuda.Stream] = None):
        """mmap -> pinned staging -> one async H2D into the slot's slab."""
        staging_idx, staging, layout = self.load_to_staging(layer_idx, expert_idx)
        if stream is None:
            stream = self.memcpy_stream
        if stream is not None and gpu_slot.device.type == "cuda":
            # the slab may still be read by kernels already queued on the compute
            # stream (an evicted expert): the overwrite waits for them
            stream.wait_stream(torch.cuda.current_stream(gpu_slot.device))
        gpu_slot.load_from_pinned(staging, layout, layer_idx, expert_idx, stream=stream)
        if stream is not None and gpu_slot.ready_event is not None:
            gpu_slot.ready_event.record(stream)
            self.staging.release(staging_idx, gpu_slot.ready_event)
            return gpu_slot.ready_event
        self.staging.release(staging_idx, None)
        return None

    def _count(self, nbytes: int) -> None:
        with self._lock:
            self.load_count += 1
            self.total_bytes_loaded += nbytes

    def get_stats(self) -> Dict:
        return {"load_count": self.load_count, "total_bytes_loaded": self.total_bytes_loaded,
                "total_mb_loaded": self.total_bytes_loaded / (1024 * 1024)}

    def close(self):
        lock = getattr(self, "_lock", None)
        if lock is not None:
            with lock:
                readers, self._readers = self._readers, None
            if readers is not None:
                readers.shutdown(wait=True)
        if self._mmap is not None:
            try:
                self._mmap.close()
            except (ValueError, OSError, BufferError):
                pass
            self._mmap = None
        if self._file is not None:
            try:
                self._file.close()
            except (ValueError, OSError):
                pass
            self._file = None

    def __del__(self):
        self.close()
