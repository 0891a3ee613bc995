"""Per-layer INT4 expert residency: which experts occupy which HBM slots.

Counterpart of the reference's cache/expert_cache.py (``PerLayerCache``
:54-787, ``ExpertCacheManager`` :790-1308) for the packed INT4 path.  The
policy is the reference's:

* slots are split into tiers PINNED / HOT / PROBATION; a new expert enters the
  first empty slot in the order probation, hot, pinned (:334-352);
* a hit counts; the second hit of a probation expert promotes it into an
  empty hot slot, or swaps it with the least-frequently-used hot expert when it
  has strictly more hits (:206-219, :255-283);
* a miss evicts the LFU (hit_count, then last_access) evictable probation
  expert, else the LFU evictable hot expert; pinned-tier slots, timed pins
  (``pin_expert``, :584-595) and adaptive pins (the top ``pin_count`` experts
  by decayed access frequency, decay 0.995 per access, refreshed by the
  manager every 16 tokens, :114-118, :221-253, :1023-1037) are never evicted;
* the manager gives layers < 12 and >= 14 one slot more than the base count
  (:890-909) and moves slots from low-miss to high-miss layers every
  ``realloc_interval_tokens`` (:1039-1136), capped at ``max_slots_per_layer``.

What is laid out differently for a 288 GB part:

* ``make_resident()`` gives a layer one slot per expert carved from ONE HBM
  arena (a single allocation of E x blob bytes) and loads every expert once.
  Mixtral (23.25 GB) and GLM-4.5-Air (51.38 GB) both fit several times over,
  so on MI355X nothing is ever evicted and the MoE layer skips the per-call
  host round trip (``is_resident``).
* Slot contents are ``GpuExpertSlot`` objects: one contiguous slab per expert
  in blob order, filled by one async copy on the store's copy stream, which
  first waits for the compute stream so that an evicted slab is not
  overwritten under a kernel still reading it.
* ``hold(experts)`` keeps the experts of one grouped launch from evicting one
  another while they are made resident together (the reference computes one
  expert at a time, so it never needs this).
* The decayed access frequency is kept with a running scale factor instead of
  multiplying every entry on every access (same values, O(1) per access).
* Tiers are a slot attribute, so a slot added to the hot or pinned tier
  belongs to that tier wherever it sits in the slot list.
"""
from __future__ import annotations

import queue
import threading
import time
from contextlib import contextmanager
from dataclasses import dataclass, field
from enum import Enum
from typing import Dict, Iterable, List, Optional, Set, Tuple

import torch

from .packed_expert_store import GpuExpertSlot

__all__ = ["SlotTier", "SlotInfo", "ExpertCacheConfig", "MoEModelConfig", "PerLayerCache",
           "ExpertCacheManager"]


class SlotTier(Enum):
    """Tier of a slot (reference cache/expert_cache.py:23-27)."""
    PINNED = "pinned"
    HOT = "hot"
    PROBATION = "probation"


@dataclass
class SlotInfo:
    """Slot metadata (reference cache/expert_cache.py:30-38)."""
    slot_idx: int
    tier: SlotTier
    expert_id: Optional[Tuple[int, int]] = None  # (layer_idx, expert_idx)
    hit_count: int = 0
    last_access: float = 0.0
    pinned_until: Optional[float] = None


@dataclass
class ExpertCacheConfig:
    """Per-layer slot configuration (reference config.py:254-283)."""
    pinned_slots: int = 1
    hot_slots: int = 1
    probation_slots: int = 1
    enable_dynamic_slots: bool = True
    realloc_interval_tokens: int = 512
    miss_rate_threshold: float = 0.3
    max_slots_per_layer: int = 4
    enable_affinity_bonus: bool = True
    affinity_bonus: float = 0.1
    affinity_entropy_threshold: float = 0.5
    enable_prefetch: bool = True
    # MI355X sizing: when a packed store is attached, every layer whose experts
    # fit the device's free HBM (less the headroom kept for activations, KV
    # cache and workspaces) becomes one resident arena; only the layers that
    # do not fit use the slot cache above (the reference's 16 GB heuristic,
    # config.py:259-267).  288 GB holds all of Mixtral-8x7B's experts (23.3 GB)
    # or GLM-4.5-Air's (51.4 GB).
    resident_when_fits: bool = True
    resident_headroom_bytes: int = 16 << 30

    @property
    def slots_per_layer(self) -> int:
        return self.pinned_slots + self.hot_slots + self.probation_slots


@dataclass
class MoEModelConfig:
    """The model dimensions the cache needs (reference config.py:22-69 for
    Mixtral; ``glm4_air()`` gives the routed-expert dims of GLM-4.5-Air)."""
    num_layers: int = 32
    num_experts: int = 8
    hidden_dim: int = 4096
    intermediate_dim: int = 14336

    @classmethod
    def glm4_air(cls) -> "MoEModelConfig":
        return cls(num_layers=45, num_experts=128, hidden_dim=4096, intermediate_dim=1408)

    @property
    def expert_params(self) -> int:
        return 3 * self.hidden_dim * self.intermediate_dim

    @property
    def expert_size_bytes(self) -> int:
        """fp16 bytes of one expert (reference config.py:55-58)."""
        return self.expert_params * 2


_ARENA_ALIGN = 256


class PerLayerCache:
    """Expert slots of one transformer layer (reference cache/expert_cache.py:54-787)."""

    def __init__(self, layer_idx: int, num_experts: int, expert_size_bytes: int,
                 config: ExpertCacheConfig, device: torch.device,
                 dtype: torch.dtype = torch.float16):
        self.layer_idx = layer_idx
        self.num_experts = num_experts
        self.expert_size_bytes = expert_size_bytes
        self.config = config
        self.device = torch.device(device)
        self.dtype = dtype
        self.slots: List[SlotInfo] = []
        for tier, n in ((SlotTier.PINNED, config.pinned_slots), (SlotTier.HOT, config.hot_slots),
                        (SlotTier.PROBATION, config.probation_slots)):
            for _ in range(n):
                self.slots.append(SlotInfo(len(self.slots), tier))
        self.expert_to_slot: Dict[int, SlotInfo] = {}
        self.gpu_int4_slots: Dict[int, GpuExpertSlot] = {}  # slot_idx -> slot buffers
        self.gpu_weights: Dict[int, Dict[str, torch.Tensor]] = {}  # slot_idx -> fp16 weights
        self.ram_weights: Dict[int, Dict[str, torch.Tensor]] = {}  # fp16 (non-packed) mode
        self.hits = 0
        self.misses = 0
        self.promotions = 0
        self.evictions = 0
        # decayed access frequency: freq[e] = _freq_raw[e] * _freq_scale
        self._freq_raw: Dict[int, float] = {}
        self._freq_scale = 1.0
        self.freq_decay = 0.995
        self.pin_count = 1
        self.adaptive_pins: Set[int] = set()
        self._held: Set[int] = set()
        self._lock = threading.RLock()
        self.packed_store = None
        self.use_packed_mode = False
        self._packed_hidden_dim = 0
        self._packed_intermediate_dim = 0
        self._packed_group_size = 0
        self._arena: Optional[torch.Tensor] = None
        self.resident = False

    # ------------------------------------------------------------------ tiers
    @property
    def pinned_slots(self) -> int:
        return sum(1 for s in self.slots if s.tier is SlotTier.PINNED)

    @property
    def hot_slots(self) -> int:
        return sum(1 for s in self.slots if s.tier is SlotTier.HOT)

    @property
    def probation_slots(self) -> int:
        return sum(1 for s in self.slots if s.tier is SlotTier.PROBATION)

    @property
    def total_slots(self) -> int:
        return len(self.slots)

    def _tier(self, tier: SlotTier) -> List[SlotInfo]:
        return [s for s in self.slots if s.tier is tier]

    def get_slot_count(self) -> int:
        return len(self.slots)

    # ------------------------------------------------------------ frequencies
    @property
    def expert_freq(self) -> Dict[int, float]:
        """Decayed access frequency per expert (reference :114-118)."""
        return {e: r * self._freq_scale for e, r in self._freq_raw.items()}

    def _record_expert_access(self, expert_idx: int):
        """Every frequency decays by freq_decay, then this expert's gains 1
        (reference :221-227)."""
        self._freq_scale *= self.freq_decay
        if self._freq_scale < 1e-200:  # renormalise long before underflow
            for e in self._freq_raw:
                self._freq_raw[e] *= self._freq_scale
            self._freq_scale = 1.0
        self._freq_raw[expert_idx] = self._freq_raw.get(expert_idx, 0.0) + 1.0 / self._freq_scale

    def refresh_adaptive_pins(self, debug: bool = False):
        """Pin the top pin_count experts by decayed frequency that are cached
        (reference :229-253)."""
        with self._lock:
            if not self._freq_raw or self.pin_count == 0:
                return
            ranked = sorted(self._freq_raw.items(), key=lambda kv: -kv[1])
            top = [e for e, _ in ranked[: self.pin_count]]
            self.adaptive_pins = {e for e in top if e in self.expert_to_slot}
            if debug:
                print(f"[L{self.layer_idx} pins] {sorted(self.adaptive_pins)}")

    # ------------------------------------------------------------ hits / tiers
    def _record_hit(self, slot: SlotInfo):
        """Count a hit; a probation expert's second hit tries promotion (:206-219)."""
        self.hits += 1
        slot.hit_count += 1
        slot.last_access = time.time()
        if slot.expert_id is not None:
            self._record_expert_access(slot.expert_id[1])
        if slot.tier is SlotTier.PROBATION and slot.hit_count >= 2:
            self._try_promote(slot)

    def _try_promote(self, slot: SlotInfo):
        """Move into an empty hot slot, else swap with the LFU hot expert when
        this one has strictly more hits (:255-283)."""
        hot = self._tier(SlotTier.HOT)
        for dst in hot:
            if dst.expert_id is None:
                self._swap_slots(slot, dst)
                self.promotions += 1
                return
        cands = [s for s in hot if s.expert_id is not None and s.pinned_until is None]
        if cands:
            lfu = min(cands, key=lambda s: (s.hit_count, s.last_access))
            if slot.hit_count > lfu.hit_count:
                self._swap_slots(slot, lfu)
                self.promotions += 1

    def _swap_slots(self, a: SlotInfo, b: SlotInfo):
        """Exchange the experts of two slots; each slot keeps its tier (:285-332).
        Buffers, counters and a timed pin move with their expert (no data copy)."""
        for table in (self.gpu_weights, self.gpu_int4_slots):
            va, vb = table.pop(a.slot_idx, None), table.pop(b.slot_idx, None)
            if va is not None:
                table[b.slot_idx] = va
            if vb is not None:
                table[a.slot_idx] = vb
        for idx in (a.slot_idx, b.slot_idx):
            if idx in self.gpu_int4_slots:
                self.gpu_int4_slots[idx].slot_idx = idx
        a.expert_id, b.expert_id = b.expert_id, a.expert_id
        a.hit_count, b.hit_count = b.hit_count, a.hit_count
        a.last_access, b.last_access = b.last_access, a.last_access
        a.pinned_until, b.pinned_until = b.pinned_until, a.pinned_until
        for s in (a, b):
            if s.expert_id is not None:
                self.expert_to_slot[s.expert_id[1]] = s

    # ------------------------------------------------------ allocate / evict
    def _evictable(self, s: SlotInfo, now: float) -> bool:
        if s.pinned_until is not None and s.pinned_until >= now:
            return False
        if s.expert_id is not None:
            e = s.expert_id[1]
            if e in self.adaptive_pins or e in self._held:
                return False
        return True

    def _allocate_slot(self, expert_idx: int) -> SlotInfo:
        """Empty probation, hot, pinned slot; else evict the LFU evictable
        probation, then hot, expert (:334-393)."""
        for tier in (SlotTier.PROBATION, SlotTier.HOT, SlotTier.PINNED):
            for s in self._tier(tier):
                if s.expert_id is None:
                    return s
        now = time.time()
        for tier in (SlotTier.PROBATION, SlotTier.HOT):
            cands = [s for s in self._tier(tier) if self._evictable(s, now)]
            if cands:
                victim = min(cands, key=lambda s: (s.hit_count, s.last_access))
                self._evict(victim)
                return victim
        raise RuntimeError(f"Layer {self.layer_idx}: No evictable slots available")

    def _evict(self, slot: SlotInfo):
        """Drop the slot's expert; its INT4 buffers stay allocated for reuse (:395-421)."""
        if slot.expert_id is None:
            return
        del self.expert_to_slot[slot.expert_id[1]]
        self.gpu_weights.pop(slot.slot_idx, None)
        gs = self.gpu_int4_slots.get(slot.slot_idx)
        if gs is not None:
            gs._cached_fp16 = None
        slot.expert_id = None
        slot.hit_count = 0
        slot.last_access = 0.0
        slot.pinned_until = None
        self.evictions += 1

    def add_slot(self, tier: SlotTier = SlotTier.PROBATION) -> bool:
        """One more slot unless at max_slots_per_layer (:423-447)."""
        with self._lock:
            if self.resident or len(self.slots) >= self.config.max_slots_per_layer:
                return False
            self.slots.append(SlotInfo(len(self.slots), tier))
            return True

    def remove_slot(self) -> bool:
        """Remove the least valuable slot: empty probation, empty hot, LFU
        probation, LFU hot; never the last one (:449-530).  Remaining slots are
        renumbered and their buffers follow them; the removed slot's buffers are
        freed."""
        with self._lock:
            if self.resident or len(self.slots) <= 1:
                return False
            target = None
            for tier in (SlotTier.PROBATION, SlotTier.HOT):
                for s in reversed(self._tier(tier)):
                    if s.expert_id is None:
                        target = s
                        break
                if target is not None:
                    break
            if target is None:
                for tier in (SlotTier.PROBATION, SlotTier.HOT):
                    occ = [s for s in self._tier(tier) if s.expert_id is not None]
                    if occ:
                        target = min(occ, key=lambda s: (s.hit_count, s.last_access))
                        break
            if target is None:
                return False
            self._evict(target)
            self.slots.remove(target)
            self.gpu_weights.pop(target.slot_idx, None)
            self.gpu_int4_slots.pop(target.slot_idx, None)
            weights = {s.slot_idx: self.gpu_weights.pop(s.slot_idx) for s in self.slots
                       if s.slot_idx in self.gpu_weights}
            bufs = {s.slot_idx: self.gpu_int4_slots.pop(s.slot_idx) for s in self.slots
                    if s.slot_idx in self.gpu_int4_slots}
            for i, s in enumerate(self.slots):
                if s.slot_idx in weights:
                    self.gpu_weights[i] = weights[s.slot_idx]
                if s.slot_idx in bufs:
                    bufs[s.slot_idx].slot_idx = i
                    self.gpu_int4_slots[i] = bufs[s.slot_idx]
                s.slot_idx = i
            return True

    # ----------------------------------------------------------------- loads
    def _gpu_slot(self, slot: SlotInfo) -> GpuExpertSlot:
        gs = self.gpu_int4_slots.get(slot.slot_idx)
        if gs is None:
            gs = GpuExpertSlot(slot.slot_idx, self._packed_hidden_dim,
                               self._packed_intermediate_dim, self._packed_group_size,
                               self.device)
            self.gpu_int4_slots[slot.slot_idx] = gs
        return gs

    def _load_int4_to_slot(self, expert_idx: int, slot: SlotInfo):
        """Async blob load into the slot's buffers on the store's copy stream;
        fp16 weights are not made (:650-679)."""
        if not self.use_packed_mode:
            raise RuntimeError(f"Layer {self.layer_idx}: no packed store attached "
                               "(ExpertCacheManager.set_packed_store)")
        gs = self._gpu_slot(slot)
        self.packed_store.load_to_gpu_slot(self.layer_idx, expert_idx, gs)
        slot.expert_id = (self.layer_idx, expert_idx)
        slot.hit_count = 1
        slot.last_access = time.time()
        slot.pinned_until = None
        self.expert_to_slot[expert_idx] = slot

    def prefetch_int4_slot(self, expert_idx: int) -> GpuExpertSlot:
        """Start loading a missing expert (may evict); no hit/miss accounting (:601-620)."""
        with self._lock:
            s = self.expert_to_slot.get(expert_idx)
            if s is not None:
                return self.gpu_int4_slots[s.slot_idx]
            s = self._allocate_slot(expert_idx)
            self._load_int4_to_slot(expert_idx, s)
            return self.gpu_int4_slots[s.slot_idx]

    def get_int4_slot(self, expert_idx: int, prefetched_miss: bool = False) -> GpuExpertSlot:
        """INT4 slot ready for compute on the current stream; records the hit or
        miss (the one place stats are counted, :622-648).  A caller that
        prefetched this expert because it was missing passes
        ``prefetched_miss=True`` so the access counts as the miss it was (the
        reference counts it as a hit, model/mixtral.py:309-320)."""
        with self._lock:
            s = self.expert_to_slot.get(expert_idx)
            if s is not None and prefetched_miss:
                self.misses += 1
                self._record_expert_access(expert_idx)
            elif s is not None:
                self._record_hit(s)
                s = self.expert_to_slot[expert_idx]  # promotion may have moved it
            else:
                self.misses += 1
                self._record_expert_access(expert_idx)
                s = self._allocate_slot(expert_idx)
                self._load_int4_to_slot(expert_idx, s)
            gs = self.gpu_int4_slots[s.slot_idx]
            gs.wait_ready()
            return gs

    @contextmanager
    def hold(self, experts: Iterable[int]):
        """Keep these experts from being evicted inside the block (they are used
        by one grouped launch)."""
        experts = set(int(e) for e in experts)
        with self._lock:
            if len(experts) > len(self.slots):
                raise RuntimeError(f"Layer {self.layer_idx}: {len(experts)} experts in one "
                                   f"call but only {len(self.slots)} slots")
            prev = self._held
            self._held = prev | experts
            try:
                yield
            finally:
                self._held = prev

    # ------------------------------------------------------- resident layer
    def make_resident(self):
        """One slot per expert in a single HBM arena; every expert is loaded once
        and nothing is evicted afterwards."""
        with self._lock:
            if not self.use_packed_mode:
                raise RuntimeError("make_resident needs a packed store")
            size = self.packed_store.layout.total_size
            stride = (size + _ARENA_ALIGN - 1) // _ARENA_ALIGN * _ARENA_ALIGN
            E = self.num_experts
            self.expert_to_slot.clear()
            self.gpu_int4_slots.clear()
            self.gpu_weights.clear()
            self._arena = None
            self._arena = torch.empty(E * stride, dtype=torch.uint8, device=self.device)
            self.slots = [SlotInfo(e, SlotTier.PINNED) for e in range(E)]
            for e in range(E):
                window = self._arena[e * stride: e * stride + size]
                self.gpu_int4_slots[e] = GpuExpertSlot(
                    e, self._packed_hidden_dim, self._packed_intermediate_dim,
                    self._packed_group_size, self.device, slab=window)
                self._load_int4_to_slot(e, self.slots[e])
            self.resident = True

    def is_resident(self) -> bool:
        return self.resident

    def resident_slots(self) -> List[GpuExpertSlot]:
        """Slots in expert order (only for a resident layer)."""
        if not self.resident:
            raise RuntimeError(f"Layer {self.layer_idx} is not resident")
        return [self.gpu_int4_slots[self.expert_to_slot[e].slot_idx]
                for e in range(self.num_experts)]

    # ------------------------------------------------- fp16 (dequant) path
    def register_expert(self, expert_idx: int, weights: Dict[str, torch.Tensor]):
        """fp16 weights kept in (pinned) host memory for the non-packed mode (:120-145)."""
        pin = torch.cuda.is_available() and self.device.type == "cuda"
        held = {}
        for name, t in weights.items():
            h = torch.empty(t.shape, dtype=self.dtype, pin_memory=pin)
            h.copy_(t)
            held[name] = h
        with self._lock:
            self.ram_weights[expert_idx] = held

    def _load_to_slot(self, expert_idx: int, slot: SlotInfo):
        if self.use_packed_mode:
            self._load_int4_to_slot(expert_idx, slot)
            return
        if expert_idx not in self.ram_weights:
            raise ValueError(f"Expert {expert_idx} not registered in RAM")
        self.gpu_weights[slot.slot_idx] = {n: t.to(self.device, non_blocking=True)
                                           for n, t in self.ram_weights[expert_idx].items()}
        slot.expert_id = (self.layer_idx, expert_idx)
        slot.hit_count = 1
        slot.last_access = time.time()
        slot.pinned_until = None
        self.expert_to_slot[expert_idx] = slot

    def get_weights(self, expert_idx: int) -> Dict[str, torch.Tensor]:
        """fp16 gate_proj/up_proj/down_proj on the device (:147-204); in packed
        mode they are dequantised (bit-exact) from the INT4 slot."""
        with self._lock:
            s = self.expert_to_slot.get(expert_idx)
            if s is not None:
                self._record_hit(s)
                s = self.expert_to_slot[expert_idx]
            else:
                self.misses += 1
                self._record_expert_access(expert_idx)
                s = self._allocate_slot(expert_idx)
                self._load_to_slot(expert_idx, s)
            if s.slot_idx not in self.gpu_weights:
                if not self.use_packed_mode:
                    self._load_to_slot(expert_idx, s)
                else:
                    gs = self.gpu_int4_slots[s.slot_idx]
                    gs.wait_ready()
                    self.gpu_weights[s.slot_idx] = gs.dequantize()
            return self.gpu_weights[s.slot_idx]

    def clear_fp16_cache(self):
        """Drop every dequantised fp16 copy; INT4 data stays (:706-738)."""
        with self._lock:
            self.gpu_weights.clear()
            for gs in self.gpu_int4_slots.values():
                gs._cached_fp16 = None

    def clear_expert_fp16(self, expert_idx: int):
        with self._lock:
            s = self.expert_to_slot.get(expert_idx)
            if s is None:
                return
            self.gpu_weights.pop(s.slot_idx, None)
            gs = self.gpu_int4_slots.get(s.slot_idx)
            if gs is not None:
                gs._cached_fp16 = None

    # ----------------------------------------------------------- misc / stats
    def pin_expert(self, expert_idx: int, duration_sec: float = 1.0):
        """Protect a cached expert from eviction for duration_sec (:584-595)."""
        with self._lock:
            s = self.expert_to_slot.get(expert_idx)
            if s is not None:
                s.pinned_until = time.time() + duration_sec

    def is_cached(self, expert_idx: int) -> bool:
        return expert_idx in self.expert_to_slot

    def set_packed_mode(self, store, hidden_dim: int, intermediate_dim: int, group_size: int):
        """Attach a PackedExpertStore (:764-787)."""
        self.packed_store = store
        self.use_packed_mode = True
        self._packed_hidden_dim = hidden_dim
        self._packed_intermediate_dim = intermediate_dim
        self._packed_group_size = group_size

    def get_stats(self) -> Dict:
        """Counters and tier occupancy (reference :681-697, same keys)."""
        with self._lock:
            total = self.hits + self.misses

            def occ(t):
                return sum(1 for s in self._tier(t) if s.expert_id is not None)
            return {"layer": self.layer_idx, "hits": self.hits, "misses": self.misses,
                    "hit_rate": self.hits / max(1, total), "promotions": self.promotions,
                    "evictions": self.evictions, "cached_count": len(self.expert_to_slot),
                    "pinned_count": occ(SlotTier.PINNED), "hot_count": occ(SlotTier.HOT),
                    "probation_count": occ(SlotTier.PROBATION)}

    def reset_stats(self):
        with self._lock:
            self.hits = self.misses = self.promotions = self.evictions = 0


class ExpertCacheManager:
    """Per-layer caches for every MoE layer (reference cache/expert_cache.py:790-1308)."""

    def __init__(self, model_config, cache_config: ExpertCacheConfig,
                 device: torch.device = torch.device("cuda"), dtype: torch.dtype = torch.float16):
        self.model_config = model_config
        self.cache_config = cache_config
        self.device = torch.device(device)
        self.dtype = dtype
        self.expert_size_bytes = model_config.expert_size_bytes
        alloc = self._compute_slot_allocation(model_config.num_layers,
                                              cache_config.slots_per_layer)
        self.layer_caches: List[PerLayerCache] = []
        for layer_idx, n in enumerate(alloc):
            # per-layer split: no pinned tier, hot = n // 2, probation = rest (:838-853)
            cfg = ExpertCacheConfig(
                pinned_slots=0, hot_slots=n // 2, probation_slots=n - n // 2,
                enable_dynamic_slots=cache_config.enable_dynamic_slots,
                realloc_interval_tokens=cache_config.realloc_interval_tokens,
                miss_rate_threshold=cache_config.miss_rate_threshold,
                max_slots_per_layer=cache_config.max_slots_per_layer,
                enable_affinity_bonus=cache_config.enable_affinity_bonus,
                affinity_bonus=cache_config.affinity_bonus,
                affinity_entropy_threshold=cache_config.affinity_entropy_threshold,
                enable_prefetch=cache_config.enable_prefetch)
            self.layer_caches.append(PerLayerCache(layer_idx, model_config.num_experts,
                                                   self.expert_size_bytes, cfg, self.device,
                                                   dtype))
        self._slot_allocations = list(alloc)
        self.tokens_since_realloc = 0
        self.tokens_since_pin_refresh = 0
        self.pin_refresh_interval = 16
        self.packed_store = None
        self.use_packed_mode = False
        self.auto_resident_layers = 0
        self.sequence_lfu: Dict[int, Dict[int, Dict[int, float]]] = {}
        self.lfu_decay_rate = 0.95
        self.active_sequence_id: Optional[int] = None
        self.miss_burst_count = 0
        self.miss_burst_threshold = 8
        self.total_burst_events = 0
        self.total_load_time_ms = 0.0
        self.prefetch_queue: "queue.Queue" = queue.Queue()
        self._running = True
        self._prefetch_thread = threading.Thread(target=self._prefetch_worker, daemon=True)
        self._prefetch_thread.start()

    def _compute_slot_allocation(self, num_layers: int, base_slots: int) -> List[int]:
        """base + 1 slots for layers < 12 and >= 14 (:890-909)."""
        return [base_slots + 1 if (i < 12 or i >= 14) else base_slots for i in range(num_layers)]

    def set_packed_store(self, store):
        """Attach the packed INT4 store to every layer (:911-936), then make
        resident as many layers as the device's free HBM holds
        (``resident_plan``)."""
        self.packed_store = store
        self.use_packed_mode = True
        H = store.model_config["hidden_dim"]
        I = store.model_config["intermediate_dim"]
        g = store.quant_config["group_size"]
        for c in self.layer_caches:
            c.set_packed_mode(store, H, I, g)
        n = self.resident_plan()
        if n:
            self.make_resident(range(n))
        self.auto_resident_layers = n

    def _free_device_bytes(self) -> Optional[int]:
        """Free memory of the cache's device (None off the GPU)."""
        if self.device.type != "cuda" or not torch.cuda.is_available():
            return None
        return int(torch.cuda.mem_get_info(self.device)[0])

    def layer_resident_bytes(self) -> int:
        """HBM one resident layer takes (its arena)."""
        size = self.packed_store.layout.total_size
        stride = (size + _ARENA_ALIGN - 1) // _ARENA_ALIGN * _ARENA_ALIGN
        return stride * self.model_config.num_experts

    def resident_plan(self) -> int:
        """How many layers (from layer 0) to make resident: those whose arenas
        fit the free device memory less ``resident_headroom_bytes``; 0 when
        ``resident_when_fits`` is off or the device reports no figure."""
        if not self.cache_config.resident_when_fits or self.packed_store is None:
            return 0
        free = self._free_device_bytes()
        if free is None:
            return 0
        room = free - int(self.cache_config.resident_headroom_bytes)
        per = self.layer_resident_bytes()
        return int(max(0, min(len(self.layer_caches), room // per if per > 0 else 0)))

    def resident_bytes(self) -> int:
        """HBM that make_resident() needs for every layer."""
        if self.packed_store is None:
            raise RuntimeError("no packed store attached")
        return self.layer_resident_bytes() * len(self.layer_caches)

    def make_resident(self, layers: Optional[Iterable[int]] = None):
        """Load every expert of the given layers (all by default) into per-layer
        HBM arenas; those layers never evict or miss afterwards."""
        for i in (range(len(self.layer_caches)) if layers is None else layers):
            self.layer_caches[i].make_resident()

    def is_resident(self, layer_idx: int) -> bool:
        return self.layer_caches[layer_idx].is_resident()

    def resident_slots(self, layer_idx: int) -> List[GpuExpertSlot]:
        return self.layer_caches[layer_idx].resident_slots()

    def hold(self, layer_idx: int, experts: Iterable[int]):
        return self.layer_caches[layer_idx].hold(experts)

    def register_expert(self, layer_idx: int, expert_idx: int, weights: Dict[str, torch.Tensor]):
        self.layer_caches[layer_idx].register_expert(expert_idx, weights)

    def get_expert_weights(self, layer_idx: int, expert_idx: int) -> Dict[str, torch.Tensor]:
        t0 = time.time()
        w = self.layer_caches[layer_idx].get_weights(expert_idx)
        self.total_load_time_ms += (time.time() - t0) * 1000
        return w

    def is_cached(self, layer_idx: int, expert_idx: int) -> bool:
        return self.layer_caches[layer_idx].is_cached(expert_idx)

    def prefetch_int4_slot(self, layer_idx: int, expert_idx: int) -> GpuExpertSlot:
        return self.layer_caches[layer_idx].prefetch_int4_slot(expert_idx)

    def get_int4_slot(self, layer_idx: int, expert_idx: int,
                      prefetched_miss: bool = False) -> GpuExpertSlot:
        t0 = time.time()
        s = self.layer_caches[layer_idx].get_int4_slot(expert_idx, prefetched_miss)
        self.total_load_time_ms += (time.time() - t0) * 1000
        return s

    def clear_layer_fp16(self, layer_idx: int):
        self.layer_caches[layer_idx].clear_fp16_cache()

    def clear_expert_fp16(self, layer_idx: int, expert_idx: int):
        self.layer_caches[layer_idx].clear_expert_fp16(expert_idx)

    def prefetch(self, layer_idx: int, expert_indices: List[int]):
        """Queue loads of uncached experts for the background worker (:1000-1009)."""
        for e in expert_indices:
            if not self.is_cached(layer_idx, e):
                self.prefetch_queue.put((layer_idx, e))

    def _prefetch_worker(self):
        """Loads queued experts: packed mode starts the async INT4 load (no stats),
        fp16 mode copies the registered weights (:1138-1161)."""
        while self._running:
            try:
                layer_idx, e = self.prefetch_queue.get(timeout=0.01)
            except queue.Empty:
                continue
            try:
                if self.is_cached(layer_idx, e):
                    continue
                if self.use_packed_mode:
                    self.layer_caches[layer_idx].prefetch_int4_slot(e)
                else:
                    self.layer_caches[layer_idx].get_weights(e)
            except Exception as exc:  # the worker must survive a bad request
                print(f"Prefetch error: {exc}")
            finally:
                self.prefetch_queue.task_done()

    def pin_experts(self, expert_ids: List[Tuple[int, int]], duration_sec: float = 1.0):
        for layer_idx, e in expert_ids:
            self.layer_caches[layer_idx].pin_expert(e, duration_sec)

    def maybe_reallocate_slots(self, token_count: int = 1):
        """Pin refresh every pin_refresh_interval tokens, reallocation every
        realloc_interval_tokens when enabled (:1023-1047)."""
        self.tokens_since_pin_refresh += token_count
        if self.tokens_since_pin_refresh >= self.pin_refresh_interval:
            self.tokens_since_pin_refresh = 0
            self.refresh_adaptive_pins()
        if not self.cache_config.enable_dynamic_slots:
            return
        self.tokens_since_realloc += token_count
        if self.tokens_since_realloc < self.cache_config.realloc_interval_tokens:
            return
        self.tokens_since_realloc = 0
        self._do_reallocation()

    def refresh_adaptive_pins(self):
        for c in self.layer_caches:
            c.refresh_adaptive_pins()

    def _do_reallocation(self) -> int:
        """Move up to two slots from layers with miss rate < threshold/2 (most
        hits first) to layers above the threshold (most misses first) (:1062-1136).
        Returns the number of slots moved."""
        thr = self.cache_config.miss_rate_threshold
        cap = self.cache_config.max_slots_per_layer
        donors, recipients = [], []
        for c in self.layer_caches:
            if c.is_resident():
                continue
            miss = 1.0 - c.get_stats()["hit_rate"]
            n = c.get_slot_count()
            if miss > thr and n < cap:
                recipients.append((c.layer_idx, miss))
            elif miss < thr / 2 and n > 1:
                donors.append((c.layer_idx, miss))
        recipients.sort(key=lambda x: -x[1])
        donors.sort(key=lambda x: x[1])
        moved = 0
        for (r, _), (d, _) in zip(recipients, donors):
            if moved >= 2:
                break
            dc, rc = self.layer_caches[d], self.layer_caches[r]
            if dc.get_slot_count() <= 1 or rc.get_slot_count() >= cap:
                continue
            if dc.remove_slot() and rc.add_slot():
                self._slot_allocations[d] -= 1
                self._slot_allocations[r] += 1
                moved += 1
        return moved

    # per-sequence LFU (:1163-1258)
    def register_sequence(self, seq_id: int):
        if seq_id not in self.sequence_lfu:
            self.sequence_lfu[seq_id] = {i: {} for i in range(self.model_config.num_layers)}

    def unregister_sequence(self, seq_id: int):
        self.sequence_lfu.pop(seq_id, None)

    def set_active_sequence(self, seq_id: int):
        self.active_sequence_id = seq_id
        self.register_sequence(seq_id)

    def record_expert_use(self, seq_id: int, layer_idx: int, expert_idx: int):
        self.register_sequence(seq_id)
        lfu = self.sequence_lfu[seq_id][layer_idx]
        lfu[expert_idx] = lfu.get(expert_idx, 0.0) + 1.0

    def decay_sequence_lfu(self, seq_id: int):
        """Multiply by lfu_decay_rate; entries below 0.01 are dropped."""
        for lfu in self.sequence_lfu.get(seq_id, {}).values():
            for e in list(lfu):
                lfu[e] *= self.lfu_decay_rate
                if lfu[e] < 0.01:
                    del lfu[e]

    def get_sequence_hot_experts(self, seq_id: int, layer_idx: int, top_k: int = 4) -> List[int]:
        lfu = self.sequence_lfu.get(seq_id, {}).get(layer_idx, {})
        return [e for e, _ in sorted(lfu.items(), key=lambda kv: -kv[1])[:top_k]]

    def start_token_step(self):
        self.miss_burst_count = 0

    def end_token_step(self):
        if self.miss_burst_count > self.miss_burst_threshold:
            self.total_burst_events += 1
        if self.active_sequence_id is not None:
            self.decay_sequence_lfu(self.active_sequence_id)

    def record_miss(self, layer_idx: int):
        self.miss_burst_count += 1

    def get_stats(self) -> Dict:
        """Aggregate counters (reference :1260-1289, same keys)."""
        per = [c.get_stats() for c in self.layer_caches]
        hits = sum(s["hits"] for s in per)
        misses = sum(s["misses"] for s in per)
        rates = sorted(s["hit_rate"] for s in per)
        return {"total_hits": hits, "total_misses": misses,
                "hit_rate": hits / max(1, hits + misses),
                "total_evictions": sum(s["evictions"] for s in per),
                "total_promotions": sum(s["promotions"] for s in per),
                "avg_load_time_ms": self.total_load_time_ms / max(1, misses),
                "per_layer_stats": per,
                "layer_hit_rate_min": rates[0] if rates else 0.0,
                "layer_hit_rate_median": rates[len(rates) // 2] if rates else 0.0,
                "layer_hit_rate_max": rates[-1] if rates else 0.0,
                "miss_burst_events": self.total_burst_events,
                "active_sequences": len(self.sequence_lfu),
                "resident_layers": sum(1 for c in self.layer_caches if c.is_resident())}

    def reset_stats(self):
        for c in self.layer_caches:
            c.reset_stats()
        self.total_load_time_ms = 0.0
        self.total_burst_events = 0
        self.miss_burst_count = 0

    def shutdown(self):
        self._running = False
        t = getattr(self, "_prefetch_thread", None)
        if t is not None and t.is_alive() and t is not threading.current_thread():
            t.join(timeout=1.0)

    def __del__(self):
        self.shutdown()
