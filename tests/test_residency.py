"""Behavioural CPU tests of the INT4 residency cache (PerLayerCache /
ExpertCacheManager), mirroring the reference's tests/test_int4_loader.py:279-379
(packed mode, eviction counts) and tests/test_glm4_synthetic.py:474-536
(add/remove slot), plus the policy the reference's cache/expert_cache.py fixes:
allocation order (:334-352), promotion on the second hit (:206-219,
:255-283), LFU eviction that skips pins (:354-393), per-layer slot counts
(:890-909), reallocation (:1062-1136) and hit/miss accounting (:601-648).
Slot contents are checked byte for byte against the blobs in experts.bin.
"""
import time

import pytest
import torch

from hydranet_amd.cache.expert_cache import (ExpertCacheConfig, ExpertCacheManager,
                                             MoEModelConfig, PerLayerCache, SlotTier)
from hydranet_amd.cache.packed_expert_store import PackedExpertStore
from tests._store import make_store

CPU = torch.device("cpu")
H, I, G = 256, 512, 128


@pytest.fixture
def store4(tmp_path):
    experts = make_store(tmp_path, num_layers=2, num_experts=4, H=H, I=I, g=G)
    st = PackedExpertStore(tmp_path / "experts.idx", device=CPU)
    yield st, experts
    st.close()


def _layer(store, pinned=1, hot=1, prob=1, E=4, max_slots=4, layer=0):
    c = PerLayerCache(layer, E, 0, ExpertCacheConfig(pinned, hot, prob,
                                                      max_slots_per_layer=max_slots), CPU)
    c.set_packed_mode(store, H, I, G)
    return c


def _same(slot, tensors):
    return all(torch.equal(getattr(slot, n), v) for n, v in tensors.items())


def _tier_of(c, e):
    return c.expert_to_slot[e].tier


def test_manager_packed_mode_eviction(store4):
    """test_int4_loader.py:330-379: 4 experts through 3 slots evict."""
    st, experts = store4
    cfg = MoEModelConfig(num_layers=1, num_experts=4, hidden_dim=H, intermediate_dim=I)
    cm = ExpertCacheManager(cfg, ExpertCacheConfig(1, 1, 1), device=CPU)
    try:
        # layer 0 < 12 gets base + 1 = 4 slots, split hot 2 / probation 2
        assert cm.layer_caches[0].get_slot_count() == 4
        cm.layer_caches[0].remove_slot()
        cm.set_packed_store(st)
        for e in range(4):
            s = cm.get_int4_slot(0, e)
            assert _same(s, experts[(0, e)])
            assert cm.is_cached(0, e)
        stats = cm.get_stats()
        assert stats["total_evictions"] > 0 and stats["total_misses"] == 4
        assert stats["total_hits"] == 0
    finally:
        cm.shutdown()


def test_allocation_order_and_promotion(store4):
    st, experts = store4
    c = _layer(st)
    for e in range(3):
        c.get_int4_slot(e)
    # empty probation, then empty hot, then empty pinned
    assert [_tier_of(c, e) for e in range(3)] == [SlotTier.PROBATION, SlotTier.HOT,
                                                  SlotTier.PINNED]
    assert c.get_stats()["misses"] == 3 and c.evictions == 0
    # expert 3 evicts the only probation expert (0): LFU over probation first
    c.get_int4_slot(3)
    assert not c.is_cached(0) and c.evictions == 1 and _tier_of(c, 3) is SlotTier.PROBATION
    # a hit on expert 3 (hit_count 2) beats hot expert 1 (hit_count 1): swap
    c.get_int4_slot(3)
    assert _tier_of(c, 3) is SlotTier.HOT and _tier_of(c, 1) is SlotTier.PROBATION
    assert c.promotions == 1 and c.hits == 1
    # buffers moved with their experts
    assert _same(c.gpu_int4_slots[c.expert_to_slot[3].slot_idx], experts[(0, 3)])
    assert _same(c.gpu_int4_slots[c.expert_to_slot[1].slot_idx], experts[(0, 1)])
    assert c.get_stats()["hot_count"] == 1 and c.get_stats()["pinned_count"] == 1


def test_promotion_into_empty_hot_slot(store4):
    st, _ = store4
    c = _layer(st, pinned=0, hot=1, prob=2)
    c.get_int4_slot(0)  # probation
    c.get_int4_slot(1)  # second probation slot
    assert _tier_of(c, 0) is SlotTier.PROBATION and _tier_of(c, 1) is SlotTier.PROBATION
    c.get_int4_slot(0)  # second hit -> empty hot slot
    assert _tier_of(c, 0) is SlotTier.HOT and c.promotions == 1


def test_no_promotion_without_more_hits(store4):
    st, _ = store4
    c = _layer(st, pinned=0, hot=1, prob=1)
    c.get_int4_slot(0)
    c.get_int4_slot(1)  # hot (empty) slot
    for _ in range(3):
        c.get_int4_slot(1)  # hot expert at 4 hits
    c.get_int4_slot(0)  # probation at 2 hits < 4: stays
    assert _tier_of(c, 0) is SlotTier.PROBATION and c.promotions == 0


def test_lfu_eviction_order(store4):
    st, _ = store4
    c = _layer(st, pinned=0, hot=0, prob=3)
    for e in range(3):
        c.get_int4_slot(e)
    c.get_int4_slot(0)
    c.get_int4_slot(2)
    c.get_int4_slot(3)  # evicts 1, the only one with hit_count 1
    assert not c.is_cached(1) and all(c.is_cached(e) for e in (0, 2, 3))


def test_adaptive_and_timed_pins(store4):
    st, _ = store4
    c = _layer(st, pinned=0, hot=0, prob=2)
    c.get_int4_slot(0)
    c.get_int4_slot(1)
    c.get_int4_slot(1)
    c.refresh_adaptive_pins()
    assert c.adaptive_pins == {1}
    c.pin_expert(0, duration_sec=60.0)
    with pytest.raises(RuntimeError, match="No evictable slots"):
        c.get_int4_slot(2)
    c.expert_to_slot[0].pinned_until = time.time() - 1.0  # expired
    c.get_int4_slot(2)
    assert not c.is_cached(0) and c.is_cached(1)


def test_decayed_frequency():
    c = PerLayerCache(0, 4, 0, ExpertCacheConfig(0, 0, 1), CPU)
    for e in (0, 1, 1):
        c._record_expert_access(e)
    f = c.expert_freq
    # each access multiplies every frequency by 0.995, then adds 1 to its expert
    assert f[0] == pytest.approx(0.995 ** 2, rel=1e-12)
    assert f[1] == pytest.approx(0.995 + 1.0, rel=1e-12)
    for _ in range(100000):  # long runs renormalise instead of underflowing
        c._record_expert_access(2)
    assert c.expert_freq[2] == pytest.approx(1 / (1 - 0.995), rel=1e-6)
    assert c.expert_freq[0] >= 0.0


def test_prefetch_counts_nothing_then_get_is_hit(store4):
    st, experts = store4
    c = _layer(st)
    s = c.prefetch_int4_slot(2)
    assert c.hits == 0 and c.misses == 0 and c.is_cached(2)
    assert c.prefetch_int4_slot(2) is s
    assert c.get_int4_slot(2) is s and c.hits == 1 and c.misses == 0
    assert _same(s, experts[(0, 2)])
    # a caller that prefetched a known miss counts it as a miss
    c.prefetch_int4_slot(1)
    assert c.get_int4_slot(1, prefetched_miss=True) is c.gpu_int4_slots[
        c.expert_to_slot[1].slot_idx]
    assert c.hits == 1 and c.misses == 1


def test_slot_add_remove():
    """test_glm4_synthetic.py:474-536."""
    c = PerLayerCache(0, 8, 1024, ExpertCacheConfig(0, 1, 1, max_slots_per_layer=5), CPU,
                      torch.float32)
    n0 = c.get_slot_count()
    assert c.add_slot() and c.get_slot_count() == n0 + 1
    while c.add_slot():
        pass
    assert c.get_slot_count() == 5
    assert c.remove_slot() and c.get_slot_count() == 4
    while c.get_slot_count() > 1:
        c.remove_slot()
    assert c.get_slot_count() == 1
    assert not c.remove_slot() and c.get_slot_count() == 1


def test_remove_slot_keeps_buffers_with_experts(store4):
    st, experts = store4
    c = _layer(st, pinned=0, hot=2, prob=2)
    for e in range(4):
        c.get_int4_slot(e)
    c.get_int4_slot(3)
    c.get_int4_slot(3)
    assert c.remove_slot()  # LFU probation expert goes
    assert c.get_slot_count() == 3 and len(c.expert_to_slot) == 3
    assert [s.slot_idx for s in c.slots] == [0, 1, 2]
    for e, s in c.expert_to_slot.items():
        assert c.slots[s.slot_idx] is s
        gs = c.gpu_int4_slots[s.slot_idx]
        assert gs.slot_idx == s.slot_idx and _same(gs, experts[(0, e)])


def test_hold_protects_experts_of_one_call(store4):
    st, _ = store4
    c = _layer(st, pinned=0, hot=0, prob=2)
    c.get_int4_slot(0)
    c.get_int4_slot(1)
    with c.hold([0, 2]):
        c.get_int4_slot(2)  # must evict 1, not the held 0
    assert c.is_cached(0) and c.is_cached(2) and not c.is_cached(1)
    with pytest.raises(RuntimeError, match="only 2 slots"):
        with c.hold([0, 1, 2]):
            pass


def test_manager_slot_allocation(tmp_path):
    make_store(tmp_path, num_layers=16, num_experts=4, H=H, I=I, g=G)
    st = PackedExpertStore(tmp_path / "experts.idx", device=CPU)
    cfg = MoEModelConfig(num_layers=16, num_experts=4, hidden_dim=H, intermediate_dim=I)
    cc = ExpertCacheConfig(0, 1, 1, max_slots_per_layer=4, realloc_interval_tokens=4)
    cm = ExpertCacheManager(cfg, cc, device=CPU)
    try:
        counts = [c.get_slot_count() for c in cm.layer_caches]
        assert counts == [3] * 12 + [2, 2] + [3, 3]
        assert cm.layer_caches[12].hot_slots == 1 and cm.layer_caches[0].probation_slots == 2
    finally:
        cm.shutdown()
        st.close()


def test_manager_reallocation(tmp_path):
    make_store(tmp_path, num_layers=2, num_experts=4, H=H, I=I, g=G)
    st = PackedExpertStore(tmp_path / "experts.idx", device=CPU)
    cfg = MoEModelConfig(num_layers=2, num_experts=4, hidden_dim=H, intermediate_dim=I)
    cc = ExpertCacheConfig(0, 1, 1, max_slots_per_layer=4, realloc_interval_tokens=4)
    cm = ExpertCacheManager(cfg, cc, device=CPU)
    try:
        cm.set_packed_store(st)
        # layer 1 misses on every access, layer 0 hits after one miss
        for e in range(4):
            cm.get_int4_slot(1, e)
        for _ in range(20):
            cm.get_int4_slot(0, 0)
        cm.maybe_reallocate_slots(3)  # below the interval: nothing moves
        assert [c.get_slot_count() for c in cm.layer_caches] == [3, 3]
        cm.maybe_reallocate_slots(1)
        assert [c.get_slot_count() for c in cm.layer_caches] == [2, 4]
        assert cm._do_reallocation() == 0  # recipient at max_slots_per_layer
        stats = cm.get_stats()
        assert stats["total_misses"] == 5 and stats["total_hits"] == 19
        assert stats["layer_hit_rate_min"] == 0.0 and stats["layer_hit_rate_max"] == 0.95
        cm.reset_stats()
        assert cm.get_stats()["total_hits"] == 0
    finally:
        cm.shutdown()
        st.close()


def test_manager_pin_refresh_interval(store4):
    st, _ = store4
    cfg = MoEModelConfig(num_layers=1, num_experts=4, hidden_dim=H, intermediate_dim=I)
    cm = ExpertCacheManager(cfg, ExpertCacheConfig(0, 1, 1, enable_dynamic_slots=False),
                            device=CPU)
    try:
        cm.set_packed_store(st)
        cm.get_int4_slot(0, 1)
        cm.get_int4_slot(0, 1)
        cm.maybe_reallocate_slots(15)
        assert cm.layer_caches[0].adaptive_pins == set()
        cm.maybe_reallocate_slots(1)  # 16 tokens -> refresh
        assert cm.layer_caches[0].adaptive_pins == {1}
    finally:
        cm.shutdown()


def test_prefetch_worker_loads_in_background(store4):
    st, experts = store4
    cfg = MoEModelConfig(num_layers=2, num_experts=4, hidden_dim=H, intermediate_dim=I)
    cm = ExpertCacheManager(cfg, ExpertCacheConfig(0, 2, 2), device=CPU)
    try:
        cm.set_packed_store(st)
        cm.prefetch(1, [0, 3])
        cm.prefetch_queue.join()
        assert cm.is_cached(1, 0) and cm.is_cached(1, 3)
        assert cm.get_stats()["total_misses"] == 0  # prefetch counts nothing
        assert _same(cm.get_int4_slot(1, 3), experts[(1, 3)])
        assert cm.get_stats()["total_hits"] == 1
    finally:
        cm.shutdown()


def test_make_resident_arena(store4):
    st, experts = store4
    cfg = MoEModelConfig(num_layers=2, num_experts=4, hidden_dim=H, intermediate_dim=I)
    cm = ExpertCacheManager(cfg, ExpertCacheConfig(0, 1, 1), device=CPU)
    try:
        cm.set_packed_store(st)
        size = st.layout.total_size
        assert cm.resident_bytes() == 2 * 4 * ((size + 255) // 256 * 256)
        cm.make_resident()
        for layer in range(2):
            assert cm.is_resident(layer)
            slots = cm.resident_slots(layer)
            base = slots[0].slab.data_ptr()
            for e, s in enumerate(slots):
                assert _same(s, experts[(layer, e)])
                # one allocation per layer, 256-byte aligned windows
                assert s.slab.data_ptr() - base == e * ((size + 255) // 256 * 256)
                assert cm.get_int4_slot(layer, e) is s
        c = cm.layer_caches[0]
        assert not c.add_slot() and not c.remove_slot()
        assert cm.get_stats()["total_misses"] == 0 and cm.get_stats()["total_evictions"] == 0
    finally:
        cm.shutdown()


def test_sequence_lfu_and_bursts():
    cfg = MoEModelConfig(num_layers=2, num_experts=4, hidden_dim=H, intermediate_dim=I)
    cm = ExpertCacheManager(cfg, ExpertCacheConfig(), device=CPU)
    try:
        cm.set_active_sequence(7)
        for e in (1, 1, 2):
            cm.record_expert_use(7, 0, e)
        assert cm.get_sequence_hot_experts(7, 0) == [1, 2]
        cm.start_token_step()
        for _ in range(9):
            cm.record_miss(0)
        cm.end_token_step()  # 9 > 8 -> one burst; counts decay by 0.95
        assert cm.get_stats()["miss_burst_events"] == 1
        assert cm.sequence_lfu[7][0][1] == pytest.approx(1.9)
        for _ in range(120):  # 1.9 * 0.95**120 < 0.01
            cm.decay_sequence_lfu(7)
        assert cm.sequence_lfu[7][0] == {}  # entries below 0.01 are dropped
        cm.unregister_sequence(7)
        assert cm.get_stats()["active_sequences"] == 0
    finally:
        cm.shutdown()


def test_missing_store_is_an_error():
    c = PerLayerCache(0, 4, 0, ExpertCacheConfig(0, 1, 1), CPU)
    with pytest.raises(RuntimeError, match="no packed store"):
        c.get_int4_slot(0)


class _SizedManager(ExpertCacheManager):
    """The manager with a stated free-memory figure (the GPU's, stubbed)."""

    free_bytes = None

    def _free_device_bytes(self):
        return self.free_bytes


@pytest.mark.parametrize("free_layers,headroom,want", [(10.0, 0, 2), (1.5, 0, 1), (0.5, 0, 0),
                                                       (3.0, 1, 2), (2.5, 1, 1)])
def test_resident_plan_from_free_memory(store4, free_layers, headroom, want):
    """Layers become resident arenas, from layer 0, as long as their arenas fit
    the free memory less the headroom; the others keep the slot cache."""
    st, experts = store4
    cfg = MoEModelConfig(num_layers=2, num_experts=4, hidden_dim=H, intermediate_dim=I)
    per = 4 * ((st.layout.total_size + 255) // 256 * 256)
    cc = ExpertCacheConfig(0, 1, 1, resident_headroom_bytes=int(headroom * per))
    cm = _SizedManager(cfg, cc, device=CPU)
    cm.free_bytes = int(free_layers * per)
    try:
        cm.set_packed_store(st)
        assert cm.layer_resident_bytes() == per
        assert cm.auto_resident_layers == want
        assert [cm.is_resident(l) for l in range(2)] == [l < want for l in range(2)]
        assert cm.get_stats()["resident_layers"] == want
        for l in range(want):
            for e in range(4):
                assert _same(cm.get_int4_slot(l, e), experts[(l, e)])
        assert cm.get_stats()["total_misses"] == 0
    finally:
        cm.shutdown()


def test_resident_plan_off(store4):
    st, _ = store4
    cfg = MoEModelConfig(num_layers=2, num_experts=4, hidden_dim=H, intermediate_dim=I)
    cm = _SizedManager(cfg, ExpertCacheConfig(0, 1, 1, resident_when_fits=False), device=CPU)
    cm.free_bytes = 1 << 40
    try:
        cm.set_packed_store(st)
        assert cm.auto_resident_layers == 0 and not cm.is_resident(0)
    finally:
        cm.shutdown()
    # no figure (a CPU device): the slot cache
    cm = ExpertCacheManager(cfg, ExpertCacheConfig(0, 1, 1), device=CPU)
    try:
        cm.set_packed_store(st)
        assert cm.auto_resident_layers == 0
    finally:
        cm.shutdown()
