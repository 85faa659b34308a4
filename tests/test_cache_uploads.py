"""Order and count of slot uploads a residency call issues (host logic, CPU).

The slot numbers follow the reference's policy (cache.py:60-117) and are
checked against oracle/slots.py in test_host.py; here only the uploads are
observed: one per slot per ensure_resident call (an eviction's clear is
replaced by the new occupant's load), issued free slots first, then by the
age of each slot's last recorded reader, then slots handed out and not yet
marked.  Each load goes to an arena region no slot points at when one is
free (the arena's spare regions), else to the slot's own region; the
regions held by slots and the free ones always partition the arena.
"""

from __future__ import annotations

import numpy as np
import torch

from polylora_amd.cache import GpuAdapterCache
from tests._util import make_cache, peft_layer

SHAPES = {"m": (32, 24)}


def _cache(n_adapters: int, slots: int):
    g = torch.Generator().manual_seed(3)
    adapters = {f"a{i}": {"m": peft_layer(g, 32, 24, 2 + i % 3, 4.0)} for i in range(n_adapters)}
    return make_cache(adapters, SHAPES, slots, 4, torch.device("cpu"), torch.float32)


def _record(cache, monkeypatch):
    seen = []
    real = cache._write_slot_now

    def spy(slot, packed):
        seen.append((slot, packed is not None))
        real(slot, packed)

    monkeypatch.setattr(cache, "_write_slot_now", spy)
    return seen


def test_eviction_issues_one_upload_per_slot(monkeypatch):
    cache = _cache(6, 3)
    cache.ensure_resident(["a0", "a1", "a2"])
    seen = _record(cache, monkeypatch)
    cache.ensure_resident(["a3", "a4"])  # evicts two slots: their clears are folded into the loads
    assert sorted(s for s, _ in seen) == sorted({s for s, _ in seen}) and len(seen) == 2
    assert all(loaded for _, loaded in seen)
    for aid in ("a3", "a4"):
        slot = cache.adapter_to_slot[aid]
        assert int(cache.ranks["m"][slot]) == int(cache.store.adapters[aid].layers["m"].rank)


def test_uploads_go_oldest_reader_first(monkeypatch):
    cache = _cache(4, 4)
    seen = _record(cache, monkeypatch)
    # slot 1: handed out, readers not yet marked; slot 2: last read at use 5; slot 3: at use 2;
    # slot 4: never read
    cache._slot_last_use = {1: None, 2: object(), 3: object()}
    cache._slot_use_seq = {2: 5, 3: 2}
    cache._issue_writes({1: None, 2: None, 3: None, 4: None})
    assert [s for s, _ in seen] == [4, 3, 2, 1]


def test_slot_numbers_do_not_depend_on_upload_order():
    """Two caches, one with uploads reversed: the same slots, ranks and scales."""
    a, b = _cache(8, 3), _cache(8, 3)

    def reverse(writes, cache=b):
        for slot in sorted(writes, reverse=True):
            cache._write_slot_now(slot, writes[slot])

    b._issue_writes = reverse
    for batch in (["a0", "a1"], ["a2", "a3", "a0"], ["a4", "a5"], ["a6", "a1", "a7"], ["a0"]):
        ra = a.ensure_resident(batch)
        rb = b.ensure_resident(batch)
        assert torch.equal(ra, rb)
        assert a.slot_to_adapter == b.slot_to_adapter
        assert torch.equal(a.ranks["m"], b.ranks["m"]) and torch.equal(a.scales["m"], b.scales["m"])
        for slot in range(1, a.num_slots):  # the bytes each resident image occupies (the rest is never read)
            aid = a.slot_to_adapter[slot]
            if aid is not None:
                n = a.store.adapters[aid].image.nbytes
                oa, ob = a.slot_offset(slot), b.slot_offset(slot)  # the regions may differ
                assert torch.equal(a.arena[oa : oa + n], b.arena[ob : ob + n])


def _regions_consistent(cache):
    held = [r for r in cache._slot_region[1:] if r is not None]
    free = [r for r, _ in cache._free_regions]
    assert len(held) == len(set(held)), "two slots share a region"
    assert sorted(held + free) == list(range(cache.num_regions)), "a region is lost or listed twice"
    for slot in range(1, cache.num_slots):
        aid = cache.slot_to_adapter[slot]
        assert (aid is None) == (cache.slot_offset(slot) is None)
        if aid is not None:
            image = cache.store.adapters[aid].image
            off = cache.slot_offset(slot)
            assert torch.equal(cache.arena[off : off + image.nbytes], image.data[: image.nbytes])
            rows = cache.table[slot].numpy().view(np.int64)  # A and B offsets point into the region
            has = cache.table[slot, :, 0].numpy() > 0
            assert ((rows[has, 2] >= off) & (rows[has, 3] < off + cache.layout.slot_bytes)).all()


def test_loads_go_to_spare_regions_and_free_the_old_ones():
    """A reload copies into a region no slot points at; the evicted adapter's region is freed."""
    cache = _cache(6, 3)
    assert cache.spare_regions == 3 and cache.num_regions == 6
    cache.ensure_resident(["a0", "a1", "a2"])
    before = {cache.adapter_to_slot[a]: cache._slot_region[cache.adapter_to_slot[a]] for a in ("a0", "a1", "a2")}
    cache.ensure_resident(["a3"])  # evicts the least recently used adapter
    slot = cache.adapter_to_slot["a3"]
    assert cache._slot_region[slot] != before[slot]
    assert before[slot] in [r for r, _ in cache._free_regions]
    _regions_consistent(cache)


def test_without_spare_regions_loads_rewrite_in_place(monkeypatch):
    monkeypatch.setattr(GpuAdapterCache, "SPARE_REGION_BYTES", 0)
    cache = _cache(6, 3)
    assert cache.spare_regions == 0 and cache.num_regions == 3
    cache.ensure_resident(["a0", "a1", "a2"])
    offsets = [cache.slot_offset(s) for s in range(1, 4)]
    for batch in (["a3"], ["a4", "a0"], ["a5", "a1", "a2"]):
        cache.ensure_resident(batch)
        assert [cache.slot_offset(s) for s in range(1, 4)] == offsets
        _regions_consistent(cache)


def test_region_bookkeeping_over_random_batches():
    g = np.random.default_rng(11)
    cache = _cache(10, 4)
    for _ in range(40):
        batch = [f"a{i}" for i in g.choice(10, size=int(g.integers(1, 5)), replace=False)]
        cache.ensure_resident(batch)
        _regions_consistent(cache)
        for aid in batch:
            slot = cache.adapter_to_slot[aid]
            assert int(cache.ranks["m"][slot]) == int(cache.store.adapters[aid].layers["m"].rank)


def test_spare_region_budget_comes_from_the_config():
    """PolyLoraConfig.spare_region_bytes sets the spare regions' budget (0: none; a value: as many whole
    regions as it holds, at most one per slot); negative budgets are refused."""
    import pytest

    from polylora_amd.cache import ModuleSpec
    from polylora_amd.config import PolyLoraConfig
    from tests._util import make_store

    g = torch.Generator().manual_seed(4)
    adapters = {f"a{i}": {"m": peft_layer(g, 32, 24, 2, 4.0)} for i in range(4)}
    specs = [ModuleSpec("m", 32, 24)]

    def spares(budget):
        cfg = PolyLoraConfig(max_gpu_adapters=3, max_rank=4, spare_region_bytes=budget)
        cache = GpuAdapterCache(make_store(adapters), specs, cfg, torch.device("cpu"), torch.float32)
        return cache.spare_regions, cache.layout.slot_bytes

    assert spares(0)[0] == 0
    n, slot_bytes = spares(None)
    assert n == 3  # the default cap (4 GiB) holds a spare for every slot
    assert spares(slot_bytes)[0] == 1 and spares(2 * slot_bytes + 1)[0] == 2
    with pytest.raises(ValueError, match="spare_region_bytes"):
        PolyLoraConfig(max_gpu_adapters=1, max_rank=4, spare_region_bytes=-1)


def test_bound_launch_arguments_follow_a_reallocated_arena():
    """The fused launch's prebuilt arguments (arena and table addresses) are rebuilt after the cache
    allocates a new arena and table on a dtype change, never reused from the freed ones."""
    from polylora_amd import sgmv

    cache = _cache(4, 3)
    cache.ensure_resident(["a0", "a1"])
    before = sgmv._cache_args_c(cache, "m")
    assert before[0].value == cache.arena.data_ptr() and before[1].value == cache.table.data_ptr()
    assert sgmv._cache_args(cache, "m")[0] == cache.arena.data_ptr()
    old_arena = cache.arena
    cache.to(torch.device("cpu"), torch.float16)
    assert cache.arena is not old_arena
    after = sgmv._cache_args_c(cache, "m")
    assert after[0].value == cache.arena.data_ptr() and after[1].value == cache.table.data_ptr()
    assert sgmv._cache_args(cache, "m")[:2] == (cache.arena.data_ptr(), cache.table.data_ptr())
