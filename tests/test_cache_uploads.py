"""Order and count of slot uploads a residency call issues (host logic, CPU).

The slot numbers follow the reference's policy (cache.py:60-117) and are
checked against oracle/slots.py in test_host.py; here only the uploads are
observed: one per slot per ensure_resident call (an eviction's clear is
replaced by the new occupant's load), issued free slots first, then by the
age of each slot's last recorded reader, then slots handed out and not yet
marked.
"""

from __future__ import annotations

import torch

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
                base, n = (slot - 1) * a.layout.slot_bytes, a.store.adapters[aid].image.nbytes
                assert torch.equal(a.arena[base : base + n], b.arena[base : base + n])
