"""GPU slot bookkeeping of cache.py:60-162 as plain Python (test infrastructure).

Only the host-visible state is modelled: ``adapter_to_slot``,
``slot_to_adapter`` and the LRU order, with the same operation order as the
reference, including iteration over the ``needed`` set in ``ensure_resident``
(cache.py:73-74), whose order depends on the string hash seed.
"""

from __future__ import annotations

from collections import OrderedDict


class SlotCacheModel:
    def __init__(self, max_gpu_adapters: int, base_adapter_id: str = "__base__") -> None:
        self.base = base_adapter_id
        self.num_slots = max_gpu_adapters + 1
        self.max_gpu_adapters = max_gpu_adapters
        self.adapter_to_slot: dict[str, int] = {base_adapter_id: 0}
        self.slot_to_adapter: list[str | None] = [base_adapter_id] + [None] * max_gpu_adapters
        self.lru: OrderedDict[str, None] = OrderedDict()
        self.loads: list[tuple[str, int]] = []

    def ensure_resident(self, adapter_ids: list[str], known: set[str]) -> list[int]:
        needed = {a for a in adapter_ids if a != self.base}  # cache.py:61
        unknown = [a for a in needed if a not in known]
        if unknown:
            raise KeyError(f"Unknown LoRA adapter id(s): {unknown}")
        if len(needed) > self.max_gpu_adapters:  # cache.py:65-66
            raise RuntimeError("Batch needs more adapters than GPU cache capacity")
        for a in sorted(needed):  # cache.py:68-71
            if a not in self.adapter_to_slot:
                slot = self._allocate_or_evict(needed)
                self.adapter_to_slot[a] = slot
                self.slot_to_adapter[slot] = a
                self._touch(a)
                self.loads.append((a, slot))
        for a in needed:  # cache.py:73-74
            self._touch(a)
        return [0 if a == self.base else self.adapter_to_slot[a] for a in adapter_ids]

    def _allocate_or_evict(self, needed: set[str]) -> int:  # cache.py:97-117
        for slot in range(1, self.num_slots):
            if self.slot_to_adapter[slot] is None:
                return slot
        for a in list(self.lru.keys()):
            if a in needed:
                continue
            slot = self.adapter_to_slot.pop(a)
            self.lru.pop(a, None)
            self.slot_to_adapter[slot] = None
            return slot
        raise RuntimeError("No evictable LoRA adapter slot is available")

    def _touch(self, a: str) -> None:  # cache.py:152-157
        if a == self.base:
            return
        self.lru.pop(a, None)
        self.lru[a] = None
