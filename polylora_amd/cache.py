"""GPU adapter slots (src/polylora/cache.py:12-162) as a packed arena plus a slot table.

Reference layout: per wrapped module, dense ``A[slots, in, max_rank]``,
``B[slots, max_rank, out]``, ``ranks[slots]`` and ``scales[slots]``; an
adapter load is ~10 small default-stream ops per module and zero-fills the
whole slot.

Here every slot s >= 1 owns one contiguous region of ``slot_bytes`` in a
single device arena.  An adapter is packed once on the host (pinned, model
dtype) into a compact image: for each module it has weights for, A as
``[rank][in]`` (= PEFT lora_A) then B as ``[out][rank8]`` (= PEFT lora_B,
rank padded to a multiple of 8 with zeros), each part 256-byte aligned and
stored in MFMA blocks (``tile_rows``): the first dimension cut into tiles of
16 rows, each tile stored as consecutive 64-byte column blocks, so that a
kernel's 16-row x 64-byte operand load reads contiguous memory.
Loading is one host->device copy of that image plus one copy of the slot's
table row (32 bytes per module: rank, scale, rank8, A and B offsets), both
on a side stream that first waits for the last forward that read the slot;
the compute stream waits on the copy's event before the next forward's
kernels.  Slot 0 is the base adapter: its table row stays all zero.

``ranks[module]`` and ``scales[module]`` remain int32 / fp32 device tensors
indexed by slot (views into the table), as in the reference.  ``A`` and
``B`` return reference-layout tensors materialised from the arena on request.

Slot choice, LRU order and error behaviour follow cache.py:60-162, including
the set-iteration order of ``ensure_resident``'s touch loop.
"""

from __future__ import annotations

from collections import OrderedDict
from collections.abc import Mapping
from dataclasses import dataclass

import numpy as np
import torch

from . import _native
from .config import PolyLoraConfig
from .store import CpuAdapter, CpuAdapterStore

_ALIGN = 256
_ENTRY_INTS = _native.SLOT_ENTRY_INT32S  # int32 words per (slot, module) entry


@dataclass(frozen=True)
class ModuleSpec:
    name: str
    in_features: int
    out_features: int


def _align(n: int) -> int:
    return (n + _ALIGN - 1) // _ALIGN * _ALIGN


def _round8(r: int) -> int:
    return (r + 7) // 8 * 8


_TILE_ROWS = 16
_BLOCK_BYTES = 64


def tile_rows(m: torch.Tensor) -> torch.Tensor:
    """``[R][C]`` -> the arena's block layout, flattened (same element count).

    Rows are cut into tiles of 16 (the last may be shorter, ``rt`` rows); a
    tile is stored as its column blocks of ``W = 64 bytes`` one after the
    other, each block row-major (the last block may be narrower, ``wb``
    columns).  Element (i, c) lands at
    ``16*t*C + s*rt*W + (i % 16)*wb + (c - s*W)`` with ``t = i // 16`` and
    ``s = c // W``.  For ``C <= W`` this is the plain row-major layout.
    """
    R, C = m.shape
    w = _BLOCK_BYTES // m.element_size()
    out = torch.empty(R * C, dtype=m.dtype)
    full = C // w
    for t0 in range(0, R, _TILE_ROWS):
        tile = m[t0 : t0 + _TILE_ROWS]
        rt = tile.shape[0]
        base = t0 * C
        if full:
            out[base : base + rt * full * w] = tile[:, : full * w].reshape(rt, full, w).transpose(0, 1).reshape(-1)
        if C > full * w:
            out[base + rt * full * w : base + rt * C] = tile[:, full * w :].reshape(-1)
    return out


def untile_rows(flat: torch.Tensor, R: int, C: int) -> torch.Tensor:
    """Inverse of ``tile_rows``: the block layout back to ``[R][C]``."""
    w = _BLOCK_BYTES // flat.element_size()
    out = torch.empty((R, C), dtype=flat.dtype, device=flat.device)
    full = C // w
    for t0 in range(0, R, _TILE_ROWS):
        rt = min(_TILE_ROWS, R - t0)
        base = t0 * C
        if full:
            out[t0 : t0 + rt, : full * w] = flat[base : base + rt * full * w].view(full, rt, w).transpose(0, 1).reshape(rt, full * w)
        if C > full * w:
            out[t0 : t0 + rt, full * w :] = flat[base + rt * full * w : base + rt * C].view(rt, C - full * w)
    return out


class SlotLayout:
    """Byte budget of one slot for a module list, an element type and a rank cap."""

    def __init__(self, specs: list[ModuleSpec], dtype: torch.dtype, max_rank: int) -> None:
        self.specs = list(specs)
        self.dtype = dtype
        self.elem = torch.empty((), dtype=dtype).element_size()
        self.max_rank = int(max_rank)
        self.rank8_cap = _round8(self.max_rank)
        self.slot_bytes = sum(
            _align(self.max_rank * s.in_features * self.elem) + _align(s.out_features * self.rank8_cap * self.elem)
            for s in self.specs
        )
        self.key = (str(dtype), self.max_rank, tuple((s.name, s.in_features, s.out_features) for s in self.specs))


@dataclass
class PackedAdapter:
    image: torch.Tensor  # uint8 [nbytes], pinned when a GPU is present
    rows: np.ndarray  # int32 [num_modules, 8]; offsets relative to the slot base


def pack_adapter(adapter: CpuAdapter, layout: SlotLayout) -> PackedAdapter:
    """Pack an adapter into the compact slot image, validating like cache.py:129-136."""
    n_mod = len(layout.specs)
    rows = np.zeros((n_mod, _ENTRY_INTS), dtype=np.int32)
    rows_f = rows.view(np.float32)
    rows_64 = rows.view(np.int64)  # [n_mod, 4]: int64 word 2 = a_off, word 3 = b_off
    parts = []
    cursor = 0
    es = layout.elem
    for i, spec in enumerate(layout.specs):
        weights = adapter.layers.get(spec.name)
        if weights is None:
            continue  # missing module: rank 0, scale 0 (cache.py:127-128)
        r = int(weights.rank)
        if r > layout.max_rank:
            raise ValueError(
                f"Adapter {adapter.adapter_id!r} rank {r} exceeds max_rank {layout.max_rank}"
            )
        if tuple(weights.A.shape) != (spec.in_features, r):
            raise ValueError(f"LoRA A shape mismatch for adapter {adapter.adapter_id!r}, module {spec.name!r}")
        if tuple(weights.B.shape) != (r, spec.out_features):
            raise ValueError(f"LoRA B shape mismatch for adapter {adapter.adapter_id!r}, module {spec.name!r}")
        r8 = _round8(r)
        a_off = cursor
        cursor += _align(r * spec.in_features * es)
        b_off = cursor
        cursor += _align(spec.out_features * r8 * es)
        rows[i, 0] = r
        rows_f[i, 1] = np.float32(weights.scale)
        rows[i, 2] = r8
        rows_64[i, 2] = a_off
        rows_64[i, 3] = b_off
        parts.append((weights, spec, r, r8, a_off, b_off))
    image = torch.zeros(max(cursor, 1), dtype=torch.uint8)
    for weights, spec, r, r8, a_off, b_off in parts:
        a_bytes = r * spec.in_features * es
        a_rows = weights.A.t().to(layout.dtype)
        image[a_off : a_off + a_bytes].view(layout.dtype).copy_(tile_rows(a_rows))
        b_bytes = spec.out_features * r8 * es
        b_rows = torch.zeros(spec.out_features, r8, dtype=layout.dtype)
        b_rows[:, :r].copy_(weights.B.t())
        image[b_off : b_off + b_bytes].view(layout.dtype).copy_(tile_rows(b_rows))
    if torch.cuda.is_available():
        image = image.pin_memory()
    return PackedAdapter(image=image, rows=rows)


class _ReferenceLayoutWeights(Mapping):
    """``cache.A`` / ``cache.B`` in the reference layout, built from the arena on access."""

    def __init__(self, cache: "GpuAdapterCache", side: str) -> None:
        self._cache = cache
        self._side = side

    def __getitem__(self, name: str) -> torch.Tensor:
        return self._cache._materialize(name, self._side)

    def __iter__(self):
        return iter(self._cache.module_specs)

    def __len__(self) -> int:
        return len(self._cache.module_specs)


class GpuAdapterCache:
    def __init__(
        self,
        store: CpuAdapterStore,
        module_specs: list[ModuleSpec],
        config: PolyLoraConfig,
        device: torch.device,
        dtype: torch.dtype,
    ) -> None:
        self.store = store
        self.config = config
        self.device = torch.device(device)
        self.dtype = dtype
        self.num_slots = config.max_gpu_adapters + 1
        if self.num_slots > _native.PL_MAX_SLOTS:
            raise ValueError(f"max_gpu_adapters must be below {_native.PL_MAX_SLOTS}")
        self.adapter_to_slot: dict[str, int] = {config.base_adapter_id: 0}
        self.slot_to_adapter: list[str | None] = [config.base_adapter_id] + [None] * config.max_gpu_adapters
        self.lru: OrderedDict[str, None] = OrderedDict()
        self.module_specs = {spec.name: spec for spec in module_specs}
        self.module_index = {spec.name: i for i, spec in enumerate(module_specs)}
        # (first module, input shape) -> modules called back to back on that
        # same input tensor; learned by MultiLoraLinear, used to stack shrinks
        self.stacked_runs: dict[tuple, tuple[str, ...]] = {}
        # False: every wrapped Linear computes its own LoRA delta (no sibling runs)
        self.stack_siblings = True
        # module name -> its MultiLoraLinear, so the first Linear of a run can
        # compute its siblings' outputs
        self.wrapped: dict[str, object] = {}
        self.loads = 0  # adapters copied into a slot since construction
        self._allocate()

    # ------------------------------------------------------------------ storage
    def _allocate(self) -> None:
        self.layout = SlotLayout(list(self.module_specs.values()), self.dtype, self.config.max_rank)
        n_mod = len(self.module_specs)
        arena_bytes = max(1, (self.num_slots - 1) * self.layout.slot_bytes)
        self.arena = torch.empty(arena_bytes, dtype=torch.uint8, device=self.device)
        self.table = torch.zeros((self.num_slots, n_mod, _ENTRY_INTS), dtype=torch.int32, device=self.device)
        self.table_host = np.zeros((self.num_slots, n_mod, _ENTRY_INTS), dtype=np.int32)
        table_f = self.table.view(torch.float32)
        self.ranks = {name: self.table[:, i, 0] for name, i in self.module_index.items()}
        self.scales = {name: table_f[:, i, 1] for name, i in self.module_index.items()}
        self._row_bytes = n_mod * _ENTRY_INTS * 4
        self._side_stream = None
        if self.device.type == "cuda":
            self._side_stream = torch.cuda.Stream(self.device)
            # the table's zero fill runs on the compute stream; uploads must follow it
            self._side_stream.wait_stream(torch.cuda.current_stream(self.device))
        # slot -> the event after the last work known to read it, or None when
        # the slot was handed out by ensure_resident and no mark_used has
        # covered that hand-out yet (its readers are then somewhere on the
        # compute stream, and a rewrite waits for everything queued there)
        self._slot_last_use: dict[int, torch.cuda.Event | None] = {}
        self._slot_ready: dict[int, torch.cuda.Event] = {}
        self._pending: list[tuple] = []
        # device pointers kept by the launch helpers belong to this arena and table
        self.__dict__.pop("_launch_args", None)

    @property
    def A(self) -> Mapping:
        return _ReferenceLayoutWeights(self, "A")

    @property
    def B(self) -> Mapping:
        return _ReferenceLayoutWeights(self, "B")

    @property
    def rank8_cap(self) -> int:
        return self.layout.rank8_cap

    def _materialize(self, name: str, side: str) -> torch.Tensor:
        spec = self.module_specs[name]
        i = self.module_index[name]
        R = self.config.max_rank
        shape = (self.num_slots, spec.in_features, R) if side == "A" else (self.num_slots, R, spec.out_features)
        out = torch.zeros(shape, dtype=self.dtype, device=self.device)
        es = self.layout.elem
        for slot in range(1, self.num_slots):
            entry = self.table_host[slot, i]
            r = int(entry[0])
            if r == 0:
                continue
            offs = entry.view(np.int64)
            if side == "A":
                a = self.arena[int(offs[2]) : int(offs[2]) + r * spec.in_features * es]
                out[slot, :, :r] = untile_rows(a.view(self.dtype), r, spec.in_features).t()
            else:
                r8 = int(entry[2])
                b = self.arena[int(offs[3]) : int(offs[3]) + spec.out_features * r8 * es]
                out[slot, :r, :] = untile_rows(b.view(self.dtype), spec.out_features, r8)[:, :r].t()
        return out

    # ------------------------------------------------------------- residency
    def ensure_resident(self, adapter_ids: list[str]) -> torch.Tensor:
        """Make every id resident; return the int32 row -> slot map on the device (cache.py:60-84)."""
        base_id = self.config.base_adapter_id
        needed = {adapter_id for adapter_id in adapter_ids if adapter_id != base_id}
        unknown = [adapter_id for adapter_id in needed if adapter_id not in self.store]
        if unknown:
            raise KeyError(f"Unknown LoRA adapter id(s): {unknown}")
        if len(needed) > self.config.max_gpu_adapters:
            raise RuntimeError("Batch needs more adapters than GPU cache capacity")
        self._reap_pending()
        loaded: list[int] = []
        for adapter_id in sorted(needed):
            if adapter_id not in self.adapter_to_slot:
                slot = self._allocate_or_evict(needed)
                self._load_adapter_into_slot(adapter_id, slot)
                loaded.append(slot)
        for adapter_id in needed:  # set order, as cache.py:73-74
            self._touch(adapter_id)
        self._sync_cpu_eviction_exclusions()
        if self.device.type == "cuda" and loaded:
            compute = torch.cuda.current_stream(self.device)
            for slot in loaded:
                compute.wait_event(self._slot_ready[slot])
        slots = [0 if aid == base_id else self.adapter_to_slot[aid] for aid in adapter_ids]
        for slot in set(slots):
            if slot > 0:
                self._slot_last_use[slot] = None  # handed out: readers unknown until mark_used
        host = torch.tensor(slots, dtype=torch.int32)
        if self.device.type == "cuda":
            return host.pin_memory().to(self.device, non_blocking=True)
        return host.to(self.device)

    def mark_used(self, slots: set[int]) -> None:
        """Record that every reader of these slots is enqueued on the current stream, up to now.

        A later rewrite of such a slot then waits for this point of the stream
        only.  A slot handed out by ``ensure_resident`` and not marked since
        (the ``prepare_lora_context`` + ``use_lora_context`` path) is rewritten
        only after everything queued on the compute stream at the rewrite.
        """
        if self.device.type != "cuda" or not slots:
            return
        event = torch.cuda.Event()
        event.record(torch.cuda.current_stream(self.device))
        for slot in slots:
            if slot > 0:
                self._slot_last_use[slot] = event

    def to(self, device: torch.device, dtype: torch.dtype) -> None:
        device = torch.device(device)
        if self.device == device and self.dtype == dtype:
            return
        if self.device.type == "cuda":
            torch.cuda.synchronize(self.device)
        resident = [(slot, aid) for slot, aid in enumerate(self.slot_to_adapter) if slot > 0 and aid is not None]
        self.device = device
        self.dtype = dtype
        self._allocate()
        for slot, aid in resident:
            adapter = self.store.adapters.get(aid) or self.store.get(aid)
            self._write_slot(slot, self._packed(adapter))
        if self.device.type == "cuda" and resident:
            compute = torch.cuda.current_stream(self.device)
            for slot, _ in resident:
                compute.wait_event(self._slot_ready[slot])

    def _allocate_or_evict(self, needed: set[str]) -> int:
        for slot in range(1, self.num_slots):
            if self.slot_to_adapter[slot] is None:
                return slot
        for adapter_id in list(self.lru.keys()):
            if adapter_id in needed:
                continue
            slot = self.adapter_to_slot.pop(adapter_id)
            self.lru.pop(adapter_id, None)
            self.slot_to_adapter[slot] = None
            self._write_slot(slot, None)  # ranks and scales of the freed slot read 0
            return slot
        raise RuntimeError("No evictable LoRA adapter slot is available")

    def _load_adapter_into_slot(self, adapter_id: str, slot: int) -> None:
        adapter = self.store.get(adapter_id)
        self._write_slot(slot, self._packed(adapter))
        self.loads += 1
        self.adapter_to_slot[adapter_id] = slot
        self.slot_to_adapter[slot] = adapter_id
        self._touch(adapter_id)
        self._sync_cpu_eviction_exclusions()

    def _touch(self, adapter_id: str) -> None:
        if adapter_id == self.config.base_adapter_id:
            return
        self.lru.pop(adapter_id, None)
        self.lru[adapter_id] = None
        self.store.touch(adapter_id)

    def _sync_cpu_eviction_exclusions(self) -> None:
        self.store.set_eviction_exclusions(
            {adapter_id for adapter_id in self.slot_to_adapter[1:] if adapter_id is not None}
        )

    # ---------------------------------------------------------------- uploads
    def _packed(self, adapter: CpuAdapter) -> PackedAdapter:
        key = self.layout.key
        packed = adapter.packed.get(key)
        if packed is None:
            packed = pack_adapter(adapter, self.layout)
            adapter.packed[key] = packed
        return packed

    def _write_slot(self, slot: int, packed: PackedAdapter | None) -> None:
        """Copy an adapter image (or nothing, for a cleared slot) and its table row into `slot`."""
        base = (slot - 1) * self.layout.slot_bytes
        if packed is None:
            row = np.zeros_like(self.table_host[slot])
            image, nbytes = None, 0
        else:
            row = packed.rows.copy()
            has = row[:, 0] > 0
            row64 = row.view(np.int64)
            row64[has, 2] += base
            row64[has, 3] += base
            image, nbytes = packed.image, (int(packed.image.numel()) if has.any() else 0)
        self.table_host[slot] = row
        if self.device.type != "cuda":
            if nbytes:
                self.arena[base : base + nbytes].copy_(image[:nbytes])
            self.table[slot].copy_(torch.from_numpy(row))
            return
        lib = _native.load()
        side = self._side_stream
        if slot in self._slot_last_use:
            last = self._slot_last_use.pop(slot)
            if last is None:
                # readers not marked: they are among the work queued on the compute stream
                side.wait_stream(torch.cuda.current_stream(self.device))
            else:
                side.wait_event(last)  # the previous occupant may still be read
        previous = self._slot_ready.get(slot)
        if previous is not None:
            side.wait_event(previous)
        row_pinned = torch.from_numpy(row).pin_memory()
        with torch.cuda.device(self.device):
            _native.check(
                lib.pl_slot_upload(
                    self.arena.data_ptr() + base,
                    image.data_ptr() if nbytes else None,
                    nbytes,
                    self.table.data_ptr() + slot * self._row_bytes,
                    row_pinned.data_ptr(),
                    self._row_bytes,
                    side.cuda_stream,
                ),
                "pl_slot_upload",
            )
        ready = torch.cuda.Event()
        ready.record(side)
        self._slot_ready[slot] = ready
        self._pending.append((ready, image, row_pinned))

    def _reap_pending(self) -> None:
        self._pending = [item for item in self._pending if not item[0].query()]

    def synchronize(self) -> None:
        """Wait for every queued slot upload."""
        if self._side_stream is not None:
            self._side_stream.synchronize()
        self._pending.clear()
