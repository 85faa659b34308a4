"""GPU adapter slots (src/polylora/cache.py:12-162) as a packed arena plus a slot table.

Reference layout: per wrapped module, dense ``A[slots, in, max_rank]``,
``B[slots, max_rank, out]``, ``ranks[slots]`` and ``scales[slots]``; an
adapter load is ~10 small default-stream ops per module and zero-fills the
whole slot.

Here the weights of slot s >= 1 fill one region of ``slot_bytes`` in a
single device arena, found through the slot's table row (the kernels read
every A and B offset from it).  The arena has more regions than slots (up to
one spare per slot, within ``PolyLoraConfig.spare_region_bytes``, by default
4 GiB and an eighth of the free device memory).  The store holds each
adapter as its slot image
(``slot_image.AdapterImage``, pinned, model dtype): for each module it has
weights for, A as ``[rank][in]`` (= PEFT lora_A) then B as ``[out][rank8]``
(= PEFT lora_B, rank padded to a multiple of 8 with zeros), each part
256-byte aligned and stored in MFMA blocks (``tile_rows``): the first
dimension cut into tiles of 16 rows, each tile stored as consecutive 64-byte
column blocks, so that a kernel's 16-row x 64-byte operand load reads
contiguous memory.  The cache binds its layout to the store, which packs
every adapter added afterwards straight into that image.
Loading is one host->device copy of that image, on a side stream, into a
free region: one that no slot points at and whose last readers have finished
(the copy waits for them), so the copy runs while the forward that reads the
slot's current region is still computing.  The slot's table row (32 bytes
per module: rank, scale, rank8, A and B offsets) is then written on the
compute stream, after the copy's event and after every kernel queued before
it, and the region the slot held before becomes free once that write has run
(and the slot's last recorded reader, when mark_used recorded one).  With no
free region the image is rewritten in place, after the slot's readers.  Slot
0 is the base adapter: its table row stays all zero.

``ranks[module]`` and ``scales[module]`` remain int32 / fp32 device tensors
indexed by slot (views into the table), as in the reference.  ``A`` and
``B`` return reference-layout tensors materialised from the arena on request;
writes into them raise (``SlotWeightsSnapshot``), since they would not reach
the arena the kernels read.

Slot choice, LRU order and error behaviour follow cache.py:60-162, including
the set-iteration order of ``ensure_resident``'s touch loop.
"""

from __future__ import annotations

from collections import OrderedDict, deque
from collections.abc import Mapping

import numpy as np
import torch

from . import _native
from .config import PolyLoraConfig
from .slot_image import AdapterImage, ModuleSpec, SlotLayout, tile_rows, untile_rows
from .store import CpuAdapter, CpuAdapterStore

__all__ = ["GpuAdapterCache", "ModuleSpec", "SlotLayout", "tile_rows", "untile_rows"]

_ENTRY_INTS = _native.SLOT_ENTRY_INT32S  # int32 words per (slot, module) entry


_NOT_WRITES = {"requires_grad_", "share_memory_", "retain_grad", "__set_state__"}
_AUGMENTED = {"__setitem__", "__iadd__", "__isub__", "__imul__", "__itruediv__", "__ifloordiv__", "__imod__",
              "__ipow__", "__iand__", "__ior__", "__ixor__", "__ilshift__", "__irshift__", "__imatmul__"}


class SlotWeightsSnapshot(torch.Tensor):
    """A reference-layout copy of slot weights (``cache.A[m]`` / ``cache.B[m]``) that refuses writes.

    In the reference these are the live slot tensors the kernels read
    (cache.py:43-56).  Here the kernels read the packed arena, and this
    tensor is built from it on access, so a write into it would be lost
    without a trace: every in-place op, item assignment or ``out=`` into it
    or into a view of it raises RuntimeError instead.  Results that do not
    share its memory (``clone()``, arithmetic) are plain tensors.
    """

    @classmethod
    def __torch_function__(cls, func, types, args=(), kwargs=None):
        kwargs = kwargs or {}
        name = getattr(func, "__name__", "")
        target = args[0] if args else None
        write = name in _AUGMENTED or (name.endswith("_") and not name.endswith("__") and name not in _NOT_WRITES)
        outs = kwargs.get("out")
        outs = outs if isinstance(outs, (tuple, list)) else (outs,)
        if (write and isinstance(target, cls)) or any(isinstance(o, cls) for o in outs):
            raise RuntimeError(
                f"GpuAdapterCache.A/.B are reference-layout copies of the packed slot arena; {name} into one "
                "would not reach the kernels.  Load changed weights as an adapter instead "
                "(add_adapter_from_peft_state_dict / load_adapter_from_disk).")
        with torch._C.DisableTorchFunctionSubclass():
            ret = func(*args, **kwargs)
        return _keep_views(ret, target, cls)


def _keep_views(ret, source, cls):
    """Outputs that share ``source``'s memory stay snapshots (so writes through them raise); others are plain."""
    if isinstance(ret, (tuple, list)):
        return type(ret)(_keep_views(r, source, cls) for r in ret)
    if isinstance(ret, torch.Tensor) and isinstance(source, torch.Tensor):
        try:
            shared = ret.untyped_storage().data_ptr() == source.untyped_storage().data_ptr()
        except RuntimeError:
            shared = False
        if shared and ret.untyped_storage().nbytes() > 0:
            return ret.as_subclass(cls)
        if type(ret) is not torch.Tensor:
            return ret.as_subclass(torch.Tensor)
    return ret


class _ReferenceLayoutWeights(Mapping):
    """``cache.A`` / ``cache.B`` in the reference layout, built from the arena on access (write-protected)."""

    def __init__(self, cache: "GpuAdapterCache", side: str) -> None:
        self._cache = cache
        self._side = side

    def __getitem__(self, name: str) -> torch.Tensor:
        return self._cache._materialize(name, self._side).as_subclass(SlotWeightsSnapshot)

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
        # decode-sized batches (16-token plan groups, fewer than 2048 tokens):
        # shrink and expand in one launch (pl_lora_decode_stacked); False runs
        # them as two launches
        self.decode_handoff = True
        # module name -> its MultiLoraLinear, so the first Linear of a run can
        # compute its siblings' outputs
        self.wrapped: dict[str, object] = {}
        self.loads = 0  # adapters copied into a slot since construction
        self._allocate()

    # ------------------------------------------------------------------ storage
    # Default cap on the device memory for spare arena regions (at most one
    # per slot): a load copies into a spare region while a running forward
    # still reads the slot's current one.  PolyLoraConfig.spare_region_bytes
    # overrides it; without that the spares also stay within an eighth of
    # the device memory free at allocation.  0 turns them off (loads then
    # rewrite a slot in place, after its readers).  Read when the arena is
    # allocated.
    SPARE_REGION_BYTES = 4 << 30

    def _spare_budget(self) -> int:
        given = getattr(self.config, "spare_region_bytes", None)  # a reference config has no such field
        if given is not None:
            return int(given)
        cap = int(self.SPARE_REGION_BYTES)
        if self.device.type == "cuda" and cap > 0:
            free, _ = torch.cuda.mem_get_info(self.device)
            cap = min(cap, free // 8)
        return cap

    def _allocate(self) -> None:
        self.layout = SlotLayout(list(self.module_specs.values()), self.dtype, self.config.max_rank)
        # adapters added from now on are packed straight into this layout's slot images
        self.store.bind_layout(self.layout)
        n_mod = len(self.module_specs)
        slots = self.num_slots - 1
        self.spare_regions = int(min(slots, self._spare_budget() // max(1, self.layout.slot_bytes)))
        self.num_regions = slots + self.spare_regions
        arena_bytes = max(1, self.num_regions * self.layout.slot_bytes)
        # ordinary tensors even when the first forward under torch.inference_mode moves the cache: loads
        # write into them with in-place copies, which an inference tensor refuses outside that mode
        with torch.inference_mode(False):
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
        # compute stream, and an in-place rewrite waits for everything queued
        # there)
        self._slot_last_use: dict[int, torch.cuda.Event | None] = {}
        # slot -> the arena region holding its adapter (None: no adapter)
        self._slot_region: list[int | None] = [None] * self.num_slots
        # regions no slot points at, the longest free first, each with the
        # events a copy into it must wait for (its last readers)
        self._free_regions: deque = deque((region, ()) for region in range(self.num_regions))
        # one residency call's table rows, written together by _flush_rows:
        # the slots to write, the copies they wait for, and the regions they
        # release (with the slots' last recorded readers)
        self._rows_dirty: set[int] = set()
        self._rows_ready: list = []
        self._rows_release: list[tuple[int, tuple]] = []
        self._pending: list[tuple] = []
        self._deferred_writes: dict | None = None  # slot -> image, while ensure_resident runs
        self._use_seq = 0  # mark_used calls so far
        self._slot_use_seq: dict[int, int] = {}  # slot -> _use_seq of its last recorded use
        # device pointers kept by the launch helpers belong to this arena and table
        self.__dict__.pop("_launch_args", None)
        # the staging stream and its events belong to the device (the pinned buffers do not)
        self.__dict__.pop("_staging_stream", None)
        self.__dict__.pop("_staging_read", None)

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
        self._deferred_writes = {}
        try:
            for adapter_id in sorted(needed):
                if adapter_id not in self.adapter_to_slot:
                    slot = self._allocate_or_evict(needed)
                    self._load_adapter_into_slot(adapter_id, slot)
        finally:
            writes, self._deferred_writes = self._deferred_writes, None
            self._issue_writes(writes)
            self._flush_rows()
        for adapter_id in needed:  # set order, as cache.py:73-74
            self._touch(adapter_id)
        self._sync_cpu_eviction_exclusions()
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

        When such a slot gets a new adapter, its old region is reused only
        after this point of the stream (and after the table row's switch), and
        an in-place rewrite waits for this point only.  A slot handed out by
        ``ensure_resident`` and not marked since (the ``prepare_lora_context``
        + ``use_lora_context`` path) is taken to be read by everything queued
        on the compute stream.
        """
        if self.device.type != "cuda" or not slots:
            return
        event = torch.cuda.Event()
        event.record(torch.cuda.current_stream(self.device))
        self._use_seq += 1
        for slot in slots:
            if slot > 0:
                self._slot_last_use[slot] = event
                self._slot_use_seq[slot] = self._use_seq

    def _issue_writes(self, writes: dict) -> None:
        """Enqueue one residency call's slot writes, slots whose readers finished longest ago first.

        The slot numbers are settled (the reference's policy, cache.py:97-117);
        only the order of the uploads on the side stream is chosen here.  An
        upload waits for the last reader of its slot, and the side stream runs
        its uploads in order, so one upload into a slot the running forward
        still reads would hold back every upload queued after it, also those
        into slots nothing reads any more.  Free slots go first, then slots by
        the age of their last recorded use, then slots handed out and not yet
        marked (their readers are the latest work on the compute stream).
        """
        def age(slot: int) -> float:
            if slot not in self._slot_last_use:
                return -1.0
            if self._slot_last_use[slot] is None:
                return float("inf")
            return float(self._slot_use_seq.get(slot, 0))

        for slot in sorted(writes, key=age):
            self._write_slot_now(slot, writes[slot])

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
        self._flush_rows()

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
    def _packed(self, adapter: CpuAdapter) -> AdapterImage:
        """The adapter's slot image for this cache's layout (validated like cache.py:129-136)."""
        return self.store.image(adapter, self.layout)

    def _write_slot(self, slot: int, packed: AdapterImage | None) -> None:
        """Copy an adapter image (or nothing, for a cleared slot) and its table row into `slot`.

        Inside ``ensure_resident`` the write is only recorded (the last write
        to a slot wins: an eviction's clear is followed by the new occupant's
        load) and issued at the end of the call by ``_issue_writes``.
        """
        if self._deferred_writes is not None:
            self._deferred_writes[slot] = packed
            return
        self._write_slot_now(slot, packed)

    def slot_offset(self, slot: int) -> int | None:
        """Byte offset in the arena of the region holding slot `slot`'s adapter, or None."""
        region = self._slot_region[slot]
        return None if region is None else region * self.layout.slot_bytes

    def _take_region(self, slot: int) -> tuple[int, tuple, bool]:
        """A region for slot `slot`'s new image: (region, events to wait for, wait for the compute stream).

        The region free longest, else one this residency call released
        (its readers are queued on the compute stream), else the slot's own
        region (its readers: the slot's last recorded use, or, when none was
        recorded, the compute stream).
        """
        if self._free_regions:
            region, waits = self._free_regions.popleft()
            return region, waits, False
        if self._rows_release:
            region, waits = self._rows_release.pop(0)
            return region, waits, True
        region = self._slot_region[slot]
        if region is None:
            raise RuntimeError("no arena region is free")  # more slots than regions: cannot happen
        last = self._slot_last_use.get(slot)
        return region, (() if last is None else (last,)), slot in self._slot_last_use and last is None

    def _write_slot_now(self, slot: int, packed: AdapterImage | None) -> None:
        """Copy an image into a region for `slot` and record the slot's new table row."""
        old = self._slot_region[slot]
        if packed is None:
            region, waits, wait_compute = None, (), False
            row = np.zeros_like(self.table_host[slot])
            image, nbytes, base = None, 0, 0
        else:
            region, waits, wait_compute = self._take_region(slot)
            base = region * self.layout.slot_bytes
            row = packed.rows.copy()
            has = row[:, 0] > 0
            row64 = row.view(np.int64)
            row64[has, 2] += base
            row64[has, 3] += base
            image, nbytes = packed.data, packed.nbytes
        self.table_host[slot] = row
        self._slot_region[slot] = region
        if old is not None and old != region:
            last = self._slot_last_use.get(slot)
            self._rows_release.append((old, () if last is None else (last,)))
        self._slot_last_use.pop(slot, None)  # the old occupant's readers now guard its old region
        self._rows_dirty.add(slot)
        if self.device.type != "cuda":
            if nbytes:
                self.arena[base : base + nbytes].copy_(image[:nbytes])
            return
        if not nbytes:
            return
        lib = _native.load()
        side = self._side_stream
        if wait_compute:
            side.wait_stream(torch.cuda.current_stream(self.device))
        for event in waits:
            side.wait_event(event)
        staging, ring_index = self._stage(image, nbytes) if not packed.pinned else (None, None)
        with torch.cuda.device(self.device):
            _native.check(
                lib.pl_slot_upload(self.arena.data_ptr() + base, (staging if staging is not None else image).data_ptr(),
                                   nbytes, None, None, 0, side.cuda_stream),
                "pl_slot_upload",
            )
        ready = torch.cuda.Event()
        ready.record(side)
        self._rows_ready.append(ready)
        if ring_index is not None:
            self._staging_read[ring_index] = ready  # the buffer's next fill waits for this DMA
        # the source image and the staging buffer stay alive until the upload has run
        self._pending.append((ready, image, staging))

    def _flush_rows(self) -> None:
        """Write the recorded table rows and free the regions they no longer point at.

        On a GPU the rows go in one copy on the compute stream, after the
        uploads they describe and after every kernel queued so far (the
        readers of the rows being replaced); the released regions wait for
        that point, and for the slots' last recorded readers, before a copy
        reuses them.
        """
        dirty, self._rows_dirty = self._rows_dirty, set()
        ready, self._rows_ready = self._rows_ready, []
        release, self._rows_release = self._rows_release, []
        if not dirty:
            self._free_regions.extend(release)
            return
        lo, hi = min(dirty), max(dirty) + 1
        if self.device.type != "cuda":
            self.table[lo:hi].copy_(torch.from_numpy(self.table_host[lo:hi]))
            self._free_regions.extend(release)
            return
        compute = torch.cuda.current_stream(self.device)
        for event in ready:
            compute.wait_event(event)
        rows = torch.from_numpy(self.table_host[lo:hi].copy()).pin_memory()
        with torch.cuda.device(self.device):
            _native.check(
                _native.load().pl_slot_upload(None, None, 0, self.table.data_ptr() + lo * self._row_bytes,
                                              rows.data_ptr(), (hi - lo) * self._row_bytes, compute.cuda_stream),
                "pl_slot_upload",
            )
        written = torch.cuda.Event()
        written.record(compute)
        self._free_regions.extend((region, waits + (written,)) for region, waits in release)
        self._pending.append((written, rows))

    # Page-locked staging buffers for images held in pageable memory.  The
    # runtime's own copy from pageable memory blocks the calling thread until
    # the side stream reaches it, i.e. until the forward that last read the
    # slot has finished, so the host could no longer queue work ahead of the
    # GPU.  Instead the copy of such an image into the next buffer of a ring
    # runs as a host function on a staging stream (pl_host_copy_async, 8
    # threads), and the upload stream's DMA from that buffer waits for it with
    # an event.  The host copy waits only for the DMA that last read its
    # buffer, not for the slot's readers, so it runs while the upload stream
    # is busy with other DMAs or waiting for a forward; the calling thread
    # never waits.
    STAGING_BUFFERS = 8

    def _stage(self, image: torch.Tensor, nbytes: int) -> tuple[torch.Tensor | None, int | None]:
        """Queue the image's copy into the next staging buffer; (buffer, ring index), or (None, None)."""
        from .slot_image import host_bytes

        n = self.STAGING_BUFFERS
        ring = self.__dict__.setdefault("_staging", [None] * n)
        read = self.__dict__.setdefault("_staging_read", [None] * n)
        i = self.__dict__.get("_staging_next", 0) % n
        buf = ring[i]
        if buf is None or buf.numel() < nbytes:
            # a replaced buffer stays referenced by the pending uploads that use it
            buf, pinned = host_bytes(nbytes, pin=True)
            if not pinned:
                return None, None  # no page-locked memory left: the runtime stages the copy itself
            ring[i] = buf
            read[i] = None
        stage = self.__dict__.get("_staging_stream")
        if stage is None:
            stage = self._staging_stream = torch.cuda.Stream(self.device)
        if read[i] is not None:
            stage.wait_event(read[i])  # the DMA that last read this buffer is done
        _native.check(_native.load().pl_host_copy_async(buf.data_ptr(), image.data_ptr(), nbytes, stage.cuda_stream),
                      "pl_host_copy_async")
        filled = torch.cuda.Event()
        filled.record(stage)
        self._side_stream.wait_event(filled)
        self._staging_next = i + 1
        return buf, i

    def _reap_pending(self) -> None:
        self._pending = [item for item in self._pending if not item[0].query()]

    def synchronize(self) -> None:
        """Wait for every queued slot upload."""
        if self._side_stream is not None:
            self._side_stream.synchronize()
        self._pending.clear()
