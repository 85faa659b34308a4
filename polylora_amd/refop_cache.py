"""Reuse of the operator API's plan and repacked weights across calls.

``sgmv_lora_a_fwd`` / ``sgmv_lora_b_fwd`` (src/polylora/sgmv.py:141-175 and
:278-328) take the adapter weights in the reference's slot layout on every
call.  Their MFMA path works in three parts of device memory (the C ABI's
``pl_sgmv_lora_*_ref_parts``):

* the plan, which depends on ``weight_indices``, ``seq_lens``, B, M and the
  adapter count only, so one plan serves the shrink and the expand of every
  wrapped Linear of a forward (MultiLoraLinear passes the same context
  tensors to all of them, layers.py:36-58);
* the weights part: the slot table and the weights repacked into the MFMA
  block layout, which depends on ``weights``, ``lora_ranks``, ``stack_num``
  and ``scalings``;
* per-call scratch (the shrink's split planes).

This module keeps the first two across calls, and one scratch buffer per
device and stream that every call on that stream reuses (calls on one
stream run in order, so a call's planes are written only after the
previous call's kernels have read theirs).  An entry is found by what
identifies the tensors it was built from (storage pointer, shape, strides,
dtype, device, the stream) and is valid while their version counters are
where they were when it was built; a changed counter (any in-place write
through torch, e.g. cache.py:140-145 loading an adapter into a slot) makes
the next call rebuild it in place.  The weights part is packed lazily: the
first call after a (re)build repacks only the adapters its rows use, the
second packs the rest, and later calls launch no repack at all.

Entries hold strong references to the plan's index tensors (small) and weak
references to the weight, rank and scale tensors: an entry whose tensors
died is dropped, so a recycled storage pointer is never mistaken for the old
tensor.  Tensors without a version counter (inference tensors) are never
reused, and nothing is kept while a HIP graph is being captured.  Writes
that bypass the version counter (through ``.data``, DLPack or raw pointers)
are not seen: call :func:`clear` after them.  Entries are per stream; the
weights entries of a device share a byte budget (:func:`configure`), least
recently used first out.
"""

from __future__ import annotations

import weakref
from collections import OrderedDict

import torch

from . import _native

_DEFAULT_BUDGET_FRACTION = 4  # default weights budget: a quarter of the device's memory


def _ident_version(t: torch.Tensor):
    """(identity, version counter) of t, or None for a tensor without a version counter."""
    try:
        v = t._version
    except RuntimeError:  # inference tensors track no version
        return None
    return (t.data_ptr(), t.shape, t.stride(), t.dtype), v


def _aligned_buffer(nbytes: int, device: torch.device) -> torch.Tensor:
    """nbytes of device memory at a 256-byte aligned address; an ordinary tensor even under
    torch.inference_mode, since a kept weights part's marks are cleared in place on later calls."""
    with torch.inference_mode(False):
        buf = torch.empty(nbytes + 256, dtype=torch.uint8, device=device)
    pad = (-buf.data_ptr()) % 256
    return buf[pad : pad + nbytes]


class _PlanEntry:
    __slots__ = ("refs", "versions", "buf", "ptr", "ptrs", "live")

    def __init__(self, refs: tuple, versions: tuple, buf: torch.Tensor) -> None:
        self.refs = refs  # strong: the storage cannot be recycled while the entry lives
        self.versions = versions
        self.buf = buf
        self.ptr = buf.data_ptr()
        self.ptrs = tuple(t.data_ptr() for t in refs)
        self.live = True  # False once the cache has dropped it


class _WeightsEntry:
    __slots__ = ("refs", "versions", "buf", "ptr", "marks_bytes", "epoch", "stage", "nbytes", "wmeta", "live", "key")

    def __init__(self, refs: tuple, buf: torch.Tensor, marks_bytes: int, wmeta: tuple) -> None:
        self.refs = refs  # weak references
        self.wmeta = wmeta  # the weights' storage pointer and shape when the entry was made
        self.live = True  # False once the cache has dropped it
        self.versions = None
        self.buf = buf
        self.ptr = buf.data_ptr()
        self.marks_bytes = marks_bytes
        self.epoch = 0
        self.stage = 0  # 0: nothing packed, 1: the adapters of one call packed, 2: all packed
        self.nbytes = int(buf.numel())

    def alive(self) -> bool:
        return all(r() is not None for r in self.refs)


class ReferenceOpCache:
    """Plan and weights entries of the operator API, per device and stream."""

    def __init__(self) -> None:
        self.plans: OrderedDict = OrderedDict()
        self.weights: OrderedDict = OrderedDict()
        self.max_plans = 16
        self.max_bytes: int | None = None  # None: a quarter of the device's memory
        self.bytes: dict = {}
        self._dead: list = []
        self._device_budget: dict = {}
        self._scratch: dict = {}
        # Front memos of the lookups below, keyed by the tensors' identities: a hit is taken only for a
        # live entry that holds these very tensor objects (weakly or strongly, so an id() reused by a
        # later tensor never matches), at the same storage pointers and version counters; anything
        # else goes through the full lookup.
        self._recent_plans: dict = {}
        self._recent_weights: dict = {}
        self.stats = dict(plan_builds=0, plan_hits=0, pack_used=0, pack_all=0, weights_hits=0, uncached=0)

    def clear(self) -> None:
        for e in (*self.plans.values(), *self.weights.values()):
            e.live = False
        self.plans.clear()
        self.weights.clear()
        self.bytes.clear()
        self._dead.clear()
        self._scratch.clear()
        self._recent_plans.clear()
        self._recent_weights.clear()

    def _budget(self, device: torch.device) -> int:
        if self.max_bytes is not None:
            return self.max_bytes
        got = self._device_budget.get(device)
        if got is None:
            got = torch.cuda.get_device_properties(device).total_memory // _DEFAULT_BUDGET_FRACTION
            self._device_budget[device] = got
        return got

    def _drop(self, key) -> None:
        e = self.weights.pop(key, None)
        if e is not None:
            e.live = False
            self.bytes[key[0]] = self.bytes.get(key[0], 0) - e.nbytes

    def _reap(self) -> None:
        while self._dead:
            self._drop(self._dead.pop())

    def scratch(self, device: torch.device, stream: int, nbytes: int) -> int:
        """Address of at least nbytes of 256-byte aligned scratch for calls on `stream`, grown on demand
        (a replaced buffer goes back to torch's allocator, which hands it to later work on the stream it
        was allocated on, the same stream, only after the kernels queued so far)."""
        key = (device, stream)
        hit = self._scratch.get(key)
        if hit is None or hit[1] < nbytes:
            size = max(nbytes, 2 * hit[1]) if hit is not None else nbytes
            buf = _aligned_buffer(size, device)
            hit = self._scratch[key] = (buf.data_ptr(), size, buf)
        return hit[0]

    def plan(self, device: torch.device, stream: int, B: int, M: int, num_adapters: int, seq_lens: torch.Tensor,
             weight_indices: torch.Tensor, nbytes: int) -> tuple:
        """(plan buffer, its address, whether the call must build it)."""
        fast = (id(seq_lens), id(weight_indices), B, M, num_adapters, nbytes, stream)
        e = self._recent_plans.get(fast)
        if e is not None and e.live and e.refs[0] is seq_lens and e.refs[1] is weight_indices:
            try:
                same = (e.ptrs == (seq_lens.data_ptr(), weight_indices.data_ptr())
                        and e.versions == (seq_lens._version, weight_indices._version))
            except RuntimeError:
                same = False
            if same:
                self.stats["plan_hits"] += 1
                return e.buf, e.ptr, False
        a, b = _ident_version(seq_lens), _ident_version(weight_indices)
        if a is None or b is None:
            self.stats["plan_builds"] += 1
            buf = _aligned_buffer(nbytes, device)
            return buf, buf.data_ptr(), True
        key = (device, stream, B, M, num_adapters, nbytes, a[0], b[0])
        now = (a[1], b[1])
        e = self.plans.get(key)
        if e is not None:
            self.plans.move_to_end(key)
            self._remember(self._recent_plans, fast, e)
            if now == e.versions:
                self.stats["plan_hits"] += 1
                return e.buf, e.ptr, False
            e.versions = now
            self.stats["plan_builds"] += 1
            return e.buf, e.ptr, True
        e = _PlanEntry((seq_lens, weight_indices), now, _aligned_buffer(nbytes, device))
        self.plans[key] = e
        while len(self.plans) > self.max_plans:
            self.plans.popitem(last=False)[1].live = False
        if e.live:
            self._remember(self._recent_plans, fast, e)
        self.stats["plan_builds"] += 1
        return e.buf, e.ptr, True

    @staticmethod
    def _remember(memo: dict, fast: tuple, e) -> None:
        if len(memo) >= 256:
            memo.clear()
        memo[fast] = e

    def weights_part(self, device: torch.device, stream: int, which: int, weights: torch.Tensor,
                     lora_ranks: torch.Tensor, scalings: torch.Tensor | None, stack_num: int, dims: tuple,
                     nbytes: int, marks_bytes: int) -> tuple:
        """(weights buffer, its address, build flags, epoch) for this call."""
        if self._dead:
            self._reap()
        fast = (id(weights), id(lora_ranks), id(scalings), which, stack_num, stream)
        e = self._recent_weights.get(fast)
        if e is not None and e.live and e.stage == 2 and e.refs[0]() is weights and e.refs[1]() is lora_ranks \
                and (scalings is None or e.refs[2]() is scalings):
            try:
                now = (weights._version, lora_ranks._version) if scalings is None else (
                    weights._version, lora_ranks._version, scalings._version)
                same = now == e.versions and (weights.data_ptr(), weights.shape) == e.wmeta
            except RuntimeError:
                same = False
            if same:
                self.weights.move_to_end(e.key)
                self.stats["weights_hits"] += 1
                return e.buf, e.ptr, 0, 0
        srcs = (weights, lora_ranks) if scalings is None else (weights, lora_ranks, scalings)
        ivs = [_ident_version(t) for t in srcs]
        if None in ivs or nbytes > self._budget(device):
            self.stats["uncached"] += 1
            self.stats["pack_used"] += 1
            buf = _aligned_buffer(nbytes, device)
            return buf, buf.data_ptr(), _native.PL_REF_PACK_USED, 0
        key = (device, stream, which, stack_num, dims, nbytes) + tuple(iv[0] for iv in ivs)
        e = self.weights.get(key)
        if e is not None and not e.alive():
            self._drop(key)
            e = None
        if e is None:
            dead = self._dead
            refs = tuple(weakref.ref(t, lambda _r, k=key: dead.append(k)) for t in srcs)
            e = _WeightsEntry(refs, _aligned_buffer(nbytes, device), marks_bytes, (weights.data_ptr(), weights.shape))
            e.key = key
            self.weights[key] = e
            self.bytes[device] = self.bytes.get(device, 0) + e.nbytes
            budget = self._budget(device)
            for old in list(self.weights):
                if self.bytes[device] <= budget:
                    break
                if old != key and old[0] == device:
                    self._drop(old)
        else:
            self.weights.move_to_end(key)
        if e.live:
            self._remember(self._recent_weights, fast, e)
        now = tuple(iv[1] for iv in ivs)
        if e.versions != now or e.epoch >= 0x7FFFFFF0:
            e.versions = now
            e.stage = 0
            e.epoch = 0
            e.buf[: e.marks_bytes].zero_()
        if e.stage == 2:
            self.stats["weights_hits"] += 1
            return e.buf, e.ptr, 0, 0
        e.epoch += 1
        if e.stage == 0:
            e.stage = 1
            self.stats["pack_used"] += 1
            return e.buf, e.ptr, _native.PL_REF_PACK_USED | _native.PL_REF_KEEP_PACKED, e.epoch
        e.stage = 2
        self.stats["pack_all"] += 1
        return e.buf, e.ptr, _native.PL_REF_PACK_ALL | _native.PL_REF_KEEP_PACKED, e.epoch


CACHE = ReferenceOpCache()


def configure(max_bytes: int | None = None, max_plans: int = 16) -> None:
    """Byte budget of the kept weights parts per device (None: a quarter of the
    device's memory; 0 keeps none) and the number of kept plans.  Drops every
    kept part and zeroes the counters in ``CACHE.stats``."""
    CACHE.max_bytes = max_bytes
    CACHE.max_plans = max(0, int(max_plans))
    CACHE.clear()
    for k in CACHE.stats:
        CACHE.stats[k] = 0


def clear() -> None:
    """Drop every kept plan and weights part (after writes the version counters do not see)."""
    CACHE.clear()


def marks_bytes(num_adapters: int) -> int:
    """Bytes of the pack marks at the start of a weights part."""
    return (4 * num_adapters + 255) // 256 * 256
