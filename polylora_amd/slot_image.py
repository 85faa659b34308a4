"""Host image of one adapter in the GPU slot layout: what a slot upload copies.

A slot of the device arena holds, for every wrapped module an adapter has
weights for, two 256-byte-aligned parts in the model dtype:

* A, the ``[rank][in_features]`` matrix of PEFT's ``lora_A`` (no transpose);
* B, the ``[out_features][rank8]`` matrix of PEFT's ``lora_B``, the rank
  padded with zero columns to a multiple of 8,

each stored in MFMA blocks (``tile_rows``).  An ``AdapterImage`` is exactly
those bytes for a ``SlotLayout`` (module list, dtype, rank cap), plus the
adapter's rows of the slot table (rank, fp32 scale, rank8, A and B offsets
per module), so loading an adapter into a slot is one host-to-device copy of
the image and one of its table rows.  The image is built straight from the
PEFT tensors (``ImageBuilder``) and is the only host copy the store keeps of
an adapter once a layout is known.

Replaces the per-module ``A[slots, in, max_rank]`` / ``B[slots, max_rank,
out]`` slot tensors of cache.py:37-58 and the transposed host copies of
store.py:248-253 (``CpuLayerWeights``), which are rebuilt from an image on
request.
"""

from __future__ import annotations

import ctypes
import weakref
from dataclasses import dataclass

import numpy as np
import torch

ALIGN = 256  # bytes: alignment of every A and B part inside a slot
TILE_ROWS = 16  # rows per MFMA tile
BLOCK_BYTES = 64  # bytes per column block of a tile
ENTRY_INT32S = 8  # int32 words of one slot-table entry (pl_slot_entry)


@dataclass(frozen=True)
class ModuleSpec:
    """A wrapped nn.Linear: its name in the model and its sizes (cache.py:12-16)."""

    name: str
    in_features: int
    out_features: int


def align(n: int) -> int:
    return -(-n // ALIGN) * ALIGN


def round8(r: int) -> int:
    return -(-r // 8) * 8


def _block_elems(t: torch.Tensor) -> int:
    return BLOCK_BYTES // t.element_size()


def _tile_copy(dst: torch.Tensor, src: torch.Tensor, forward: bool) -> None:
    """Copy between a row-major ``[R][C]`` matrix and its flat block layout.

    ``forward``: ``src`` is the matrix and ``dst`` the flat image; otherwise
    the other way round.  One tensor copy per group of equally shaped tiles
    (all full tiles together, then the short last tile) and block kind (the
    full-width blocks, then the narrower last one), whatever R and C are.
    """
    mat, flat = (src, dst) if forward else (dst, src)
    R, C = mat.shape
    w = _block_elems(flat)
    nfull = C // w
    tail = C - nfull * w
    full_tiles = R // TILE_ROWS
    spans = []
    if full_tiles:
        spans.append((0, full_tiles, TILE_ROWS))
    if R % TILE_ROWS:
        spans.append((full_tiles * TILE_ROWS, 1, R % TILE_ROWS))
    for r0, count, rt in spans:
        m = mat[r0 : r0 + count * rt].view(count, rt, C)
        f = flat[r0 * C : (r0 + count * rt) * C].view(count, rt * C)
        if nfull:
            fm = f[:, : rt * nfull * w].view(count, nfull, rt, w)
            mm = m[:, :, : nfull * w].view(count, rt, nfull, w).permute(0, 2, 1, 3)
            if forward:
                fm.copy_(mm)
            else:
                mm.copy_(fm)
        if tail:
            ft = f[:, rt * nfull * w :].view(count, rt, tail)
            mt = m[:, :, nfull * w :]
            if forward:
                ft.copy_(mt)
            else:
                mt.copy_(ft)


def tile_rows_into(dst: torch.Tensor, m: torch.Tensor) -> None:
    """Write ``m [R][C]`` into the flat view ``dst`` (R*C elements of dst's dtype) in block layout.

    Rows are cut into tiles of 16 (the last may be shorter, ``rt`` rows); a
    tile is stored as its column blocks of ``W = 64 bytes`` one after the
    other, each block row-major (the last block may be narrower, ``wb``
    columns).  Element (i, c) lands at
    ``16*t*C + s*rt*W + (i % 16)*wb + (c - s*W)`` with ``t = i // 16`` and
    ``s = c // W``.  For ``C <= W`` this is the plain row-major layout.  ``m``
    is converted to ``dst``'s dtype on the way.
    """
    if m.dim() != 2 or dst.dim() != 1 or dst.numel() != m.numel():
        raise ValueError(f"tile_rows_into: {tuple(dst.shape)} cannot hold {tuple(m.shape)}")
    m = m.to(device=dst.device, dtype=dst.dtype)  # one conversion (and device copy) for the whole matrix
    _tile_copy(dst, m, forward=True)


def tile_rows(m: torch.Tensor) -> torch.Tensor:
    """``[R][C]`` -> its block layout, flattened (see ``tile_rows_into``)."""
    out = torch.empty(m.numel(), dtype=m.dtype, device=m.device)
    _tile_copy(out, m, forward=True)
    return out


def untile_rows(flat: torch.Tensor, R: int, C: int) -> torch.Tensor:
    """Inverse of ``tile_rows``: the block layout back to ``[R][C]``."""
    out = torch.empty((R, C), dtype=flat.dtype, device=flat.device)
    _tile_copy(out, flat, forward=False)
    return out


class SlotLayout:
    """Byte budget of one slot for a module list, an element type and a rank cap.

    ``slot_bytes`` covers ``max_rank`` for every module, so any adapter the
    cache accepts fits any slot; an image holds only the adapter's own ranks.
    """

    def __init__(self, specs: list[ModuleSpec], dtype: torch.dtype, max_rank: int) -> None:
        self.specs = list(specs)
        self.dtype = dtype
        self.elem = torch.empty((), dtype=dtype).element_size()
        self.max_rank = int(max_rank)
        self.rank8_cap = round8(self.max_rank)
        self.index = {s.name: i for i, s in enumerate(self.specs)}
        self.slot_bytes = sum(
            align(self.max_rank * s.in_features * self.elem) + align(s.out_features * self.rank8_cap * self.elem)
            for s in self.specs
        )
        self.key = (str(dtype), self.max_rank, tuple((s.name, s.in_features, s.out_features) for s in self.specs))


def host_bytes(nbytes: int, pin: bool | None = None) -> tuple[torch.Tensor, bool]:
    """A host byte buffer and whether it is page-locked (asked for unless ``pin`` is False, GPU only).

    Page-locked buffers are exactly ``nbytes`` from ``pl_host_alloc``; their
    memory is released when the last tensor viewing it is gone.  When the
    system refuses to lock more memory the buffer is pageable.  A page-locked
    image is copied to its slot by the DMA engine while the host runs ahead;
    a pageable one is staged by the runtime and its copy blocks the host.
    """
    n = max(1, int(nbytes))
    want = torch.cuda.is_available() if pin is None else bool(pin and torch.cuda.is_available())
    if want:
        ptr = _locked_free.get(n, [None]).pop() if _locked_free.get(n) else None
        if ptr is None:
            from . import _native

            ptr = _native.load().pl_host_alloc(n)
        if ptr:
            raw = (ctypes.c_uint8 * n).from_address(ptr)
            # when the last view of the buffer dies its memory goes back to the free list
            weakref.finalize(raw, _locked_free.setdefault(n, []).append, ptr)
            return torch.frombuffer(raw, dtype=torch.uint8), True
    return torch.empty(n, dtype=torch.uint8), False


# Page-locked buffers no image uses any more, by size, reused by the next image
# of that size: releasing page-locked memory (hipHostFree) can wait for the
# whole device, which would stall the host in the middle of serving.
_locked_free: dict[int, list[int]] = {}


def release_locked_free() -> int:
    """Return the page-locked buffers no image uses to the system; the bytes released.

    For a caller that is done with a set of adapters (e.g. between workloads)
    and wants their page-locked memory back before pinning others: the
    system limits page-locked memory per process.  ``hipHostFree`` may wait
    for the device, so this is not for the middle of serving.
    """
    from . import _native

    freed = 0
    lib = _native.load()
    for n, ptrs in list(_locked_free.items()):
        while ptrs:
            _native.check(lib.pl_host_free(ptrs.pop()), "pl_host_free")
            freed += n
    _locked_free.clear()
    return freed


class AdapterImage:
    """One adapter packed for a ``SlotLayout``.

    ``data``: uint8 bytes of the slot contents (pinned when a GPU is present);
    ``rows``: int32 ``[num_modules, 8]`` slot-table entries with A and B
    offsets relative to the slot base (rank 0 and scale 0 for modules the
    adapter lacks, cache.py:127-128).
    """

    __slots__ = ("layout", "data", "rows", "pinned")

    def __init__(self, layout: SlotLayout, data: torch.Tensor, rows: np.ndarray, pinned: bool | None = None) -> None:
        self.layout, self.data, self.rows = layout, data, rows
        self.pinned = bool(torch.cuda.is_available() and data.is_pinned()) if pinned is None else bool(pinned)

    @property
    def nbytes(self) -> int:
        """Bytes a slot load copies (0 for an adapter with no module of this layout)."""
        return int(self.data.numel()) if (self.rows[:, 0] > 0).any() else 0

    def entry(self, name: str):
        """(rank, scale, rank8, a_off, b_off) of a module, or None when the adapter lacks it."""
        row = self.rows[self.layout.index[name]]
        rank = int(row[0])
        if rank == 0:
            return None
        off = row.view(np.int64)
        return rank, float(row.view(np.float32)[1]), int(row[2]), int(off[2]), int(off[3])

    def lora_tensors(self, name: str):
        """PEFT-layout (lora_A [r, in], lora_B [out, r], scale) of a module, rebuilt from the image, or None."""
        got = self.entry(name)
        if got is None:
            return None
        rank, scale, r8, a_off, b_off = got
        spec = self.layout.specs[self.layout.index[name]]
        es, dt = self.layout.elem, self.layout.dtype
        a = untile_rows(self.data[a_off : a_off + rank * spec.in_features * es].view(dt), rank, spec.in_features)
        b = untile_rows(self.data[b_off : b_off + spec.out_features * r8 * es].view(dt), spec.out_features, r8)
        return a, b[:, :rank].contiguous(), scale


class ImageBuilder:
    """Lays out one adapter's modules in a ``SlotLayout`` and fills the image in place.

    ``modules``: name -> (rank, scale) for every module the adapter has; the
    offsets follow the layout's module order.  ``put`` copies (and converts,
    pads and tiles) one module's PEFT tensors straight into the image, so the
    image is the only buffer the weights pass through on the host.
    """

    def __init__(self, layout: SlotLayout, modules: dict[str, tuple[int, float]], pin=None) -> None:
        """``pin``: None (page-locked when a GPU is present), a bool, or a callable that gets the
        image's byte count and decides."""
        self.layout = layout
        self.rows = np.zeros((len(layout.specs), ENTRY_INT32S), dtype=np.int32)
        rows_f, rows_64 = self.rows.view(np.float32), self.rows.view(np.int64)
        es = layout.elem
        cursor = 0
        self.parts: dict[str, tuple[int, int, int]] = {}  # name -> (rank, a_off, b_off)
        for i, spec in enumerate(layout.specs):
            got = modules.get(spec.name)
            if got is None:
                continue
            rank, scale = int(got[0]), float(got[1])
            a_off = cursor
            cursor += align(rank * spec.in_features * es)
            b_off = cursor
            cursor += align(spec.out_features * round8(rank) * es)
            self.rows[i, 0] = rank
            rows_f[i, 1] = np.float32(scale)
            self.rows[i, 2] = round8(rank)
            rows_64[i, 2] = a_off
            rows_64[i, 3] = b_off
            self.parts[spec.name] = (rank, a_off, b_off)
        self.nbytes = cursor
        self.data, self.pinned = host_bytes(cursor, pin(cursor) if callable(pin) else pin)
        # the alignment gaps between parts are never read; zero them so an image is deterministic
        for name, (rank, a_off, b_off) in self.parts.items():
            spec = layout.specs[layout.index[name]]
            a_end, b_end = a_off + rank * spec.in_features * es, b_off + spec.out_features * round8(rank) * es
            self.data[a_end : a_off + align(a_end - a_off)].zero_()
            self.data[b_end : b_off + align(b_end - b_off)].zero_()
        self.filled: set[str] = set()

    def put(self, name: str, lora_a: torch.Tensor, lora_b: torch.Tensor) -> None:
        """lora_A ``[rank, in]`` and lora_B ``[out, rank]`` of one module, any float dtype."""
        rank, a_off, b_off = self.parts[name]
        spec = self.layout.specs[self.layout.index[name]]
        es, dt = self.layout.elem, self.layout.dtype
        tile_rows_into(self.data[a_off : a_off + rank * spec.in_features * es].view(dt), lora_a)
        r8 = round8(rank)
        b_flat = self.data[b_off : b_off + spec.out_features * r8 * es].view(dt)
        if r8 == rank:
            tile_rows_into(b_flat, lora_b)
        else:
            padded = torch.zeros((spec.out_features, r8), dtype=dt)
            padded[:, :rank] = lora_b
            tile_rows_into(b_flat, padded)
        self.filled.add(name)

    def finish(self) -> AdapterImage:
        missing = set(self.parts) - self.filled
        if missing:
            raise RuntimeError(f"image modules never filled: {sorted(missing)}")
        return AdapterImage(self.layout, self.data, self.rows, self.pinned)
