"""Host adapter tiers: PEFT parsing into slot images, the CPU LRU store and the disk cache.

Interface of src/polylora/store.py: the classes ``CpuLayerWeights``,
``CpuAdapter``, ``DiskAdapterEntry``, ``DiskAdapterCache`` and
``CpuAdapterStore`` with their method names, arguments, exception types and
messages, the PEFT key suffixes, the disk directory naming and the manifest
schema are kept, so callers and the reference's tests work unchanged.

How an adapter is held.  Once the GPU cache has bound its slot layout to the
store (``bind_layout``), an adapter exists on the host exactly once: as its
``AdapterImage``, the pinned bytes one slot upload copies (``slot_image``),
filled straight from the PEFT tensors -- or from a memory-mapped
``adapter_model.safetensors`` -- without an intermediate transposed copy.
Before a layout is bound (a store used on its own) an adapter keeps its PEFT
tensors as given (``lora_A [r, in]``, ``lora_B [out, r]``, source dtype) and
is packed on first use.  ``CpuAdapter.layers`` still yields the reference's
``CpuLayerWeights`` (``A = lora_A^T [in, r]``, ``B = lora_B^T [r, out]``,
``scale = lora_alpha / r``, store.py:248-253), built on access.

Reference: store.py:14-26 (types), :36-148 (disk tier), :160-436 (store).
"""

from __future__ import annotations

import json
import os
import shutil
import warnings
from collections import OrderedDict
from collections.abc import Mapping
from dataclasses import dataclass
from hashlib import sha256
from pathlib import Path
from typing import Any, Iterator

import numpy as np
import torch

from .slot_image import AdapterImage, ImageBuilder, SlotLayout


@dataclass(frozen=True)
class CpuLayerWeights:
    """One module of an adapter in the reference's host layout (store.py:14-19)."""

    A: torch.Tensor  # lora_A^T [in_features, rank]
    B: torch.Tensor  # lora_B^T [rank, out_features]
    rank: int
    scale: float


@dataclass(frozen=True)
class DiskAdapterEntry:
    adapter_id: str
    path: Path
    peft_adapter_name: str


# --------------------------------------------------------------------------- adapters


class _Module:
    """PEFT tensors of one module before packing: lora_A [r, in], lora_B [out, r]."""

    __slots__ = ("lora_a", "lora_b", "rank", "scale")

    def __init__(self, lora_a: torch.Tensor, lora_b: torch.Tensor, rank: int, scale: float) -> None:
        self.lora_a, self.lora_b, self.rank, self.scale = lora_a, lora_b, rank, scale


class _LayerView(Mapping):
    """``CpuAdapter.layers``: module name -> CpuLayerWeights, built from what the adapter holds."""

    def __init__(self, adapter: "CpuAdapter") -> None:
        self._adapter = adapter

    def __iter__(self) -> Iterator[str]:
        return iter(self._adapter.module_ranks())

    def __len__(self) -> int:
        return len(self._adapter.module_ranks())

    def __contains__(self, name: object) -> bool:
        return name in self._adapter.module_ranks()

    def __getitem__(self, name: str) -> CpuLayerWeights:
        got = self._adapter.peft_tensors(name)
        if got is None:
            raise KeyError(name)
        lora_a, lora_b, rank, scale = got
        return CpuLayerWeights(A=lora_a.t(), B=lora_b.t(), rank=rank, scale=scale)


class CpuAdapter:
    """A parsed adapter: its id, PEFT config, and its weights, held once (store.py:22-26).

    Either the PEFT tensors (no slot layout bound yet) or one ``AdapterImage``.
    """

    def __init__(self, adapter_id: str, config: dict[str, Any], modules: dict[str, _Module]) -> None:
        self.adapter_id = adapter_id
        self.config = config
        self._modules: dict[str, _Module] | None = modules
        self._image: AdapterImage | None = None
        self._ranks = {name: (m.rank, m.scale) for name, m in modules.items()}

    @classmethod
    def from_image(cls, adapter_id: str, config: dict[str, Any], image: AdapterImage) -> "CpuAdapter":
        """An adapter held only as an already packed slot image."""
        adapter = cls(adapter_id, config, {})
        adapter._modules = None
        adapter._image = image
        adapter._ranks = {}
        for spec in image.layout.specs:
            got = image.entry(spec.name)
            if got is not None:
                adapter._ranks[spec.name] = (got[0], got[1])
        return adapter

    @property
    def layers(self) -> Mapping:
        return _LayerView(self)

    @property
    def image(self) -> AdapterImage | None:
        """The packed slot image, once there is one."""
        return self._image

    def module_ranks(self) -> dict[str, tuple[int, float]]:
        """module name -> (rank, scale) of every module the adapter has weights for."""
        return self._ranks

    def peft_tensors(self, name: str):
        """(lora_A [r, in], lora_B [out, r], rank, scale) of a module, or None if the adapter lacks it."""
        if name not in self._ranks:
            return None
        if self._modules is not None:
            m = self._modules[name]
            return m.lora_a, m.lora_b, m.rank, m.scale
        lora_a, lora_b, scale = self._image.lora_tensors(name)
        return lora_a, lora_b, self._ranks[name][0], scale

    def image_for(self, layout: SlotLayout, keep_source: bool = True, pin=None) -> AdapterImage:
        """The adapter packed for ``layout``, packing it first if needed.

        Raises the reference's slot-load errors (cache.py:129-136) for a rank
        above the layout's cap or a module of the wrong shape.  With
        ``keep_source=False`` the PEFT tensors are dropped once packed, unless
        packing rounded them (a source dtype wider than the layout's).
        """
        if self._image is not None and self._image.layout.key == layout.key:
            return self._image
        specs = {s.name: s for s in layout.specs}
        present = {}
        for spec in layout.specs:  # the reference's check order: module order of the cache
            got = self.peft_tensors(spec.name)
            if got is None:
                continue
            lora_a, lora_b, rank, scale = got
            if rank > layout.max_rank:
                raise ValueError(f"Adapter {self.adapter_id!r} rank {rank} exceeds max_rank {layout.max_rank}")
            if tuple(lora_a.shape) != (rank, spec.in_features):
                raise ValueError(f"LoRA A shape mismatch for adapter {self.adapter_id!r}, module {spec.name!r}")
            if tuple(lora_b.shape) != (spec.out_features, rank):
                raise ValueError(f"LoRA B shape mismatch for adapter {self.adapter_id!r}, module {spec.name!r}")
            present[spec.name] = (lora_a, lora_b, rank, scale)
        builder = ImageBuilder(layout, {n: (v[2], v[3]) for n, v in present.items()}, pin=pin)
        for name, (lora_a, lora_b, _, _) in present.items():
            builder.put(name, lora_a, lora_b)
        image = builder.finish()
        # the source tensors stay whenever packing rounded them: a later layout of
        # another dtype packs from them, as the reference converts its source-dtype
        # copy at every slot load (store.py:240-241, cache.py:139)
        keep_source = keep_source or (self._modules is not None and any(
            rounds(a.dtype, layout.dtype) or rounds(b.dtype, layout.dtype) for a, b, _, _ in present.values()))
        # modules outside the layout are not part of any slot and are not kept
        self._ranks = {n: self._ranks[n] for n in self._ranks if n in specs} if not keep_source else self._ranks
        self._image = image
        if not keep_source:
            self._modules = None
        return image


def rounds(src: torch.dtype, dst: torch.dtype) -> bool:
    """Whether converting values of dtype ``src`` to ``dst`` can change them."""
    return src != dst and not (dst == torch.float32 and src in (torch.bfloat16, torch.float16))


# --------------------------------------------------------------------------- PEFT files


_ST_DTYPES = {
    "F32": (np.float32, None),
    "F64": (np.float64, None),
    "F16": (np.float16, None),
    "BF16": (np.uint16, torch.bfloat16),
}


def read_safetensors(path: Path) -> dict[str, torch.Tensor]:
    """Tensors of a .safetensors file as views of a private memory map of it.

    The format is an 8-byte little-endian header length, a JSON header of
    ``name -> {dtype, shape, data_offsets}`` (offsets relative to the end of
    the header) and the raw little-endian data.  Nothing is read until a
    tensor is touched, so packing copies each weight from the page cache
    straight into its slot image.
    """
    with open(path, "rb") as fh:
        head_len = int.from_bytes(fh.read(8), "little")
        header = json.loads(fh.read(head_len))
    base = 8 + head_len
    mapped = np.memmap(path, dtype=np.uint8, mode="c")  # copy-on-write: never writes the file
    out: dict[str, torch.Tensor] = {}
    for name, info in header.items():
        if name == "__metadata__":
            continue
        kind = info["dtype"]
        if kind not in _ST_DTYPES:
            raise ValueError(f"unsupported safetensors dtype {kind!r} for {name!r} in {path}")
        np_dtype, torch_view = _ST_DTYPES[kind]
        start, end = (int(v) for v in info["data_offsets"])
        raw = mapped[base + start : base + end]
        if (base + start) % np.dtype(np_dtype).itemsize:
            raw = np.array(raw)  # an unaligned tensor is copied rather than viewed
        arr = raw.view(np_dtype).reshape([int(v) for v in info["shape"]])
        t = torch.from_numpy(arr)
        out[name] = t.view(torch_view) if torch_view is not None else t
    return out


def _peft_state_dict(adapter_path: Path) -> dict[str, torch.Tensor]:
    """adapter_model.safetensors (memory-mapped) or adapter_model.bin (tensors only) of a PEFT directory."""
    st = adapter_path / "adapter_model.safetensors"
    if st.exists():
        return read_safetensors(st)
    pt = adapter_path / "adapter_model.bin"
    if pt.exists():
        # weights_only: the file is a state dict and nothing else in it is executed
        try:
            return torch.load(pt, map_location="cpu", weights_only=True, mmap=True)
        except RuntimeError:  # legacy (non-zip) files cannot be mapped
            return torch.load(pt, map_location="cpu", weights_only=True)
    raise FileNotFoundError(f"No PEFT adapter weights found in {adapter_path}")


def _has_peft_weights(adapter_path: Path) -> bool:
    return any((adapter_path / f).exists() for f in ("adapter_model.safetensors", "adapter_model.bin"))


def _check_peft_config_file(config: dict[str, Any]) -> None:
    """The adapter_config.json options the runtime cannot serve (store.py:402-415)."""
    kind = config.get("peft_type")
    if kind not in (None, "LORA"):
        raise ValueError(f"Unsupported PEFT adapter type: {kind!r}")
    refused = (("use_dora", "DoRA adapters are not supported"), ("use_rslora", "RS-LoRA adapters are not supported"),
               ("lora_bias", "LoRA bias is not supported"))
    for key, message in refused:
        if config.get(key, False):
            raise ValueError(message)
    if float(config.get("lora_dropout", 0.0)) != 0.0:
        raise ValueError("LoRA dropout is not supported by the inference runtime")
    if "lora_alpha" not in config:
        raise ValueError("adapter_config.json is missing lora_alpha")


def _check_peft_config_object(config: Any) -> None:
    """The same for a live PEFT LoraConfig (store.py:389-400)."""
    for option in ("use_dora", "lora_bias", "use_rslora"):
        if hasattr(config, option):
            value = getattr(config, option)
            if value != False:  # noqa: E712 -- any value but False is refused, as store.py:397
                raise ValueError(f"Unsupported PEFT LoRA option: {option}={value!r}")
    if getattr(config, "lora_dropout", 0.0) not in (0, 0.0):
        raise ValueError("LoRA dropout is not supported by the inference runtime")


def _config_as_dict(config: Any) -> dict[str, Any]:
    for convert in (lambda c: c.to_dict(), lambda c: vars(c)):
        try:
            return dict(convert(config))
        except (AttributeError, TypeError):
            continue
    return {}


class _PeftKeys:
    """LoRA keys of a PEFT state dict, parsed once.

    A live PeftModel names weights ``<module>.lora_A.<adapter>.weight``;
    ``save_pretrained`` drops the adapter name: ``<module>.lora_A.weight``.
    A target module's key is the first key, in state-dict order, that ends
    with ``<module>.<side>.<adapter>.weight`` or ``<module>.<side>.weight``
    (store.py:330-342); a key's module is the text before its first
    ``.lora_A.`` / ``.lora_B.`` (store.py:361-369).
    """

    def __init__(self, state_dict: Mapping[str, torch.Tensor]) -> None:
        self.keys = list(state_dict)
        self.modules: set[str] = set()
        # (dot-aligned suffix of a key's text before its side, rest of the key) -> first key
        self._index: dict[tuple[str, str], str] = {}
        for key in self.keys:
            cut = min((i for i in (key.find(".lora_A."), key.find(".lora_B.")) if i >= 0), default=-1)
            if cut < 0:
                continue
            head, rest = key[:cut], key[cut:]
            self.modules.add(head)
            parts = head.split(".")
            for i in range(len(parts)):
                self._index.setdefault((".".join(parts[i:]), rest), key)

    def find(self, module_name: str, side: str, adapter_name: str) -> str | None:
        rests = (f".{side}.{adapter_name}.weight", f".{side}.weight")
        hits = [self._index[(module_name, r)] for r in rests if (module_name, r) in self._index]
        if not hits:
            # a suffix that does not start at a dot still matches, as the plain endswith rule has it
            wanted = tuple(module_name + r for r in rests)
            hits = [k for k in self.keys if k.endswith(wanted)] if module_name else []
        if not hits:
            return None
        order = {k: i for i, k in enumerate(self.keys) if k in hits}
        return min(hits, key=order.__getitem__)

    def outside(self, module_names: list[str]) -> list[str]:
        def allowed(m: str) -> bool:
            return any(m == t or m.endswith(f".{t}") for t in module_names)

        return sorted(m for m in self.modules if not allowed(m))


# --------------------------------------------------------------------------- disk tier


class DiskAdapterCache:
    """Bounded LRU of PEFT adapter directories under ``cache_dir`` with a JSON manifest (store.py:36-148).

    Entries live in ``<cache_dir>/<safe id>-<sha256(id)[:12]>``; the manifest
    ``manifest.json`` lists ``{adapter_id, path, peft_adapter_name}`` oldest
    first, so a restarted process finds the same entries in the same order.
    """

    _MANIFEST_NAME = "manifest.json"

    def __init__(self, cache_dir: str | Path, max_adapters: int | None = None) -> None:
        if max_adapters is not None and max_adapters < 1:
            raise ValueError("max_adapters must be at least 1")
        self.cache_dir = Path(cache_dir)
        self.max_adapters = max_adapters
        self.cache_dir.mkdir(parents=True, exist_ok=True)
        self.entries: OrderedDict[str, DiskAdapterEntry] = OrderedDict(self._read_manifest())
        self._evict_if_needed()

    def __contains__(self, adapter_id: str) -> bool:
        return adapter_id in self.entries

    def get(self, adapter_id: str) -> DiskAdapterEntry:
        entry = self.entries.get(adapter_id)
        if entry is None:
            raise KeyError(f"Unknown disk LoRA adapter id: {adapter_id}")
        self.touch(adapter_id)
        return entry

    def touch(self, adapter_id: str) -> None:
        if adapter_id not in self.entries:
            return
        self.entries.move_to_end(adapter_id)
        self._write_manifest()

    def add_adapter(self, adapter_id: str, adapter_path: str | Path, peft_adapter_name: str = "default") -> Path:
        source = Path(adapter_path)
        self._validate_adapter_dir(source)
        home = self.cache_dir / self._entry_dirname(adapter_id)
        if source.resolve() != home.resolve():
            shutil.rmtree(home, ignore_errors=True)
            shutil.copytree(source, home)
        self.entries.pop(adapter_id, None)
        self.entries[adapter_id] = DiskAdapterEntry(adapter_id, home, peft_adapter_name)
        self._evict_if_needed(exclude={adapter_id})
        self._write_manifest()
        return home

    def _read_manifest(self) -> Iterator[tuple[str, DiskAdapterEntry]]:
        manifest = self.cache_dir / self._MANIFEST_NAME
        if not manifest.exists():
            return
        for record in json.loads(manifest.read_text(encoding="utf-8")).get("adapters", []):
            home = self.cache_dir / str(record["path"])
            if home.exists():  # directories removed behind the cache's back are forgotten
                aid = str(record["adapter_id"])
                yield aid, DiskAdapterEntry(aid, home, str(record.get("peft_adapter_name", "default")))

    def _write_manifest(self) -> None:
        # written beside the manifest and renamed over it: a process that dies
        # mid-write leaves the previous manifest, never a truncated one
        listing = [{"adapter_id": e.adapter_id, "path": e.path.name, "peft_adapter_name": e.peft_adapter_name}
                   for e in self.entries.values()]
        target = self.cache_dir / self._MANIFEST_NAME
        staging = target.with_name(f".{target.name}.{os.getpid()}.tmp")
        staging.write_text(json.dumps({"adapters": listing}, indent=2, sort_keys=True), encoding="utf-8")
        os.replace(staging, target)

    def _evict_if_needed(self, exclude: set[str] | None = None) -> None:
        if self.max_adapters is None or len(self.entries) <= self.max_adapters:
            return
        keep = exclude or set()
        while len(self.entries) > self.max_adapters:
            victim = next((e for aid, e in self.entries.items() if aid not in keep), None)
            if victim is None:
                raise RuntimeError("No evictable disk LoRA adapter is available")
            del self.entries[victim.adapter_id]
            shutil.rmtree(victim.path, ignore_errors=True)
        self._write_manifest()

    @staticmethod
    def _entry_dirname(adapter_id: str) -> str:
        # the directory naming of store.py:135-139, so caches written by the reference still resolve
        safe = "".join(c if (c.isalnum() or c in "-_.") else "_" for c in adapter_id) or "adapter"
        return f"{safe}-{sha256(adapter_id.encode('utf-8')).hexdigest()[:12]}"

    @staticmethod
    def _validate_adapter_dir(adapter_path: Path) -> None:
        config = adapter_path / "adapter_config.json"
        if not config.exists():
            raise FileNotFoundError(f"PEFT adapter config not found: {config}")
        if not _has_peft_weights(adapter_path):
            raise FileNotFoundError(f"No PEFT adapter weights found in {adapter_path}")


# --------------------------------------------------------------------------- CPU tier


class CpuAdapterStore:
    """CPU LRU of parsed adapters over an optional disk tier (store.py:160-436).

    Adapters that are resident on the GPU (``set_eviction_exclusions``) are
    never evicted.  With a slot layout bound (``bind_layout``, done by the GPU
    cache) every adapter added is packed into its pinned slot image at once
    and its PEFT tensors are not kept, unless packing rounded them (source
    dtype wider than the layout's): those stay, in their own dtype, so that a
    later layout of another dtype packs from them.
    """

    def __init__(
        self,
        base_adapter_id: str = "__base__",
        max_adapters: int | None = None,
        disk_cache: DiskAdapterCache | None = None,
        module_names: list[str] | None = None,
        *,
        pinned_bytes_limit: int | None = None,
    ) -> None:
        """``pinned_bytes_limit`` (not in the reference): page-lock slot images only up to this many
        bytes in total; later images stay pageable (their slot loads are staged copies that block the
        host).  None pins every image, as far as the system allows."""
        if max_adapters is not None and max_adapters < 1:
            raise ValueError("max_adapters must be at least 1")
        self.base_adapter_id = base_adapter_id
        self.max_adapters = max_adapters
        self.disk_cache = disk_cache
        self.module_names = module_names
        self.adapters: OrderedDict[str, CpuAdapter] = OrderedDict()
        self.eviction_exclusions: set[str] = set()
        self.layout: SlotLayout | None = None
        self.pinned_bytes_limit = pinned_bytes_limit

    # ---------------------------------------------------------------- lookup
    def __contains__(self, adapter_id: str) -> bool:
        if adapter_id == self.base_adapter_id or adapter_id in self.adapters:
            return True
        return self.disk_cache is not None and adapter_id in self.disk_cache

    def get(self, adapter_id: str) -> CpuAdapter:
        if adapter_id == self.base_adapter_id:
            raise KeyError(f"Base adapter {adapter_id!r} has no LoRA weights")
        if adapter_id not in self.adapters:
            if self.disk_cache is None or adapter_id not in self.disk_cache:
                raise KeyError(f"Unknown LoRA adapter id: {adapter_id}")
            self._load_adapter_from_disk_cache(adapter_id)
        self.touch(adapter_id)
        return self.adapters[adapter_id]

    def touch(self, adapter_id: str) -> None:
        if adapter_id in self.adapters:
            self.adapters.move_to_end(adapter_id)

    def set_eviction_exclusions(self, adapter_ids: set[str]) -> None:
        self.eviction_exclusions = set(adapter_ids) - {self.base_adapter_id}

    def set_module_names(self, module_names: list[str]) -> None:
        self.module_names = list(module_names)

    # ---------------------------------------------------------------- images
    def bind_layout(self, layout: SlotLayout) -> None:
        """Pack adapters for this slot layout from now on (adapters already held are packed on first use)."""
        self.layout = layout

    def image(self, adapter: CpuAdapter, layout: SlotLayout) -> AdapterImage:
        """``adapter`` packed for ``layout``; its PEFT tensors are dropped when that is the bound layout
        and packing did not round them."""
        bound = self.layout is not None and self.layout.key == layout.key
        return adapter.image_for(layout, keep_source=not bound, pin=self.pin_image)

    def pinned_bytes(self) -> int:
        """Bytes of page-locked slot images the store holds."""
        total = 0
        for adapter in self.adapters.values():
            img = adapter.image
            if img is not None and img.pinned:
                total += int(img.data.numel())
        return total

    def pin_image(self, nbytes: int) -> bool:
        """Whether a new image of ``nbytes`` is page-locked under ``pinned_bytes_limit``."""
        if self.pinned_bytes_limit is None:
            return True
        return self.pinned_bytes() + nbytes <= self.pinned_bytes_limit

    # ---------------------------------------------------------------- adding
    def add_adapter(
        self,
        adapter_id: str,
        layers: dict[str, CpuLayerWeights],
        config: dict[str, Any] | None = None,
    ) -> None:
        modules = {name: _Module(w.A.t(), w.B.t(), int(w.rank), float(w.scale)) for name, w in layers.items()}
        self._insert(adapter_id, modules, config)

    def add_adapter_image(self, adapter_id: str, image: AdapterImage, config: dict[str, Any] | None = None) -> None:
        """Add an adapter that is already packed in a slot image (``slot_image.ImageBuilder``).

        No counterpart in the reference: for callers that keep or build
        images themselves (a reload without parsing, a synthetic catalog).
        The image must be for the store's bound layout, if it has one.
        """
        if self.layout is not None and image.layout.key != self.layout.key:
            raise ValueError(f"Adapter {adapter_id!r}: image layout does not match the store's slot layout")
        self._check_new(adapter_id, bool(CpuAdapter.from_image(adapter_id, {}, image).module_ranks()))
        self._place(CpuAdapter.from_image(adapter_id, config or {}, image))

    def _check_new(self, adapter_id: str, has_modules: bool) -> None:
        if adapter_id == self.base_adapter_id:
            raise ValueError(f"{self.base_adapter_id!r} is reserved for base-only rows")
        if not has_modules:
            raise ValueError("Adapter must contain at least one target layer")

    def _insert(self, adapter_id: str, modules: dict[str, _Module], config: dict[str, Any] | None) -> None:
        self._check_new(adapter_id, bool(modules))
        adapter = CpuAdapter(adapter_id, config or {}, modules)
        if self.layout is not None:
            try:
                adapter.image_for(self.layout, keep_source=False, pin=self.pin_image)
            except ValueError:
                pass  # kept as given: the slot load raises the reference's error (cache.py:129-136)
        self._place(adapter)

    def _place(self, adapter: CpuAdapter) -> None:
        """Newest entry of the LRU (replacing one of the same id), then evict down to the capacity."""
        self.adapters.pop(adapter.adapter_id, None)
        self.adapters[adapter.adapter_id] = adapter
        self._evict_if_needed(exclude={adapter.adapter_id})

    def add_adapter_from_peft_state_dict(
        self,
        adapter_id: str,
        state_dict: dict[str, torch.Tensor],
        module_names: list[str],
        lora_alpha: float,
        peft_adapter_name: str = "default",
        config: dict[str, Any] | None = None,
    ) -> None:
        keys = _PeftKeys(state_dict)
        outside = keys.outside(module_names)
        if outside:
            raise ValueError(f"Adapter {adapter_id!r} contains LoRA weights outside the configured module set: {outside}")
        modules: dict[str, _Module] = {}
        for name in module_names:
            key_a = keys.find(name, "lora_A", peft_adapter_name)
            key_b = keys.find(name, "lora_B", peft_adapter_name)
            if key_a is None and key_b is None:
                continue  # the adapter does not touch this module: rank 0 there
            if key_a is None or key_b is None:
                raise ValueError(f"Adapter {adapter_id!r} has incomplete LoRA weights for {name!r}")
            lora_a, lora_b = state_dict[key_a].detach(), state_dict[key_b].detach()
            rank = int(lora_a.shape[0])
            if rank <= 0:
                raise ValueError(f"Adapter {adapter_id!r} has non-positive rank for {name!r}")
            if int(lora_b.shape[1]) != rank:
                raise ValueError(f"LoRA A/B rank mismatch for adapter {adapter_id!r}, module {name!r}")
            if self.layout is None or rounds(lora_a.dtype, self.layout.dtype) or rounds(lora_b.dtype, self.layout.dtype):
                # held beside or instead of the image (no layout bound yet, or packing rounds
                # them): an owned CPU copy in the source dtype, independent of the caller's tensors
                lora_a, lora_b = lora_a.to("cpu", copy=True), lora_b.to("cpu", copy=True)
            modules[name] = _Module(lora_a, lora_b, rank, float(lora_alpha) / rank)
        self._insert(adapter_id, modules, config)

    def add_adapter_from_peft_model(
        self,
        adapter_id: str,
        peft_model: torch.nn.Module,
        module_names: list[str],
        peft_adapter_name: str | None = None,
    ) -> None:
        name = peft_adapter_name or adapter_id
        lora_config = getattr(peft_model, "peft_config", {}).get(name)
        if lora_config is None:
            raise ValueError(f"PEFT model does not contain adapter {name!r}")
        _check_peft_config_object(lora_config)
        self.add_adapter_from_peft_state_dict(
            adapter_id,
            peft_model.state_dict(),
            module_names,
            float(lora_config.lora_alpha),
            peft_adapter_name=name,
            config=_config_as_dict(lora_config),
        )

    def load_adapter_from_disk(
        self,
        adapter_id: str,
        adapter_path: str | Path,
        module_names: list[str],
        peft_adapter_name: str = "default",
    ) -> None:
        if self.disk_cache is not None:
            adapter_path = self.disk_cache.add_adapter(adapter_id, adapter_path, peft_adapter_name)
        self._load_adapter_from_disk_path(adapter_id, adapter_path, module_names, peft_adapter_name)

    def _load_adapter_from_disk_cache(self, adapter_id: str) -> None:
        if self.disk_cache is None:
            raise KeyError(f"Unknown LoRA adapter id: {adapter_id}")
        if self.module_names is None:
            raise RuntimeError("module_names must be configured before loading adapters from disk cache")
        entry = self.disk_cache.get(adapter_id)
        self._load_adapter_from_disk_path(adapter_id, entry.path, self.module_names, entry.peft_adapter_name)

    def _load_adapter_from_disk_path(
        self,
        adapter_id: str,
        adapter_path: str | Path,
        module_names: list[str],
        peft_adapter_name: str = "default",
    ) -> None:
        home = Path(adapter_path)
        config_file = home / "adapter_config.json"
        if not config_file.exists():
            raise FileNotFoundError(f"PEFT adapter config not found: {config_file}")
        config = json.loads(config_file.read_text(encoding="utf-8"))
        _check_peft_config_file(config)
        with warnings.catch_warnings():
            warnings.simplefilter("ignore", UserWarning)  # torch notes that mapped views are not writable
            state_dict = _peft_state_dict(home)
            self.add_adapter_from_peft_state_dict(adapter_id, state_dict, module_names, float(config["lora_alpha"]),
                                                  peft_adapter_name, config)

    # ---------------------------------------------------------------- eviction
    def _evict_if_needed(self, exclude: set[str] | None = None) -> None:
        if self.max_adapters is None:
            return
        keep = (exclude or set()) | self.eviction_exclusions
        while len(self.adapters) > self.max_adapters:
            victim = next((aid for aid in self.adapters if aid not in keep), None)
            if victim is None:
                raise RuntimeError("No evictable CPU LoRA adapter is available")
            del self.adapters[victim]
