"""Host adapter tiers: PEFT parsing, CPU LRU store and disk cache.

Follows src/polylora/store.py (classes, method names, arguments, exception
types and messages are kept so that callers and tests of the reference work
unchanged).  This tier does no GPU work; ``GpuAdapterCache`` turns a
``CpuAdapter`` into the packed slot image it uploads (cached on the adapter
in ``CpuAdapter.packed``).

Layout fixed by store.py:248-253: ``CpuLayerWeights.A`` is lora_A^T
``[in_features, rank]``, ``.B`` is lora_B^T ``[rank, out_features]``,
``scale = lora_alpha / rank``; tensors keep their source dtype.
"""

from __future__ import annotations

import json
import shutil
from collections import OrderedDict
from dataclasses import dataclass, field
from hashlib import sha256
from pathlib import Path
from typing import Any

import torch


@dataclass(frozen=True)
class CpuLayerWeights:
    A: torch.Tensor
    B: torch.Tensor
    rank: int
    scale: float


@dataclass(frozen=True)
class CpuAdapter:
    adapter_id: str
    config: dict[str, Any]
    layers: dict[str, CpuLayerWeights]
    # slot-image cache: layout key -> packed pinned image (filled by GpuAdapterCache)
    packed: dict = field(default_factory=dict, compare=False, repr=False)


@dataclass(frozen=True)
class DiskAdapterEntry:
    adapter_id: str
    path: Path
    peft_adapter_name: str


class DiskAdapterCache:
    """Bounded LRU of PEFT adapter directories with a JSON manifest (store.py:36-148)."""

    _MANIFEST_NAME = "manifest.json"

    def __init__(self, cache_dir: str | Path, max_adapters: int | None = None) -> None:
        if max_adapters is not None and max_adapters < 1:
            raise ValueError("max_adapters must be at least 1")
        self.cache_dir = Path(cache_dir)
        self.max_adapters = max_adapters
        self.cache_dir.mkdir(parents=True, exist_ok=True)
        self.entries: OrderedDict[str, DiskAdapterEntry] = OrderedDict()
        self._load_manifest()
        self._evict_if_needed()

    def __contains__(self, adapter_id: str) -> bool:
        return adapter_id in self.entries

    def get(self, adapter_id: str) -> DiskAdapterEntry:
        if adapter_id not in self.entries:
            raise KeyError(f"Unknown disk LoRA adapter id: {adapter_id}")
        entry = self.entries[adapter_id]
        self.touch(adapter_id)
        return entry

    def touch(self, adapter_id: str) -> None:
        if adapter_id in self.entries:
            self.entries.move_to_end(adapter_id)
            self._write_manifest()

    def add_adapter(
        self,
        adapter_id: str,
        adapter_path: str | Path,
        peft_adapter_name: str = "default",
    ) -> Path:
        source = Path(adapter_path)
        self._validate_adapter_dir(source)
        target = self.cache_dir / self._entry_dirname(adapter_id)
        if source.resolve() != target.resolve():
            if target.exists():
                shutil.rmtree(target)
            shutil.copytree(source, target)
        self.entries[adapter_id] = DiskAdapterEntry(adapter_id, target, peft_adapter_name)
        self.entries.move_to_end(adapter_id)
        self._evict_if_needed(exclude={adapter_id})
        self._write_manifest()
        return target

    def _load_manifest(self) -> None:
        manifest = self.cache_dir / self._MANIFEST_NAME
        if not manifest.exists():
            return
        data = json.loads(manifest.read_text(encoding="utf-8"))
        for item in data.get("adapters", []):
            path = self.cache_dir / str(item["path"])
            if not path.exists():
                continue
            adapter_id = str(item["adapter_id"])
            self.entries[adapter_id] = DiskAdapterEntry(
                adapter_id=adapter_id,
                path=path,
                peft_adapter_name=str(item.get("peft_adapter_name", "default")),
            )

    def _write_manifest(self) -> None:
        records = [
            {"adapter_id": e.adapter_id, "path": e.path.name, "peft_adapter_name": e.peft_adapter_name}
            for e in self.entries.values()
        ]
        text = json.dumps({"adapters": records}, indent=2, sort_keys=True)
        (self.cache_dir / self._MANIFEST_NAME).write_text(text, encoding="utf-8")

    def _evict_if_needed(self, exclude: set[str] | None = None) -> None:
        if self.max_adapters is None:
            return
        keep = exclude or set()
        changed = False
        while len(self.entries) > self.max_adapters:
            victim = next((aid for aid in self.entries if aid not in keep), None)
            if victim is None:
                raise RuntimeError("No evictable disk LoRA adapter is available")
            entry = self.entries.pop(victim)
            if entry.path.exists():
                shutil.rmtree(entry.path)
            changed = True
        if changed:
            self._write_manifest()

    @staticmethod
    def _entry_dirname(adapter_id: str) -> str:
        # Directory naming rule of store.py:135-139 (kept so existing caches resolve).
        safe = "".join(ch if ch.isalnum() or ch in "-_." else "_" for ch in adapter_id)
        return f"{safe or 'adapter'}-{sha256(adapter_id.encode('utf-8')).hexdigest()[:12]}"

    @staticmethod
    def _validate_adapter_dir(adapter_path: Path) -> None:
        if not (adapter_path / "adapter_config.json").exists():
            raise FileNotFoundError(f"PEFT adapter config not found: {adapter_path / 'adapter_config.json'}")
        if not (adapter_path / "adapter_model.safetensors").exists() and not (
            adapter_path / "adapter_model.bin"
        ).exists():
            raise FileNotFoundError(f"No PEFT adapter weights found in {adapter_path}")


def _pin_if_possible(tensor: torch.Tensor) -> torch.Tensor:
    if torch.cuda.is_available():
        try:
            return tensor.pin_memory()
        except RuntimeError:
            return tensor
    return tensor


class CpuAdapterStore:
    """CPU LRU of parsed adapters with an optional disk tier (store.py:160-436)."""

    def __init__(
        self,
        base_adapter_id: str = "__base__",
        max_adapters: int | None = None,
        disk_cache: DiskAdapterCache | None = None,
        module_names: list[str] | None = None,
    ) -> None:
        if max_adapters is not None and max_adapters < 1:
            raise ValueError("max_adapters must be at least 1")
        self.base_adapter_id = base_adapter_id
        self.max_adapters = max_adapters
        self.disk_cache = disk_cache
        self.module_names = module_names
        self.adapters: OrderedDict[str, CpuAdapter] = OrderedDict()
        self.eviction_exclusions: set[str] = set()

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
        adapter = self.adapters[adapter_id]
        self.touch(adapter_id)
        return adapter

    def touch(self, adapter_id: str) -> None:
        if adapter_id in self.adapters:
            self.adapters.move_to_end(adapter_id)

    def set_eviction_exclusions(self, adapter_ids: set[str]) -> None:
        self.eviction_exclusions = {aid for aid in adapter_ids if aid != self.base_adapter_id}

    def set_module_names(self, module_names: list[str]) -> None:
        self.module_names = list(module_names)

    def add_adapter(
        self,
        adapter_id: str,
        layers: dict[str, CpuLayerWeights],
        config: dict[str, Any] | None = None,
    ) -> None:
        if adapter_id == self.base_adapter_id:
            raise ValueError(f"{self.base_adapter_id!r} is reserved for base-only rows")
        if not layers:
            raise ValueError("Adapter must contain at least one target layer")
        self.adapters[adapter_id] = CpuAdapter(adapter_id, config or {}, layers)
        self.adapters.move_to_end(adapter_id)
        self._evict_if_needed(exclude={adapter_id})

    def add_adapter_from_peft_state_dict(
        self,
        adapter_id: str,
        state_dict: dict[str, torch.Tensor],
        module_names: list[str],
        lora_alpha: float,
        peft_adapter_name: str = "default",
        config: dict[str, Any] | None = None,
    ) -> None:
        self._validate_lora_keys_within_modules(adapter_id, state_dict, module_names)
        layers: dict[str, CpuLayerWeights] = {}
        for module_name in module_names:
            key_a = self._find_lora_key(state_dict, module_name, "lora_A", peft_adapter_name)
            key_b = self._find_lora_key(state_dict, module_name, "lora_B", peft_adapter_name)
            if key_a is None and key_b is None:
                continue
            if key_a is None or key_b is None:
                raise ValueError(f"Adapter {adapter_id!r} has incomplete LoRA weights for {module_name!r}")
            lora_a = state_dict[key_a].detach().to("cpu").contiguous()  # [rank, in]
            lora_b = state_dict[key_b].detach().to("cpu").contiguous()  # [out, rank]
            rank = int(lora_a.shape[0])
            if rank <= 0:
                raise ValueError(f"Adapter {adapter_id!r} has non-positive rank for {module_name!r}")
            if int(lora_b.shape[1]) != rank:
                raise ValueError(f"LoRA A/B rank mismatch for adapter {adapter_id!r}, module {module_name!r}")
            layers[module_name] = CpuLayerWeights(
                A=_pin_if_possible(lora_a.t().contiguous()),
                B=_pin_if_possible(lora_b.t().contiguous()),
                rank=rank,
                scale=float(lora_alpha) / rank,
            )
        self.add_adapter(adapter_id, layers, config)

    def add_adapter_from_peft_model(
        self,
        adapter_id: str,
        peft_model: torch.nn.Module,
        module_names: list[str],
        peft_adapter_name: str | None = None,
    ) -> None:
        name = peft_adapter_name or adapter_id
        adapter_config = getattr(peft_model, "peft_config", {}).get(name)
        if adapter_config is None:
            raise ValueError(f"PEFT model does not contain adapter {name!r}")
        self._validate_peft_config(adapter_config)
        self.add_adapter_from_peft_state_dict(
            adapter_id=adapter_id,
            state_dict=peft_model.state_dict(),
            module_names=module_names,
            lora_alpha=float(getattr(adapter_config, "lora_alpha")),
            peft_adapter_name=name,
            config=self._config_to_dict(adapter_config),
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
        self._load_adapter_from_disk_path(
            adapter_id=adapter_id,
            adapter_path=entry.path,
            module_names=self.module_names,
            peft_adapter_name=entry.peft_adapter_name,
        )

    def _load_adapter_from_disk_path(
        self,
        adapter_id: str,
        adapter_path: str | Path,
        module_names: list[str],
        peft_adapter_name: str = "default",
    ) -> None:
        adapter_path = Path(adapter_path)
        config_path = adapter_path / "adapter_config.json"
        if not config_path.exists():
            raise FileNotFoundError(f"PEFT adapter config not found: {config_path}")
        config = json.loads(config_path.read_text(encoding="utf-8"))
        self._validate_peft_config_dict(config)
        self.add_adapter_from_peft_state_dict(
            adapter_id=adapter_id,
            state_dict=self._load_peft_state_dict(adapter_path),
            module_names=module_names,
            lora_alpha=float(config["lora_alpha"]),
            peft_adapter_name=peft_adapter_name,
            config=config,
        )

    @staticmethod
    def _find_lora_key(
        state_dict: dict[str, torch.Tensor],
        module_name: str,
        side: str,
        peft_adapter_name: str,
    ) -> str | None:
        # PEFT live models name weights "<module>.lora_A.<adapter>.weight";
        # save_pretrained drops the adapter name: "<module>.lora_A.weight".
        suffixes = (f"{module_name}.{side}.{peft_adapter_name}.weight", f"{module_name}.{side}.weight")
        return next((key for key in state_dict if key.endswith(suffixes)), None)

    @classmethod
    def _validate_lora_keys_within_modules(
        cls,
        adapter_id: str,
        state_dict: dict[str, torch.Tensor],
        module_names: list[str],
    ) -> None:
        unexpected = sorted(
            name
            for name in cls._state_dict_lora_module_names(state_dict)
            if not cls._matches_module_name(name, module_names)
        )
        if unexpected:
            raise ValueError(
                f"Adapter {adapter_id!r} contains LoRA weights outside the configured module set: {unexpected}"
            )

    @staticmethod
    def _state_dict_lora_module_names(state_dict: dict[str, torch.Tensor]) -> set[str]:
        names: set[str] = set()
        markers = (".lora_A.", ".lora_B.", ".lora_A.weight", ".lora_B.weight")
        for key in state_dict:
            marker = next((m for m in markers if m in key), None)
            if marker is not None:
                names.add(key.split(marker, 1)[0])
        return names

    @staticmethod
    def _matches_module_name(module_name: str, allowed_module_names: list[str]) -> bool:
        return any(module_name == allowed or module_name.endswith(f".{allowed}") for allowed in allowed_module_names)

    @staticmethod
    def _load_peft_state_dict(adapter_path: Path) -> dict[str, torch.Tensor]:
        safetensors_path = adapter_path / "adapter_model.safetensors"
        bin_path = adapter_path / "adapter_model.bin"
        if safetensors_path.exists():
            try:
                from safetensors.torch import load_file
            except ImportError as exc:
                raise ImportError("safetensors is required to load adapter_model.safetensors") from exc
            return load_file(str(safetensors_path), device="cpu")
        if bin_path.exists():
            # Tensors only: adapter .bin files are state dicts; nothing else is unpickled.
            return torch.load(bin_path, map_location="cpu", weights_only=True)
        raise FileNotFoundError(f"No PEFT adapter weights found in {adapter_path}")

    @staticmethod
    def _validate_peft_config(config: Any) -> None:
        for name in ("use_dora", "lora_bias", "use_rslora"):
            if hasattr(config, name) and getattr(config, name) != False:  # noqa: E712 (store.py:397)
                raise ValueError(f"Unsupported PEFT LoRA option: {name}={getattr(config, name)!r}")
        if getattr(config, "lora_dropout", 0.0) not in (0, 0.0):
            raise ValueError("LoRA dropout is not supported by the inference runtime")

    @staticmethod
    def _validate_peft_config_dict(config: dict[str, Any]) -> None:
        if config.get("peft_type") not in (None, "LORA"):
            raise ValueError(f"Unsupported PEFT adapter type: {config.get('peft_type')!r}")
        if config.get("use_dora", False):
            raise ValueError("DoRA adapters are not supported")
        if config.get("use_rslora", False):
            raise ValueError("RS-LoRA adapters are not supported")
        if config.get("lora_bias", False):
            raise ValueError("LoRA bias is not supported")
        if float(config.get("lora_dropout", 0.0)) != 0.0:
            raise ValueError("LoRA dropout is not supported by the inference runtime")
        if "lora_alpha" not in config:
            raise ValueError("adapter_config.json is missing lora_alpha")

    @staticmethod
    def _config_to_dict(config: Any) -> dict[str, Any]:
        if hasattr(config, "to_dict"):
            return dict(config.to_dict())
        if hasattr(config, "__dict__"):
            return dict(config.__dict__)
        return {}

    def _evict_if_needed(self, exclude: set[str] | None = None) -> None:
        if self.max_adapters is None:
            return
        keep = (exclude or set()) | self.eviction_exclusions
        while len(self.adapters) > self.max_adapters:
            victim = next((aid for aid in self.adapters if aid not in keep), None)
            if victim is None:
                raise RuntimeError("No evictable CPU LoRA adapter is available")
            self.adapters.pop(victim)
