"""Shared test helpers: synthetic PEFT adapters, caches and the matching oracle tensors."""

from __future__ import annotations

import torch

from oracle.lora import dense_slot_tensors
from polylora_amd.cache import GpuAdapterCache, ModuleSpec
from polylora_amd.config import PolyLoraConfig
from polylora_amd.store import CpuAdapterStore, CpuLayerWeights

BF16_TOL = dict(rtol=2e-2, atol=1e-2)
FP32_TOL = dict(rtol=1e-5, atol=1e-5)


def tol_for(dtype: torch.dtype) -> dict:
    return FP32_TOL if dtype == torch.float32 else BF16_TOL


def peft_layer(gen: torch.Generator, fin: int, fout: int, rank: int, alpha: float, std: float = 0.02):
    """PEFT-layout weights: lora_A [rank, in], lora_B [out, rank] ~ N(0, std)."""
    a = torch.randn(rank, fin, generator=gen) * std
    b = torch.randn(fout, rank, generator=gen) * std
    return a, b, float(alpha)


def make_store(adapters: dict, base_id: str = "__base__") -> CpuAdapterStore:
    """adapters: id -> {module: (lora_A, lora_B, alpha)} -> a CpuAdapterStore."""
    store = CpuAdapterStore(base_id)
    for aid, layers in adapters.items():
        store.add_adapter(
            aid,
            {
                m: CpuLayerWeights(A=a.t().contiguous(), B=b.t().contiguous(), rank=a.shape[0], scale=alpha / a.shape[0])
                for m, (a, b, alpha) in layers.items()
            },
        )
    return store


def make_cache(adapters: dict, module_shapes: dict, max_gpu_adapters: int, max_rank: int, device, dtype, tiled=True):
    config = PolyLoraConfig(max_gpu_adapters=max_gpu_adapters, max_rank=max_rank, use_triton_kernels=tiled)
    specs = [ModuleSpec(n, fin, fout) for n, (fin, fout) in module_shapes.items()]
    return GpuAdapterCache(make_store(adapters), specs, config, device, dtype)


def oracle_slot_tensors(cache: GpuAdapterCache, adapters: dict, module: str, dtype: torch.dtype):
    """Reference-layout dense tensors following the cache's current slot assignment."""
    spec = cache.module_specs[module]
    per_slot = [None]
    for slot in range(1, cache.num_slots):
        aid = cache.slot_to_adapter[slot]
        per_slot.append(None if aid is None else adapters[aid].get(module))
    return dense_slot_tensors(per_slot, spec.in_features, spec.out_features, cache.config.max_rank, dtype)
