"""PolyLoraConfig — same fields, defaults and validation as src/polylora/config.py:6-32.

``use_triton_kernels`` keeps its name so existing configs load unchanged.
There is no Triton here: True selects the MFMA-tiled HIP kernels, False the
portable row-based HIP kernels.  Both run on the GPU; neither falls back to
the CPU.
"""

from __future__ import annotations

from dataclasses import dataclass
from pathlib import Path


@dataclass(frozen=True)
class PolyLoraConfig:
    max_gpu_adapters: int
    max_rank: int
    target_modules: list[str] | None = None
    max_cpu_adapters: int | None = None
    disk_cache_dir: str | Path | None = None
    max_disk_adapters: int | None = None
    base_adapter_id: str = "__base__"
    enforce_right_padding: bool = True
    use_triton_kernels: bool = True
    # Device memory for spare slot regions (not in the reference, which
    # rewrites a slot in place): a load copies an adapter into a spare region
    # while a forward still reads the slot's current one.  None: at most
    # GpuAdapterCache.SPARE_REGION_BYTES (4 GiB) and at most an eighth of
    # the device memory free when the cache allocates; 0: no spares (loads
    # then rewrite a slot in place, after its readers).
    spare_region_bytes: int | None = None

    def __post_init__(self) -> None:
        # Same checks and messages as config.py:17-29.
        if self.max_gpu_adapters < 1:
            raise ValueError("max_gpu_adapters must be at least 1")
        if self.max_cpu_adapters is not None and self.max_cpu_adapters < self.max_gpu_adapters:
            raise ValueError("max_cpu_adapters must be at least max_gpu_adapters")
        if self.max_disk_adapters is not None and self.max_disk_adapters < 1:
            raise ValueError("max_disk_adapters must be at least 1")
        if self.max_disk_adapters is not None and self.disk_cache_dir is None:
            raise ValueError("disk_cache_dir must be set when max_disk_adapters is set")
        if self.max_rank < 1:
            raise ValueError("max_rank must be at least 1")
        if self.target_modules is not None and not self.target_modules:
            raise ValueError("target_modules must not be empty when provided")
        if self.spare_region_bytes is not None and self.spare_region_bytes < 0:
            raise ValueError("spare_region_bytes must be at least 0")

    @property
    def use_hip_kernels(self) -> bool:
        """True: MFMA-tiled HIP kernels; False: row-based HIP kernels."""
        return self.use_triton_kernels


CustomLoraConfig = PolyLoraConfig
