"""polylora_amd — multi-LoRA inference with gfx950 HIP SGMV kernels.

Same public names as the reference package ``polylora`` (src/polylora/__init__.py:1-18).
"""

from .cache import GpuAdapterCache
from .config import CustomLoraConfig, PolyLoraConfig
from .context import LoraBatchContext
from .layers import MultiLoraLinear
from .model import CustomPeftModel, PolyLoraModel
from .store import CpuAdapterStore, DiskAdapterCache

__all__ = [
    "CpuAdapterStore",
    "CustomLoraConfig",
    "CustomPeftModel",
    "DiskAdapterCache",
    "GpuAdapterCache",
    "LoraBatchContext",
    "MultiLoraLinear",
    "PolyLoraConfig",
    "PolyLoraModel",
]
