"""Reference fallback forward of a whole model (test infrastructure).

Restates PolyLoraModel.forward + MultiLoraLinear with the torch fallback
(model.py:75-131, layers.py:33-62, :112-134): every target nn.Linear is
replaced by ``OracleLoraLinear``, which adds ``lora.reference_forward`` to the
base output using dense reference-layout slot tensors (cache.py:43-58).
Slot numbers here are simply 1 + the adapter's index in sorted id order; the
LoRA output depends only on which adapter a row uses.
"""

from __future__ import annotations

import torch
from torch import nn

from .lora import dense_slot_tensors, prepare_batched_inputs, reference_forward


def matches_target(name: str, targets: list[str] | None) -> bool:
    """model.py:113-115."""
    return targets is None or any(name == t or name.endswith(f".{t}") for t in targets)


class OracleBank:
    """Dense per-module slot tensors for a fixed adapter set plus the current batch."""

    def __init__(self, adapters: dict, module_shapes: dict, max_rank: int, dtype: torch.dtype, device) -> None:
        # adapters: id -> {module_name: (lora_A [r, in], lora_B [out, r], alpha)}
        self.ids = sorted(adapters)
        self.slot_of = {aid: i + 1 for i, aid in enumerate(self.ids)}
        self.tensors = {}
        for name, (fin, fout) in module_shapes.items():
            per_slot = [None] + [adapters[aid].get(name) for aid in self.ids]
            A, B, ranks, scales = dense_slot_tensors(per_slot, fin, fout, max_rank, dtype)
            self.tensors[name] = (A.to(device), B.to(device), ranks.to(device), scales.to(device))
        self.batch = None  # (weight_indices, seq_lens)


class OracleLoraLinear(nn.Module):
    def __init__(self, base_layer: nn.Linear, name: str, bank: OracleBank) -> None:
        super().__init__()
        self.base_layer = base_layer
        self.name = name
        self.bank = bank

    def forward(self, x: torch.Tensor) -> torch.Tensor:
        base = self.base_layer(x)
        if self.bank.batch is None:
            return base
        weight_indices, seq_lens = self.bank.batch
        x3, b3, seq, widx = prepare_batched_inputs(x, base, weight_indices, seq_lens)
        A, B, ranks, scales = self.bank.tensors[self.name]
        return reference_forward(x3, b3, seq, widx, A, B, ranks, scales).reshape(base.shape)


def wrap_model(model: nn.Module, targets: list[str] | None, bank: OracleBank) -> list[str]:
    """Replace target nn.Linear modules in place (model.py:117-131); returns their names."""
    names = [n for n, m in model.named_modules() if isinstance(m, nn.Linear) and matches_target(n, targets)]
    for name in names:
        parts = name.split(".")
        parent = model
        for p in parts[:-1]:
            parent = getattr(parent, p)
        setattr(parent, parts[-1], OracleLoraLinear(getattr(parent, parts[-1]), name, bank))
    return names


def run(model: nn.Module, bank: OracleBank, adapter_ids: list[str], base_id: str = "__base__", **kwargs):
    """One forward with per-row adapters (model.py:75-111 without residency)."""
    tensor = kwargs.get("input_ids")
    if tensor is None:
        tensor = kwargs.get("inputs_embeds")
    batch, seq_len = int(tensor.shape[0]), int(tensor.shape[1])
    device = tensor.device
    widx = torch.tensor([0 if a == base_id else bank.slot_of[a] for a in adapter_ids], dtype=torch.int64, device=device)
    mask = kwargs.get("attention_mask")
    if mask is None:
        seq_lens = torch.full((batch,), seq_len, dtype=torch.int32, device=device)
    else:
        seq_lens = mask.to(device=device, dtype=torch.int32).sum(dim=-1)
    bank.batch = (widx, seq_lens)
    try:
        return model(**kwargs)
    finally:
        bank.batch = None
