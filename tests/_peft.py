"""PEFT-layout adapter fixtures written without PEFT (it is not installed).

Key names follow PEFT's LoRA layer naming: a live PeftModel's state dict uses
``base_model.model.<module>.lora_A.<adapter>.weight`` (shape [r, in]) and
``...lora_B.<adapter>.weight`` ([out, r]); ``save_pretrained`` drops the
adapter name: ``base_model.model.<module>.lora_A.weight``.  The directory
holds ``adapter_config.json`` plus ``adapter_model.safetensors`` or
``adapter_model.bin``, as the reference's tests write them
(tests/test_polylora_peft.py:86-100, :164).
"""

from __future__ import annotations

import json
from pathlib import Path

import torch


def linear_shapes(model: torch.nn.Module, targets: list[str] | None) -> dict[str, tuple[int, int]]:
    out = {}
    for name, mod in model.named_modules():
        if isinstance(mod, torch.nn.Linear) and (targets is None or any(name == t or name.endswith("." + t) for t in targets)):
            out[name] = (mod.in_features, mod.out_features)
    return out


def make_lora_weights(gen: torch.Generator, shapes: dict, rank: int, std: float = 0.02, modules=None):
    """{module: (lora_A [r, in], lora_B [out, r])} with N(0, std) entries (B != 0, like init_lora_weights=False)."""
    mods = modules if modules is not None else list(shapes)
    return {m: (torch.randn(rank, shapes[m][0], generator=gen) * std, torch.randn(shapes[m][1], rank, generator=gen) * std) for m in mods}


def state_dict(weights: dict, adapter_name: str | None = None) -> dict[str, torch.Tensor]:
    sd = {}
    for mod, (a, b) in weights.items():
        mid = f".{adapter_name}" if adapter_name else ""
        sd[f"base_model.model.{mod}.lora_A{mid}.weight"] = a.contiguous()
        sd[f"base_model.model.{mod}.lora_B{mid}.weight"] = b.contiguous()
    return sd


def write_adapter_dir(path: Path, weights: dict, rank: int, alpha: float, fmt: str = "safetensors",
                      adapter_name: str | None = None, extra_config: dict | None = None) -> Path:
    path = Path(path)
    path.mkdir(parents=True, exist_ok=True)
    cfg = {"peft_type": "LORA", "r": rank, "lora_alpha": alpha, "lora_dropout": 0.0,
           "target_modules": sorted({m.rsplit(".", 1)[-1] for m in weights})}
    cfg.update(extra_config or {})
    (path / "adapter_config.json").write_text(json.dumps(cfg), encoding="utf-8")
    sd = state_dict(weights, adapter_name)
    if fmt == "safetensors":
        from safetensors.torch import save_file

        save_file(sd, str(path / "adapter_model.safetensors"))
    else:
        torch.save(sd, path / "adapter_model.bin")
    return path


def tiny_deberta(seed: int, vocab: int = 97, relative_attention: bool = False):
    """The reference tests' fixture model (tests/test_polylora_peft.py:40-52)."""
    from transformers import DebertaV2Config, DebertaV2Model

    torch.manual_seed(seed)
    cfg = DebertaV2Config(
        vocab_size=vocab,
        hidden_size=32,
        num_hidden_layers=1,
        num_attention_heads=4,
        intermediate_size=64,
        hidden_dropout_prob=0.0,
        attention_probs_dropout_prob=0.0,
        max_position_embeddings=32,
        relative_attention=relative_attention,
        type_vocab_size=0,
        **({"share_att_key": True, "position_buckets": 8, "pos_att_type": ["p2c", "c2p"]} if relative_attention else {}),
    )
    return DebertaV2Model(cfg).eval()
