"""Seeded random models through PolyLoraModel, every wrapped Linear against the oracle.

Each case draws a dtype, a tiny Llama (hidden and FFN sizes drawn too), a random
subset of the seven target modules (so sibling runs can be partial: q and v
without k, gate without up), adapters that cover random subsets of the targets
with a rank drawn per module, a right-padded batch (prefill) or one-token rows
(decode-sized), and rows on __base__.  Two forwards run under the per-layer
check (tests/test_gpu_model.py::_per_layer_check: each wrapped Linear's output
against oracle.lora.reference_forward on the inputs it saw); the second
forward, which runs the sibling runs learned from the first in stacked
launches, must equal the first bit for bit, and __base__ rows equal the base
model's output bit for bit.

Reference: PolyLoraModel.forward and MultiLoraLinear.forward (model.py:75-85,
layers.py:33-62) against the fallback of layers.py:112-134.
"""

from __future__ import annotations

import copy

import numpy as np
import pytest
import torch

from polylora_amd import PolyLoraConfig, PolyLoraModel
from tests import _peft
from tests.test_gpu_model import LLAMA_TARGETS, _announce, _per_layer_check, _shapes

pytestmark = pytest.mark.gpu

_DTYPES = (torch.bfloat16, torch.float16, torch.float32)


def _llama(seed, dtype, device, hidden, ffn):
    from transformers import LlamaConfig, LlamaModel

    from bench import register_attention

    register_attention()
    torch.manual_seed(seed)
    cfg = LlamaConfig(hidden_size=hidden, num_hidden_layers=2, num_attention_heads=4, num_key_value_heads=2,
                      head_dim=hidden // 4, intermediate_size=ffn, vocab_size=211)
    cfg._attn_implementation = "pl_safe_fp32"
    return LlamaModel(cfg).to(device=device, dtype=dtype).eval()


@pytest.mark.parametrize("seed", range(24))
def test_random_models_every_layer_against_the_oracle(gpu, seed):
    r = np.random.default_rng(7000 + seed)
    dtype = _DTYPES[int(r.integers(3))]
    hidden = int(r.choice([64, 128, 192]))
    ffn = int(r.choice([128, 256, 352]))
    k = int(r.integers(1, len(LLAMA_TARGETS) + 1))
    targets = sorted(r.choice(LLAMA_TARGETS, size=k, replace=False).tolist(), key=LLAMA_TARGETS.index)
    max_rank = int(r.choice([8, 16, 32]))
    n_ad = int(r.integers(1, 7))
    decode = bool(r.integers(2))
    B = int(r.integers(1, 13))
    S = 1 if decode else int(r.integers(2, 301))
    _announce(test="model_sweep", seed=seed, dtype=dtype, hidden=hidden, ffn=ffn, targets=targets,
              max_rank=max_rank, adapters=n_ad, B=B, S=S)
    base = _llama(seed, dtype, gpu, hidden, ffn)
    pm = PolyLoraModel(copy.deepcopy(base), PolyLoraConfig(target_modules=targets, max_gpu_adapters=n_ad,
                                                           max_rank=max_rank)).eval()
    shapes = _shapes(pm)
    names = list(shapes)
    g = torch.Generator().manual_seed(seed)
    ads = {}
    for i in range(n_ad):
        mods = [m for m in names if r.random() < 0.7] or [names[0]]
        weights = {}
        for m in mods:  # a rank per module
            weights.update(_peft.make_lora_weights(g, shapes, int(r.integers(1, max_rank + 1)), std=0.05, modules=[m]))
        alpha = float(r.choice([1.0, 8.0, 16.0]))
        ads[f"ad{i}"] = (weights, alpha)
        pm.adapter_store.add_adapter_from_peft_state_dict(f"ad{i}", _peft.state_dict(weights), pm.target_module_names,
                                                          alpha)
    pool = ["__base__", *ads]
    adapter_ids = [pool[int(i)] for i in r.integers(0, len(pool), B)]
    ids = torch.randint(0, 211, (B, S), generator=g).to(gpu)
    if decode:
        mask = torch.ones(B, S, dtype=torch.long, device=gpu)
    else:
        lens = torch.randint(1, S + 1, (B,), generator=g)
        mask = (torch.arange(S)[None, :] < lens[:, None]).long().to(gpu)
    with torch.inference_mode(), _per_layer_check(pm, ads, dtype, f"model sweep seed {seed}") as checked:
        first = pm(input_ids=ids, attention_mask=mask, adapter_ids=adapter_ids).last_hidden_state
        second = pm(input_ids=ids, attention_mask=mask, adapter_ids=adapter_ids).last_hidden_state
    assert checked.calls == 2 * len(pm.target_module_names), (checked.calls, len(pm.target_module_names))
    assert torch.equal(first, second), "the stacked second forward differs from the first"
    with torch.inference_mode():
        plain = base(input_ids=ids, attention_mask=mask).last_hidden_state
    valid = mask.bool()
    for b, aid in enumerate(adapter_ids):
        if aid == "__base__":
            assert torch.equal(first[b][valid[b]], plain[b][valid[b]]), b


@pytest.mark.parametrize("seed", range(8))
def test_random_churn_every_layer_against_the_oracle(gpu, seed):
    """A catalog larger than the slots through random batches: each step loads the adapters it lacks into
    free or evicted slots (spare regions on or off, so loads copy beside the readers or rewrite a slot in
    place after them), and every wrapped Linear of every step is checked against the oracle on the
    cache's slot assignment at that step."""
    r = np.random.default_rng(8000 + seed)
    dtype = (torch.bfloat16, torch.float16)[int(r.integers(2))]
    slots = int(r.integers(2, 6))
    catalog = int(r.integers(slots + 1, 3 * slots + 2))
    max_rank = int(r.choice([8, 16]))
    spare = int(r.choice([0, 1 << 30]))
    steps = 6
    _announce(test="churn_sweep", seed=seed, dtype=dtype, slots=slots, catalog=catalog, max_rank=max_rank,
              spare_bytes=spare)
    base = _llama(seed, dtype, gpu, 128, 256)
    pm = PolyLoraModel(copy.deepcopy(base), PolyLoraConfig(target_modules=LLAMA_TARGETS, max_gpu_adapters=slots,
                                                           max_rank=max_rank, spare_region_bytes=spare)).eval()
    shapes = _shapes(pm)
    g = torch.Generator().manual_seed(seed)
    ads = {}
    for i in range(catalog):
        weights = {}
        for m in shapes:
            if r.random() < 0.85:
                weights.update(_peft.make_lora_weights(g, shapes, int(r.integers(1, max_rank + 1)), std=0.05,
                                                       modules=[m]))
        weights = weights or _peft.make_lora_weights(g, shapes, max_rank, std=0.05, modules=[next(iter(shapes))])
        ads[f"c{i:02d}"] = (weights, 2.0 * max_rank)
        pm.adapter_store.add_adapter_from_peft_state_dict(f"c{i:02d}", _peft.state_dict(weights),
                                                          pm.target_module_names, 2.0 * max_rank)
    names = list(ads)
    with torch.inference_mode(), _per_layer_check(pm, ads, dtype, f"churn sweep seed {seed}") as checked:
        for step in range(steps):
            B = int(r.integers(1, 9))
            S = int(r.choice([1, 1, 5, 40]))
            pick = r.choice(len(names), size=int(r.integers(1, slots + 1)), replace=False)
            adapter_ids = [names[int(pick[int(i)])] if r.random() > 0.15 else "__base__"
                           for i in r.integers(0, len(pick), B)]
            ids = torch.randint(0, 211, (B, S), generator=g).to(gpu)
            pm(input_ids=ids, adapter_ids=adapter_ids)
    assert checked.calls == steps * len(pm.target_module_names)


@pytest.mark.parametrize("seed", range(10))
def test_random_debertas_every_layer_against_the_oracle(gpu, seed):
    """Tiny fp32 DeBERTas (the reference tests' fixture shape), relative attention on or off (with it the
    shared relative-position projections reach the wrapped Linears as [1, M, K] inputs and take row 0's
    adapter, layers.py:91-97), random target subsets, adapters over random modules and ranks, right-padded
    batches; every wrapped Linear against the oracle at fp32 tolerance."""
    from tests.test_gpu_model import TARGETS

    r = np.random.default_rng(9500 + seed)
    rel = bool(r.integers(2))
    k = int(r.integers(1, len(TARGETS) + 1))
    targets = sorted(r.choice(TARGETS, size=k, replace=False).tolist(), key=TARGETS.index)
    max_rank = int(r.choice([4, 8, 16]))
    n_ad = int(r.integers(1, 5))
    B, S = int(r.integers(1, 9)), int(r.integers(2, 33))
    _announce(test="deberta_sweep", seed=seed, relative_attention=rel, targets=targets, max_rank=max_rank,
              adapters=n_ad, B=B, S=S)
    base = _peft.tiny_deberta(seed, relative_attention=rel).to(gpu)
    pm = PolyLoraModel(copy.deepcopy(base), PolyLoraConfig(target_modules=targets, max_gpu_adapters=n_ad,
                                                           max_rank=max_rank)).eval()
    shapes = _shapes(pm)
    names = list(shapes)
    g = torch.Generator().manual_seed(seed)
    ads = {}
    for i in range(n_ad):
        mods = [m for m in names if r.random() < 0.75] or [names[-1]]
        weights = {}
        for m in mods:
            weights.update(_peft.make_lora_weights(g, shapes, int(r.integers(1, max_rank + 1)), std=0.05, modules=[m]))
        ads[f"d{i}"] = (weights, 2.0 * max_rank)
        pm.adapter_store.add_adapter_from_peft_state_dict(f"d{i}", _peft.state_dict(weights), pm.target_module_names,
                                                          2.0 * max_rank)
    pool = ["__base__", *ads]
    adapter_ids = [pool[int(i)] for i in r.integers(0, len(pool), B)]
    ids = torch.randint(1, 90, (B, S), generator=g).to(gpu)
    lens = torch.randint(1, S + 1, (B,), generator=g)
    mask = (torch.arange(S)[None, :] < lens[:, None]).long().to(gpu)
    with torch.inference_mode(), _per_layer_check(pm, ads, torch.float32, f"deberta sweep seed {seed}") as checked:
        pm(input_ids=ids, attention_mask=mask, adapter_ids=adapter_ids)
    assert checked.calls >= len(pm.target_module_names), (checked.calls, len(pm.target_module_names))
