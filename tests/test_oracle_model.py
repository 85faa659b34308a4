"""Pins the model-level oracle (oracle.model: wrap_model, OracleBank, run).

oracle.model restates PolyLoraModel.forward with the torch fallback
(model.py:75-131, layers.py:33-62, :112-134) and is the expected output of
every model-level GPU test.  Here it is checked, on the CPU in fp32, against a
forward that shares none of its code: every target nn.Linear is replaced by a
closed-form module built straight from the PEFT tensors,

    y = F.linear(x, W, b) + (alpha / r) * F.linear(F.linear(x, lora_A), lora_B)

on each row's first min(seq_len, M) tokens only, with the row's own adapter
(no dense slot tensors, no slot numbers, no reference_forward).  Cases: a
tiny DeBERTa with and without relative attention (its shared batch-1 position
projections take row 0's adapter), a tiny Llama in prefill and in decode over
a KV cache (mask [B, past + 1], one token per row), right-padded masks, a
``__base__`` row and a sparse adapter.  Planted mistakes in the oracle (a
wrong target set, the mask ignored, the row -> adapter map shifted) must each
be caught by the same comparison.
"""

from __future__ import annotations

import copy

import pytest
import torch
import torch.nn.functional as F
from torch import nn

from oracle import model as oracle_model
from tests import _peft

FP32 = dict(rtol=1e-5, atol=1e-5)
DEBERTA_TARGETS = ["query_proj", "key_proj", "value_proj", "dense"]
LLAMA_TARGETS = ["q_proj", "k_proj", "v_proj", "o_proj", "gate_proj", "up_proj", "down_proj"]


class _Batch:
    """Per-forward row -> adapter ids and row lengths that the closed-form Linears read."""

    def __init__(self) -> None:
        self.ids: list[str] | None = None
        self.lens: list[int] | None = None


class _ClosedFormLinear(nn.Module):
    """x W^T + b, plus (alpha / r) (x lora_A^T) lora_B^T on each row's valid tokens."""

    def __init__(self, base: nn.Linear, name: str, adapters: dict, batch: _Batch) -> None:
        super().__init__()
        self.weight, self.bias = base.weight, base.bias
        self.name, self.adapters, self.batch = name, adapters, batch

    def _delta(self, x_row: torch.Tensor, adapter_id: str) -> torch.Tensor | None:
        entry = self.adapters.get(adapter_id, {}).get(self.name)
        if entry is None:
            return None
        lora_a, lora_b, alpha = entry
        r = lora_a.shape[0]
        return (float(alpha) / r) * F.linear(F.linear(x_row, lora_a), lora_b)

    def forward(self, x: torch.Tensor) -> torch.Tensor:
        y = F.linear(x, self.weight, self.bias)
        if self.batch.ids is None:
            return y
        ids, lens = self.batch.ids, self.batch.lens
        rows = len(ids)
        out = y.clone()
        if x.shape[0] == rows:
            xv, ov = x.reshape(rows, -1, x.shape[-1]), out.view(rows, -1, out.shape[-1])
            todo = [(b, ids[b], lens[b]) for b in range(rows)]
        elif x.dim() == 3 and x.shape[0] == 1:
            # one tensor shared by the whole batch: row 0's adapter and length
            xv, ov = x, out
            todo = [(0, ids[0], lens[0])]
        else:
            xv = x.reshape(rows, -1, x.shape[-1])
            ov = out.view(rows, -1, out.shape[-1])
            todo = [(b, ids[b], lens[b]) for b in range(rows)]
        for b, aid, length in todo:
            n = max(0, min(length, xv.shape[1]))
            if n == 0:
                continue
            d = self._delta(xv[b, :n], aid)
            if d is not None:
                ov[b, :n] = ov[b, :n] + d
        return out


def _closed_form_model(base: nn.Module, targets: list[str], adapters: dict, batch: _Batch) -> nn.Module:
    m = copy.deepcopy(base)
    names = [n for n, mod in m.named_modules()
             if isinstance(mod, nn.Linear) and any(n == t or n.endswith("." + t) for t in targets)]
    for name in names:
        parent_name, _, child = name.rpartition(".")
        parent = m.get_submodule(parent_name) if parent_name else m
        setattr(parent, child, _ClosedFormLinear(getattr(parent, child), name, adapters, batch))
    return m


def _oracle_model(base: nn.Module, targets: list[str], adapters: dict, max_rank: int):
    m = copy.deepcopy(base)
    names = oracle_model.wrap_model(m, targets, None)
    shapes = {n: (m.get_submodule(n).base_layer.in_features, m.get_submodule(n).base_layer.out_features)
              for n in names}
    bank = oracle_model.OracleBank(adapters, shapes, max_rank, torch.float32, torch.device("cpu"))
    for n in names:
        m.get_submodule(n).bank = bank
    return m, bank


def _adapters(gen, shapes: dict, spec: dict) -> dict:
    """spec: id -> (rank, alpha, modules or None) -> id -> {module: (lora_A, lora_B, alpha)}."""
    out = {}
    for aid, (rank, alpha, mods) in spec.items():
        w = _peft.make_lora_weights(gen, shapes, rank, std=0.05, modules=mods)
        out[aid] = {m: (a, b, float(alpha)) for m, (a, b) in w.items()}
    return out


def _deberta_case(relative_attention: bool):
    base = _peft.tiny_deberta(21, relative_attention=relative_attention)
    shapes = _peft.linear_shapes(base, DEBERTA_TARGETS)
    g = torch.Generator().manual_seed(21)
    qv = [n for n in shapes if n.endswith(("query_proj", "value_proj"))]
    adapters = _adapters(g, shapes, {"a": (4, 8.0, None), "b": (2, 6.0, None), "sparse": (3, 6.0, qv)})
    ids = torch.randint(1, 90, (4, 7), generator=g)
    mask = torch.tensor([[1] * 7, [1] * 5 + [0] * 2, [1] * 3 + [0] * 4, [1] * 6 + [0]])
    adapter_ids = ["b", "a", "__base__", "sparse"]
    return base, DEBERTA_TARGETS, adapters, 4, adapter_ids, dict(input_ids=ids, attention_mask=mask)


def _tiny_llama(seed: int):
    from transformers import LlamaConfig, LlamaModel

    torch.manual_seed(seed)
    cfg = LlamaConfig(hidden_size=64, num_hidden_layers=2, num_attention_heads=4, num_key_value_heads=2, head_dim=16,
                      intermediate_size=96, vocab_size=101)
    cfg._attn_implementation = "eager"
    return LlamaModel(cfg).eval(), cfg


def _llama_adapters(base, seed):
    shapes = _peft.linear_shapes(base, LLAMA_TARGETS)
    g = torch.Generator().manual_seed(seed)
    qv = [n for n in shapes if n.endswith(("q_proj", "v_proj"))]
    return g, _adapters(g, shapes, {"p": (8, 16.0, None), "q": (4, 4.0, None), "s": (2, 4.0, qv)})


def _llama_prefill_case():
    base, _ = _tiny_llama(22)
    g, adapters = _llama_adapters(base, 22)
    S = 9
    lens = [9, 4, 6, 1, 7]
    mask = (torch.arange(S)[None, :] < torch.tensor(lens)[:, None]).long()
    ids = torch.randint(0, 101, (5, S), generator=g)
    adapter_ids = ["p", "q", "__base__", "s", "p"]
    return base, LLAMA_TARGETS, adapters, 8, adapter_ids, dict(input_ids=ids, attention_mask=mask)


def _llama_decode_case():
    """One new token per row over a 6-token KV cache: seq_len = 7 while each Linear sees M = 1."""
    from transformers import DynamicCache

    base, cfg = _tiny_llama(23)
    g, adapters = _llama_adapters(base, 23)
    B, past = 4, 6
    kv = [(torch.randn(B, 2, past, 16, generator=g), torch.randn(B, 2, past, 16, generator=g)) for _ in range(2)]

    def cache():
        c = DynamicCache(config=cfg)
        for layer, (k, v) in enumerate(kv):
            c.update(k.clone(), v.clone(), layer)
        return c

    ids = torch.randint(0, 101, (B, 1), generator=g)
    mask = torch.ones(B, past + 1, dtype=torch.long)
    adapter_ids = ["q", "__base__", "s", "p"]
    return base, LLAMA_TARGETS, adapters, 8, adapter_ids, dict(input_ids=ids, attention_mask=mask, use_cache=True,
                                                                 past_key_values=cache)


CASES = {
    "deberta": lambda: _deberta_case(False),
    "deberta_relative_attention": lambda: _deberta_case(True),
    "llama_prefill": _llama_prefill_case,
    "llama_decode": _llama_decode_case,
}


def _inputs(kwargs: dict) -> dict:
    """Fresh inputs per forward (a KV cache is consumed by the forward that extends it)."""
    return {k: (v() if callable(v) else v) for k, v in kwargs.items()}


def _outputs(case):
    base, targets, adapters, max_rank, adapter_ids, kwargs = case
    batch = _Batch()
    closed = _closed_form_model(base, targets, adapters, batch)
    oracle_m, bank = _oracle_model(base, targets, adapters, max_rank)
    inputs = _inputs(kwargs)
    mask = inputs.get("attention_mask")
    rows, seq = inputs["input_ids"].shape
    batch.ids = list(adapter_ids)
    batch.lens = [int(v) for v in mask.sum(-1)] if mask is not None else [seq] * rows
    with torch.no_grad():
        want = closed(**inputs).last_hidden_state
        got = oracle_model.run(oracle_m, bank, adapter_ids, **_inputs(kwargs)).last_hidden_state
        plain = base(**_inputs(kwargs)).last_hidden_state
    return got, want, plain, adapter_ids


@pytest.mark.parametrize("name", list(CASES))
def test_oracle_model_matches_closed_form(name):
    got, want, plain, adapter_ids = _outputs(CASES[name]())
    torch.testing.assert_close(got, want, **FP32)
    # the adapters change every non-base row, and the __base__ row is the base model's
    for b, aid in enumerate(adapter_ids):
        if aid == "__base__":
            torch.testing.assert_close(got[b], plain[b], **FP32)
        else:
            assert not torch.allclose(got[b], plain[b], **FP32), (name, b)


def _mutant_wrong_targets(monkeypatch):
    """The oracle wraps all targets but the last one."""
    orig = oracle_model.matches_target
    monkeypatch.setattr(oracle_model, "matches_target", lambda n, t: orig(n, None if t is None else t[:-1]))


def _mutant_mask_ignored(monkeypatch):
    """Every row's length is its full width (LoRA also on padding tokens)."""
    orig = oracle_model.prepare_batched_inputs

    def full(x, base, widx, seq):
        x3, b3, s, w = orig(x, base, widx, seq)
        return x3, b3, torch.full_like(s, x3.shape[1]), w

    monkeypatch.setattr(oracle_model, "prepare_batched_inputs", full)


def _mutant_shifted_rows(monkeypatch):
    """Row b takes row b+1's adapter."""
    orig = oracle_model.prepare_batched_inputs

    def shifted(x, base, widx, seq):
        x3, b3, s, w = orig(x, base, widx, seq)
        return x3, b3, s, torch.roll(w, 1)

    monkeypatch.setattr(oracle_model, "prepare_batched_inputs", shifted)


MUTANTS = [_mutant_wrong_targets, _mutant_mask_ignored, _mutant_shifted_rows]


@pytest.mark.parametrize("mutant", MUTANTS, ids=lambda f: f.__name__)
@pytest.mark.parametrize("name", ["deberta", "llama_prefill"])
def test_closed_form_catches_planted_oracle_mistakes(monkeypatch, mutant, name):
    case = CASES[name]()
    mutant(monkeypatch)
    got, want, _, _ = _outputs(case)
    assert not torch.allclose(got, want, **FP32), (mutant.__name__, name)


def test_counted_parity_exempts_one_operand_ulp_at_a_cancellation_and_nothing_else():
    """The per-layer GPU check: plain rtol/atol everywhere; a cancellation one ulp of the operands off is exempt
    but counted and capped; wrong deltas, two-ulp misses and too many exemptions fail."""
    from tests._util import CountedParity, ulp_of

    assert float(ulp_of(torch.tensor(2.5), torch.bfloat16)) == 2.0 ** -6
    assert float(ulp_of(torch.tensor(1.0), torch.bfloat16)) == 2.0 ** -7
    assert float(ulp_of(torch.tensor(3.0), torch.float32)) == 2.0 ** -22
    assert float(ulp_of(torch.tensor(0.0), torch.bfloat16)) == 0.0
    g = torch.Generator().manual_seed(7)
    base = (torch.randn(512, 256, generator=g) * 2).bfloat16()
    delta = (torch.randn(512, 256, generator=g) * 2).bfloat16()
    want = (base.float() + delta.float()).bfloat16()
    base[0, 0], delta[0, 0] = 2.25, -2.125  # want 0.125, one ulp of the operands is 2**-6
    want[0, 0] = 0.125
    got = want.clone()
    got[0, 0] = 0.125 + 2.0 ** -6  # beyond atol + rtol * |want| = 0.0125
    p = CountedParity(torch.bfloat16, "t")
    p.check(got, want, base)
    assert p.exempt == 1 and p.checked == got.numel()
    p.finish()  # 1 <= 1e-5 * 131072
    two = got.clone()
    two[0, 0] = 0.125 + 2.0 ** -5  # two ulps: not exempt
    with pytest.raises(AssertionError):
        CountedParity(torch.bfloat16).check(two, want, base)
    p = CountedParity(torch.bfloat16)
    p.check(got[:64], want[:64], base[:64])  # one exemption in 16384 elements: over the cap
    with pytest.raises(AssertionError):
        p.finish()
    for wrong in (base.float() + 2 * delta.float(), base.float(), base.float() - delta.float()):
        with pytest.raises(AssertionError):
            CountedParity(torch.bfloat16).check(wrong.bfloat16(), want, base)
