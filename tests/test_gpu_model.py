"""Model-level GPU parity: PolyLoraModel (HIP kernels) against the fallback forward.

The reference's tests (tests/test_polylora_peft.py) compare PolyLoRA with
PEFT on a tiny DeBERTa.  PEFT is not installed, so each is restated with the
oracle's fallback forward (oracle.model, the torch restatement of
layers.py:112-134 over dense reference-layout slot tensors) as the expected
output, computed on the same GPU from the same base weights; the fallback is
pinned against the textbook LoRA closed form in tests/test_oracle.py.  Their
slot, rank and scale assertions are kept as they are.
"""

from __future__ import annotations

import copy
from types import SimpleNamespace

import pytest
import torch

from oracle import model as oracle_model
from polylora_amd import sgmv
from polylora_amd import PolyLoraConfig, PolyLoraModel
from tests import _peft
from tests._util import CountedParity

pytestmark = pytest.mark.gpu

TARGETS = ["query_proj", "key_proj", "value_proj", "dense"]
FP32 = dict(rtol=1e-5, atol=1e-5)
BF16 = dict(rtol=2e-2, atol=1e-2)


def _announce(**kw):
    print("case:", ", ".join(f"{k}={v}" for k, v in kw.items()), flush=True)


class _PeftModelStandIn(torch.nn.Module):
    """What add_adapter_from_peft_model reads from a PeftModel: ``peft_config`` and ``state_dict()``."""

    def __init__(self, base: torch.nn.Module, adapters: dict) -> None:
        super().__init__()
        self.peft_config = {}
        self._sd = {}
        for name, (weights, rank, alpha) in adapters.items():
            self.peft_config[name] = SimpleNamespace(
                r=rank, lora_alpha=alpha, lora_dropout=0.0, use_dora=False, lora_bias=False, use_rslora=False
            )
            self._sd.update(_peft.state_dict(weights, name))

    def state_dict(self, *a, **kw):
        return dict(self._sd)


def _shapes(pm: PolyLoraModel) -> dict:
    return {s.name: (s.in_features, s.out_features) for s in pm.module_specs}


def _oracle(base_model, targets, adapters: dict, max_rank: int, dtype, device):
    """adapters: id -> ({module: (lora_A, lora_B)}, alpha) -> (wrapped model copy, bank)."""
    m = copy.deepcopy(base_model)
    bank_ad = {aid: {mod: (a, b, alpha) for mod, (a, b) in w.items()} for aid, (w, alpha) in adapters.items()}
    names = oracle_model.wrap_model(m, targets, None)
    shapes = {n: (m.get_submodule(n).base_layer.in_features, m.get_submodule(n).base_layer.out_features) for n in names}
    bank = oracle_model.OracleBank(bank_ad, shapes, max_rank, dtype, device)
    for n in names:
        m.get_submodule(n).bank = bank
    return m, bank


def _dev():
    return torch.device("cuda", 0)


class _per_layer_check:
    """Check every wrapped Linear's output against the oracle on the inputs that layer actually saw.

    A forward hook on each MultiLoraLinear recomputes the base output, applies
    the fallback LoRA (oracle.lora.reference_forward over dense slot tensors
    that follow the cache's slot assignment) and compares the exact layer
    output of the HIP path at the dtype's tolerance on every element
    (tests._util.CountedParity: fp32 rtol/atol 1e-5, bf16/fp16 rtol 2e-2 /
    atol 1e-2, with cancellation exemptions counted and capped).
    """

    def __init__(self, pm, adapters: dict, dtype, label: str = "per-layer") -> None:
        self.pm, self.adapters, self.dtype = pm, adapters, dtype
        self.count = 0
        self.calls = 0
        self.handles = []
        self.parity = CountedParity(dtype, label)

    def __enter__(self):
        from oracle.lora import dense_slot_tensors, prepare_batched_inputs, reference_forward
        from polylora_amd.context import get_lora_context

        cache = self.pm.adapter_cache
        seen = set()

        def hook(module, inputs, output):
            ctx = get_lora_context()
            if ctx is None:
                return
            x = inputs[0]
            spec = cache.module_specs[module.module_name]
            per_slot = [None]
            for slot in range(1, cache.num_slots):
                aid = cache.slot_to_adapter[slot]
                entry = None if aid is None else self.adapters[aid][0].get(module.module_name)
                per_slot.append(None if entry is None else (*entry, self.adapters[aid][1]))
            A, B, rk, sc = (t.to(x.device) for t in dense_slot_tensors(per_slot, spec.in_features, spec.out_features,
                                                                      cache.config.max_rank, self.dtype))
            base = module.base_layer(x)
            x3, b3, seq, widx = prepare_batched_inputs(x, base, ctx.weight_indices.long(), ctx.seq_lens)
            want = reference_forward(x3, b3, seq, widx, A, B, rk, sc).reshape(output.shape)
            self.parity.check(output, want, base, where=f" {module.module_name}")
            self.calls += 1
            if module.module_name not in seen:
                seen.add(module.module_name)
                self.count += 1

        for name in self.pm.target_module_names:
            self.handles.append(self.pm.base_model.get_submodule(name).register_forward_hook(hook))
        return self

    def __exit__(self, exc_type, *exc):
        for h in self.handles:
            h.remove()
        if exc_type is None:
            self.parity.finish()
        return False


def test_mixed_batch_matches_fallback(gpu, tmp_path):
    """tests/test_polylora_peft.py:36-122: adapters from a PEFT model and from disk, plus __base__ rows."""
    _announce(test="mixed_batch")
    base = _peft.tiny_deberta(0).to(gpu)
    pm = PolyLoraModel(copy.deepcopy(base), PolyLoraConfig(target_modules=TARGETS, max_gpu_adapters=2, max_rank=3)).eval()
    g = torch.Generator().manual_seed(0)
    wa = _peft.make_lora_weights(g, _shapes(pm), 2)
    wb = _peft.make_lora_weights(g, _shapes(pm), 3)
    peft_like = _PeftModelStandIn(base, {"a": (wa, 2, 8), "b": (wb, 3, 6)})
    pm.add_adapter_from_peft_model("a", peft_like, peft_adapter_name="a")
    path = tmp_path / "adapter_b"
    path.mkdir()
    (path / "adapter_config.json").write_text('{"peft_type": "LORA", "r": 3, "lora_alpha": 6, "lora_dropout": 0.0}')
    torch.save(peft_like.state_dict(), path / "adapter_model.bin")  # both adapters, named keys
    pm.load_adapter_from_disk("b", str(path), peft_adapter_name="b")
    ids = torch.tensor([[1, 5, 6, 7, 2], [1, 8, 9, 4, 2], [1, 3, 3, 3, 2], [1, 11, 12, 13, 2]], device=gpu)
    mask = torch.ones(4, 5, dtype=torch.long, device=gpu)
    adapter_ids = ["a", "b", "__base__", "a"]
    om, bank = _oracle(base, TARGETS, {"a": (wa, 8), "b": (wb, 6)}, 3, torch.float32, gpu)
    with torch.inference_mode():
        got = pm(input_ids=ids, attention_mask=mask, adapter_ids=adapter_ids).last_hidden_state
        want = oracle_model.run(om, bank, adapter_ids, input_ids=ids, attention_mask=mask).last_hidden_state
        plain = base(input_ids=ids, attention_mask=mask).last_hidden_state
    torch.testing.assert_close(got, want, **FP32)
    torch.testing.assert_close(got[2], plain[2], **FP32)
    assert not torch.allclose(got[0], plain[0], **FP32)


def test_three_disk_adapters_batched(gpu, tmp_path):
    """tests/test_polylora_peft.py:125-213: save_pretrained layout, ranks 2/3/4, alpha 4/9/8 (scale 3.0)."""
    _announce(test="three_disk")
    base = _peft.tiny_deberta(3, vocab=101).to(gpu)
    pm = PolyLoraModel(copy.deepcopy(base), PolyLoraConfig(target_modules=TARGETS, max_gpu_adapters=3, max_rank=4)).eval()
    specs = [("adapter_0", 2, 4), ("adapter_1", 3, 9), ("adapter_2", 4, 8)]
    ads = {}
    for seed, (aid, r, alpha) in enumerate(specs, start=10):
        w = _peft.make_lora_weights(torch.Generator().manual_seed(seed), _shapes(pm), r)
        pm.load_adapter_from_disk(aid, str(_peft.write_adapter_dir(tmp_path / aid, w, r, alpha, fmt="bin")))
        ads[aid] = (w, alpha)
    ids = torch.tensor([[1, 5, 6, 7, 2, 0], [1, 8, 9, 4, 3, 2], [1, 11, 12, 13, 14, 2]], device=gpu)
    mask = torch.ones(3, 6, dtype=torch.long, device=gpu)
    adapter_ids = [a for a, _, _ in specs]
    om, bank = _oracle(base, TARGETS, ads, 4, torch.float32, gpu)
    with torch.inference_mode():
        got = pm(input_ids=ids, attention_mask=mask, adapter_ids=adapter_ids).last_hidden_state
        want = oracle_model.run(om, bank, adapter_ids, input_ids=ids, attention_mask=mask).last_hidden_state
    torch.testing.assert_close(got, want, **FP32)
    slot = pm.adapter_cache.adapter_to_slot["adapter_1"]
    assert all(float(pm.adapter_cache.scales[m][slot]) == 3.0 for m in pm.target_module_names)


def test_gpu_slot_reload_cycle(gpu):
    """tests/test_polylora_peft.py:216-273: one GPU slot cycles a -> b -> a; outputs reproduce."""
    _announce(test="slot_reload")
    base = _peft.tiny_deberta(1).to(gpu)
    pm = PolyLoraModel(
        copy.deepcopy(base), PolyLoraConfig(target_modules=TARGETS, max_gpu_adapters=1, max_cpu_adapters=2, max_rank=2)
    ).eval()
    g = torch.Generator().manual_seed(1)
    wa, wb = _peft.make_lora_weights(g, _shapes(pm), 2), _peft.make_lora_weights(g, _shapes(pm), 2)
    peft_like = _PeftModelStandIn(base, {"a": (wa, 2, 4), "b": (wb, 2, 4)})
    pm.add_adapter_from_peft_model("a", peft_like, peft_adapter_name="a")
    pm.add_adapter_from_peft_model("b", peft_like, peft_adapter_name="b")
    ids = torch.tensor([[1, 5, 6, 2]], device=gpu)
    mask = torch.ones(1, 4, dtype=torch.long, device=gpu)
    with torch.inference_mode():
        out_a1 = pm(input_ids=ids, attention_mask=mask, adapter_ids=["a"]).last_hidden_state
        assert pm.adapter_cache.slot_to_adapter[1] == "a"
        out_b = pm(input_ids=ids, attention_mask=mask, adapter_ids=["b"]).last_hidden_state
        assert pm.adapter_cache.slot_to_adapter[1] == "b"
        out_a2 = pm(input_ids=ids, attention_mask=mask, adapter_ids=["a"]).last_hidden_state
        assert pm.adapter_cache.slot_to_adapter[1] == "a"
    assert "a" in pm.adapter_store and "b" in pm.adapter_store
    assert not torch.allclose(out_a1, out_b, **FP32)
    assert torch.equal(out_a1, out_a2)


def test_base_adapter_slot_zero_rank_zero(gpu):
    """tests/test_polylora_peft.py:276-328."""
    _announce(test="base_slot")
    base = _peft.tiny_deberta(2).to(gpu)
    pm = PolyLoraModel(copy.deepcopy(base), PolyLoraConfig(target_modules=TARGETS, max_gpu_adapters=1, max_rank=2)).eval()
    wa = _peft.make_lora_weights(torch.Generator().manual_seed(2), _shapes(pm), 2)
    pm.add_adapter_from_peft_model("a", _PeftModelStandIn(base, {"a": (wa, 2, 4)}), peft_adapter_name="a")
    ids = torch.tensor([[1, 5, 6, 2], [1, 8, 9, 2]], device=gpu)
    mask = torch.ones(2, 4, dtype=torch.long, device=gpu)
    with torch.inference_mode():
        mixed = pm(input_ids=ids, attention_mask=mask, adapter_ids=["__base__", "a"]).last_hidden_state
        plain = base(input_ids=ids, attention_mask=mask).last_hidden_state
    assert pm.adapter_cache.adapter_to_slot["__base__"] == 0
    for m in pm.target_module_names:
        assert int(pm.adapter_cache.ranks[m][0].item()) == 0
        assert float(pm.adapter_cache.scales[m][0].item()) == 0.0
    torch.testing.assert_close(mixed[0], plain[0], **FP32)
    assert not torch.allclose(mixed[1], plain[1], **FP32)


def test_sparse_adapter_rank_zero_modules(gpu):
    """tests/test_polylora_peft.py:331-383: value_proj-only adapter; no target_modules (all Linears)."""
    _announce(test="sparse")
    base = _peft.tiny_deberta(4).to(gpu)
    pm = PolyLoraModel(copy.deepcopy(base), PolyLoraConfig(max_gpu_adapters=1, max_rank=2)).eval()
    vmods = [n for n in pm.target_module_names if n.endswith("value_proj")]
    w = _peft.make_lora_weights(torch.Generator().manual_seed(4), _shapes(pm), 2, modules=vmods)
    pm.add_adapter_from_peft_model("sparse", _PeftModelStandIn(base, {"sparse": (w, 2, 4)}), peft_adapter_name="sparse")
    ids = torch.tensor([[1, 5, 6, 2], [1, 8, 9, 2]], device=gpu)
    mask = torch.ones(2, 4, dtype=torch.long, device=gpu)
    om, bank = _oracle(base, None, {"sparse": (w, 4)}, 2, torch.float32, gpu)
    with torch.inference_mode():
        got = pm(input_ids=ids, attention_mask=mask, adapter_ids=["sparse", "sparse"]).last_hidden_state
        want = oracle_model.run(om, bank, ["sparse", "sparse"], input_ids=ids, attention_mask=mask).last_hidden_state
    q = next(n for n in pm.target_module_names if n.endswith("query_proj"))
    slot = pm.adapter_cache.adapter_to_slot["sparse"]
    assert int(pm.adapter_cache.ranks[q][slot].item()) == 0
    assert float(pm.adapter_cache.scales[q][slot].item()) == 0.0
    assert int(pm.adapter_cache.ranks[vmods[0]][slot].item()) == 2
    torch.testing.assert_close(got, want, **FP32)


def test_cpu_miss_reloads_from_disk_cache(gpu, tmp_path):
    """tests/test_polylora_peft.py:484-550."""
    _announce(test="disk_reload")
    base = _peft.tiny_deberta(7).to(gpu)
    pm = PolyLoraModel(
        copy.deepcopy(base),
        PolyLoraConfig(target_modules=TARGETS, max_gpu_adapters=1, max_cpu_adapters=1, disk_cache_dir=tmp_path / "disk",
                       max_disk_adapters=2, max_rank=2),
    ).eval()
    ws = {}
    for seed, aid in enumerate(["a", "b"], start=20):
        ws[aid] = _peft.make_lora_weights(torch.Generator().manual_seed(seed), _shapes(pm), 2)
        pm.load_adapter_from_disk(aid, str(_peft.write_adapter_dir(tmp_path / f"source_{aid}", ws[aid], 2, 4, fmt="bin")))
    assert "a" not in pm.adapter_store.adapters and "a" in pm.adapter_store
    ids = torch.tensor([[1, 5, 6, 2]], device=gpu)
    mask = torch.ones(1, 4, dtype=torch.long, device=gpu)
    om, bank = _oracle(base, TARGETS, {"a": (ws["a"], 4)}, 2, torch.float32, gpu)
    with torch.inference_mode():
        got = pm(input_ids=ids, attention_mask=mask, adapter_ids=["a"]).last_hidden_state
        want = oracle_model.run(om, bank, ["a"], input_ids=ids, attention_mask=mask).last_hidden_state
    assert "a" in pm.adapter_store.adapters
    assert pm.adapter_cache.slot_to_adapter[1] == "a"
    torch.testing.assert_close(got, want, **FP32)


def test_right_padding_enforced_and_padded_rows(gpu):
    """context.py:37-45 through forward: right-padded masks work, others raise ValueError."""
    _announce(test="right_padding")
    base = _peft.tiny_deberta(5).to(gpu)
    pm = PolyLoraModel(copy.deepcopy(base), PolyLoraConfig(target_modules=TARGETS, max_gpu_adapters=2, max_rank=4)).eval()
    g = torch.Generator().manual_seed(5)
    ads = {aid: (_peft.make_lora_weights(g, _shapes(pm), r), 2.0 * r) for aid, r in (("x", 4), ("y", 3))}
    for aid, (w, alpha) in ads.items():
        pm.adapter_store.add_adapter_from_peft_state_dict(aid, _peft.state_dict(w), pm.target_module_names, alpha)
    ids = torch.randint(1, 90, (3, 7), generator=g).to(gpu)
    mask = torch.tensor([[1] * 7, [1] * 4 + [0] * 3, [1] * 2 + [0] * 5], device=gpu)
    om, bank = _oracle(base, TARGETS, ads, 4, torch.float32, gpu)
    with torch.inference_mode():
        got = pm(input_ids=ids, attention_mask=mask, adapter_ids=["x", "y", "x"]).last_hidden_state
        want = oracle_model.run(om, bank, ["x", "y", "x"], input_ids=ids, attention_mask=mask).last_hidden_state
        torch.testing.assert_close(got, want, **FP32)
        bad = mask.clone()
        bad[1] = torch.tensor([0, 1, 1, 1, 1, 0, 0])
        with pytest.raises(ValueError, match="right-padded attention_mask"):
            pm(input_ids=ids, attention_mask=bad, adapter_ids=["x", "y", "x"])
        with pytest.raises(ValueError, match="right-padded attention_mask"):
            pm.prepare_lora_context(["x", "y", "x"], bad, 3, 7, gpu)


def test_deberta_relative_attention_shared_rows(gpu):
    """Batch-1 branch of layers.py:91-97: shared relative-position projections take row 0's adapter."""
    _announce(test="deberta_rel_att")
    base = _peft.tiny_deberta(6, relative_attention=True).to(gpu)
    pm = PolyLoraModel(copy.deepcopy(base), PolyLoraConfig(target_modules=TARGETS, max_gpu_adapters=2, max_rank=4)).eval()
    g = torch.Generator().manual_seed(6)
    ads = {aid: (_peft.make_lora_weights(g, _shapes(pm), r), 2.0 * r) for aid, r in (("p", 4), ("q", 2))}
    for aid, (w, alpha) in ads.items():
        pm.adapter_store.add_adapter_from_peft_state_dict(aid, _peft.state_dict(w), pm.target_module_names, alpha)
    ids = torch.randint(1, 90, (2, 6), generator=g).to(gpu)
    mask = torch.tensor([[1] * 6, [1] * 3 + [0] * 3], device=gpu)
    om, bank = _oracle(base, TARGETS, ads, 4, torch.float32, gpu)
    for adapter_ids in (["p", "q"], ["__base__", "p"]):
        with torch.inference_mode():
            got = pm(input_ids=ids, attention_mask=mask, adapter_ids=adapter_ids).last_hidden_state
            want = oracle_model.run(om, bank, adapter_ids, input_ids=ids, attention_mask=mask).last_hidden_state
        torch.testing.assert_close(got, want, **FP32)


def test_deberta_base_shape_fp32_config(gpu):
    """DeBERTa-v3-base shape (12 layers, 768, FFN 3072), 5 adapters r {4,8,8,16,16}, alpha 2r, B=8, S=128."""
    _announce(test="deberta_base_fp32")
    from bench import deberta_workload

    wl = deberta_workload(gpu, seed=1001)
    with torch.inference_mode():
        got = wl.model(**wl.inputs, adapter_ids=wl.adapter_ids).last_hidden_state
        om, bank = _oracle(wl.base, TARGETS, wl.adapters, 16, torch.float32, gpu)
        want = oracle_model.run(om, bank, wl.adapter_ids, **wl.inputs).last_hidden_state
    torch.testing.assert_close(got, want, **FP32)
    # and every one of the 72 wrapped Linears on the inputs it saw, at the fp32 tolerance
    with torch.inference_mode(), _per_layer_check(wl.model, wl.adapters, torch.float32, "deberta") as checked:
        again = wl.model(**wl.inputs, adapter_ids=wl.adapter_ids).last_hidden_state
    assert checked.count == len(wl.model.target_module_names) == 72
    assert torch.equal(again, got)


def _tiny_llama(seed, dtype, device, attn="pl_safe_fp32"):
    """Tiny Llama; attention in fp32 on contiguous operands (no bf16 batched product) unless `attn` says otherwise."""
    from transformers import LlamaConfig, LlamaModel

    from bench import register_attention

    register_attention()
    torch.manual_seed(seed)
    cfg = LlamaConfig(hidden_size=128, num_hidden_layers=2, num_attention_heads=4, num_key_value_heads=2, head_dim=32,
                      intermediate_size=256, vocab_size=211)
    cfg._attn_implementation = attn
    return LlamaModel(cfg).to(device=device, dtype=dtype).eval(), cfg


LLAMA_TARGETS = ["q_proj", "k_proj", "v_proj", "o_proj", "gate_proj", "up_proj", "down_proj"]


@pytest.mark.parametrize("use_tiled", [True, False])
def test_llama_decode_with_kv_cache_bf16(gpu, use_tiled):
    """Decode: mask [B, past+1] gives seq_len 513 while each Linear sees one token per row."""
    _announce(test="llama_decode", tiled=use_tiled)
    from transformers import DynamicCache

    base, cfg = _tiny_llama(11, torch.bfloat16, gpu)
    pm = PolyLoraModel(copy.deepcopy(base), PolyLoraConfig(target_modules=LLAMA_TARGETS, max_gpu_adapters=6, max_rank=16,
                                                           use_triton_kernels=use_tiled)).eval()
    g = torch.Generator().manual_seed(11)
    ads = {f"ad{i}": (_peft.make_lora_weights(g, _shapes(pm), r, std=0.05), 2.0 * r) for i, r in enumerate([8, 16, 4, 16, 8, 2])}
    for aid, (w, alpha) in ads.items():
        pm.adapter_store.add_adapter_from_peft_state_dict(aid, _peft.state_dict(w), pm.target_module_names, alpha)
    B, past = 10, 512
    adapter_ids = [["__base__", *ads][int(i)] for i in torch.randint(0, 7, (B,), generator=g)]
    om, bank = _oracle(base, LLAMA_TARGETS, ads, 16, torch.bfloat16, gpu)
    kv = [(torch.randn(B, 2, past, 32, generator=g).to(gpu, torch.bfloat16), torch.randn(B, 2, past, 32, generator=g).to(gpu, torch.bfloat16))
          for _ in range(2)]

    def cache():
        c = DynamicCache(config=cfg)
        for layer, (k, v) in enumerate(kv):
            c.update(k.clone(), v.clone(), layer)
        return c

    ids = torch.randint(0, 211, (B, 1), generator=g).to(gpu)
    mask = torch.ones(B, past + 1, dtype=torch.long, device=gpu)
    with torch.inference_mode():
        got = pm(input_ids=ids, attention_mask=mask, past_key_values=cache(), use_cache=True, adapter_ids=adapter_ids).last_hidden_state
        want = oracle_model.run(om, bank, adapter_ids, input_ids=ids, attention_mask=mask, past_key_values=cache(),
                                use_cache=True).last_hidden_state
        plain = base(input_ids=ids, attention_mask=mask, past_key_values=cache(), use_cache=True).last_hidden_state
    torch.testing.assert_close(got.float(), want.float(), **BF16)
    for b, aid in enumerate(adapter_ids):
        if aid == "__base__":
            assert torch.equal(got[b], plain[b])


def test_llama_prefill_right_padded_bf16(gpu):
    """Prefill: right-padded rows of different lengths, 2 rows per adapter, MFMA tiled path."""
    _announce(test="llama_prefill")
    base, cfg = _tiny_llama(12, torch.bfloat16, gpu)
    pm = PolyLoraModel(copy.deepcopy(base), PolyLoraConfig(target_modules=LLAMA_TARGETS, max_gpu_adapters=4, max_rank=32)).eval()
    g = torch.Generator().manual_seed(12)
    ads = {f"p{i}": (_peft.make_lora_weights(g, _shapes(pm), r, std=0.05), 2.0 * r) for i, r in enumerate([16, 16, 32, 32])}
    for aid, (w, alpha) in ads.items():
        pm.adapter_store.add_adapter_from_peft_state_dict(aid, _peft.state_dict(w), pm.target_module_names, alpha)
    B, S = 8, 200
    lens = torch.randint(100, S + 1, (B,), generator=g)
    mask = (torch.arange(S)[None, :] < lens[:, None]).long().to(gpu)
    ids = torch.randint(0, 211, (B, S), generator=g).to(gpu)
    adapter_ids = [f"p{i // 2}" for i in range(B)]
    om, bank = _oracle(base, LLAMA_TARGETS, ads, 32, torch.bfloat16, gpu)
    with torch.inference_mode(), _per_layer_check(pm, ads, torch.bfloat16) as checked:
        got = pm(input_ids=ids, attention_mask=mask, adapter_ids=adapter_ids).last_hidden_state
        want = oracle_model.run(om, bank, adapter_ids, input_ids=ids, attention_mask=mask).last_hidden_state
    assert checked.count == len(pm.target_module_names)
    # end to end, bf16 rounding differences compound through two layers: bound the relative error norm
    valid = mask.bool()
    diff = (got[valid].float() - want[valid].float()).norm() / want[valid].float().norm()
    assert float(diff) < 1e-2, float(diff)
    # the first forward learned q/k/v and gate/up as siblings; the second runs each
    # run in one stacked fused launch and gives the same output bit for bit
    runs = set(pm.adapter_cache.stacked_runs.values())
    assert len(runs) == 2 * cfg.num_hidden_layers, runs
    calls = []
    stacked_fused = sgmv.lora_fused_stacked

    def counting(*a, **k):
        calls.append(tuple(a[3]))
        return stacked_fused(*a, **k)

    sgmv.lora_fused_stacked = counting
    try:
        with torch.inference_mode():
            again = pm(input_ids=ids, attention_mask=mask, adapter_ids=adapter_ids).last_hidden_state
    finally:
        sgmv.lora_fused_stacked = stacked_fused
    assert sorted(calls) == sorted(runs), (calls, runs)
    assert torch.equal(again, got)


def test_llama_fp16_prefill_then_decode(gpu):
    """An fp16 model: right-padded prefill (fused kernel, stacked siblings on the second forward), then a
    decode step on a KV cache (split kernels); every wrapped Linear against the oracle."""
    _announce(test="llama_fp16")
    from transformers import DynamicCache

    dt = torch.float16
    base, cfg = _tiny_llama(15, dt, gpu)
    pm = PolyLoraModel(copy.deepcopy(base), PolyLoraConfig(target_modules=LLAMA_TARGETS, max_gpu_adapters=4, max_rank=32)).eval()
    g = torch.Generator().manual_seed(15)
    ads = {f"h{i}": (_peft.make_lora_weights(g, _shapes(pm), r, std=0.05), 2.0 * r) for i, r in enumerate([8, 16, 32, 24])}
    for aid, (w, alpha) in ads.items():
        pm.adapter_store.add_adapter_from_peft_state_dict(aid, _peft.state_dict(w), pm.target_module_names, alpha)
    B, S = 8, 160
    lens = torch.randint(80, S + 1, (B,), generator=g)
    mask = (torch.arange(S)[None, :] < lens[:, None]).long().to(gpu)
    ids = torch.randint(0, 211, (B, S), generator=g).to(gpu)
    adapter_ids = [f"h{i // 2}" for i in range(B)]
    om, bank = _oracle(base, LLAMA_TARGETS, ads, 32, dt, gpu)
    for _ in range(2):  # the second forward takes the stacked sibling launches
        with torch.inference_mode(), _per_layer_check(pm, ads, dt) as checked:
            got = pm(input_ids=ids, attention_mask=mask, adapter_ids=adapter_ids).last_hidden_state
        assert checked.count == len(pm.target_module_names)
    with torch.inference_mode():
        want = oracle_model.run(om, bank, adapter_ids, input_ids=ids, attention_mask=mask).last_hidden_state
    valid = mask.bool()
    diff = (got[valid].float() - want[valid].float()).norm() / want[valid].float().norm()
    assert float(diff) < 5e-3, float(diff)
    # decode: one token per row on a 64-position cache, a base row among them
    past = 64
    kv = [(torch.randn(B, 2, past, 32, generator=g).to(gpu, dt), torch.randn(B, 2, past, 32, generator=g).to(gpu, dt))
          for _ in range(2)]

    def cache():
        c = DynamicCache(config=cfg)
        for layer, (k, v) in enumerate(kv):
            c.update(k.clone(), v.clone(), layer)
        return c

    step_ids = ["__base__"] + adapter_ids[1:]
    tok = torch.randint(0, 211, (B, 1), generator=g).to(gpu)
    dmask = torch.ones(B, past + 1, dtype=torch.long, device=gpu)
    with torch.inference_mode(), _per_layer_check(pm, ads, dt) as checked:
        got = pm(input_ids=tok, attention_mask=dmask, past_key_values=cache(), use_cache=True,
                 adapter_ids=step_ids).last_hidden_state
    assert checked.count == len(pm.target_module_names)
    with torch.inference_mode():
        want = oracle_model.run(om, bank, step_ids, input_ids=tok, attention_mask=dmask, past_key_values=cache(),
                                use_cache=True).last_hidden_state
        plain = base(input_ids=tok, attention_mask=dmask, past_key_values=cache(), use_cache=True).last_hidden_state
    torch.testing.assert_close(got.float(), want.float(), **BF16)
    assert torch.equal(got[0], plain[0])


def test_adapter_churn_matches_fallback(gpu):
    """Many adapters through few slots: uploads on the side stream, every step against the fallback."""
    _announce(test="churn")
    base, cfg = _tiny_llama(13, torch.bfloat16, gpu)
    pm = PolyLoraModel(copy.deepcopy(base), PolyLoraConfig(target_modules=LLAMA_TARGETS, max_gpu_adapters=4, max_rank=16)).eval()
    g = torch.Generator().manual_seed(13)
    ads = {f"c{i:02d}": (_peft.make_lora_weights(g, _shapes(pm), 16, std=0.05), 32.0) for i in range(12)}
    for aid, (w, alpha) in ads.items():
        pm.adapter_store.add_adapter_from_peft_state_dict(aid, _peft.state_dict(w), pm.target_module_names, alpha)
    om, bank = _oracle(base, LLAMA_TARGETS, ads, 16, torch.bfloat16, gpu)
    ids_all = list(ads)
    B = 6
    with torch.inference_mode():
        for step in range(12):
            pick = torch.randperm(12, generator=g)[:4].tolist()
            adapter_ids = [ids_all[pick[int(i)]] for i in torch.randint(0, 4, (B,), generator=g)]
            ids = torch.randint(0, 211, (B, 3), generator=g).to(gpu)
            got = pm(input_ids=ids, adapter_ids=adapter_ids).last_hidden_state
            want = oracle_model.run(om, bank, adapter_ids, input_ids=ids).last_hidden_state
            torch.testing.assert_close(got.float(), want.float(), **BF16)


def test_llama_decode_step_graph_replays(gpu):
    """A decode step (shrinks on the side stream, expands joined back) captured in a HIP graph:
    every replay, with eager work between replays, equals the eager step bit for bit."""
    _announce(test="decode_graph_replay")
    from transformers import StaticCache

    from polylora_amd.context import use_lora_context

    # torch's fused SDPA kernels (never the math path); a single decode query gets no mask, so
    # the step has no host-side mask work and can be captured
    base, cfg = _tiny_llama(14, torch.bfloat16, gpu, attn="pl_fused_sdpa")
    pm = PolyLoraModel(base, PolyLoraConfig(target_modules=LLAMA_TARGETS, max_gpu_adapters=6, max_rank=32)).eval()
    g = torch.Generator().manual_seed(14)
    ads = {f"d{i}": (_peft.make_lora_weights(g, _shapes(pm), r, std=0.05), 2.0 * r) for i, r in enumerate([8, 16, 32, 4])}
    for aid, (w, alpha) in ads.items():
        pm.adapter_store.add_adapter_from_peft_state_dict(aid, _peft.state_dict(w), pm.target_module_names, alpha)
    B, past = 24, 40
    adapter_ids = [["__base__", *ads][int(i)] for i in torch.randint(0, 5, (B,), generator=g)]
    kv = StaticCache(config=cfg, max_cache_len=past + 1)
    for layer in range(cfg.num_hidden_layers):
        kv.update(torch.randn(B, 2, past, 32, generator=g).to(gpu, torch.bfloat16),
                  torch.randn(B, 2, past, 32, generator=g).to(gpu, torch.bfloat16), layer)
    ids = torch.randint(0, 211, (B, 1), generator=g).to(gpu)
    pos = torch.tensor([past], device=gpu)
    with torch.inference_mode():
        ctx = pm.prepare_lora_context(adapter_ids, None, B, 1, gpu)

        def step():
            for layer in kv.layers:
                layer.cumulative_length.fill_(past)
            with use_lora_context(ctx):
                return pm.base_model(input_ids=ids, past_key_values=kv, cache_position=pos, use_cache=True).last_hidden_state

        s = torch.cuda.Stream()
        s.wait_stream(torch.cuda.current_stream())
        with torch.cuda.stream(s):
            want = step().clone()
            step()
        torch.cuda.current_stream().wait_stream(s)
        torch.cuda.synchronize()
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph):
            out = step()
        for i in range(3):
            out.fill_(float(i))  # eager work between replays
            torch.cuda.synchronize()
            graph.replay()
            torch.cuda.synchronize()
            assert torch.equal(out, want), i
        # and the step still equals the fallback forward
        om, bank = _oracle(_tiny_llama(14, torch.bfloat16, gpu, attn="pl_fused_sdpa")[0], LLAMA_TARGETS, ads, 32,
                           torch.bfloat16, gpu)
        for layer in kv.layers:
            layer.cumulative_length.fill_(past)
        ref = oracle_model.run(om, bank, adapter_ids, input_ids=ids, past_key_values=kv, cache_position=pos,
                               use_cache=True).last_hidden_state
    torch.testing.assert_close(want.float(), ref.float(), **BF16)


@pytest.mark.parametrize("handoff", [True, False])
def test_sibling_shrinks_are_stacked(gpu, handoff):
    """q/k/v and gate/up are learned as siblings in the first forward; the second forward serves each run in
    one launch (shrink and expand with the hand-off inside it), or with `decode_handoff` off one stacked shrink
    and one stacked expand, and gives the same output bit for bit; both match the fallback."""
    _announce(test="stacked_siblings", handoff=handoff)
    base, cfg = _tiny_llama(15, torch.bfloat16, gpu)
    pm = PolyLoraModel(copy.deepcopy(base), PolyLoraConfig(target_modules=LLAMA_TARGETS, max_gpu_adapters=4, max_rank=32)).eval()
    g = torch.Generator().manual_seed(15)
    ads = {f"t{i}": (_peft.make_lora_weights(g, _shapes(pm), r, std=0.05), 2.0 * r) for i, r in enumerate([8, 32, 16])}
    for aid, (w, alpha) in ads.items():
        pm.adapter_store.add_adapter_from_peft_state_dict(aid, _peft.state_dict(w), pm.target_module_names, alpha)
    ids = torch.randint(0, 211, (12, 1), generator=g).to(gpu)
    adapter_ids = [["__base__", *ads][int(i)] for i in torch.randint(0, 4, (12,), generator=g)]
    with torch.inference_mode():
        first = pm(input_ids=ids, adapter_ids=adapter_ids).last_hidden_state.clone()
        runs = set(pm.adapter_cache.stacked_runs.values())
        for layer in range(cfg.num_hidden_layers):
            p = f"layers.{layer}."
            assert (p + "self_attn.q_proj", p + "self_attn.k_proj", p + "self_attn.v_proj") in runs
            assert (p + "mlp.gate_proj", p + "mlp.up_proj") in runs
        pm.adapter_cache.decode_handoff = handoff
        calls = []
        name = "lora_decode_stacked" if handoff else "lora_expand_stacked"
        launch = getattr(sgmv, name)

        def counting(*a, **k):
            if len(a[3]) > 1:
                calls.append(tuple(a[3]))
            return launch(*a, **k)

        setattr(sgmv, name, counting)
        try:
            second = pm(input_ids=ids, adapter_ids=adapter_ids).last_hidden_state
        finally:
            setattr(sgmv, name, launch)
        # every run was computed whole by its first Linear: one stacked launch each
        assert sorted(calls) == sorted(runs), (calls, runs)
        om, bank = _oracle(base, LLAMA_TARGETS, ads, 32, torch.bfloat16, gpu)
        want = oracle_model.run(om, bank, adapter_ids, input_ids=ids).last_hidden_state
    assert torch.equal(first, second)
    torch.testing.assert_close(second.float(), want.float(), **BF16)


@pytest.mark.parametrize("rows,seq", [(64, 1), (16, 64), (4, 600)])
def test_batches_without_lora_work_equal_the_base_model(gpu, rows, seq):
    """Every row on the base adapter: the wrapped Linears still run their LoRA launches, on a plan with no
    groups (64 x 1: the one-launch decode kernel; 16 x 64: the fused kernel; 4 x 600: the fused kernel past
    the side-stream overlap threshold), and the output equals the base model's bit for bit."""
    _announce(test="no_lora_work", rows=rows, seq=seq)
    base, cfg = _tiny_llama(21, torch.bfloat16, gpu)
    pm = PolyLoraModel(copy.deepcopy(base), PolyLoraConfig(target_modules=LLAMA_TARGETS, max_gpu_adapters=2,
                                                           max_rank=16)).eval()
    g = torch.Generator().manual_seed(21)
    w = _peft.make_lora_weights(g, _shapes(pm), 8, std=0.05)
    pm.adapter_store.add_adapter_from_peft_state_dict("a", _peft.state_dict(w), pm.target_module_names, 16.0)
    ids = torch.randint(0, 211, (rows, seq), generator=g).to(gpu)
    mask = torch.ones(rows, seq, dtype=torch.long, device=gpu)
    with torch.inference_mode():
        pm(input_ids=ids, attention_mask=mask, adapter_ids=["a"] * rows)  # the adapter resident, siblings learned
        for _ in range(2):
            got = pm(input_ids=ids, attention_mask=mask, adapter_ids=["__base__"] * rows).last_hidden_state
            plain = base(input_ids=ids, attention_mask=mask).last_hidden_state
            assert torch.equal(got, plain)
    assert not sgmv.decode_waits_timed_out(gpu)
