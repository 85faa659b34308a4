"""GPU regression tests of fixed host-path bugs (each runs the fixed code and must pass).

* Launch arguments cached per adapter cache (arena and table pointers) are
  dropped when ``GpuAdapterCache.to`` reallocates them: fused-path forward in
  fp32, ``.to(bfloat16)``, fused-path forward again, against the oracle.
* A slot handed out by ``prepare_lora_context`` and read by a forward run
  under ``use_lora_context`` (no ``mark_used``) is rewritten by a later
  eviction only after that forward's queued kernels: the forward's output
  equals the oracle for the evicted adapter.
* A sibling Linear's output kept by the first Linear of a run is returned only
  to the very next wrapped call: an interrupting call plus an in-place edit
  of x under inference mode make the sibling compute its own.
"""

from __future__ import annotations

import copy

import pytest
import torch

from oracle import model as oracle_model
from oracle.lora import dense_slot_tensors, reference_forward
from polylora_amd import PolyLoraConfig, PolyLoraModel, sgmv
from polylora_amd.context import use_lora_context
from tests import _peft
from tests.test_gpu_model import BF16, LLAMA_TARGETS, _announce, _oracle, _per_layer_check, _shapes, _tiny_llama

pytestmark = pytest.mark.gpu


def _add_adapters(pm, g, ranks, prefix, std=0.05):
    ads = {f"{prefix}{i}": (_peft.make_lora_weights(g, _shapes(pm), r, std=std), 2.0 * r) for i, r in enumerate(ranks)}
    for aid, (w, alpha) in ads.items():
        pm.adapter_store.add_adapter_from_peft_state_dict(aid, _peft.state_dict(w), pm.target_module_names, alpha)
    return ads


def _oracle_linear(pm, ads, module_name: str, x: torch.Tensor, ctx, dtype) -> torch.Tensor:
    """One wrapped Linear's expected output on x under ctx (fallback over dense slot tensors)."""
    from oracle.lora import prepare_batched_inputs

    cache = pm.adapter_cache
    spec = cache.module_specs[module_name]
    per_slot = [None]
    for slot in range(1, cache.num_slots):
        aid = cache.slot_to_adapter[slot]
        entry = None if aid is None else ads[aid][0].get(module_name)
        per_slot.append(None if entry is None else (*entry, ads[aid][1]))
    A, B, rk, sc = (t.to(x.device) for t in dense_slot_tensors(per_slot, spec.in_features, spec.out_features,
                                                              cache.config.max_rank, dtype))
    base = pm.base_model.get_submodule(module_name).base_layer(x)
    x3, b3, seq, widx = prepare_batched_inputs(x, base, ctx.weight_indices.long(), ctx.seq_lens)
    return reference_forward(x3, b3, seq, widx, A, B, rk, sc).reshape(base.shape)


def test_dtype_change_after_fused_forward(gpu):
    """fp32 forward on the fused path, .to(bfloat16), bf16 forward on the fused path: both match the oracle."""
    _announce(test="dtype_change_fused")
    base, cfg = _tiny_llama(41, torch.float32, gpu)
    pm = PolyLoraModel(copy.deepcopy(base), PolyLoraConfig(target_modules=LLAMA_TARGETS, max_gpu_adapters=4,
                                                           max_rank=16)).eval()
    g = torch.Generator().manual_seed(41)
    ads = _add_adapters(pm, g, [8, 16, 4, 16], "f")
    B, S = 8, 160  # 1280 tokens, 4 adapters: long segments take the fused kernel
    ids = torch.randint(0, 211, (B, S), generator=g).to(gpu)
    adapter_ids = [f"f{i // 2}" for i in range(B)]
    calls = []
    fused, stacked = sgmv._fused_launch, sgmv.lora_fused_stacked

    def count_fused(*a, **k):
        calls.append("fused")
        return fused(*a, **k)

    def count_stacked(*a, **k):
        calls.append("stacked")
        return stacked(*a, **k)

    sgmv._fused_launch, sgmv.lora_fused_stacked = count_fused, count_stacked
    try:
        with torch.inference_mode(), _per_layer_check(pm, ads, torch.float32) as checked:
            pm(input_ids=ids, adapter_ids=adapter_ids)
            pm(input_ids=ids, adapter_ids=adapter_ids)  # the second forward takes the stacked launches
        assert checked.count == len(pm.target_module_names)
        assert "fused" in calls and "stacked" in calls, calls
        old_arena = pm.adapter_cache.arena.data_ptr()
        pm.to(torch.bfloat16)
        calls.clear()
        with torch.inference_mode(), _per_layer_check(pm, ads, torch.bfloat16) as checked:
            got = pm(input_ids=ids, adapter_ids=adapter_ids).last_hidden_state
        assert pm.adapter_cache.dtype == torch.bfloat16 and pm.adapter_cache.arena.data_ptr() != old_arena
        assert checked.count == len(pm.target_module_names)
        assert calls, "the bf16 forward did not take the fused kernel"
    finally:
        sgmv._fused_launch, sgmv.lora_fused_stacked = fused, stacked
    om, bank = _oracle(base.to(torch.bfloat16), LLAMA_TARGETS, ads, 16, torch.bfloat16, gpu)
    with torch.inference_mode():
        want = oracle_model.run(om, bank, adapter_ids, input_ids=ids).last_hidden_state
    diff = (got.float() - want.float()).norm() / want.float().norm()
    assert float(diff) < 1e-2, float(diff)


def test_dtype_widening_repacks_from_source_weights(gpu):
    """fp32 PEFT adapters added to a bf16 model, a bf16 forward, then .to(float32): the fp32 forward (a resident
    adapter rewritten into the new arena, and one loaded for the first time) matches the fp32 oracle at rtol
    1e-5, which the bf16-rounded weights would miss (store.py:240-241, cache.py:139 convert at every load)."""
    _announce(test="dtype_widening")
    base, cfg = _tiny_llama(43, torch.bfloat16, gpu)
    pm = PolyLoraModel(copy.deepcopy(base), PolyLoraConfig(target_modules=LLAMA_TARGETS, max_gpu_adapters=2,
                                                           max_rank=16)).eval()
    g = torch.Generator().manual_seed(43)
    ads = _add_adapters(pm, g, [8, 16, 4], "w")
    ids = torch.randint(0, 211, (4, 5), generator=g).to(gpu)
    with torch.inference_mode(), _per_layer_check(pm, ads, torch.bfloat16, label="bf16") as checked:
        pm(input_ids=ids, adapter_ids=["w0", "w1", "__base__", "w0"])
    assert checked.count == len(pm.target_module_names)
    pm.to(torch.float32)  # the adapter cache follows at the next forward (model.py:75-85 infers the dtype)
    with torch.inference_mode(), _per_layer_check(pm, ads, torch.float32, label="fp32") as checked:
        pm(input_ids=ids, adapter_ids=["w0", "w2", "w2", "__base__"])  # w0 resident since bf16, w2 loaded now
    assert pm.adapter_cache.dtype == torch.float32
    assert checked.count == len(pm.target_module_names)


def test_prepare_context_eviction_waits_for_queued_readers(gpu):
    """max_gpu_adapters=1: a forward for "a" under prepare_lora_context/use_lora_context sits behind a long
    queue of GPU work when prepare_lora_context(["b"]) evicts "a"; its output is still "a"'s."""
    _announce(test="eviction_ordering")
    base, cfg = _tiny_llama(42, torch.bfloat16, gpu)
    pm = PolyLoraModel(copy.deepcopy(base), PolyLoraConfig(target_modules=LLAMA_TARGETS, max_gpu_adapters=1,
                                                           max_rank=16)).eval()
    g = torch.Generator().manual_seed(42)
    ads = _add_adapters(pm, g, [16, 8], "e", std=0.1)
    B, S = 6, 4
    ids = torch.randint(0, 211, (B, S), generator=g).to(gpu)
    m1 = torch.randn(4096, 4096, device=gpu, dtype=torch.bfloat16) * 0.01
    m2 = torch.empty_like(m1)

    def hold_the_queue(module, args):
        # ~hundreds of ms of GPU work queued inside the forward, ahead of every LoRA kernel of the layers
        for _ in range(400):
            torch.mm(m1, m1, out=m2)

    cache = pm.adapter_cache
    cache._packed(pm.adapter_store.get("e1"))  # packed (and pinned) ahead: the eviction below only copies
    with torch.inference_mode():
        ctx_a = pm.prepare_lora_context(["e0"] * B, None, B, S, gpu)
        assert pm.adapter_cache.slot_to_adapter[1] == "e0"
        handle = pm.base_model.layers[0].register_forward_pre_hook(hold_the_queue)
        try:
            with use_lora_context(ctx_a):
                out_a = pm.base_model(input_ids=ids).last_hidden_state
        finally:
            handle.remove()
        pm.prepare_lora_context(["e1"] * B, None, B, S, gpu)  # evicts e0 from slot 1
        assert pm.adapter_cache.slot_to_adapter[1] == "e1"
        torch.cuda.synchronize()
        om, bank = _oracle(base, LLAMA_TARGETS, ads, 16, torch.bfloat16, gpu)
        want = oracle_model.run(om, bank, ["e0"] * B, input_ids=ids).last_hidden_state
        other = oracle_model.run(om, bank, ["e1"] * B, input_ids=ids).last_hidden_state
    assert not torch.allclose(want.float(), other.float(), **BF16)
    diff = (out_a.float() - want.float()).norm() / want.float().norm()
    assert float(diff) < 1e-2, float(diff)


@pytest.mark.parametrize("B,S", [(12, 1), (8, 160)], ids=["decode_split", "prefill_fused"])
def test_sibling_output_not_reused_after_interrupting_call(gpu, B, S):
    """Under inference mode: q(x) keeps k's and v's outputs; an o_proj call and an in-place edit of x come
    before k(x), which must then compute its own output on the edited x."""
    _announce(test="sibling_interrupt", B=B, S=S)
    base, cfg = _tiny_llama(43, torch.bfloat16, gpu)
    pm = PolyLoraModel(copy.deepcopy(base), PolyLoraConfig(target_modules=LLAMA_TARGETS, max_gpu_adapters=4,
                                                           max_rank=16)).eval()
    g = torch.Generator().manual_seed(43)
    ads = _add_adapters(pm, g, [8, 16, 4], "s")
    ids = torch.randint(0, 211, (B, S), generator=g).to(gpu)
    adapter_ids = [["__base__", *ads][i % 4] if S == 1 else f"s{i % 3}" for i in range(B)]
    attn = pm.base_model.layers[0].self_attn
    hidden = cfg.hidden_size
    with torch.inference_mode():
        pm(input_ids=ids, adapter_ids=adapter_ids)  # learns the sibling runs
        assert any(r[0].endswith("layers.0.self_attn.q_proj") for r in pm.adapter_cache.stacked_runs.values())
        ctx = pm.prepare_lora_context(adapter_ids, None, B, S, gpu)
        x = torch.randn(B, S, hidden, generator=g).to(gpu, torch.bfloat16)
        other = torch.randn(B, S, hidden, generator=g).to(gpu, torch.bfloat16)
        with use_lora_context(ctx):
            attn.q_proj(x)
            attn.o_proj(other)  # interrupts the q/k/v run
            x.add_(1.0)  # no version counter under inference mode
            k_out = attn.k_proj(x)
            # a fresh, uninterrupted run still serves its siblings
            x2 = torch.randn(B, S, hidden, generator=g).to(gpu, torch.bfloat16)
            attn.q_proj(x2)
            k2, v2 = attn.k_proj(x2), attn.v_proj(x2)
        for name, xin, got in (("k_proj", x, k_out), ("k_proj", x2, k2), ("v_proj", x2, v2)):
            want = _oracle_linear(pm, ads, f"layers.0.self_attn.{name}", xin, ctx, torch.bfloat16)
            torch.testing.assert_close(got.float(), want.float(), **BF16)
