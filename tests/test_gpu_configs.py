"""Parity at the benchmark configurations' own shapes, against the oracle (oracle.lora.reference_forward).

* Prefill size (32 rows x 1024, U[512,1024] lengths, 8 adapters of ranks 16
  and 32): the o launch, the stacked gate/up launch (N = 14336) and the down
  launch (K = 14336) of the fused kernel, every token.
* Adapter churn (the Llama-3-8B layer shapes, all 7 targets, 32 GPU slots,
  rank-16 adapters): a catalog of 96 distinct PEFT adapters added through the
  store's PEFT path, some held in pageable memory (their loads go through the
  staging ring), batches of 128 rows drawn Zipf(0.9) and split into
  sub-batches of at most 24 distinct adapters, every wrapped layer of every
  sub-batch against the oracle on the inputs it saw; and at the catalog's own
  size, 1024 adapters (images built as the churn bench builds them, half of
  them pageable), steps of 128 rows, sub-batches of up to 32 distinct: 8 steps
  on 2 layers, and 3 steps on the configuration's 32 layers.
* Decode (32 Llama-3-8B layers, 64 slots, ranks {8,16,32,64}, 256 rows over
  a 512-token KV cache, Zipf(1.1) with 10% base rows): one decode step with
  all 224 wrapped layers checked; and the same rows and adapters on two
  layers in fp16 and in fp32 (the one-launch decode path in those dtypes).
* Prefill through the model (2 Llama-3-8B layers, 32 rows x 1024, U[512,1024]
  right-padded lengths, 8 adapters of ranks 16 and 32, 4 rows each): two
  forwards of PolyLoraModel, one fused launch per Linear and then the stacked
  fused launches, all 14 wrapped layers checked each time.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

from oracle.lora import reference_forward
from polylora_amd import PolyLoraConfig, PolyLoraModel, sgmv
from tests import _peft
from tests._util import make_cache, oracle_slot_tensors, peft_layer
from tests.test_gpu_model import BF16, LLAMA_TARGETS, _announce, _per_layer_check

pytestmark = pytest.mark.gpu


def test_prefill_config_o_gateup_down_fused_bf16(gpu):
    """o (4096 -> 4096), gate/up stacked (4096 -> 14336 each) and down (14336 -> 4096) at prefill size."""
    _announce(test="prefill_config_o_gateup_down")
    g = torch.Generator().manual_seed(1014)
    B, S = 32, 1024
    shapes = {"o": (4096, 4096), "gate": (4096, 14336), "up": (4096, 14336), "down": (14336, 4096)}
    adapters = {f"p{i}": {m: peft_layer(g, fi, fo, 16 if i < 4 else 32, 2.0 * (16 if i < 4 else 32))
                          for m, (fi, fo) in shapes.items()} for i in range(8)}
    cache = make_cache(adapters, shapes, 8, 32, gpu, torch.bfloat16)
    row_slot = cache.ensure_resident([f"p{i // 4}" for i in range(B)])
    seq_lens = torch.randint(512, S + 1, (B,), generator=g, dtype=torch.int32)
    plan = sgmv.SgmvPlan(row_slot, seq_lens.to(gpu), S, cache.num_slots, distinct_slots=8)
    assert plan.group_tokens == 64 and sgmv.fused_ok(plan, cache, 14336)
    gg = torch.Generator(device=gpu).manual_seed(1014)
    xs = {k: torch.randn(B * S, k, generator=gg, device=gpu).to(torch.bfloat16) for k in (4096, 14336)}
    base = {m: torch.randn(B * S, fo, generator=gg, device=gpu).to(torch.bfloat16) for m, (fi, fo) in shapes.items()}
    ys = {m: base[m].clone() for m in shapes}
    sgmv.lora_fused(xs[4096], ys["o"], cache, "o", plan)
    sgmv.lora_fused_stacked(xs[4096], [ys["gate"], ys["up"]], cache, ["gate", "up"], plan)
    sgmv.lora_fused(xs[14336], ys["down"], cache, "down", plan)
    torch.cuda.synchronize()
    pad = (torch.arange(S)[None, :] >= seq_lens[:, None]).to(gpu)
    for m, (fi, fo) in shapes.items():
        A, Bm, rk, sc = (t.to(gpu) for t in oracle_slot_tensors(cache, adapters, m, torch.bfloat16))
        expect = reference_forward(xs[fi].view(B, S, fi), base[m].view(B, S, fo), seq_lens.to(gpu), row_slot, A, Bm,
                                   rk, sc)
        torch.testing.assert_close(ys[m].view(B, S, fo), expect, **BF16)
        assert torch.equal(ys[m].view(B, S, fo)[pad], base[m].view(B, S, fo)[pad])  # padding keeps the base output


def _sub_batches(ids, limit):
    """Rows in order, cut whenever a new adapter would make `limit + 1` distinct ones (as the churn bench)."""
    out, cur, seen = [], [], set()
    for a in ids:
        if a not in seen and len(seen) == limit:
            out.append(cur)
            cur, seen = [], set()
        cur.append(a)
        seen.add(a)
    out.append(cur)
    return out


@pytest.mark.parametrize("limit,spare", [(24, True), (32, True), (32, False)])
def test_churn_config_every_layer_against_the_oracle(gpu, limit, spare, monkeypatch):
    """Config 5 shapes on 2 layers: 96 distinct rank-16 adapters (40 pinned, 56 pageable) through 32 slots,
    in sub-batches of at most `limit` distinct adapters (at 32 every slot is in use, and each load copies
    into a spare arena region while the previous sub-batch's forward reads the slot's old one; without
    spare regions each load rewrites its slot in place after that forward)."""
    _announce(test="churn_config", limit=limit, spare=spare)
    from transformers import DynamicCache

    from bench import build_llama
    from polylora_amd.cache import GpuAdapterCache

    if not spare:
        monkeypatch.setattr(GpuAdapterCache, "SPARE_REGION_BYTES", 0)
    model = build_llama(gpu, layers=2, seed=1005)
    pm = PolyLoraModel(model, PolyLoraConfig(target_modules=LLAMA_TARGETS, max_gpu_adapters=32, max_rank=16)).eval()
    assert pm.adapter_cache.spare_regions == (32 if spare else 0)
    shapes = {s.name: (s.in_features, s.out_features) for s in pm.module_specs}
    image_bytes = sum(16 * (fi + fo) * 2 for fi, fo in shapes.values())
    pm.adapter_store.pinned_bytes_limit = 40 * image_bytes  # the rest stay pageable: loads go through staging
    g = torch.Generator().manual_seed(1005)
    ads = {}
    for i in range(96):
        w = _peft.make_lora_weights(g, shapes, 16, std=0.02)  # N(0, 0.02), as the configurations specify
        ads[f"c{i:03d}"] = (w, 32.0)
        pm.adapter_store.add_adapter_from_peft_state_dict(f"c{i:03d}", _peft.state_dict(w), pm.target_module_names, 32.0)
    store = pm.adapter_store
    pinned = sum(1 for a in store.adapters.values() if a.image.pinned)
    assert pinned == 40, pinned
    rng = np.random.default_rng(1005)
    w = 1.0 / np.arange(1, 97) ** 0.9
    w /= w.sum()
    names = list(ads)
    vocab = model.config.vocab_size
    gen = torch.Generator(device=gpu).manual_seed(1005)
    loads0, forwards = pm.adapter_cache.loads, 0
    with torch.inference_mode(), _per_layer_check(pm, ads, torch.bfloat16) as checked:
        for step in range(3):
            ids = [names[int(i)] for i in rng.choice(96, size=128, p=w)]
            for sub in _sub_batches(ids, limit):
                x = torch.randint(0, vocab, (len(sub), 1), generator=gen, device=gpu)
                pm(input_ids=x, adapter_ids=sub, past_key_values=DynamicCache(config=model.config), use_cache=True)
                forwards += 1
    assert checked.count == len(pm.target_module_names)
    loads = pm.adapter_cache.loads - loads0
    assert forwards >= 6 and loads > 32, (forwards, loads)  # slots were reused: evictions and reloads happened


class _StoreWeights(dict):
    """PEFT-layout (lora_A, lora_B) of an adapter, read from the store's image on demand."""

    def __init__(self, adapter) -> None:
        super().__init__()
        self.adapter = adapter

    def get(self, module, default=None):
        got = self.adapter.peft_tensors(module)
        return default if got is None else (got[0], got[1])


@pytest.mark.parametrize("layers,n_steps", [(2, 8), (32, 3)])
def test_churn_catalog_of_1024_adapters_every_layer_against_the_oracle(gpu, layers, n_steps):
    """Config 5 at its catalog size: 1024 rank-16 adapters on all 7 targets (images as the churn bench builds
    them; about half of them pageable, loaded through the staging ring), 32 slots with spare regions, steps of
    128 rows drawn Zipf(0.9) over the catalog, each cut into sub-batches of at most 32 distinct adapters; every
    wrapped layer of every sub-batch against the oracle, with the weights read back from the store's images.
    On 2 layers for more steps, and on the configuration's 32 layers (an 86 GB catalog) for 3 steps."""
    _announce(test="churn_catalog", catalog=1024, layers=layers, steps=n_steps)
    import gc

    from transformers import DynamicCache

    from bench import build_llama, random_image_catalog
    from polylora_amd.slot_image import release_locked_free

    n_cat, rows = 1024, 128
    model = build_llama(gpu, layers=layers, seed=1006)
    pm = PolyLoraModel(model, PolyLoraConfig(target_modules=LLAMA_TARGETS, max_gpu_adapters=32, max_rank=16)).eval()
    assert pm.adapter_cache.spare_regions == 32
    shapes = {s.name: (s.in_features, s.out_features) for s in pm.module_specs}
    image_bytes = sum(16 * (fi + fo) * 2 for fi, fo in shapes.values())
    store = pm.adapter_store
    store.pinned_bytes_limit = n_cat // 2 * (image_bytes + (1 << 16))  # room for about half of the images
    catalog = random_image_catalog(pm, n_cat, rank=16, seed=1006)
    pinned = sum(1 for a in catalog if store.adapters[a].image.pinned)
    assert 0 < pinned < n_cat, pinned
    ads = {aid: (_StoreWeights(store.adapters[aid]), 32.0) for aid in catalog}  # alpha = 2 r
    rng = np.random.default_rng(1006)
    w = 1.0 / np.arange(1, n_cat + 1) ** 0.9
    w /= w.sum()
    vocab = model.config.vocab_size
    gen = torch.Generator(device=gpu).manual_seed(1006)
    loads0, forwards, distinct = pm.adapter_cache.loads, 0, set()
    with torch.inference_mode(), _per_layer_check(pm, ads, torch.bfloat16, "churn catalog") as checked:
        for step in range(n_steps):
            ids = [catalog[int(i)] for i in rng.choice(n_cat, size=rows, p=w)]
            distinct.update(ids)
            for sub in _sub_batches(ids, 32):
                x = torch.randint(0, vocab, (len(sub), 1), generator=gen, device=gpu)
                pm(input_ids=x, adapter_ids=sub, past_key_values=DynamicCache(config=model.config), use_cache=True)
                forwards += 1
            print(f"step {step + 1}/{n_steps}: {forwards} forwards, {pm.adapter_cache.loads - loads0} loads", flush=True)
    assert checked.count == len(pm.target_module_names) == 7 * layers
    assert checked.calls == 7 * layers * forwards
    loads = pm.adapter_cache.loads - loads0
    # every step meets more distinct adapters than there are slots: loads far beyond the slot count
    assert len(distinct) > 150 and loads > 4 * 32, (len(distinct), loads)
    print(f"churn catalog: {forwards} forwards, {loads} loads, {len(distinct)} distinct adapters", flush=True)
    # the catalog's page-locked images back to the system before the next test pins its own
    del ads, catalog, store, pm, model, checked
    gc.collect()
    torch.cuda.synchronize()
    release_locked_free()


def test_decode_config_step_every_layer_against_the_oracle(gpu):
    """One decode step of the 32-layer decode configuration with all 224 wrapped Linears checked."""
    _announce(test="decode_config_step")
    from bench import _reset_kv, decode_workload

    wl = decode_workload(gpu, layers=32)
    pm = wl.model
    store = pm.adapter_store
    # the oracle's weights: the random bf16 adapters as the store holds them (alpha = 2 r)
    ads = {aid: (_StoreWeights(store.adapters[aid]), 2.0 * r) for aid, r in wl.ranks.items()}
    _reset_kv(wl)
    with torch.inference_mode(), _per_layer_check(pm, ads, torch.bfloat16) as checked:
        out = pm(input_ids=wl.input_ids, past_key_values=wl.cache, cache_position=wl.cache_position, use_cache=True,
                 adapter_ids=wl.adapter_ids).last_hidden_state
    assert checked.count == len(pm.target_module_names) == 224
    assert torch.isfinite(out.float()).all()


@pytest.mark.parametrize("dtype", [torch.float16, torch.float32])
def test_decode_shapes_in_fp16_and_fp32_every_layer_against_the_oracle(gpu, dtype):
    """The decode configuration's rows and adapters (256 rows of one token, 64 slots, ranks {8,16,32,64},
    Zipf(1.1) with 10% base rows) on two Llama-3-8B-shaped layers in fp16 and in fp32: every wrapped Linear
    runs the one-launch decode path (one module per launch, then the sibling sets stacked) and is checked
    against the oracle at the dtype's tolerance."""
    _announce(test="decode_shapes", dtype=dtype)
    from bench import add_random_adapters, build_llama, zipf_ids

    model = build_llama(gpu, layers=2, seed=1007, attn="pl_safe_fp32").to(dtype)  # attention in fp32, any dtype
    pm = PolyLoraModel(model, PolyLoraConfig(target_modules=LLAMA_TARGETS, max_gpu_adapters=64, max_rank=64)).eval()
    assert pm.adapter_cache.dtype == dtype and pm.adapter_cache.decode_handoff
    rng = np.random.default_rng(1007)
    names = [f"h{i:02d}" for i in range(64)]
    ranks = add_random_adapters(pm, {n: int(rng.choice([8, 16, 32, 64])) for n in names}, seed=1007, device=gpu)
    ids = zipf_ids(rng, 256, 64, 1.1, 0.10, names)
    store = pm.adapter_store
    ads = {aid: (_StoreWeights(store.adapters[aid]), 2.0 * r) for aid, r in ranks.items()}
    x = torch.randint(0, model.config.vocab_size, (256, 1), generator=torch.Generator().manual_seed(1007)).to(gpu)
    with torch.inference_mode(), _per_layer_check(pm, ads, dtype, f"decode shapes {dtype}") as checked:
        # the first forward launches per Linear and learns the sibling runs; the second stacks q/k/v and gate/up
        out = [pm(input_ids=x, adapter_ids=ids).last_hidden_state for _ in range(2)]
    assert checked.count == len(pm.target_module_names) == 14 and checked.calls == 28
    assert pm.adapter_cache.stacked_runs
    assert torch.isfinite(out[0].float()).all() and torch.equal(out[0], out[1])
    assert not sgmv.decode_waits_timed_out(gpu)


def test_prefill_config_through_the_model_every_layer_against_the_oracle(gpu, monkeypatch):
    """PolyLoraModel.forward (model.py:75-85) -> MultiLoraLinear (layers.py:33-62) at the prefill batch on two
    Llama-3-8B-shaped layers: the plan takes 64-token groups; the first forward runs one fused launch per
    Linear, the second the stacked fused launches for q/k/v and gate/up; every wrapped layer against the
    oracle on the inputs it saw, both times."""
    _announce(test="prefill_config_model")
    from bench import add_random_adapters, build_llama

    model = build_llama(gpu, layers=2, seed=1004, attn="pl_safe_fp32")
    pm = PolyLoraModel(model, PolyLoraConfig(target_modules=LLAMA_TARGETS, max_gpu_adapters=64, max_rank=64)).eval()
    names = [f"pf{i}" for i in range(8)]
    ranks = {n: (16 if i < 4 else 32) for i, n in enumerate(names)}
    add_random_adapters(pm, ranks, seed=1004, device=gpu)
    ads = {aid: (_StoreWeights(pm.adapter_store.adapters[aid]), 2.0 * r) for aid, r in ranks.items()}
    rng = np.random.default_rng(1004)
    B, S = 32, 1024
    lens = rng.integers(512, S + 1, size=B)
    adapter_ids = [names[i // 4] for i in range(B)]
    mask = (torch.arange(S)[None, :] < torch.as_tensor(lens)[:, None]).long().to(gpu)
    gen = torch.Generator(device=gpu).manual_seed(1004)
    ids = torch.randint(0, model.config.vocab_size, (B, S), generator=gen, device=gpu)
    launches = []
    single, stacked = sgmv._fused_launch, sgmv.lora_fused_stacked

    def record_single(x, y, cache, module_name, plan, *a, **k):
        launches.append(("single", module_name.rsplit(".", 1)[-1], plan.group_tokens))
        return single(x, y, cache, module_name, plan, *a, **k)

    def record_stacked(x, ys, cache, module_names, plan, *a, **k):
        launches.append(("stacked", tuple(n.rsplit(".", 1)[-1] for n in module_names), plan.group_tokens))
        return stacked(x, ys, cache, module_names, plan, *a, **k)

    monkeypatch.setattr(sgmv, "_fused_launch", record_single)
    monkeypatch.setattr(sgmv, "lora_fused_stacked", record_stacked)
    outs = []
    for forward in range(2):
        launches.clear()
        with torch.inference_mode(), _per_layer_check(pm, ads, torch.bfloat16, label=f"prefill forward {forward}") as chk:
            outs.append(pm(input_ids=ids, attention_mask=mask, adapter_ids=adapter_ids).last_hidden_state.clone())
        assert chk.count == len(pm.target_module_names) == 14 and chk.calls == 14
        assert {gt for _, _, gt in launches} == {64}, launches  # 64-token groups: the prefill plan
        kinds = sorted(launches)
        if forward == 0:
            assert kinds == sorted(("single", m, 64) for m in LLAMA_TARGETS * 2), kinds
        else:
            want = [("single", "o_proj", 64), ("single", "down_proj", 64), ("stacked", ("q_proj", "k_proj", "v_proj"), 64),
                    ("stacked", ("gate_proj", "up_proj"), 64)] * 2
            assert kinds == sorted(want), kinds
    valid = mask.bool()
    assert torch.isfinite(outs[1][valid].float()).all()
    assert torch.equal(outs[0], outs[1])  # stacked launches give the single launches' results bit for bit

