"""Benchmark of the multi-LoRA SGMV path on one MI355X.

Headline (``value``): SGMV achieved HBM GB/s on the isolated op, bf16:
T=4096 tokens, K=N=4096, 16 adapter slots + the base slot, ranks cycling
{0,4,8,16} by slot, alpha=32 (scale 32/r), tokens sorted into contiguous
per-slot segments with Dirichlet(1) lengths, X and base Y ~N(0,1), A and B
~N(0,0.02).  One step = the LoRA shrink + expand of all tokens
(``pl_lora_apply``) with the device plan already built (one plan per forward
is shared by every wrapped Linear).  Inputs rotate over enough X/Y sets
(> 512 MB) that the 256 MB Infinity Cache cannot hold them.

Also reported in the same JSON line (``workloads``):

* ``decode``  Llama-3-8B-shaped decoder (32 layers, hidden 4096, 32/8 heads,
  head_dim 128, FFN 14336, random init, bf16), LoRA on q/k/v/o/gate/up/down,
  64 slots, max_rank 64, ranks {8,16,32,64}, alpha 2r; batch 256 rows x one
  new token over a 512-token random KV cache; adapter_ids Zipf(1.1) over 64
  adapters with 10% __base__ rows.  Multi-LoRA tokens/s against the same
  model with no adapters (HIP-graph replay of one decode step, and eager),
  and the 224 shrink+expand pairs of one step timed alone (HBM GB/s).
* ``prefill`` the same model, 8 adapters (r16 x4, r32 x4), B=32, S=1024
  right-padded, U[512,1024] lengths: LoRA kernel GB/s and MFMA fraction,
  forward time with and without adapters.
* ``churn`` 1024 rank-16 adapters through 32 slots, batch 128, Zipf(0.9):
  tokens/s against an all-resident hot set, H2D bytes, copy/compute overlap.
* ``deberta`` DeBERTa-v3-base shape, fp32, 5 adapters, B=8, S=128 (tokens/s).

``--gpus`` above 1 exits: the library runs and measures on one GPU.
"""

from __future__ import annotations

import argparse
from collections import Counter
import json
import os
import re
import platform
import sys
import time
from dataclasses import dataclass, field

import numpy as np
import torch

HBM_PEAK_GBS = 8000.0
MFMA_BF16_PEAK_TFLOPS = 2500.0
METRIC = "SGMV achieved HBM GB/s (% peak); multi-LoRA decode tokens/s, 1 MI355X"

LLAMA_TARGETS = ["q_proj", "k_proj", "v_proj", "o_proj", "gate_proj", "up_proj", "down_proj"]
DEBERTA_TARGETS = ["query_proj", "key_proj", "value_proj", "dense"]


def _log(msg: str) -> None:
    print(f"[bench] {msg}", file=sys.stderr, flush=True)


def cpu_model() -> str:
    """The host CPU's model name from /proc/cpuinfo (platform.processor() is often empty on Linux)."""
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return platform.processor() or platform.machine()


def _cpu_record(value: float, unit: str, threads: int, sample: str) -> dict:
    """A cpu_baseline object: the oracle's restatement of the fallback timed on the host cores."""
    return {"value": value, "unit": unit, "cores": threads, "kind": "port", "cpu_model": cpu_model(),
            "host_logical_cpus": os.cpu_count(), "sample": sample}


# ----------------------------------------------------------------------------- base-model attention
def _safe_fp32_attention(module, query, key, value, attention_mask, scaling=None, dropout=0.0, **kwargs):
    """Attention in fp32 with contiguous operands (no bf16 batched product on a transposed view)."""
    groups = query.shape[1] // key.shape[1]
    q, k, v = query.float(), key.float(), value.float()
    if groups > 1:
        k = k.repeat_interleave(groups, dim=1)
        v = v.repeat_interleave(groups, dim=1)
    scale = scaling if scaling is not None else q.shape[-1] ** -0.5
    w = torch.matmul(q, k.transpose(2, 3).contiguous()) * scale
    if attention_mask is not None:
        m = attention_mask[..., : k.shape[2]]
        w = w.masked_fill(~m, float("-inf")) if m.dtype == torch.bool else w + m.float()
    w = torch.softmax(w, dim=-1)
    out = torch.matmul(w, v.contiguous()).transpose(1, 2).contiguous()
    return out.to(query.dtype), None


_GQA_NATIVE = {"ok": None}  # None: untried; True/False once a fused kernel accepted or refused enable_gqa


def _fused_sdpa_attention(module, query, key, value, attention_mask, scaling=None, dropout=0.0, is_causal=None,
                          **kwargs):
    """torch SDPA restricted to its fused kernels (raises instead of taking the math path).

    Grouped-query heads go to the kernel as they are (enable_gqa) when it
    accepts them; otherwise K/V are expanded to the query heads first.
    """
    import torch.nn.functional as F
    from torch.nn.attention import SDPBackend, sdpa_kernel

    groups = query.shape[1] // key.shape[1]
    if is_causal is None:
        is_causal = query.shape[2] > 1 and attention_mask is None and getattr(module, "is_causal", True)
    kw = dict(attn_mask=attention_mask, dropout_p=0.0, scale=scaling, is_causal=bool(is_causal))
    with sdpa_kernel([SDPBackend.FLASH_ATTENTION, SDPBackend.EFFICIENT_ATTENTION]):
        out = None
        if groups > 1 and _GQA_NATIVE["ok"] is not False:
            try:
                out = F.scaled_dot_product_attention(query, key, value, enable_gqa=True, **kw)
                _GQA_NATIVE["ok"] = True
            except RuntimeError:
                if _GQA_NATIVE["ok"]:
                    raise
                _GQA_NATIVE["ok"] = False
        if out is None:
            if groups > 1:
                key = key.repeat_interleave(groups, dim=1)
                value = value.repeat_interleave(groups, dim=1)
            out = F.scaled_dot_product_attention(query, key, value, **kw)
    return out.transpose(1, 2).contiguous(), None


def _fused_sdpa_mask(*args, **kwargs):
    """sdpa masks, except a single decode query with no padding mask gets none.

    The decode workloads here attend over a cache that is exactly full (512
    cached positions + the new one), so every key is visible and the mask
    would be all true; passing none lets SDPA's flash kernel take the step.
    """
    from transformers.masking_utils import sdpa_mask

    q_length = kwargs.get("q_length", args[1] if len(args) > 1 else None)
    if kwargs.get("attention_mask") is None and q_length == 1:
        return None
    return sdpa_mask(*args, **kwargs)


def register_attention() -> None:
    """Register "pl_safe_fp32" (eager masks) and "pl_fused_sdpa" (sdpa masks) with transformers."""
    from transformers import AttentionInterface
    from transformers.masking_utils import AttentionMaskInterface, eager_mask

    AttentionInterface.register("pl_safe_fp32", _safe_fp32_attention)
    AttentionMaskInterface.register("pl_safe_fp32", eager_mask)
    AttentionInterface.register("pl_fused_sdpa", _fused_sdpa_attention)
    AttentionMaskInterface.register("pl_fused_sdpa", _fused_sdpa_mask)


# ----------------------------------------------------------------------------- adapters
def _lora_pair(gen, fin, fout, rank, std, device):
    """PEFT-layout lora_A [rank, in] and lora_B [out, rank], N(0, std), bf16, generated on `device`."""
    a = (torch.randn(rank, fin, generator=gen, device=device) * std).to(torch.bfloat16)
    b = (torch.randn(fout, rank, generator=gen, device=device) * std).to(torch.bfloat16)
    return a, b


def add_random_adapters(pm, ranks: dict, std: float = 0.02, seed: int = 0, device="cpu", alpha_per_rank: float = 2.0):
    """Random PEFT-layout adapters (all target modules) added to pm's CPU store; returns id -> rank.

    The store packs each straight into its pinned slot image (its layout is
    bound by the GPU cache), so the tensors generated here are not kept.
    """
    from polylora_amd.store import CpuLayerWeights

    gen = torch.Generator(device=device).manual_seed(seed)
    progress = _Progress("random adapters")
    for i, (aid, r) in enumerate(ranks.items()):
        progress.tick(f"adapter {i + 1}/{len(ranks)}")
        layers = {}
        for spec in pm.module_specs:
            a, b = _lora_pair(gen, spec.in_features, spec.out_features, r, std, device)
            layers[spec.name] = CpuLayerWeights(A=a.t(), B=b.t(), rank=r, scale=alpha_per_rank)
        pm.adapter_store.add_adapter(aid, layers)
    return ranks


def random_image_catalog(pm, n: int, rank: int, seed: int, std: float = 0.02, alpha_per_rank: float = 2.0) -> list:
    """n adapters of one rank on every target module, each with its own pinned slot image of N(0, std) weights.

    Each image is laid out by ImageBuilder for the cache's slot layout (so its
    slot-table rows are the ones a PEFT adapter of these ranks gets) and its
    A and B parts are filled with one draw of random bf16 values generated on
    the GPU; with i.i.d. weights the order of the values inside a part does
    not matter, so no per-module packing is needed.  Added with
    add_adapter_image: one host copy per adapter.
    """
    from polylora_amd.slot_image import AdapterImage, ImageBuilder

    layout = pm.adapter_cache.layout
    device = pm.adapter_cache.device
    modules = {spec.name: (rank, alpha_per_rank) for spec in pm.module_specs}
    gen = torch.Generator(device=device).manual_seed(seed)
    ids = [f"cat{i:04d}" for i in range(n)]
    progress = _Progress("catalog")
    data_ranges = None
    for i, aid in enumerate(ids):
        progress.tick(f"{i}/{n} images")
        builder = ImageBuilder(layout, modules, pin=pm.adapter_store.pin_image)
        data = builder.data
        if data_ranges is None:  # the A and B parts; the alignment gaps between them stay zero
            data_ranges = []
            for name, (r, a_off, b_off) in builder.parts.items():
                spec = layout.specs[layout.index[name]]
                data_ranges.append((a_off, a_off + r * spec.in_features * layout.elem))
                data_ranges.append((b_off, b_off + spec.out_features * ((r + 7) // 8 * 8) * layout.elem))
            data_ranges.sort()
            merged = [list(data_ranges[0])]
            for lo, hi in data_ranges[1:]:
                if lo == merged[-1][1]:
                    merged[-1][1] = hi
                else:
                    merged.append([lo, hi])
            data_ranges = merged
        vals = (torch.randn(data.numel() // 2, generator=gen, device=device) * std).to(torch.bfloat16).view(torch.uint8)
        for lo, hi in data_ranges:
            data[lo:hi].copy_(vals[lo:hi])
        pm.adapter_store.add_adapter_image(aid, AdapterImage(layout, data, builder.rows, builder.pinned))
    torch.cuda.synchronize()
    return ids


class _Progress:
    """Log a line from inside a long loop at most every `every` seconds (a profiler run must not look silent)."""

    def __init__(self, what: str, every: float = 20.0) -> None:
        self.what, self.every = what, every
        self.t0 = self.last = time.perf_counter()

    def tick(self, where: str) -> None:
        now = time.perf_counter()
        if now - self.last >= self.every:
            self.last = now
            _log(f"{self.what}: {where} ({now - self.t0:.0f} s)")


def _rank_of(pm, adapter_id: str, module: str) -> int:
    """An adapter's rank in a module (0 where it has no weights), without materializing its weights."""
    return pm.adapter_store.adapters[adapter_id].module_ranks().get(module, (0, 0.0))[0]


# ----------------------------------------------------------------------------- config 1: DeBERTa fp32
@dataclass
class DebertaWorkload:
    model: object  # PolyLoraModel
    base: object  # plain DebertaV2Model with the same weights
    inputs: dict
    adapter_ids: list
    adapters: dict  # id -> ({module: (lora_A, lora_B)}, alpha)


def deberta_workload(device, seed: int = 1001, layers: int = 12) -> DebertaWorkload:
    """DeBERTa-v3-base shape fp32, q/k/v/dense targets, 5 adapters r {4,8,8,16,16} (last: q/v only), B=8, S=128."""
    import copy

    from transformers import DebertaV2Config, DebertaV2Model

    from polylora_amd import PolyLoraConfig, PolyLoraModel

    torch.manual_seed(seed)
    cfg = DebertaV2Config(vocab_size=32000, hidden_size=768, num_hidden_layers=layers, num_attention_heads=12,
                          intermediate_size=3072, hidden_dropout_prob=0.0, attention_probs_dropout_prob=0.0,
                          initializer_range=0.02)
    base = DebertaV2Model(cfg).to(device).eval()
    pm = PolyLoraModel(copy.deepcopy(base), PolyLoraConfig(target_modules=DEBERTA_TARGETS, max_gpu_adapters=4, max_rank=16)).eval()
    gen = torch.Generator().manual_seed(seed)
    adapters = {}
    for i, r in enumerate([4, 8, 8, 16, 16]):
        mods = [s for s in pm.module_specs if i < 4 or s.name.endswith(("query_proj", "value_proj"))]
        w = {s.name: (torch.randn(r, s.in_features, generator=gen) * 0.02, torch.randn(s.out_features, r, generator=gen) * 0.02) for s in mods}
        aid = f"deb{i}"
        from polylora_amd.store import CpuLayerWeights

        pm.adapter_store.add_adapter(aid, {m: CpuLayerWeights(a.t().contiguous(), b.t().contiguous(), r, 2.0) for m, (a, b) in w.items()})
        adapters[aid] = (w, 2.0 * r)
    B, S = 8, 128
    choices = list(adapters) + ["__base__"]
    while True:  # at most 4 distinct adapters per batch (4 GPU slots)
        pick = torch.randint(0, len(choices), (B,), generator=gen).tolist()
        ids = [choices[i] for i in pick]
        if len({a for a in ids if a != "__base__"}) <= 4:
            break
    lens = torch.randint(32, S + 1, (B,), generator=gen)
    mask = (torch.arange(S)[None, :] < lens[:, None]).long()
    input_ids = torch.randint(0, 32000, (B, S), generator=gen)
    inputs = {"input_ids": input_ids.to(device), "attention_mask": mask.to(device)}
    return DebertaWorkload(pm, base, inputs, ids, adapters)


def cpu_baseline_deberta(wl: DebertaWorkload, budget_s: float) -> dict:
    """The whole 12-layer fp32 forward on the host through the reference fallback.

    The base weights are a CPU copy of the GPU model's; every target Linear
    adds the oracle's restatement of layers.py:112-134 (oracle.model), on
    the same batch, mask and adapters.
    """
    import copy

    from oracle import model as oracle_model

    m = copy.deepcopy(wl.base).cpu().eval()
    names = oracle_model.wrap_model(m, DEBERTA_TARGETS, None)
    shapes = {n: (m.get_submodule(n).base_layer.in_features, m.get_submodule(n).base_layer.out_features) for n in names}
    bank = oracle_model.OracleBank({aid: {mod: (a, b, alpha) for mod, (a, b) in w.items()}
                                    for aid, (w, alpha) in wl.adapters.items()}, shapes, 16, torch.float32, "cpu")
    for n in names:
        m.get_submodule(n).bank = bank
    inputs = {k: v.cpu() for k, v in wl.inputs.items()}
    valid = int(inputs["attention_mask"].sum())
    threads = torch.get_num_threads()
    with torch.inference_mode():
        oracle_model.run(m, bank, wl.adapter_ids, **inputs)  # warm-up
        reps, t0 = 0, time.perf_counter()
        while True:
            oracle_model.run(m, bank, wl.adapter_ids, **inputs)
            reps += 1
            el = time.perf_counter() - t0
            if el >= budget_s:
                break
    per = el / reps
    return _cpu_record(round(valid / per, 1), "tokens/s", threads,
                       f"{reps} full 12-layer fp32 forwards (8 rows x 128, {valid} valid tokens, 72 wrapped Linears) "
                       f"through the fallback, {per * 1e3:.1f} ms each; torch {threads} threads")


def run_deberta(device, reps: int = 20, cpu_budget_s: float | None = None) -> dict:
    wl = deberta_workload(device)
    valid = int(wl.inputs["attention_mask"].sum())
    with torch.inference_mode():
        for _ in range(3):
            wl.model(**wl.inputs, adapter_ids=wl.adapter_ids)
            wl.model(**wl.inputs)
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        for _ in range(reps):
            wl.model(**wl.inputs, adapter_ids=wl.adapter_ids)
        torch.cuda.synchronize()
        lora_s = (time.perf_counter() - t0) / reps
        t0 = time.perf_counter()
        for _ in range(reps):
            wl.model(**wl.inputs)
        torch.cuda.synchronize()
        base_s = (time.perf_counter() - t0) / reps
    out = {"dtype": "f32", "valid_tokens": valid, "lora_tokens_per_s": round(valid / lora_s, 1),
           "base_tokens_per_s": round(valid / base_s, 1), "ratio": round(base_s / lora_s, 4), "timing": "eager wall clock"}
    # The same forwards replayed from HIP graphs, which take the host out: the LoRA context (residency,
    # row -> slot map, lengths, right-padding check) is prepared once outside the capture, as a serving
    # loop that replays a graph per batch shape would; the base is the plain DeBERTa model.
    from polylora_amd.context import use_lora_context

    try:
        with torch.inference_mode():
            B, S = wl.inputs["input_ids"].shape
            ctx = wl.model.prepare_lora_context(wl.adapter_ids, wl.inputs["attention_mask"], B, S, device)

            def lora_fwd():
                with use_lora_context(ctx):
                    return wl.model.base_model(**wl.inputs).last_hidden_state

            g_lora = _graph_ms(lora_fwd, reps)
            g_base = _graph_ms(lambda: wl.base(**wl.inputs).last_hidden_state, reps)
        out["graph_ms_lora"] = round(g_lora, 4)
        out["graph_ms_base"] = round(g_base, 4)
        out["graph_lora_tokens_per_s"] = round(valid / g_lora * 1e3, 1)
        out["graph_base_tokens_per_s"] = round(valid / g_base * 1e3, 1)
        out["graph_ratio"] = round(g_base / g_lora, 4)
        out["graph_timing"] = "HIP graph replay of one forward, LoRA context prepared outside the capture"
    except Exception as exc:  # noqa: BLE001 - report and keep the eager numbers
        out["graph_error"] = f"{type(exc).__name__}: {str(exc)[:300]}"
    if cpu_budget_s is not None:
        _log("deberta: CPU baseline (full fp32 forward through the fallback)")
        out["cpu_baseline"] = cpu_baseline_deberta(wl, cpu_budget_s)
    return out


# ----------------------------------------------------------------------------- config 2: isolated SGMV
@dataclass
class IsolatedSgmv:
    cache: object
    adapters: dict
    ranks: list
    x: torch.Tensor  # [T, K]
    base: torch.Tensor  # [T, N] pristine base output
    y: torch.Tensor  # [T, N] working output
    row_slot: torch.Tensor  # int32 [T]
    seq_lens: torch.Tensor  # int32 [T] (ones: one token per row)
    plan: object
    seg_lens: np.ndarray  # tokens per slot (slot 0 = base)


def _dirichlet_segments(rng: np.random.Generator, total: int, parts: int) -> np.ndarray:
    w = rng.dirichlet(np.ones(parts))
    lens = np.floor(w * total).astype(np.int64)
    lens[-1] += total - lens.sum()
    return lens


def isolated_sgmv_workload(device, seed: int = 1002, T: int = 4096, K: int = 4096, N: int = 4096, slots: int = 16,
                           alpha: float = 32.0, dtype=torch.bfloat16) -> IsolatedSgmv:
    from polylora_amd import sgmv
    from polylora_amd.cache import GpuAdapterCache, ModuleSpec
    from polylora_amd.config import PolyLoraConfig
    from polylora_amd.store import CpuAdapterStore, CpuLayerWeights

    rng = np.random.default_rng(seed)
    gen = torch.Generator().manual_seed(seed)
    S = slots + 1
    rank_cycle = [0, 4, 8, 16]
    ranks = [rank_cycle[s % 4] for s in range(S)]
    r_max = max(rank_cycle)
    A = torch.randn(S, r_max, K, generator=gen) * 0.02  # PEFT lora_A per slot
    B = torch.randn(S, N, r_max, generator=gen) * 0.02  # PEFT lora_B per slot
    store = CpuAdapterStore()
    adapters = {}
    for s in range(1, S):
        r = ranks[s]
        layers = {"pad": (torch.randn(1, 8, generator=gen) * 0.02, torch.randn(8, 1, generator=gen) * 0.02, 1.0)}
        if r > 0:
            layers["op"] = (A[s, :r].clone(), B[s, :, :r].clone(), alpha)
        adapters[f"s{s:02d}"] = layers
        store.add_adapter(
            f"s{s:02d}",
            {m: CpuLayerWeights(A=a.t().contiguous(), B=b.t().contiguous(), rank=a.shape[0], scale=al / a.shape[0])
             for m, (a, b, al) in layers.items()},
        )
    config = PolyLoraConfig(max_gpu_adapters=slots, max_rank=r_max)
    cache = GpuAdapterCache(store, [ModuleSpec("op", K, N), ModuleSpec("pad", 8, 8)], config, device, dtype)
    seg = _dirichlet_segments(rng, T, S)
    token_ids = []
    for s in range(S):
        token_ids += ["__base__" if s == 0 else f"s{s:02d}"] * int(seg[s])
    row_slot = cache.ensure_resident(token_ids)
    seq_lens = torch.ones(T, dtype=torch.int32, device=device)
    x = torch.randn(T, K, generator=gen).to(dtype).to(device)
    base = torch.randn(T, N, generator=gen).to(dtype).to(device)
    # the op's plan: tokens of rank-0 slots need no work and take no group positions
    plan = sgmv.SgmvPlan(row_slot, seq_lens, 1, cache.num_slots, distinct_slots=slots, active=cache.ranks["op"])
    return IsolatedSgmv(cache, adapters, ranks, x, base, base.clone(), row_slot, seq_lens, plan, seg)


def isolated_sgmv_bytes(wl: IsolatedSgmv, K: int, N: int) -> dict:
    """Algorithmic bytes: X of active tokens, Y read+write, each active adapter's A and B once, the row maps."""
    active = [s for s in range(len(wl.ranks)) if wl.ranks[s] > 0]
    t_active = int(sum(wl.seg_lens[s] for s in active))
    r_tok = int(sum(wl.seg_lens[s] * wl.ranks[s] for s in active))
    shrink = 2 * t_active * K + sum(2 * wl.ranks[s] * K for s in active)
    expand = 4 * t_active * N + sum(2 * wl.ranks[s] * N for s in active)
    total = shrink + expand + 4 * len(wl.ranks) * 2
    flops = 2 * r_tok * (K + N)
    return {"total": total, "shrink": shrink, "expand": expand, "t_active": t_active, "flops": flops}


def cpu_baseline_isolated(wl: IsolatedSgmv, nbytes: int, budget_s: float) -> dict:
    """The reference fallback (oracle restatement of layers.py:112-134) on the host.

    Segment view: one row per slot holding its contiguous tokens, seq_len = segment length.
    """
    from oracle.lora import dense_slot_tensors, reference_forward

    K = wl.x.shape[1]
    N = wl.y.shape[1]
    S = len(wl.ranks)
    lmax = int(wl.seg_lens.max())
    xs = torch.zeros(S, lmax, K, dtype=wl.x.dtype)
    bs = torch.zeros(S, lmax, N, dtype=wl.x.dtype)
    x_cpu, b_cpu = wl.x.cpu(), wl.base.cpu()
    off = 0
    for s in range(S):
        n = int(wl.seg_lens[s])
        xs[s, :n] = x_cpu[off : off + n]
        bs[s, :n] = b_cpu[off : off + n]
        off += n
    per_slot = [None] + [wl.adapters[f"s{s:02d}"].get("op") for s in range(1, S)]
    A, B, ranks, scales = dense_slot_tensors(per_slot, K, N, 16, wl.x.dtype)
    seq = torch.tensor(wl.seg_lens, dtype=torch.int32)
    widx = torch.arange(S)
    threads = torch.get_num_threads()
    reps = 0
    t0 = time.perf_counter()
    while True:
        reference_forward(xs, bs, seq, widx, A, B, ranks, scales)
        reps += 1
        el = time.perf_counter() - t0
        if el >= budget_s:
            break
    per = el / reps
    return _cpu_record(round(nbytes / per / 1e9, 4), "GB/s", threads,
                       f"{reps} full ops (17 segment rows, {int(wl.seg_lens.sum())} tokens) of the fallback loop, "
                       f"{per * 1e3:.1f} ms each, torch {threads} threads")


class SgmvLaunch:
    """The shrink and the expand of one wrapped Linear as separate launches (pl_sgmv_shrink, pl_sgmv_expand)."""

    def __init__(self, x, y, cache, module, plan, k_splits=None):
        from polylora_amd import _native, sgmv

        self.lib, self.n = _native.load(), _native
        self.stream = torch.cuda.current_stream()
        dt = _native.dtype_code(x.dtype)
        K, N = int(x.shape[1]), int(y.shape[1])
        splits = k_splits if k_splits is not None else sgmv.choose_k_splits(plan.group_cap, K, x.dtype)
        rows = max(1, plan.tokens_cap)
        ldt = cache.rank8_cap
        gt = plan.group_tokens
        nbytes = int(self.lib.pl_shrink_workspace_bytes(dt, K, splits, gt, rows, ldt))
        planes = int(self.lib.pl_shrink_planes(dt, K, splits, gt))
        ws = sgmv._workspace(x.device, self.stream.cuda_stream)
        buf = ws.get(nbytes)
        ws.owner = None
        common = (cache.arena.data_ptr(), cache.table.data_ptr(), len(cache.module_index), cache.module_index[module],
                  plan.tok.data_ptr(), plan.groups.data_ptr(), plan.meta.data_ptr(), max(1, plan.group_cap), gt)
        s = self.stream.cuda_stream
        self.shrink_args = (dt, x.data_ptr(), x.stride(0), K, *common, buf.data_ptr(), buf.numel(), ldt, rows, splits, s)
        self.expand_args = (dt, buf.data_ptr(), ldt, rows, planes, *common, y.data_ptr(), y.stride(0), N,
                            _native.PL_EPI_FALLBACK, s)
        self.keep = (x, y, buf, plan)

    def shrink(self):
        self.n.check(self.lib.pl_sgmv_shrink(*self.shrink_args), "pl_sgmv_shrink")

    def expand(self):
        self.n.check(self.lib.pl_sgmv_expand(*self.expand_args), "pl_sgmv_expand")


class StackedLaunch:
    """Sibling Linears fed the same x: one stacked shrink launch and one stacked expand launch."""

    def __init__(self, x, ys, cache, modules, plan, k_splits=None):
        import ctypes

        from polylora_amd import _native, sgmv

        self.lib, self.n = _native.load(), _native
        self.stream = torch.cuda.current_stream()
        dt = _native.dtype_code(x.dtype)
        K = int(x.shape[1])
        splits = k_splits if k_splits is not None else sgmv.choose_k_splits(plan.group_cap, K, x.dtype)
        rows = max(1, plan.tokens_cap)
        ldt = cache.rank8_cap
        gt = plan.group_tokens
        nbytes = int(self.lib.pl_shrink_workspace_bytes(dt, K, splits, gt, rows, ldt))
        planes = int(self.lib.pl_shrink_planes(dt, K, splits, gt))
        bufs = [torch.empty(nbytes, dtype=torch.uint8, device=x.device) for _ in modules]
        n_mod = len(cache.module_index)
        s = self.stream.cuda_stream
        self.mods = (ctypes.c_int32 * len(modules))(*(cache.module_index[m] for m in modules))
        self.ptrs = (ctypes.c_void_p * len(modules))(*(b.data_ptr() for b in bufs))
        self.shrink_args = (dt, x.data_ptr(), x.stride(0), K, cache.arena.data_ptr(), cache.table.data_ptr(), n_mod,
                            len(modules), self.mods, self.ptrs, plan.tok.data_ptr(), plan.groups.data_ptr(),
                            plan.meta.data_ptr(), max(1, plan.group_cap), gt, nbytes, ldt, rows, splits, s)
        self.yptrs = (ctypes.c_void_p * len(modules))(*(y.data_ptr() for y in ys))
        self.ldys = (ctypes.c_int64 * len(modules))(*(y.stride(0) for y in ys))
        self.Ns = (ctypes.c_int32 * len(modules))(*(int(y.shape[1]) for y in ys))
        self.expand_args = (dt, self.ptrs, ldt, rows, planes, cache.arena.data_ptr(), cache.table.data_ptr(), n_mod,
                            len(modules), self.mods, plan.tok.data_ptr(), plan.groups.data_ptr(), plan.meta.data_ptr(),
                            max(1, plan.group_cap), gt, self.yptrs, self.ldys, self.Ns, _native.PL_EPI_FALLBACK, s)
        self.keep = (x, ys, bufs, plan)

    def shrink(self):
        self.n.check(self.lib.pl_sgmv_shrink_stacked(*self.shrink_args), "pl_sgmv_shrink_stacked")

    def expand(self):
        self.n.check(self.lib.pl_sgmv_expand_stacked(*self.expand_args), "pl_sgmv_expand_stacked")


class DecodeLaunch:
    """Sibling Linears fed the same x: shrink and expand in one launch with the hand-off inside it
    (pl_lora_decode_stacked), arguments bound once; its own planes and zeroed hand-off counters."""

    def __init__(self, x, ys, cache, modules, plan, k_splits=None):
        import ctypes

        from polylora_amd import _native, sgmv

        self.lib, self.n = _native.load(), _native
        s = torch.cuda.current_stream().cuda_stream
        dt = _native.dtype_code(x.dtype)
        K = int(x.shape[1])
        n = len(modules)
        splits = k_splits if k_splits is not None else sgmv.choose_k_splits(plan.group_cap, K, x.dtype)
        rows = max(1, plan.tokens_cap)
        ldt = -(-cache.rank8_cap // 32) * 32
        gt = plan.group_tokens
        cap = max(1, plan.group_cap)
        nbytes = int(self.lib.pl_shrink_workspace_bytes(dt, K, splits, gt, rows, ldt))
        bufs = [torch.empty(nbytes, dtype=torch.uint8, device=x.device) for _ in modules]
        ints = int(self.lib.pl_decode_counter_ints(cap, n))
        self.counters = torch.zeros(ints, dtype=torch.int32, device=x.device)
        self.mods = (ctypes.c_int32 * n)(*(cache.module_index[m] for m in modules))
        self.ptrs = (ctypes.c_void_p * n)(*(b.data_ptr() for b in bufs))
        self.yptrs = (ctypes.c_void_p * n)(*(y.data_ptr() for y in ys))
        self.ldys = (ctypes.c_int64 * n)(*(y.stride(0) for y in ys))
        self.Ns = (ctypes.c_int32 * n)(*(int(y.shape[1]) for y in ys))
        self.args = (dt, x.data_ptr(), x.stride(0), K, cache.arena.data_ptr(), cache.table.data_ptr(),
                     len(cache.module_index), n, self.mods, self.ptrs, plan.tok.data_ptr(), plan.groups.data_ptr(),
                     plan.meta.data_ptr(), cap, gt, nbytes, ldt, rows, splits, self.yptrs, self.ldys, self.Ns,
                     _native.PL_EPI_FALLBACK, self.counters.data_ptr(), ints, sgmv.DECODE_SPIN_LIMIT, s)
        self.keep = (x, ys, bufs, plan)

    def __call__(self):
        self.n.check(self.lib.pl_lora_decode_stacked(*self.args), "pl_lora_decode_stacked")


class FusedLaunch:
    """One wrapped Linear's fused shrink+expand (pl_lora_fused) with its arguments bound once."""

    def __init__(self, x, y, cache, module, plan, slices=None):
        from polylora_amd import _native, sgmv

        self.lib, self.n = _native.load(), _native
        n_slices = slices if slices is not None else sgmv.choose_slices(plan, int(y.shape[1]))
        self.args = (_native.dtype_code(x.dtype), x.data_ptr(), x.stride(0), int(x.shape[1]), y.data_ptr(),
                     y.stride(0), int(y.shape[1]), cache.arena.data_ptr(), cache.table.data_ptr(),
                     len(cache.module_index), cache.module_index[module], cache.rank8_cap, plan.tok.data_ptr(),
                     plan.groups.data_ptr(), plan.meta.data_ptr(), max(1, plan.group_cap), plan.group_tokens, n_slices,
                     _native.PL_EPI_FALLBACK, torch.cuda.current_stream().cuda_stream)
        self.keep = (x, y, plan)

    def __call__(self):
        self.n.check(self.lib.pl_lora_fused(*self.args), "pl_lora_fused")


class StackedFusedLaunch:
    """Sibling Linears fed the same x: one fused shrink+expand launch for all (pl_lora_fused_stacked)."""

    def __init__(self, x, ys, cache, modules, plan, slices=None):
        import ctypes

        from polylora_amd import _native, sgmv

        self.lib, self.n = _native.load(), _native
        n = len(modules)
        n_slices = slices if slices is not None else sgmv.choose_slices(plan, min(int(y.shape[1]) for y in ys))
        self.mods = (ctypes.c_int32 * n)(*(cache.module_index[m] for m in modules))
        self.yptrs = (ctypes.c_void_p * n)(*(y.data_ptr() for y in ys))
        self.ldys = (ctypes.c_int64 * n)(*(y.stride(0) for y in ys))
        self.Ns = (ctypes.c_int32 * n)(*(int(y.shape[1]) for y in ys))
        self.args = (_native.dtype_code(x.dtype), x.data_ptr(), x.stride(0), int(x.shape[1]), n, self.mods,
                     self.yptrs, self.ldys, self.Ns, cache.arena.data_ptr(), cache.table.data_ptr(),
                     len(cache.module_index), cache.rank8_cap, plan.tok.data_ptr(), plan.groups.data_ptr(),
                     plan.meta.data_ptr(), max(1, plan.group_cap), plan.group_tokens, n_slices,
                     _native.PL_EPI_FALLBACK, torch.cuda.current_stream().cuda_stream)
        self.keep = (x, ys, plan)

    def __call__(self):
        self.n.check(self.lib.pl_lora_fused_stacked(*self.args), "pl_lora_fused_stacked")


def time_launches(fns: list, reps: int, warmup: int = 2) -> float:
    """Milliseconds per pass over `fns`, launched back to back on the current stream between two events."""
    stream = torch.cuda.current_stream()
    for _ in range(warmup):
        for f in fns:
            f()
    t0 = torch.cuda.Event(enable_timing=True)
    t1 = torch.cuda.Event(enable_timing=True)
    t0.record(stream)
    progress = _Progress("timed launches")
    for i in range(reps):
        progress.tick(f"pass {i}/{reps} of {len(fns)} launches")
        for f in fns:
            f()
    t1.record(stream)
    torch.cuda.synchronize()
    return t0.elapsed_time(t1) / reps


def _profiled(workload: str, *keys):
    """A figure of the committed launch profile of `workload` (profiles/sgmv_<workload>_traffic.json), or None.

    Those files are --reduce-profile's JSON of rocprofv3 kernel-trace,
    FETCH_SIZE and WRITE_SIZE runs of --launch-profile <workload>.
    """
    path = os.path.join(os.path.dirname(os.path.abspath(__file__)), "profiles", f"sgmv_{workload}_traffic.json")
    try:
        with open(path, encoding="utf-8") as fh:
            data = json.load(fh)
        for k in keys:
            data = data[k]
        return int(round(float(data)))
    except (OSError, ValueError, KeyError, TypeError):
        return None


def _profiled_plan_us(workload: str):
    """Average pl_plan_kernel duration (us) in the committed launch profile of `workload`, or None."""
    path = os.path.join(os.path.dirname(os.path.abspath(__file__)), "profiles", f"sgmv_{workload}_traffic.json")
    try:
        with open(path, encoding="utf-8") as fh:
            return round(float(json.load(fh)["plan_avg_us"]), 2)
    except (OSError, ValueError, KeyError, TypeError):
        return None


def _profiled_traffic(kernel: str):
    """HBM bytes per launch of `kernel` in the isolated op's profile, or None."""
    return _profiled("isolated", "kernels", kernel, "traffic_bytes_per_launch")


def sequence_roofline(what: str, nbytes: int, ms: float, launches: int, workload: str) -> dict:
    """Roofline block of a launch sequence: algorithmic bytes over the sequence's back-to-back time."""
    gbs = nbytes / (ms * 1e-3) / 1e9
    return {"kernel": what, "bound": "hbm", "achieved": round(gbs, 2), "peak": HBM_PEAK_GBS, "unit": "GB/s",
            "frac": round(gbs / HBM_PEAK_GBS, 4), "traffic": _profiled(workload, "pass_traffic_bytes"),
            "algorithmic_bytes_per_sequence": nbytes, "launches": launches, "sequence_ms": round(ms, 4),
            "traffic_note": f"HBM bytes of one sequence from profiles/sgmv_{workload}_traffic.json"}


def time_operator_api(sets: list, reps: int, keep: bool = False) -> dict:
    """sgmv_lora_a_fwd then sgmv_lora_b_fwd (the reference's operator API) on the isolated op's shapes.

    The adapters of the workload in the reference's slot layout (A
    [17, 4096, 16], B [17, 16, 4096], zero past each rank; index = the
    cache slot, 0 = rank 0), each token a row of one position; x and the base
    output rotate over the same input sets as the other timings.
    """
    from polylora_amd import sgmv

    wl = sets[0]
    cache = wl.cache
    S, K, N, R = cache.num_slots, wl.x.shape[1], wl.y.shape[1], 16
    wa = torch.zeros(S, K, R, dtype=wl.x.dtype)
    wb = torch.zeros(S, R, N, dtype=wl.x.dtype)
    ranks = torch.zeros(S, dtype=torch.int32)
    scal = torch.zeros(S, dtype=torch.float32)
    for slot in range(1, S):
        aid = cache.slot_to_adapter[slot]
        got = None if aid is None else wl.adapters[aid].get("op")
        if got is None:
            continue
        a, b, alpha = got
        r = a.shape[0]
        wa[slot, :, :r] = a.t()
        wb[slot, :r, :] = b.t()
        ranks[slot], scal[slot] = r, alpha / r
    dev = wl.x.device
    wa, wb, ranks, scal = wa.to(dev), wb.to(dev), ranks.to(dev), scal.to(dev)
    widx = wl.row_slot
    seq = wl.seq_lens
    xs = [w.x.view(-1, 1, K) for w in sets]
    ys = [w.y.view(-1, 1, N) for w in sets]

    def pair(i):
        tmp = sgmv.sgmv_lora_a_fwd(xs[i], wa, seq, widx, ranks)
        sgmv.sgmv_lora_b_fwd(tmp, wb, seq, widx, ranks, scal, ys[i])

    if keep:
        return {"pair": pair}
    for i in range(2 * len(sets)):
        pair(i % len(sets))
    torch.cuda.synchronize()
    t0, t1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    t0.record()
    for i in range(reps):
        pair(i % len(sets))
    t1.record()
    torch.cuda.synchronize()
    return {"pair_ms": t0.elapsed_time(t1) / reps}


def run_isolated(args) -> dict:
    from polylora_amd import sgmv

    device = torch.device("cuda", 0)
    K = N = 4096
    base_set = isolated_sgmv_workload(device)
    set_bytes = 2 * base_set.x.numel() * base_set.x.element_size()
    n_sets = max(3, int(np.ceil(600e6 / set_bytes)))
    sets = [base_set]
    for _ in range(1, n_sets):
        sets.append(IsolatedSgmv(base_set.cache, base_set.adapters, base_set.ranks,
                                 torch.randn_like(base_set.x), base_set.base, torch.randn_like(base_set.y),
                                 base_set.row_slot, base_set.seq_lens, base_set.plan, base_set.seg_lens))
    nb = isolated_sgmv_bytes(base_set, K, N)

    def apply(wl):
        sgmv.lora_apply(wl.x, wl.y, wl.cache, "op", wl.plan)

    # Per-kernel timings first (they also bring the GPU to its working clocks
    # before the timed steps): the split shrink + expand, for comparison (the
    # kernels a plan with few tokens per adapter would use), and the fused
    # kernel alone with its arguments bound once.
    reps = max(10, args.steps // n_sets)
    launches = [SgmvLaunch(wl.x, wl.y, wl.cache, "op", wl.plan) for wl in sets]
    sh_ms = time_launches([l.shrink for l in launches], reps) / n_sets
    ex_ms = time_launches([l.expand for l in launches], reps) / n_sets
    fused = sgmv.fused_ok(base_set.plan, base_set.cache, K)
    if fused:
        f_ms = time_launches([FusedLaunch(wl.x, wl.y, wl.cache, "op", wl.plan) for wl in sets], reps) / n_sets

    from polylora_amd import refop_cache

    op_ms = time_operator_api(sets, max(20, args.steps // 2))["pair_ms"]
    try:
        refop_cache.configure(max_bytes=0, max_plans=0)
        op_nk_ms = time_operator_api(sets, max(20, args.steps // 2))["pair_ms"]
    finally:
        refop_cache.configure()
    # the op with its plan: the device plan build and the op's launch(es), back to back
    stream_h = torch.cuda.current_stream().cuda_stream
    if fused:
        with_plan = [f for wl in sets for f in (lambda: base_set.plan.rebuild(stream_h),
                                                FusedLaunch(wl.x, wl.y, wl.cache, "op", wl.plan))]
    else:
        with_plan = [f for l in launches for f in (lambda: base_set.plan.rebuild(stream_h), l.shrink, l.expand)]
    wp_ms = time_launches(with_plan, reps) / n_sets

    # a step is one lora_apply call through the Python host API (plan already
    # built, inputs resident); the calls queue back to back, so the device,
    # not the host, sets the pace
    for i in range(args.warmup):
        apply(sets[i % n_sets])
    torch.cuda.synchronize()
    start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    start.record()
    for i in range(args.steps):
        apply(sets[i % n_sets])
    end.record()
    torch.cuda.synchronize()
    ms = start.elapsed_time(end) / args.steps
    value = nb["total"] / (ms * 1e-3) / 1e9
    if fused:
        # lora_apply runs the fused kernel: one launch carries all of the op's bytes
        kernel, k_bytes, k_ms = "pl_lora_fused_tile<bf16>", nb["total"], f_ms
    else:
        kernel, k_bytes, k_ms = "pl_expand_short<bf16>", nb["expand"], ex_ms
    k_gbs = k_bytes / (k_ms * 1e-3) / 1e9
    out = {
        "value": round(value, 2),
        "ms_per_step": round(ms, 5),
        "config": {
            "workload": "isolated SGMV shrink+expand, T=4096 tokens, K=N=4096, 16 slots + base, ranks {0,4,8,16}, "
                        "Dirichlet(1) segments, alpha 32",
            "tokens_active": nb["t_active"],
            "algorithmic_bytes_per_step": nb["total"],
            "pct_of_hbm_peak": round(100 * value / HBM_PEAK_GBS, 2),
            "input_sets_rotated": n_sets,
            "timing": "lora_apply calls back to back, device events around the timed steps; the device plan "
                      "(pl_plan_build_active over the 4096 rows) is built once before the timed region, as a "
                      "model forward builds it once for all of its wrapped Linears",
            "plan_kernel_us_profiled": _profiled_plan_us("isolated"),
            "op_with_plan_ms": round(wp_ms, 5),
            "op_with_plan_gbs": round(nb["total"] / (wp_ms * 1e-3) / 1e9, 1),
            "op_with_plan_note": "the plan build and the op's launch back to back per step, arguments bound once; "
                                 "GB/s counts the op's bytes",
            "plan_group_tokens": base_set.plan.group_tokens,
            "lora_apply_kernels": "pl_lora_fused (one launch)" if fused else "pl_sgmv_shrink + pl_sgmv_expand",
            "split_shrink_ms": round(sh_ms, 5),
            "split_expand_ms": round(ex_ms, 5),
            "split_pair_gbs": round(nb["total"] / ((sh_ms + ex_ms) * 1e-3) / 1e9, 1),
            "operator_api_pair_ms": round(op_ms, 5),
            "operator_api_pair_gbs": round(nb["total"] / (op_ms * 1e-3) / 1e9, 1),
            "operator_api_note": "sgmv_lora_a_fwd + sgmv_lora_b_fwd with the reference's slot layout and a "
                                 "model-dtype intermediate, host calls back to back; the plan and the packed "
                                 "weights are kept from the warm-up calls (the tensors do not change), so a pair "
                                 "is 2 launches: the fused kernel's shrink phase and its expand phase; GB/s counts "
                                 "the op's bytes",
            "operator_api_nothing_kept_pair_ms": round(op_nk_ms, 5),
            "operator_api_nothing_kept_note": "the same with nothing kept: each call builds the plan and repacks "
                                              "the adapters its rows use (one more launch per call)",
        },
        "roofline": {
            "kernel": kernel,
            "bound": "hbm",
            "achieved": round(k_gbs, 2),
            "peak": HBM_PEAK_GBS,
            "unit": "GB/s",
            "frac": round(k_gbs / HBM_PEAK_GBS, 4),
            "traffic": _profiled_traffic(kernel.split("<")[0]),
            "algorithmic_bytes_per_launch": k_bytes,
            "avg_launch_ms": round(k_ms, 5),
        },
    }
    if not args.no_cpu_baseline:
        out["cpu_baseline"] = cpu_baseline_isolated(base_set, nb["total"], args.cpu_seconds)
    return out


# ----------------------------------------------------------------------------- Llama-3-8B shape
def llama_config(layers: int = 32, attn: str = "pl_fused_sdpa"):
    from transformers import LlamaConfig

    cfg = LlamaConfig(hidden_size=4096, num_hidden_layers=layers, num_attention_heads=32, num_key_value_heads=8,
                      head_dim=128, intermediate_size=14336, vocab_size=128256, max_position_embeddings=8192,
                      rms_norm_eps=1e-5, rope_theta=500000.0)
    cfg._attn_implementation = attn
    return cfg


def build_llama(device, layers: int = 32, seed: int = 0, attn: str = "pl_fused_sdpa"):
    """Random-init Llama-3-8B-shaped LlamaModel, built directly on the GPU in bf16."""
    from transformers import LlamaModel

    register_attention()
    torch.manual_seed(seed)
    prev = torch.get_default_dtype()
    torch.set_default_dtype(torch.bfloat16)
    try:
        with torch.device(device):
            model = LlamaModel(llama_config(layers, attn))
    finally:
        torch.set_default_dtype(prev)
    return model.eval()


def zipf_ids(rng: np.random.Generator, n_rows: int, n_adapters: int, s: float, base_frac: float, names: list) -> list:
    w = 1.0 / np.arange(1, n_adapters + 1) ** s
    w /= w.sum()
    picks = rng.choice(n_adapters, size=n_rows, p=w)
    base = rng.random(n_rows) < base_frac
    return ["__base__" if b else names[int(p)] for p, b in zip(picks, base)]


@dataclass
class DecodeWorkload:
    model: object  # PolyLoraModel over the Llama stack
    cache: object  # transformers StaticCache with 512 filled positions + 1 free
    input_ids: torch.Tensor
    cache_position: torch.Tensor
    adapter_ids: list
    ranks: dict
    past: int
    extra: dict = field(default_factory=dict)


def decode_workload(device, layers: int = 32, batch: int = 256, past: int = 512, slots: int = 64, seed: int = 1003,
                    attn: str = "pl_fused_sdpa", kv_cache: bool = True) -> DecodeWorkload:
    from transformers import StaticCache

    from polylora_amd import PolyLoraConfig, PolyLoraModel

    rng = np.random.default_rng(seed)
    model = build_llama(device, layers, seed, attn)
    pm = PolyLoraModel(model, PolyLoraConfig(target_modules=LLAMA_TARGETS, max_gpu_adapters=slots, max_rank=64)).eval()
    names = [f"ad{i:02d}" for i in range(slots)]
    ranks = {n: int(rng.choice([8, 16, 32, 64])) for n in names}
    _log(f"decode: generating {slots} adapters")
    add_random_adapters(pm, ranks, seed=seed, device=device)
    ids = zipf_ids(rng, batch, slots, 1.1, 0.10, names)
    cfg = model.config
    gen = torch.Generator(device=device).manual_seed(seed)
    if not kv_cache:  # the LoRA launches alone (launch profiles): no KV cache, no inputs
        return DecodeWorkload(pm, None, None, None, ids, ranks, past)
    kv = StaticCache(config=cfg, max_cache_len=past + 1)
    for layer in range(cfg.num_hidden_layers):
        k = torch.randn(batch, cfg.num_key_value_heads, past, cfg.head_dim, generator=gen, device=device, dtype=torch.bfloat16)
        v = torch.randn(batch, cfg.num_key_value_heads, past, cfg.head_dim, generator=gen, device=device, dtype=torch.bfloat16)
        kv.update(k, v, layer)
    input_ids = torch.randint(0, cfg.vocab_size, (batch, 1), generator=gen, device=device)
    cache_position = torch.tensor([past], device=device)
    return DecodeWorkload(pm, kv, input_ids, cache_position, ids, ranks, past)


def _reset_kv(wl: DecodeWorkload) -> None:
    for layer in wl.cache.layers:
        layer.cumulative_length.fill_(wl.past)


def _decode_step(wl: DecodeWorkload, lora: bool):
    _reset_kv(wl)
    return wl.model.base_model(input_ids=wl.input_ids, past_key_values=wl.cache, cache_position=wl.cache_position,
                               use_cache=True).last_hidden_state


def decode_lora_bytes(pm, adapter_ids: list, rows: int) -> dict:
    """Algorithmic bytes of one decode step's 224 shrink+expand pairs: active X, Y RMW, unique A+B once."""
    base_id = pm.config.base_adapter_id
    active = [a for a in adapter_ids if a != base_id]
    uniq = sorted(set(active))
    es = 2
    total = xy = ab = flops = 0
    for spec in pm.module_specs:
        for aid in uniq:
            ab += es * _rank_of(pm, aid, spec.name) * (spec.in_features + spec.out_features)
        t_act = sum(1 for a in active if _rank_of(pm, a, spec.name) > 0)
        xy += es * t_act * spec.in_features + 2 * es * t_act * spec.out_features
        flops += sum(2 * _rank_of(pm, a, spec.name) * (spec.in_features + spec.out_features) for a in active)
    total = xy + ab
    return {"total": total, "xy": xy, "ab": ab, "flops": flops, "active_rows": len(active), "distinct": len(uniq)}


@dataclass
class LaunchEntry:
    """One launch of a forward's LoRA sequence: what it serves and how to issue it."""

    label: str  # launch type, e.g. "q/k/v stacked shrink"
    part: str  # "shrink", "expand" or "fused"
    modules: list  # wrapped Linear names served
    fn: object  # issues the launch
    owner: object  # the launch object (shared by a shrink and its expand)


_SIBLINGS = {"q_proj": ("q_proj", "k_proj", "v_proj"), "gate_proj": ("gate_proj", "up_proj")}


def forward_launch_sequence(pm, plan, xs: dict, T: int, gen) -> list:
    """The LoRA launches of one forward, in MultiLoraLinear's order, without the base model.

    Sibling Linears that read the same input (q/k/v, gate/up) share one
    stacked launch, as MultiLoraLinear does once it has seen a forward.  Where
    the plan suits the fused kernel each set takes one pl_lora_fused(_stacked)
    launch; decode-sized batches one pl_lora_decode_stacked launch (split
    shrink and expand with the hand-off inside the launch); otherwise one
    stacked shrink and one stacked expand.  Every module type writes its own
    y, so siblings in one launch never share an output.
    """
    from polylora_amd import layers, sgmv

    cache = pm.adapter_cache
    device = cache.device
    by_name = {s.name: s for s in pm.module_specs}
    leaf_ys = {}
    for s in pm.module_specs:
        leaf = s.name.rsplit(".", 1)[-1]
        if leaf not in leaf_ys:
            leaf_ys[leaf] = torch.randn(T, s.out_features, generator=gen, device=device, dtype=torch.bfloat16)
    out = []
    for s in pm.module_specs:
        parent, leaf = s.name.rsplit(".", 1)
        if leaf in ("k_proj", "v_proj", "up_proj"):
            continue
        group = _SIBLINGS.get(leaf, (leaf,))
        names = [f"{parent}.{g}" for g in group if f"{parent}.{g}" in by_name]
        tag = "/".join(n.rsplit(".", 1)[-1].replace("_proj", "") for n in names)
        tag += " stacked" if len(names) > 1 else ""
        k = by_name[names[0]].in_features
        outs = [leaf_ys[n.rsplit(".", 1)[-1]] for n in names]
        if sgmv.fused_ok(plan, cache, k):
            f = (FusedLaunch(xs[k], outs[0], cache, names[0], plan) if len(names) == 1
                 else StackedFusedLaunch(xs[k], outs, cache, names, plan))
            out.append(LaunchEntry(f"{tag} fused", "fused", names, f, f))
            continue
        if T < layers.OVERLAP_MIN_TOKENS and cache.decode_handoff and sgmv.decode_ok(plan):
            d = DecodeLaunch(xs[k], outs, cache, names, plan)
            out.append(LaunchEntry(f"{tag} decode", "fused", names, d, d))
            continue
        st = StackedLaunch(xs[k], outs, cache, names, plan)
        out.append(LaunchEntry(f"{tag} shrink", "shrink", names, st.shrink, st))
        out.append(LaunchEntry(f"{tag} expand", "expand", names, st.expand, st))
    return out


def launch_bytes(pm, modules: list, part: str, adapter_ids: list, lens: list) -> int:
    """Algorithmic HBM bytes of one launch serving `modules` over a batch (bf16).

    shrink: x once for the tokens of rows whose adapter has a rank for one of
    the modules, plus each distinct adapter's A once per module; expand: y
    read and written for the tokens the module adapts, plus each distinct
    adapter's B once per module; fused: both.
    """
    base_id = pm.config.base_adapter_id
    specs = {s.name: s for s in pm.module_specs}
    rows = [(a, int(n)) for a, n in zip(adapter_ids, lens) if a != base_id and int(n) > 0]
    uniq = sorted({a for a, _ in rows})
    k = specs[modules[0]].in_features
    total = 0
    if part in ("shrink", "fused"):
        total += 2 * k * sum(n for a, n in rows if any(_rank_of(pm, a, m) > 0 for m in modules))
        total += sum(2 * _rank_of(pm, a, m) * k for m in modules for a in uniq)
    if part in ("expand", "fused"):
        for m in modules:
            nout = specs[m].out_features
            total += 4 * nout * sum(n for a, n in rows if _rank_of(pm, a, m) > 0)
            total += sum(2 * _rank_of(pm, a, m) * nout for a in uniq)
    return total


def time_lora_ops(pm, adapter_ids: list, tokens_per_row: int, seq_lens: torch.Tensor, reps: int, seed: int = 0) -> dict:
    """Every wrapped Linear's shrink+expand over one batch, launched back to back without the base model."""
    from polylora_amd import sgmv

    device = pm.adapter_cache.device
    cache = pm.adapter_cache
    row_slot = cache.ensure_resident(adapter_ids)
    distinct = len({a for a in adapter_ids if a != pm.config.base_adapter_id})
    plan = sgmv.SgmvPlan(row_slot, seq_lens, tokens_per_row, cache.num_slots, distinct_slots=distinct)
    T = len(adapter_ids) * tokens_per_row
    gen = torch.Generator(device=device).manual_seed(seed)
    shapes = sorted({(s.in_features, s.out_features) for s in pm.module_specs})
    xs = {k: torch.randn(T, k, generator=gen, device=device, dtype=torch.bfloat16) for k, _ in shapes}
    ys = {n: torch.randn(T, n, generator=gen, device=device, dtype=torch.bfloat16) for _, n in shapes}
    launches = [SgmvLaunch(xs[s.in_features], ys[s.out_features], cache, s.name, plan) for s in pm.module_specs]
    per_type = {}
    for key in sorted({s.name.rsplit(".", 1)[-1] for s in pm.module_specs}):
        sel = [l for l, s in zip(launches, pm.module_specs) if s.name.rsplit(".", 1)[-1] == key]
        per_type[key] = [round(1e3 * time_launches([l.shrink for l in sel], reps) / len(sel), 2),
                         round(1e3 * time_launches([l.expand for l in sel], reps) / len(sel), 2)]
    entries = forward_launch_sequence(pm, plan, xs, T, gen)
    lens = [min(int(v), tokens_per_row) for v in seq_lens.cpu().tolist()]
    seq_bytes = sum(launch_bytes(pm, e.modules, e.part, adapter_ids, lens) for e in entries)
    seq = [e.fn for e in entries]
    stacks = list({id(e.owner): e.owner for e in entries if e.part != "fused"}.values())
    fused = [e.fn for e in entries if e.part == "fused"]
    total_ms = time_launches(seq, reps)
    sh_ms = time_launches([st.shrink for st in stacks], reps) if stacks else 0.0
    ex_ms = time_launches([st.expand for st in stacks], reps) if stacks else 0.0
    fu_ms = time_launches(fused, reps) if fused else 0.0
    return {"pairs_ms": total_ms, "shrink_ms": sh_ms, "expand_ms": ex_ms, "fused_ms": fu_ms, "per_type_us": per_type,
            "group_tokens": plan.group_tokens, "launches": len(seq), "fused_launches": len(fused), "bytes": seq_bytes}


def cpu_baseline_layer(pm, adapter_ids: list, budget_s: float, lens: list | None = None, seq: int = 1,
                       seed: int = 1003) -> dict:
    """The reference fallback (oracle restatement of layers.py:112-134) for one decoder layer's 7 LoRA ops.

    Same adapters, slots and row -> slot map as the GPU run; x and the base
    outputs are random bf16 of the run's shapes ([rows, seq, in] and
    [rows, seq, out]) with the run's valid lengths (`lens`, default: all
    `seq` tokens).  A full 8B forward on the host is out of reach, so the
    LoRA ops of one layer are timed and the per-forward figure scales them
    by the layer count.
    """
    from oracle.lora import dense_slot_tensors, reference_forward

    cache = pm.adapter_cache
    base_id = pm.config.base_adapter_id
    rows = len(adapter_ids)
    widx = torch.tensor([0 if a == base_id else cache.adapter_to_slot[a] for a in adapter_ids])
    lens = [seq] * rows if lens is None else [int(v) for v in lens]
    seq_lens = torch.tensor(lens, dtype=torch.int32)
    layer0 = [s for s in pm.module_specs if ".0." in f".{s.name}."][:7]
    gen = torch.Generator().manual_seed(seed)
    ops, xs = [], {}
    for spec in layer0:
        per_slot = [None] * cache.num_slots
        for slot, aid in enumerate(cache.slot_to_adapter):
            if slot == 0 or aid is None:
                continue
            w = pm.adapter_store.adapters[aid].layers.get(spec.name)
            if w is not None:  # stored A [in, r], B [r, out] -> PEFT lora_A [r, in], lora_B [out, r], alpha
                per_slot[slot] = (w.A.t(), w.B.t(), float(w.scale) * int(w.rank))
        A, B, ranks, scales = dense_slot_tensors(per_slot, spec.in_features, spec.out_features,
                                                 pm.config.max_rank, torch.bfloat16)
        if spec.in_features not in xs:  # one input per width, as the layer's siblings share theirs
            xs[spec.in_features] = torch.randn(rows, seq, spec.in_features, generator=gen, dtype=torch.bfloat16)
        base = torch.randn(rows, seq, spec.out_features, generator=gen, dtype=torch.bfloat16)
        ops.append((xs[spec.in_features], base, A, B, ranks, scales))
    threads = torch.get_num_threads()
    reps = 0
    t0 = time.perf_counter()
    while True:
        for x, base, A, B, ranks, scales in ops:
            reference_forward(x, base, seq_lens, widx, A, B, ranks, scales)
        reps += 1
        el = time.perf_counter() - t0
        if el >= budget_s:
            break
    per_layer = el / reps
    layers = pm.base_model.config.num_hidden_layers
    valid = sum(min(n, seq) for n in lens)
    return _cpu_record(round(valid / (per_layer * layers), 3), "tokens/s (LoRA ops only)", threads,
                       f"{reps} passes over one layer's 7 LoRA ops ({rows} rows x {seq} positions, {valid} valid "
                       f"tokens, {int((widx > 0).sum())} rows with an adapter) of the fallback loop, "
                       f"{per_layer * 1e3:.1f} ms each, scaled by {layers} layers; torch {threads} threads")


def _graph_ms(fn, reps: int) -> float:
    """Capture fn() in a HIP graph (after eager warm-up) and time replays."""
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        for _ in range(2):
            fn()
    torch.cuda.current_stream().wait_stream(s)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        fn()
    for _ in range(3):
        g.replay()
    torch.cuda.synchronize()
    t0 = torch.cuda.Event(enable_timing=True)
    t1 = torch.cuda.Event(enable_timing=True)
    t0.record()
    progress = _Progress("graph replays")
    for i in range(reps):
        progress.tick(f"replay {i}/{reps}")
        g.replay()
    t1.record()
    torch.cuda.synchronize()
    return t0.elapsed_time(t1) / reps


def _eager_ms(fn, reps: int) -> float:
    for _ in range(2):
        fn()
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    progress = _Progress("eager steps")
    for i in range(reps):
        progress.tick(f"step {i}/{reps}")
        fn()
    torch.cuda.synchronize()
    return (time.perf_counter() - t0) / reps * 1e3


def decode_graph_trace(args) -> int:
    """Replay the decode step's HIP graph without adapters, then with them, for a kernel trace.

    Each graph is warmed up and captured as in _graph_ms and replayed twice
    (one burst of kernels), then, after a pause, `--profile-passes` times (the
    timed burst); pauses of 0.3 s separate the bursts, so that
    reduce_graph_trace can tell them apart in the trace.
    """
    from polylora_amd.context import use_lora_context

    device = torch.device("cuda", 0)
    wl = decode_workload(device, layers=args.decode_layers)
    pm = wl.model
    B = len(wl.adapter_ids)
    ctx = pm.prepare_lora_context(wl.adapter_ids, None, B, 1, device)

    def lora_step():
        with use_lora_context(ctx):
            return _decode_step(wl, True)

    reps = args.profile_passes
    with torch.inference_mode():
        for name, fn in (("base", lambda: _decode_step(wl, False)), ("lora", lora_step)):
            s = torch.cuda.Stream()
            s.wait_stream(torch.cuda.current_stream())
            with torch.cuda.stream(s):
                for _ in range(2):
                    fn()
            torch.cuda.current_stream().wait_stream(s)
            torch.cuda.synchronize()
            g = torch.cuda.CUDAGraph()
            with torch.cuda.graph(g):
                fn()
            for _ in range(2):
                g.replay()
            torch.cuda.synchronize()
            time.sleep(0.3)
            t0 = torch.cuda.Event(enable_timing=True)
            t1 = torch.cuda.Event(enable_timing=True)
            t0.record()
            for _ in range(reps):
                g.replay()
            t1.record()
            torch.cuda.synchronize()
            _log(f"graph trace: {name} step {t0.elapsed_time(t1) / reps:.3f} ms per replay")
            time.sleep(0.3)
    print(json.dumps({"graph_trace": "decode", "replays": reps}), flush=True)
    return 0


def reduce_graph_trace(args) -> int:
    """Per-kernel time of one decode step replay, without and with adapters, from a kernel trace.

    The trace's kernels are cut into bursts at idle stretches of over 100 ms:
    per graph, base first, a warm-up burst and then the burst of its
    `--profile-passes` timed replays, so the timed bursts are the third and
    the first from the end.
    """
    import csv
    from collections import defaultdict

    with open(args.trace, newline="") as f:
        rows = sorted((int(r["Start_Timestamp"]), int(r["End_Timestamp"]), r["Kernel_Name"]) for r in csv.DictReader(f))
    bursts, cur = [], rows[:1]
    for r in rows[1:]:
        if r[0] - cur[-1][1] > 100_000_000:
            bursts.append(cur)
            cur = [r]
        else:
            cur.append(r)
    bursts.append(cur)
    n = args.profile_passes
    if len(bursts) < 3 or len(bursts[-3]) % n or len(bursts[-1]) % n:
        print("the trace does not end with a --graph-trace run's bursts", file=sys.stderr)
        return 1
    steps = {"base": bursts[-3], "lora": bursts[-1]}
    per = {}
    for name, b in steps.items():
        us, cnt = defaultdict(float), defaultdict(int)
        for s, e, k in b:
            key = k.split("(")[0].split("<")[0].strip().removeprefix("void ")[:60]
            us[key] += (e - s) / 1e3 / n
            cnt[key] += 1
        idle = sum(max(0, s1 - e0) for (_, e0, _), (s1, _, _) in zip(b, b[1:])) / 1e3 / n
        per[name] = {"wall_ms": (b[-1][1] - b[0][0]) / 1e6 / n, "busy_ms": sum(us.values()) / 1e3,
                     "idle_ms": idle / 1e3, "kernels": len(b) / n, "us": us, "count": cnt}
    lines = ["| kernel | base (us per step) | with adapters (us per step) | difference | launches per step (base / with) |",
             "|---|---|---|---|---|"]
    keys = sorted(set(per["base"]["us"]) | set(per["lora"]["us"]),
                  key=lambda k: -(per["base"]["us"].get(k, 0.0) + per["lora"]["us"].get(k, 0.0)))
    for k in keys:
        b, l = per["base"]["us"].get(k, 0.0), per["lora"]["us"].get(k, 0.0)
        lines.append(f"| {k} | {b:.1f} | {l:.1f} | {l - b:+.1f} | {per['base']['count'].get(k, 0) // n} / "
                     f"{per['lora']['count'].get(k, 0) // n} |")
    lines.append("")
    for name in ("base", "lora"):
        p = per[name]
        lines.append(f"{name}: {p['wall_ms']:.3f} ms per replay from first kernel start to last kernel end, "
                     f"{p['busy_ms']:.3f} ms of kernel time, {p['idle_ms']:.3f} ms between kernels, "
                     f"{p['kernels']:.0f} kernels.")
    print("\n".join(lines))
    return 0


def operator_decode_layer_tensors(pm, adapter_ids: list) -> tuple:
    """One decode layer's seven wrapped Linears in the reference cache's own layout (cache.py:37-58).

    Per module A [65, K, 64] and B [65, 64, N] bf16 (slot 0 the base adapter
    with rank 0, the decode batch's 64 adapters at their slots and ranks,
    zero past each rank), ranks [65] int32 and scales [65] fp32, and the
    Linear's x [256, 1, K] and base output [256, 1, N].  Weight values are
    random: no timing depends on them.  Returns (modules, seq_lens,
    weight_indices) with modules a list of (module name, A, B, ranks, scales, x, y).
    """
    cache = pm.adapter_cache
    device = cache.device
    B = len(adapter_ids)
    S, R = cache.num_slots, cache.config.max_rank
    gen = torch.Generator(device=device).manual_seed(7)
    widx = cache.ensure_resident(adapter_ids)
    seq = torch.ones(B, dtype=torch.int32, device=device)
    layer0 = [s for s in pm.module_specs if re.search(r"(^|\.)layers\.0\.", s.name)]
    assert len(layer0) == 7, [s.name for s in pm.module_specs[:8]]
    mods = []
    for spec in layer0:
        K, N = spec.in_features, spec.out_features
        ranks = torch.zeros(S, dtype=torch.int32)
        for slot in range(1, S):
            aid = cache.slot_to_adapter[slot]
            if aid is not None:
                ranks[slot] = _rank_of(pm, aid, spec.name)
        rk = ranks.to(device)
        keep = torch.arange(R, device=device).view(1, R) < rk.view(S, 1)
        A = (torch.randn(S, K, R, generator=gen, device=device) * 0.02 * keep.view(S, 1, R)).bfloat16()
        Bw = (torch.randn(S, R, N, generator=gen, device=device) * 0.02 * keep.view(S, R, 1)).bfloat16()
        sc = torch.where(rk > 0, 2.0, 0.0).float()
        x = torch.randn(B, 1, K, generator=gen, device=device).bfloat16()
        y = torch.randn(B, 1, N, generator=gen, device=device).bfloat16()
        mods.append((spec.name, A, Bw, rk, sc, x, y))
    return mods, seq, widx


def operator_api_decode_layer(pm, adapter_ids: list, reps: int = 30) -> dict:
    """One decode layer's seven wrapped Linears through the reference's operator API.

    As MultiLoraLinear calls it (layers.py:42-58: sgmv_lora_a_fwd then
    sgmv_lora_b_fwd per Linear) on operator_decode_layer_tensors.  Times one
    layer on its first call (the plan built, each module's used adapters
    packed), its second (the rest packed), then layers back to back with the
    plan and packed weights kept, and the same with nothing kept (every call
    builds the plan and repacks the adapters its rows use).
    """
    from polylora_amd import refop_cache, sgmv

    mods, seq, widx = operator_decode_layer_tensors(pm, adapter_ids)

    def layer():
        for _, A, Bw, rk, sc, x, y in mods:
            tmp = sgmv.sgmv_lora_a_fwd(x, A, seq, widx, rk)
            sgmv.sgmv_lora_b_fwd(tmp, Bw, seq, widx, rk, sc, y)

    def timed(n: int) -> float:
        torch.cuda.synchronize()
        t0, t1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        t0.record()
        for _ in range(n):
            layer()
        t1.record()
        torch.cuda.synchronize()
        return t0.elapsed_time(t1) / n

    try:
        refop_cache.configure()
        first = timed(1)
        second = timed(1)
        timed(2)
        kept = timed(reps)
        stats = dict(refop_cache.CACHE.stats)
        refop_cache.configure(max_bytes=0, max_plans=0)
        timed(2)
        uncached = timed(reps)
    finally:
        refop_cache.configure()
    del mods
    return {"first_call_ms": round(first, 4), "second_call_ms": round(second, 4), "kept_ms": round(kept, 4),
            "nothing_kept_ms": round(uncached, 4), "cache_stats": stats,
            "config": "7 wrapped Linears of one Llama-3-8B layer, 256 decode rows, reference layout [65, K, 64] / "
                      "[65, 64, N] bf16, host calls back to back (14 operator calls per layer)"}


def run_decode(args) -> dict:
    from polylora_amd.context import use_lora_context

    device = torch.device("cuda", 0)
    t_build = time.perf_counter()
    wl = decode_workload(device, layers=args.decode_layers)
    pm = wl.model
    B = len(wl.adapter_ids)
    ctx = pm.prepare_lora_context(wl.adapter_ids, None, B, 1, device)  # uploads the step's adapters
    torch.cuda.synchronize()
    _log(f"decode: model + adapters ready in {time.perf_counter() - t_build:.1f}s")
    nb = decode_lora_bytes(pm, wl.adapter_ids, B)
    out = {"rows": B, "layers": args.decode_layers, "distinct_adapters": nb["distinct"], "active_rows": nb["active_rows"],
           "lora_bytes_per_step": nb["total"], "lora_adapter_bytes_per_step": nb["ab"], "lora_flops_per_step": nb["flops"]}

    with torch.no_grad():
        op = operator_api_decode_layer(pm, wl.adapter_ids)
    per_layer_bytes = nb["total"] / args.decode_layers
    op["gbs_kept"] = round(per_layer_bytes / (op["kept_ms"] * 1e-3) / 1e9, 1)
    op["bytes_note"] = "GB/s counts the layer's LoRA bytes (x read per Linear, y read and written, A and B once)"
    out["operator_api_layer"] = op
    _log(f"decode: operator API layer kept {op['kept_ms']} ms, nothing kept {op['nothing_kept_ms']} ms")

    def base_step():
        return _decode_step(wl, False)

    def lora_step():
        with use_lora_context(ctx):
            return _decode_step(wl, True)

    with torch.inference_mode():
        kt = time_lora_ops(pm, wl.adapter_ids, 1, torch.ones(B, dtype=torch.int32, device=device), reps=5)
        kern_ms = kt["pairs_ms"]
        out["lora_bytes_per_step"] = kt["bytes"]  # x read once per stacked launch, as the launches do
        out["lora_bytes_per_step_x_per_module"] = nb["total"]
        out["plan_group_tokens"] = kt["group_tokens"]
        out["lora_kernels_ms"] = round(kern_ms, 4)
        out["operator_api_layer"]["native_layer_ms"] = round(kern_ms / args.decode_layers, 4)
        out["lora_kernels_gbs"] = round(kt["bytes"] / (kern_ms * 1e-3) / 1e9, 1)
        out["lora_kernels_pct_hbm"] = round(100 * kt["bytes"] / (kern_ms * 1e-3) / 1e9 / HBM_PEAK_GBS, 2)
        out["roofline"] = sequence_roofline("one decode step's LoRA launches (pl_decode_fused: split-K shrink and "
                                            "expand with the hand-off inside each launch)",
                                            kt["bytes"], kern_ms, kt["launches"], "decode")
        out["per_op_us_shrink_expand"] = kt["per_type_us"]
        out["lora_kernel_launches_per_step"] = kt["launches"]
        out["lora_kernels_timing"] = ("the forward's launch sequence (one launch each for q/k/v stacked, o, "
                                      "gate/up stacked and down, shrink and expand inside it) back to back without "
                                      "the base model")
        # the same sequence as separate shrink and expand launches, for comparison
        pm.adapter_cache.decode_handoff = False
        try:
            ks = time_lora_ops(pm, wl.adapter_ids, 1, torch.ones(B, dtype=torch.int32, device=device), reps=5)
        finally:
            pm.adapter_cache.decode_handoff = True
        out["lora_kernels_ms_split_pairs"] = round(ks["pairs_ms"], 4)
        out["lora_kernel_launches_split_pairs"] = ks["launches"]
        out["lora_kernels_split_pairs_shrink_ms"] = round(ks["shrink_ms"], 4)
        out["lora_kernels_split_pairs_expand_ms"] = round(ks["expand_ms"], 4)
        if not args.no_cpu_baseline:
            out["cpu_baseline"] = cpu_baseline_layer(pm, wl.adapter_ids, args.cpu_seconds)
        _log(f"decode: kernels {out['lora_kernels_gbs']} GB/s")
        e_base = _eager_ms(base_step, args.decode_steps)
        e_lora = _eager_ms(lora_step, args.decode_steps)
        out["eager_ms_base"] = round(e_base, 3)
        out["eager_ms_lora"] = round(e_lora, 3)
        out["eager_tokens_per_s_lora"] = round(B / e_lora * 1e3, 1)
        out["eager_tokens_per_s_base"] = round(B / e_base * 1e3, 1)
        _log(f"decode: eager base {e_base:.2f} ms, lora {e_lora:.2f} ms")
        try:
            g_base = _graph_ms(base_step, args.decode_steps)
            g_lora = _graph_ms(lora_step, args.decode_steps)
            out["graph_ms_base"] = round(g_base, 3)
            out["graph_ms_lora"] = round(g_lora, 3)
            out["tokens_per_s_lora"] = round(B / g_lora * 1e3, 1)
            out["tokens_per_s_base"] = round(B / g_base * 1e3, 1)
            out["ratio_lora_to_base"] = round(g_base / g_lora, 4)
            # the base step is far from its own floor (attention over the 512-token cache
            # dominates it), which flatters the ratio: also state it against that floor
            cfg = pm.base_model.config
            layer_bytes = 2 * sum(p.numel() for n, p in pm.base_model.named_parameters() if "embed" not in n)
            kv_bytes = 2 * cfg.num_hidden_layers * 2 * B * cfg.num_key_value_heads * (wl.past + 1) * cfg.head_dim
            floor_ms = (layer_bytes + kv_bytes) / (HBM_PEAK_GBS * 1e9) * 1e3
            out["base_step_floor_ms"] = round(floor_ms, 3)
            out["ratio_at_base_floor"] = round(floor_ms / (floor_ms + g_lora - g_base), 4)
            out["ratio_note"] = ("the base step runs far above its floor (its weights and KV cache read once at 8 TB/s); "
                                 "ratio_at_base_floor adds the measured LoRA time to that floor instead")
            out["timing"] = "HIP graph replay of one decode step"
            out["attention"] = "torch SDPA fused kernel, " + ("native GQA" if _GQA_NATIVE["ok"] else "K/V expanded to 32 heads")
            _log(f"decode: graph base {g_base:.2f} ms, lora {g_lora:.2f} ms")
        except Exception as exc:  # noqa: BLE001 - report and keep the eager numbers
            out["graph_error"] = f"{type(exc).__name__}: {str(exc)[:300]}"
            out["tokens_per_s_lora"] = out["eager_tokens_per_s_lora"]
            out["tokens_per_s_base"] = out["eager_tokens_per_s_base"]
            out["ratio_lora_to_base"] = round(e_base / e_lora, 4)
            out["timing"] = "eager wall clock (graph capture failed)"
    if getattr(args, "keep_model", False):
        out["_model"] = pm
    del wl, ctx
    torch.cuda.empty_cache()
    return out


def prefill_bytes(pm, adapter_ids: list, lens: list) -> dict:
    """Algorithmic bytes and flops of one prefill forward's 224 shrink+expand pairs over the valid tokens.

    "total" reads x once per module; "shared_x" reads it once per set of
    sibling Linears fed the same input (q/k/v, gate/up), as one stacked launch
    does.
    """
    es = 2
    xy = ab = flops = repeat_x = 0
    uniq = sorted(set(adapter_ids))
    for spec in pm.module_specs:
        sibling = spec.name.rsplit(".", 1)[-1] in ("k_proj", "v_proj", "up_proj")
        for aid, n in zip(adapter_ids, lens):
            xy += es * n * spec.in_features + 2 * es * n * spec.out_features
            repeat_x += es * n * spec.in_features if sibling else 0
            flops += 2 * n * _rank_of(pm, aid, spec.name) * (spec.in_features + spec.out_features)
        for aid in uniq:
            ab += es * _rank_of(pm, aid, spec.name) * (spec.in_features + spec.out_features)
    return {"total": xy + ab, "shared_x": xy + ab - repeat_x, "flops": flops}


def run_prefill(args, pm) -> dict:
    """Prefill: 8 adapters (4 x r16, 4 x r32), B=32, S=1024, right-padded, lengths U[512,1024], 4 rows per adapter.

    The base model runs causal attention without the padding mask: rows are
    right-padded, so every valid token attends exactly the same keys, and
    torch's flash kernel (no masks) takes the step.  LoRA lengths come from
    the mask, as in the reference (model.py:99-104).
    """
    from polylora_amd.context import use_lora_context

    device = torch.device("cuda", 0)
    rng = np.random.default_rng(1004)
    names = [f"pf{i}" for i in range(8)]
    add_random_adapters(pm, {n: (16 if i < 4 else 32) for i, n in enumerate(names)}, seed=1004, device=device)
    B, S = 32, 1024
    lens = rng.integers(512, S + 1, size=B)
    adapter_ids = [names[i // 4] for i in range(B)]
    mask = (torch.arange(S)[None, :] < torch.as_tensor(lens)[:, None]).long().to(device)
    ids = torch.randint(0, pm.base_model.config.vocab_size, (B, S), device=device)
    ctx = pm.prepare_lora_context(adapter_ids, mask, B, S, device)
    nb = prefill_bytes(pm, adapter_ids, [int(v) for v in lens])
    out = {"rows": B, "seq": S, "valid_tokens": int(lens.sum()), "lora_bytes_per_forward": nb["shared_x"],
           "lora_bytes_per_forward_x_per_module": nb["total"], "lora_flops_per_forward": nb["flops"]}
    with torch.inference_mode():
        kt = time_lora_ops(pm, adapter_ids, S, torch.as_tensor(lens, dtype=torch.int32, device=device), reps=2)
        kern_ms = kt["pairs_ms"]
        out["plan_group_tokens"] = kt["group_tokens"]
        out["lora_kernels_ms"] = round(kern_ms, 3)
        # x read once per set of sibling Linears, as the stacked launches do
        out["lora_kernels_gbs"] = round(nb["shared_x"] / (kern_ms * 1e-3) / 1e9, 1)
        out["lora_kernels_pct_hbm"] = round(100 * nb["shared_x"] / (kern_ms * 1e-3) / 1e9 / HBM_PEAK_GBS, 2)
        out["lora_kernels_gbs_x_per_module"] = round(nb["total"] / (kern_ms * 1e-3) / 1e9, 1)
        out["lora_kernels_mfma_tflops"] = round(nb["flops"] / (kern_ms * 1e-3) / 1e12, 2)
        out["lora_kernels_pct_mfma_bf16"] = round(100 * nb["flops"] / (kern_ms * 1e-3) / 1e12 / MFMA_BF16_PEAK_TFLOPS, 3)
        out["roofline"] = sequence_roofline("one prefill forward's LoRA launches (pl_lora_fused_tile)",
                                            nb["shared_x"], kern_ms, kt["launches"], "prefill")
        out["lora_kernels_shrink_ms"] = round(kt["shrink_ms"], 3)
        out["lora_kernels_expand_ms"] = round(kt["expand_ms"], 3)
        out["lora_kernels_fused_ms"] = round(kt["fused_ms"], 3)
        out["lora_kernel_launches"] = kt["launches"]
        out["lora_fused_launches"] = kt["fused_launches"]

        def base_fwd():
            return pm.base_model(input_ids=ids, use_cache=False).last_hidden_state

        def lora_fwd():
            with use_lora_context(ctx):
                return pm.base_model(input_ids=ids, use_cache=False).last_hidden_state

        out["ms_base"] = round(_eager_ms(base_fwd, 3), 2)
        out["ms_lora"] = round(_eager_ms(lora_fwd, 3), 2)
        out["tokens_per_s_base"] = round(int(lens.sum()) / out["ms_base"] * 1e3, 1)
        out["tokens_per_s_lora"] = round(int(lens.sum()) / out["ms_lora"] * 1e3, 1)
        out["ratio_lora_to_base"] = round(out["ms_base"] / out["ms_lora"], 4)
        out["timing"] = "eager wall clock of one forward (valid tokens per second)"
    if not args.no_cpu_baseline:
        _log("prefill: CPU baseline (one layer's LoRA ops at the prefill shapes)")
        out["cpu_baseline"] = cpu_baseline_layer(pm, adapter_ids, args.cpu_seconds, lens=lens, seq=S, seed=1004)
    _log(f"prefill: kernels {out['lora_kernels_gbs']} GB/s, base {out['ms_base']} ms, lora {out['ms_lora']} ms")
    return out


def run_churn(args) -> dict:
    """Adapter churn: 1024 rank-16 adapters on all 7 targets, 32 GPU slots, batch 128, Zipf(0.9) ids.

    Each step's rows are split, when the step starts, into sub-batches of at
    most `--churn-sub-distinct` distinct adapters (at most 32, the slot count:
    the reference raises beyond it, cache.py:65-66): the adapters resident
    then first, each sub-batch taking every row of its adapters (see
    sub_batches).  Every sub-batch is one
    forward of one new token per row (empty KV cache), preceded by the loads
    its adapters need.  Loads go to the side stream, into the arena's spare
    regions, so they copy while the forward that reads the slots' current
    regions computes; a slot's table row switches to its new region after
    that forward.  The host never waits for the GPU,
    so it queues the next sub-batch's loads and forward while the device is
    still copying and computing.  Every adapter of the catalog is its own
    84 MB slot image (the store's one host copy of it; 86 GB for 1024
    adapters), page-locked up to `--churn-pinned-gib` and pageable beyond
    (loaded through the staging ring).  Compared with the same rows restricted to 32 resident adapters
    (no loads).
    """
    from transformers import DynamicCache

    from polylora_amd import PolyLoraConfig, PolyLoraModel

    device = torch.device("cuda", 0)
    rng = np.random.default_rng(1005)
    model = build_llama(device, args.decode_layers, seed=1005)
    pm = PolyLoraModel(model, PolyLoraConfig(target_modules=LLAMA_TARGETS, max_gpu_adapters=32, max_rank=16)).eval()
    # page-locked host memory is limited per process (about 65 GiB on MI355X hosts measured
    # so far): the Zipf head of the catalog is pinned, the tail stays pageable (its loads
    # go through the pinned staging ring)
    pm.adapter_store.pinned_bytes_limit = int(args.churn_pinned_gib * (1 << 30))
    n_cat = args.churn_catalog
    t_cat = time.perf_counter()
    catalog = random_image_catalog(pm, n_cat, rank=16, seed=1005)
    t_cat = time.perf_counter() - t_cat
    store = pm.adapter_store
    w = 1.0 / np.arange(1, n_cat + 1) ** 0.9
    w /= w.sum()
    B = 128
    draws = [rng.choice(n_cat, size=B, p=w) for _ in range(args.churn_steps + 2)]
    steps = [[catalog[int(i)] for i in d] for d in draws]

    limit = args.churn_sub_distinct

    seen = Counter()  # rows per adapter in the steps split so far: the harness's popularity estimate

    def sub_batches(ids):
        """A step's rows cut into sub-batches of at most `limit` distinct adapters.

        The adapters already resident when the step starts come first (no
        loads), then the step's others from the least to the most often seen
        in earlier steps (ties in order of first appearance), so the step ends
        with its most popular adapters resident for the next one; a sub-batch
        takes every row of its adapters (rows keep their order).  Against
        cutting the rows in order, this loads fewer adapters (an adapter is
        never met again in a later sub-batch of the step) and runs fewer
        forwards (ceil(distinct / limit) per step); against taking the others
        in order of first appearance, 74.9 instead of 81.3 loads per step for
        this workload under the reference's LRU policy (cache.py:97-117).
        """
        resident_now = pm.adapter_cache.adapter_to_slot
        distinct = list(dict.fromkeys(ids))
        rest = sorted((a for a in distinct if a not in resident_now), key=lambda a: seen[a])
        order = [a for a in distinct if a in resident_now] + rest
        seen.update(ids)
        out = []
        for i in range(0, len(order), limit):
            chunk = set(order[i : i + limit])
            out.append([a for a in ids if a in chunk])
        return out

    hot = catalog[:32]

    def resident(sub):
        """The same sub-batch with its distinct adapters renamed to resident ones (no loads)."""
        names = {}
        for a in sub:
            if a not in names:
                names[a] = hot[len(names)]
        return [names[a] for a in sub]

    vocab = pm.base_model.config.vocab_size
    gen = torch.Generator(device=device).manual_seed(1005)

    def run(batches, split=False):
        """Forward every sub-batch (or, with split, every step cut at its start); (s, tokens, loads, sub-batches)."""
        n_tok = 0
        loads0 = pm.adapter_cache.loads
        done = []
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        progress = _Progress("churn")
        with torch.inference_mode():
            for i, item in enumerate(batches):
                progress.tick(f"{'step' if split else 'sub-batch'} {i + 1}/{len(batches)}")
                for sub in sub_batches(item) if split else [item]:
                    x = torch.randint(0, vocab, (len(sub), 1), generator=gen, device=device)
                    # a (fresh) KV cache, as in decoding; without one, transformers
                    # checks position_ids for packed sequences, which waits for the
                    # GPU every forward
                    pm(input_ids=x, adapter_ids=sub, past_key_values=DynamicCache(config=pm.base_model.config),
                       use_cache=True)
                    n_tok += len(sub)
                    done.append(sub)
        torch.cuda.synchronize()
        return time.perf_counter() - t0, n_tok, pm.adapter_cache.loads - loads0, done

    _, _, _, warm_batches = run(steps[:2], split=True)
    churn_s, n_tok, loads, churn_batches = run(steps[2:], split=True)
    # compute alone: the same sub-batches, every adapter resident
    run([resident(sub) for sub in warm_batches])
    comp_s, _, comp_loads, _ = run([resident(sub) for sub in churn_batches])
    # the all-resident hot set: the same rows with ids folded onto 32 adapters, whole 128-row steps
    hot_steps = [[hot[int(i) % 32] for i in d] for d in draws]
    run(hot_steps[:2])
    hot_s, hot_tok, hot_loads, _ = run(hot_steps[2:])
    img = store.adapters[catalog[0]].image.data
    image_bytes = int(img.numel())
    pinned_images = sum(1 for a in catalog if store.adapters[a].image.pinned)
    # pinned host -> device bandwidth of one adapter image
    dst = torch.empty(image_bytes, dtype=torch.uint8, device=device)
    for _ in range(3):
        dst.copy_(img, non_blocking=True)
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for _ in range(10):
        dst.copy_(img, non_blocking=True)
    torch.cuda.synchronize()
    h2d_gbs = 10 * image_bytes / (time.perf_counter() - t0) / 1e9
    copy_s = loads * image_bytes / (h2d_gbs * 1e9)
    overlap = (copy_s + comp_s - churn_s) / max(1e-9, min(copy_s, comp_s))
    out = {"steps": args.churn_steps, "batch": B, "slots": 32, "catalog": n_cat, "distinct_images": n_cat,
           "host_copies_per_adapter": 1, "catalog_bytes": n_cat * image_bytes, "pinned_images": pinned_images,
           "pageable_images": n_cat - pinned_images,
           "pinned_note": "page-locked memory is limited to about 65 GiB per process on this host; the "
                          "first (Zipf-hottest) images are pinned, the rest pageable and staged",
           "catalog_build_s": round(t_cat, 1),
           "sub_batch_max_distinct": limit, "sub_batches": len(churn_batches),
           "split": "per step: resident adapters first, then the others from least to most often seen in earlier steps; all rows of an adapter in one sub-batch", "slot_loads": loads, "loads_per_step": round(loads / args.churn_steps, 1),
           "adapter_image_bytes": image_bytes, "h2d_bytes_per_step": round(loads * image_bytes / args.churn_steps),
           "pinned_h2d_gbs": round(h2d_gbs, 1),
           "tokens_per_s_churn": round(n_tok / churn_s, 1), "tokens_per_s_hot_set": round(hot_tok / hot_s, 1),
           "ratio_churn_to_hot": round(hot_s / churn_s * n_tok / hot_tok, 4),
           "wall_s_churn": round(churn_s, 3), "copy_s_at_measured_h2d": round(copy_s, 3),
           "compute_s_same_sub_batches_resident": round(comp_s, 3), "resident_run_loads": comp_loads,
           "overlap_efficiency": round(overlap, 3), "hot_set_loads": hot_loads,
           "overlap_definition": "(copy + compute - wall) / min(copy, compute); compute = the same sub-batches "
                                 "with every adapter resident",
           "timing": "eager wall clock; one new token per row on an empty KV cache"}
    _log(f"churn: {out['tokens_per_s_churn']} tok/s vs hot {out['tokens_per_s_hot_set']}, overlap {out['overlap_efficiency']}")
    del pm, model
    torch.cuda.empty_cache()
    return out


# ----------------------------------------------------------------------------- main
# ----------------------------------------------------------------------------- launch profiles
SEQUENCE_KERNELS = ("pl_shrink", "pl_expand", "pl_lora_fused", "pl_decode_fused", "pl_refop", "pl_plan")
PLAN_KERNEL = "pl_plan_kernel"
COPY_KERNEL = "__amd_rocclr_copyBuffer"


def launch_profile(args) -> int:
    """Issue one workload's LoRA launches in fixed passes, for rocprofv3, and write the manifest.

    After `--profile-plans` device plan builds, the launch sequence (a
    forward's launches for decode and prefill; the fused launch and the split
    shrink + expand for the isolated op, over rotated input sets) is issued
    `--profile-warmup` + `--profile-passes` times back to back.  The manifest
    lists one pass's launches (label, part, algorithmic bytes) in issue
    order, so `--reduce-profile` labels the profiler's dispatches by their
    position in the pass.
    """
    from polylora_amd import sgmv

    device = torch.device("cuda", 0)
    kind = args.launch_profile
    gen = torch.Generator(device=device).manual_seed(7)
    t_build = time.perf_counter()
    if kind in ("isolated", "operator"):
        base_set = isolated_sgmv_workload(device)
        nb = isolated_sgmv_bytes(base_set, 4096, 4096)
        sets = [base_set] + [IsolatedSgmv(base_set.cache, base_set.adapters, base_set.ranks,
                                          torch.randn_like(base_set.x), base_set.base, torch.randn_like(base_set.y),
                                          base_set.row_slot, base_set.seq_lens, base_set.plan, base_set.seg_lens)
                             for _ in range(8)]
        seq = []
        if kind == "isolated":
            for wl in sets:
                seq.append(("fused op", "fused", FusedLaunch(wl.x, wl.y, wl.cache, "op", wl.plan), nb["total"]))
            for wl in sets:
                sp = SgmvLaunch(wl.x, wl.y, wl.cache, "op", wl.plan)
                seq += [("split shrink", "shrink", sp.shrink, nb["shrink"]),
                        ("split expand", "expand", sp.expand, nb["expand"])]
            desc = ("isolated SGMV bf16, T=4096 tokens, K=N=4096, 16 slots + base, ranks {0,4,8,16}, 9 rotated input "
                    "sets: the fused launch on each set, then the split shrink + expand on each")
        else:
            pair = time_operator_api(sets, 1, keep=True)["pair"]
            for i in range(len(sets)):
                # one host call pair issues 2 dispatches: these shapes have long adapter segments, so
                # each call runs a phase of the fused kernel, and the plan and the packed weights are
                # kept from the first two pairs (whose extra pl_refop_prep dispatches fall in the
                # first warm-up pass); the first entry issues both
                steps = ["shrink: fused phase", "expand: fused phase"]
                part_bytes = {"shrink: fused phase": nb["shrink"], "expand: fused phase": nb["expand"]}
                for j, label in enumerate(steps):
                    fn = (lambda i=i: pair(i)) if j == 0 else (lambda: None)
                    seq.append((label, "operator", fn, part_bytes.get(label, 0)))
            desc = ("reference operator API (sgmv_lora_a_fwd + sgmv_lora_b_fwd) on the isolated op's shapes, "
                    "reference slot layout, 9 rotated input sets, plan and packed weights kept across calls")
        cache, row_slot, seq_lens, tpr, distinct = base_set.cache, base_set.row_slot, base_set.seq_lens, 1, 16
    elif kind == "operator-decode":
        from polylora_amd import refop_cache

        wl = decode_workload(device, layers=args.decode_layers, kv_cache=False)
        pm, ids = wl.model, wl.adapter_ids
        mods, op_seq, op_widx = operator_decode_layer_tensors(pm, ids)
        refop_cache.configure()
        seq = []
        for name, A, Bw, rk, sc, x, y in mods:
            def pair(A=A, Bw=Bw, rk=rk, sc=sc, x=x, y=y):
                tmp = sgmv.sgmv_lora_a_fwd(x, A, op_seq, op_widx, rk)
                sgmv.sgmv_lora_b_fwd(tmp, Bw, op_seq, op_widx, rk, sc, y)

            leaf = name.rsplit(".", 1)[-1]
            # one host call pair issues 2 dispatches once the plan and packed weights are kept (the first
            # two layers' pl_refop_prep dispatches fall in the first warm-up pass): the split shrink,
            # whose last K split of each tile writes the intermediate, and the short expand reading
            # that intermediate; the first entry issues both
            seq += [(f"{leaf} shrink: split shrink + finish", "shrink", pair,
                     launch_bytes(pm, [name], "shrink", ids, [1] * len(ids))),
                    (f"{leaf} expand: short expand", "expand", lambda: None,
                     launch_bytes(pm, [name], "expand", ids, [1] * len(ids)))]
        desc = ("reference operator API (sgmv_lora_a_fwd + sgmv_lora_b_fwd) on one Llama-3-8B-shaped decode "
                "layer's 7 Linears, 256 rows x 1 token, reference layout [65, K, 64] / [65, 64, N] bf16, 64 "
                "adapters of ranks {8,16,32,64}, Zipf(1.1) with 10% base rows, plan and packed weights kept "
                "across calls")
        cache, row_slot, seq_lens, tpr = pm.adapter_cache, op_widx, op_seq, 1
        distinct = len({a for a in ids if a != pm.config.base_adapter_id})
    else:
        if kind == "decode":
            wl = decode_workload(device, layers=args.decode_layers, kv_cache=False)
            pm, ids, tpr, lens = wl.model, wl.adapter_ids, 1, [1] * len(wl.adapter_ids)
            split = getattr(args, "profile_split_pairs", False)
            pm.adapter_cache.decode_handoff = not split
            desc = (f"Llama-3-8B-shaped decode, {args.decode_layers} layers, 256 rows x 1 token, 64 slots, ranks "
                    "{8,16,32,64}, Zipf(1.1) with 10% base rows: one forward's LoRA launches"
                    + (" as separate shrink and expand launches" if split else
                       " (shrink and expand in one launch per module set)"))
        else:
            from polylora_amd import PolyLoraConfig, PolyLoraModel

            model = build_llama(device, args.decode_layers, seed=1003)
            pm = PolyLoraModel(model, PolyLoraConfig(target_modules=LLAMA_TARGETS, max_gpu_adapters=64,
                                                     max_rank=64)).eval()
            names = [f"pf{i}" for i in range(8)]
            add_random_adapters(pm, {n: (16 if i < 4 else 32) for i, n in enumerate(names)}, seed=1004, device=device)
            rng = np.random.default_rng(1004)
            tpr = 1024
            lens = [int(v) for v in rng.integers(512, tpr + 1, size=32)]
            ids = [names[i // 4] for i in range(32)]
            desc = (f"Llama-3-8B-shaped prefill, {args.decode_layers} layers, 32 rows x 1024 positions, lengths "
                    f"U[512,1024] ({sum(lens)} valid tokens), 8 adapters (4 x r16, 4 x r32): one forward's LoRA launches")
        cache = pm.adapter_cache
        row_slot = cache.ensure_resident(ids)
        seq_lens = torch.tensor(lens, dtype=torch.int32, device=device)
        distinct = len({a for a in ids if a != pm.config.base_adapter_id})
        plan = sgmv.SgmvPlan(row_slot, seq_lens, tpr, cache.num_slots, distinct_slots=distinct)
        T = len(ids) * tpr
        xs = {k: torch.randn(T, k, generator=gen, device=device, dtype=torch.bfloat16)
              for k in sorted({s.in_features for s in pm.module_specs})}
        seq = [(e.label, e.part, e.fn, launch_bytes(pm, e.modules, e.part, ids, lens))
               for e in forward_launch_sequence(pm, plan, xs, T, gen)]
    torch.cuda.synchronize()
    _log(f"profile {kind}: {len(seq)} launches per pass, built in {time.perf_counter() - t_build:.1f}s")
    for _ in range(args.profile_plans):
        sgmv.SgmvPlan(row_slot, seq_lens, tpr, cache.num_slots, distinct_slots=distinct)
    torch.cuda.synchronize()
    progress = _Progress(f"profile {kind}")
    stream = torch.cuda.current_stream()
    t0, t1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    for p in range(args.profile_warmup + args.profile_passes):
        if p == args.profile_warmup:
            t0.record(stream)
        progress.tick(f"pass {p + 1}/{args.profile_warmup + args.profile_passes}")
        for _, _, fn, _ in seq:
            fn()
    t1.record(stream)
    torch.cuda.synchronize()
    manifest = {"workload": desc, "kind": kind, "warmup": args.profile_warmup, "passes": args.profile_passes,
                "plan_builds": args.profile_plans, "event_ms_per_pass": t0.elapsed_time(t1) / args.profile_passes,
                "sequence": [{"label": l, "part": part, "bytes": int(b)} for l, part, _, b in seq]}
    os.makedirs(os.path.dirname(os.path.abspath(args.manifest)), exist_ok=True)
    with open(args.manifest, "w", encoding="utf-8") as fh:
        json.dump(manifest, fh, indent=1)
    _log(f"profile {kind}: {manifest['event_ms_per_pass']:.4f} ms per pass; manifest {args.manifest}")
    return 0


def kernel_base_name(name: str) -> str:
    """'void pl_expand_short<__hip_bfloat16, 2>(args...)' -> 'pl_expand_short'."""
    n = name.strip().strip('"')
    if n.startswith("void "):
        n = n[5:]
    for ch in "<(":
        i = n.find(ch)
        if i >= 0:
            n = n[:i]
    return n.strip()


def read_dispatches(path: str, counter: str | None = None) -> list:
    """[(dispatch id, kernel, value, workgroups)] in dispatch order from a rocprofv3 CSV.

    value: duration in ns (kernel trace, counter None) or the counter's value
    summed over its rows for the dispatch (counter collection).
    """
    import csv

    def workgroups(row):
        if "Grid_Size_X" in row:
            g = [int(row.get(f"Grid_Size_{a}") or 1) for a in "XYZ"]
            w = [int(row.get(f"Workgroup_Size_{a}") or 1) for a in "XYZ"]
            return (g[0] * g[1] * g[2]) // max(1, w[0] * w[1] * w[2])
        return int(row.get("Grid_Size") or 0) // max(1, int(row.get("Workgroup_Size") or 1))

    out = {}
    with open(path, newline="", encoding="utf-8") as fh:
        for row in csv.DictReader(fh):
            if counter is not None and row.get("Counter_Name") != counter:
                continue
            did = int(row["Dispatch_Id"])
            if counter is None:
                val = float(int(row["End_Timestamp"]) - int(row["Start_Timestamp"]))
            else:
                val = float(row["Counter_Value"])
            if did in out:
                out[did][2] += val
            else:
                out[did] = [did, kernel_base_name(row["Kernel_Name"]), val, workgroups(row)]
    return [tuple(v) for _, v in sorted(out.items())]


def label_dispatches(dispatches: list, manifest: dict) -> dict:
    """label -> [(kernel, value, workgroups, algorithmic bytes)] of the timed passes.

    The sequence kernels' dispatches are taken in order; the last
    (warmup + passes) x len(sequence) of them are the profiled passes, of
    which the warm-up passes are dropped.  Every pass must dispatch the same
    kernel at the same position, or the labels would be wrong.
    """
    seq = manifest["sequence"]
    n = len(seq)
    run = [d for d in dispatches if d[1].startswith(SEQUENCE_KERNELS)]
    need = (manifest["warmup"] + manifest["passes"]) * n
    if len(run) < need:
        raise ValueError(f"{len(run)} sequence dispatches in the profile, the manifest needs {need}")
    run = run[len(run) - need:][manifest["warmup"] * n:]
    out = {}
    for i, (_, kernel, val, wgs) in enumerate(run):
        if kernel != run[i % n][1]:
            raise ValueError(f"dispatch {i}: {kernel} where the first pass had {run[i % n][1]}")
        e = seq[i % n]
        out.setdefault(e["label"], []).append((kernel, val, wgs, e["bytes"]))
    return out


def _calibration(path: str | None, counter: str, copy_bytes: int) -> float:
    """Scale for `counter` so that a plain copy of `copy_bytes` reads (or writes) exactly that many bytes."""
    if not path:
        return 1.0
    vals = [v for _, k, v, _ in read_dispatches(path, counter) if k == COPY_KERNEL]
    if not vals:
        raise ValueError(f"no {COPY_KERNEL} dispatch in {path}")
    return (copy_bytes / 1024.0) / (sum(vals) / len(vals))


def reduce_profile(args) -> int:
    """Print the markdown tables of a launch profile (and write its JSON) from rocprofv3 CSVs."""
    with open(args.manifest, encoding="utf-8") as fh:
        manifest = json.load(fh)
    trace = read_dispatches(args.trace)
    timed = label_dispatches(trace, manifest)
    fetch = label_dispatches(read_dispatches(args.fetch, "FETCH_SIZE"), manifest) if args.fetch else None
    write = label_dispatches(read_dispatches(args.write, "WRITE_SIZE"), manifest) if args.write else None
    fs = _calibration(args.copy_fetch, "FETCH_SIZE", args.copy_bytes)
    ws = _calibration(args.copy_write, "WRITE_SIZE", args.copy_bytes)
    per_pass = {}
    for e in manifest["sequence"]:
        per_pass[e["label"]] = per_pass.get(e["label"], 0) + 1
    lines = [f"Workload: {manifest['workload']}.", "",
             f"{manifest['passes']} profiled passes after {manifest['warmup']} warm-up passes; "
             f"bench HIP-event time {manifest['event_ms_per_pass'] * 1e3:.1f} us per pass.", "",
             "| launch | kernel | per pass | workgroups | dispatches | avg (us) | median (us) | min (us) | "
             "algorithmic MB | GB/s at avg | % of 8 TB/s |",
             "|---|---|---|---|---|---|---|---|---|---|---|"]
    report = {"workload": manifest["workload"], "fetch_scale": fs, "write_scale": ws, "labels": {}, "kernels": {}}
    pass_us = pass_bytes = 0.0
    for label, rows in timed.items():
        durs = sorted(v / 1e3 for _, v, _, _ in rows)
        avg = sum(durs) / len(durs)
        mb = sum(b for *_, b in rows) / len(rows)
        kernels = sorted({k for k, *_ in rows})
        wgs = sorted({w for _, _, w, _ in rows})
        gbs = mb / (avg * 1e-6) / 1e9
        pass_us += avg * per_pass[label]
        pass_bytes += mb * per_pass[label]
        rate = f"{gbs:.0f} | {100 * gbs / HBM_PEAK_GBS:.1f}" if mb else "- | -"
        lines.append(f"| {label} | {', '.join(kernels)} | {per_pass[label]} | {', '.join(map(str, wgs))} | {len(rows)} "
                     f"| {avg:.2f} | {durs[len(durs) // 2]:.2f} | {durs[0]:.2f} | {mb / 1e6:.2f} | {rate} |")
        report["labels"][label] = {"kernels": kernels, "per_pass": per_pass[label], "avg_us": avg,
                                   "algorithmic_bytes_per_launch": mb}
    lines += ["", f"One pass: {pass_us:.1f} us summed over its launches' average durations, "
              f"{pass_bytes / 1e6:.1f} MB algorithmic, {pass_bytes / (pass_us * 1e-6) / 1e9:.0f} GB/s "
              f"({100 * pass_bytes / (pass_us * 1e-6) / 1e9 / HBM_PEAK_GBS:.1f}% of 8 TB/s)."]
    report["pass_us"], report["pass_bytes"] = pass_us, pass_bytes
    plans = [v / 1e3 for _, k, v, _ in trace if k == PLAN_KERNEL]
    if plans:
        lines += ["", f"{PLAN_KERNEL}: {len(plans)} dispatches, avg {sum(plans) / len(plans):.2f} us, "
                  f"min {min(plans):.2f} us."]
        report["plan_avg_us"] = sum(plans) / len(plans)
    if fetch and write:
        lines += ["", f"HBM bytes per launch: FETCH_SIZE x {fs:.4f}, WRITE_SIZE x {ws:.4f} (KiB; the scales make a "
                  f"plain {args.copy_bytes}-byte copy read and write exactly its size).", "",
                  "| launch | FETCH_SIZE (KiB, raw) | WRITE_SIZE (KiB, raw) | measured MB | algorithmic MB | ratio |",
                  "|---|---|---|---|---|---|"]
        t_pass = 0.0
        for label in timed:
            f = sum(v for _, v, _, _ in fetch[label]) / len(fetch[label])
            w = sum(v for _, v, _, _ in write[label]) / len(write[label])
            meas = 1024.0 * (f * fs + w * ws)
            alg = report["labels"][label]["algorithmic_bytes_per_launch"]
            t_pass += meas * per_pass[label]
            ratio = f"{meas / alg:.3f}" if alg else "-"
            lines.append(f"| {label} | {f:.1f} | {w:.1f} | {meas / 1e6:.2f} | {alg / 1e6:.2f} | {ratio} |")
            report["labels"][label].update(fetch_kib=f, write_kib=w, traffic_bytes_per_launch=meas)
            for k in report["labels"][label]["kernels"]:
                report["kernels"].setdefault(k, {"traffic_bytes_per_launch": meas, "algorithmic_bytes_per_launch": alg})
        report["pass_traffic_bytes"] = t_pass
        lines += ["", f"One pass moves {t_pass / 1e6:.1f} MB measured against {pass_bytes / 1e6:.1f} MB algorithmic "
                  f"({t_pass / max(1.0, pass_bytes):.3f})."]
    print("\n".join(lines))
    if args.reduce_json:
        with open(args.reduce_json, "w", encoding="utf-8") as fh:
            json.dump(report, fh, indent=1)
    return 0


def _release_between_workloads() -> None:
    """Free what the previous workload left: its model and adapters, and their page-locked memory.

    Page-locked host memory is limited per process; the decode workload's
    adapter images (~10 GB) would otherwise stay locked in the recycle pool
    next to the churn catalog's 56 GiB.
    """
    import gc

    from polylora_amd.slot_image import release_locked_free

    gc.collect()
    torch.cuda.synchronize()
    torch.cuda.empty_cache()
    freed = release_locked_free()
    if freed:
        _log(f"released {freed / 2**30:.1f} GiB of page-locked memory")


def main(argv=None) -> int:
    p = argparse.ArgumentParser(description=__doc__, formatter_class=argparse.RawDescriptionHelpFormatter)
    p.add_argument("--gpus", type=int, default=1)
    p.add_argument("--steps", type=int, default=200)
    p.add_argument("--warmup", type=int, default=20)
    p.add_argument("--cpu-seconds", type=float, default=10.0, help="budget of the CPU baseline sample")
    p.add_argument("--no-cpu-baseline", action="store_true")
    p.add_argument("--only-isolated", action="store_true", help="skip the model workloads")
    p.add_argument("--decode-layers", type=int, default=32)
    p.add_argument("--decode-steps", type=int, default=20)
    p.add_argument("--no-decode", action="store_true", help="skip the decode and prefill workloads")
    p.add_argument("--no-deberta", action="store_true")
    p.add_argument("--no-prefill", action="store_true")
    p.add_argument("--no-churn", action="store_true")
    p.add_argument("--churn-steps", type=int, default=200, help="decode steps of the churn workload")
    p.add_argument("--churn-catalog", type=int, default=1024, help="adapters in the churn catalog, each its own image")
    p.add_argument("--churn-pinned-gib", type=float, default=56.0,
                   help="page-locked bytes for churn catalog images; the rest are pageable")
    p.add_argument("--churn-sub-distinct", type=int, default=32, choices=range(1, 33), metavar="1..32",
                   help="most distinct adapters per churn sub-batch (the cache has 32 slots)")
    p.add_argument("--copy-probe", type=int, default=0, metavar="BYTES",
                   help="only copy a BYTES-sized device buffer 5 times (calibrates HBM byte counters) and exit")
    p.add_argument("--launch-profile", choices=["isolated", "decode", "prefill", "operator", "operator-decode"],
                   help="only issue this workload's LoRA launches in fixed passes (for rocprofv3) and write --manifest")
    p.add_argument("--manifest", default="launch_profile/manifest.json")
    p.add_argument("--profile-passes", type=int, default=20)
    p.add_argument("--profile-warmup", type=int, default=3)
    p.add_argument("--profile-plans", type=int, default=20, help="device plan builds before the passes")
    p.add_argument("--profile-split-pairs", action="store_true",
                   help="decode: separate shrink and expand launches instead of the one-launch hand-off")
    p.add_argument("--reduce-profile", action="store_true",
                   help="no GPU: reduce rocprofv3 CSVs of a --launch-profile run into markdown tables")
    p.add_argument("--trace", help="kernel_trace.csv of the profiled run")
    p.add_argument("--fetch", help="counter_collection.csv of a --pmc FETCH_SIZE run")
    p.add_argument("--write", help="counter_collection.csv of a --pmc WRITE_SIZE run")
    p.add_argument("--copy-fetch", help="counter_collection.csv of --pmc FETCH_SIZE over --copy-probe")
    p.add_argument("--copy-write", help="counter_collection.csv of --pmc WRITE_SIZE over --copy-probe")
    p.add_argument("--copy-bytes", type=int, default=268435456)
    p.add_argument("--reduce-json", help="write the reduced figures here as JSON")
    p.add_argument("--graph-trace", action="store_true",
                   help="replay the decode step's graph without and with adapters, for a kernel trace")
    p.add_argument("--reduce-graph-trace", action="store_true",
                   help="print per-kernel time per step from the --trace of a --graph-trace run")
    args = p.parse_args(argv)
    if args.reduce_profile:
        return reduce_profile(args)
    if args.reduce_graph_trace:
        return reduce_graph_trace(args)
    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) > 1:
        print("bench.py measures one GPU only: the library has no multi-GPU path; run with --gpus 1", file=sys.stderr)
        return 2
    if not torch.cuda.is_available():
        print("bench.py needs a ROCm GPU", file=sys.stderr)
        return 1
    if args.copy_probe:
        src = torch.ones(args.copy_probe, dtype=torch.uint8, device="cuda")
        dst = torch.empty_like(src)
        for _ in range(5):
            dst.copy_(src)
        torch.cuda.synchronize()
        print(json.dumps({"copy_probe_bytes": args.copy_probe, "copies": 5}), flush=True)
        return 0
    if args.launch_profile:
        return launch_profile(args)
    if args.graph_trace:
        return decode_graph_trace(args)
    iso = run_isolated(args)
    _log(f"isolated: {iso['value']} GB/s")
    result = {
        "metric": METRIC,
        "value": iso["value"],
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": iso["ms_per_step"],
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": "synthetic",
        "config": iso["config"],
        "roofline": iso["roofline"],
    }
    if "cpu_baseline" in iso:
        result["cpu_baseline"] = iso["cpu_baseline"]
    if not args.only_isolated:
        workloads = {}
        if not args.no_decode:
            args.keep_model = not args.no_prefill
            workloads["decode"] = run_decode(args)
            pm = workloads["decode"].pop("_model", None)
            if pm is not None:
                workloads["prefill"] = run_prefill(args, pm)
                del pm
                torch.cuda.empty_cache()
        if not args.no_churn:
            _release_between_workloads()
            workloads["churn"] = run_churn(args)
        if not args.no_deberta:
            _release_between_workloads()
            workloads["deberta"] = run_deberta(torch.device("cuda", 0),
                                                cpu_budget_s=None if args.no_cpu_baseline else args.cpu_seconds)
        result["workloads"] = workloads
    print(json.dumps(result), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
