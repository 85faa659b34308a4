"""Benchmark: SGMV achieved HBM GB/s on one MI355X (isolated op, bf16).

Default workload: T=4096 tokens, K=N=4096, 16 adapter slots + the base slot,
ranks cycling {0,4,8,16} by slot, alpha=32 (scale 32/r), tokens sorted into
contiguous per-slot segments with Dirichlet(1) lengths, X and base Y ~N(0,1),
A and B ~N(0,0.02).  One step = the LoRA shrink + expand of all tokens
(``pl_lora_apply``) with the device plan already built (it is built once per
forward and shared by every wrapped Linear).  Inputs rotate over enough X/Y
sets (> 512 MB) that the 256 MB Infinity Cache cannot hold them.

Prints one JSON line (see ``--help``).  ``--gpus`` above 1 exits: this build
measures one GPU.
"""

from __future__ import annotations

import argparse
import json
import os
import platform
import sys
import time
from dataclasses import dataclass

import numpy as np
import torch

HBM_PEAK_GBS = 8000.0
MFMA_BF16_PEAK_TFLOPS = 2500.0


# ----------------------------------------------------------------------------- workloads
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
    plan = sgmv.SgmvPlan(row_slot, seq_lens, 1, cache.num_slots)
    return IsolatedSgmv(cache, adapters, ranks, x, base, base.clone(), row_slot, seq_lens, plan, seg)


def isolated_sgmv_bytes(wl: IsolatedSgmv, K: int, N: int) -> dict:
    """Algorithmic bytes: X of active tokens, Y read+write, each active adapter's A and B once, the row maps."""
    active = [s for s in range(len(wl.ranks)) if wl.ranks[s] > 0]
    t_active = int(sum(wl.seg_lens[s] for s in active))
    r_tok = int(sum(wl.seg_lens[s] * wl.ranks[s] for s in active))
    ab = sum(2 * wl.ranks[s] * (K + N) for s in active)
    shrink = 2 * t_active * K + sum(2 * wl.ranks[s] * K for s in active)
    expand = 4 * t_active * N + sum(2 * wl.ranks[s] * N for s in active)
    total = 2 * t_active * K + 4 * t_active * N + ab + 4 * len(wl.ranks) * 2
    flops = 2 * r_tok * (K + N)
    return {"total": total, "shrink": shrink, "expand": expand, "t_active": t_active, "flops": flops}


# ----------------------------------------------------------------------------- CPU baseline
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
        if el >= budget_s or reps >= 50:
            break
    per = el / reps
    return {
        "value": round(nbytes / per / 1e9, 4),
        "unit": "GB/s",
        "cores": threads,
        "kind": "port",
        "sample": f"{reps} full ops (17 segment rows, {int(wl.seg_lens.sum())} tokens) of the fallback loop, "
                  f"{per * 1e3:.1f} ms each, torch {threads} threads, {platform.processor() or platform.machine()}",
    }


# ----------------------------------------------------------------------------- GPU timing
def _time_isolated(wl_sets, steps: int, warmup: int, lib_apply) -> tuple[float, list]:
    for i in range(warmup):
        lib_apply(wl_sets[i % len(wl_sets)])
    torch.cuda.synchronize()
    start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    start.record()
    for i in range(steps):
        lib_apply(wl_sets[i % len(wl_sets)])
    end.record()
    torch.cuda.synchronize()
    return start.elapsed_time(end) / steps, []


def _kernel_times(wl_sets, reps: int) -> tuple[float, float]:
    """Average shrink and expand durations, each bracketed by events on the launch stream."""
    from polylora_amd import _native, sgmv

    lib = _native.load()
    stream = torch.cuda.current_stream()
    ev = [[torch.cuda.Event(enable_timing=True) for _ in range(3)] for _ in range(reps)]
    for i in range(reps):
        wl = wl_sets[i % len(wl_sets)]
        cache, plan = wl.cache, wl.plan
        ldt = cache.rank8_cap
        ws = sgmv._workspace(wl.x.device, stream.cuda_stream)
        splits = sgmv.choose_k_splits(plan.group_cap, wl.x.shape[1], wl.x.dtype)
        need = plan.tokens_cap * ldt
        slot, buf, zp, zc = ws.acquire(need)
        common = (cache.arena.data_ptr(), cache.table.data_ptr(), len(cache.module_index), cache.module_index["op"],
                  plan.tok.data_ptr(), plan.groups.data_ptr(), plan.meta.data_ptr(), plan.group_cap)
        ev[i][0].record(stream)
        st = lib.pl_sgmv_shrink(_native.PL_BF16, wl.x.data_ptr(), wl.x.stride(0), wl.x.shape[1], *common,
                                buf.data_ptr(), ldt, splits, zp or None, zc, stream.cuda_stream)
        ev[i][1].record(stream)
        st2 = lib.pl_sgmv_expand(_native.PL_BF16, buf.data_ptr(), ldt, *common, wl.y.data_ptr(), wl.y.stride(0),
                                 wl.y.shape[1], _native.PL_EPI_FALLBACK, stream.cuda_stream)
        ev[i][2].record(stream)
        ws.commit(slot, need, st == 0 and st2 == 0)
        _native.check(st, "pl_sgmv_shrink")
        _native.check(st2, "pl_sgmv_expand")
    torch.cuda.synchronize()
    sh = sum(e[0].elapsed_time(e[1]) for e in ev) / reps
    ex = sum(e[1].elapsed_time(e[2]) for e in ev) / reps
    return sh, ex


def run_isolated(args) -> dict:
    from polylora_amd import sgmv

    device = torch.device("cuda", 0)
    K = N = 4096
    base_set = isolated_sgmv_workload(device)
    set_bytes = 2 * base_set.x.numel() * base_set.x.element_size()
    n_sets = max(3, int(np.ceil(600e6 / set_bytes)))
    sets = [base_set]
    for i in range(1, n_sets):
        sets.append(IsolatedSgmv(base_set.cache, base_set.adapters, base_set.ranks,
                                 torch.randn_like(base_set.x), base_set.base, torch.randn_like(base_set.y),
                                 base_set.row_slot, base_set.seq_lens, base_set.plan, base_set.seg_lens))
    nb = isolated_sgmv_bytes(base_set, K, N)

    def apply(wl):
        sgmv.lora_apply(wl.x, wl.y, wl.cache, "op", wl.plan)

    ms, _ = _time_isolated(sets, args.steps, args.warmup, apply)
    sh_ms, ex_ms = _kernel_times(sets, max(20, args.steps))
    value = nb["total"] / (ms * 1e-3) / 1e9
    exp_gbs = nb["expand"] / (ex_ms * 1e-3) / 1e9
    result = {
        "metric": "SGMV achieved HBM GB/s (% peak); multi-LoRA decode tokens/s, 1 MI355X",
        "value": round(value, 2),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms, 5),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": "synthetic",
        "config": {
            "workload": "isolated SGMV shrink+expand, T=4096 tokens, K=N=4096, 16 slots + base, ranks {0,4,8,16}, "
                        "Dirichlet(1) segments, alpha 32",
            "tokens_active": nb["t_active"],
            "algorithmic_bytes_per_step": nb["total"],
            "pct_of_hbm_peak": round(100 * value / HBM_PEAK_GBS, 2),
            "input_sets_rotated": n_sets,
            "shrink_ms": round(sh_ms, 5),
            "expand_ms": round(ex_ms, 5),
        },
        "roofline": {
            "kernel": "pl_expand_tiled<bf16>",
            "bound": "hbm",
            "achieved": round(exp_gbs, 2),
            "peak": HBM_PEAK_GBS,
            "unit": "GB/s",
            "frac": round(exp_gbs / HBM_PEAK_GBS, 4),
            "traffic": None,
            "algorithmic_bytes_per_launch": nb["expand"],
        },
    }
    if not args.no_cpu_baseline:
        result["cpu_baseline"] = cpu_baseline_isolated(base_set, nb["total"], args.cpu_seconds)
    return result


def main(argv=None) -> int:
    p = argparse.ArgumentParser(description=__doc__, formatter_class=argparse.RawDescriptionHelpFormatter)
    p.add_argument("--gpus", type=int, default=1)
    p.add_argument("--steps", type=int, default=200)
    p.add_argument("--warmup", type=int, default=20)
    p.add_argument("--cpu-seconds", type=float, default=10.0, help="budget of the CPU baseline sample")
    p.add_argument("--no-cpu-baseline", action="store_true")
    args = p.parse_args(argv)
    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) > 1:
        print("bench.py measures one GPU only: this build has no multi-GPU path; run with --gpus 1", file=sys.stderr)
        return 2
    if not torch.cuda.is_available():
        print("bench.py needs a ROCm GPU", file=sys.stderr)
        return 1
    result = run_isolated(args)
    print(json.dumps(result), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
