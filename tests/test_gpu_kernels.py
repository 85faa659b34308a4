"""GPU parity of the HIP kernels against the oracle (run with `-m gpu`)."""

from __future__ import annotations

import numpy as np
import pytest
import torch

from oracle.lora import reference_forward, sgmv_expand_reference, sgmv_shrink_reference
from oracle.plan import check_plan
from polylora_amd import sgmv
from tests._util import make_cache, oracle_slot_tensors, peft_layer, tol_for

pytestmark = pytest.mark.gpu


def _announce(**kw):
    print("case:", ", ".join(f"{k}={v}" for k, v in kw.items()), flush=True)


def _adapters(gen, ranks, fin, fout, module="m", extra_module=None):
    """One adapter per rank; rank 0 means the adapter lacks `module` (needs extra_module)."""
    out = {}
    for i, r in enumerate(ranks):
        layers = {}
        if r > 0:
            layers[module] = peft_layer(gen, fin, fout, r, alpha=2.0 * r)
        if extra_module is not None:
            layers[extra_module] = peft_layer(gen, 8, 8, 2, alpha=4.0)
        out[f"a{i:03d}"] = layers
    return out


@pytest.mark.parametrize("group_tokens", [16, 64])
@pytest.mark.parametrize(
    "rows,row_len,num_slots,seed",
    [(1, 1, 2, 0), (7, 3, 5, 1), (256, 1, 65, 2), (32, 1024, 9, 3), (4096, 1, 17, 4), (3, 200, 4096, 5), (0, 5, 3, 6),
     (10000, 1, 33, 7), (9000, 2, 5, 8),
     # at most 256 slots one wave scans the slot counts; from 257 on every wave takes part
     (5000, 1, 256, 9), (5000, 1, 257, 10), (3000, 2, 1025, 11)],
)
def test_plan_matches_oracle(gpu, rows, row_len, num_slots, seed, group_tokens):
    _announce(test="plan", rows=rows, row_len=row_len, num_slots=num_slots, group_tokens=group_tokens)
    g = torch.Generator().manual_seed(seed)
    row_slot = torch.randint(-1, num_slots + 1, (rows,), generator=g, dtype=torch.int32)
    seq_lens = torch.randint(-2, row_len + 3, (rows,), generator=g, dtype=torch.int32)
    plan = sgmv.SgmvPlan(row_slot.to(gpu), seq_lens.to(gpu), row_len, num_slots, group_tokens=group_tokens)
    torch.cuda.synchronize()
    check_plan(
        plan.tok.cpu().numpy(),
        plan.groups.cpu().numpy(),
        plan.meta.cpu().numpy(),
        row_slot.tolist(),
        seq_lens.tolist(),
        row_len,
        num_slots,
        group_tokens=group_tokens,
    )


@pytest.mark.parametrize("rows,row_len,num_slots,group_tokens", [(4096, 1, 17, 16), (2049, 16, 3, 64), (8192, 4, 65, 16)])
def test_plan_of_sorted_rows_matches_oracle(gpu, rows, row_len, num_slots, group_tokens):
    """Rows sorted by slot: whole waves of one slot claim their counts and places with one atomic, and
    waves that straddle two slots take the per-thread path; 2049 rows leave the last wave one row, 8192 rows
    take two passes of the workgroup."""
    _announce(test="plan_sorted", rows=rows, row_len=row_len, num_slots=num_slots, group_tokens=group_tokens)
    g = torch.Generator().manual_seed(rows)
    row_slot = torch.sort(torch.randint(0, num_slots, (rows,), generator=g, dtype=torch.int32)).values
    seq_lens = torch.randint(0, row_len + 1, (rows,), generator=g, dtype=torch.int32)
    seq_lens[: rows // 2] = row_len  # half the rows full: runs of equal lengths as well as ragged ones
    plan = sgmv.SgmvPlan(row_slot.to(gpu), seq_lens.to(gpu), row_len, num_slots, group_tokens=group_tokens)
    torch.cuda.synchronize()
    check_plan(plan.tok.cpu().numpy(), plan.groups.cpu().numpy(), plan.meta.cpu().numpy(), row_slot.tolist(),
               seq_lens.tolist(), row_len, num_slots, group_tokens=group_tokens)


@pytest.mark.parametrize("rows,row_len,num_slots,group_tokens,seed",
                         [(4096, 1, 17, 16, 20), (300, 3, 40, 16, 21), (32, 1024, 9, 64, 22), (9000, 1, 70, 16, 23)])
def test_plan_active_mask_matches_oracle(gpu, rows, row_len, num_slots, group_tokens, seed):
    """Rows of inactive slots are left out exactly as rows of slot 0; the mask is read through its stride."""
    _announce(test="plan_active", rows=rows, row_len=row_len, num_slots=num_slots)
    g = torch.Generator().manual_seed(seed)
    row_slot = torch.randint(-1, num_slots + 1, (rows,), generator=g, dtype=torch.int32)
    seq_lens = torch.randint(-1, row_len + 2, (rows,), generator=g, dtype=torch.int32)
    table = torch.randint(-2, 3, (num_slots, 8), generator=g, dtype=torch.int32)  # column 3: the mask
    active = table[:, 3]
    plan = sgmv.SgmvPlan(row_slot.to(gpu), seq_lens.to(gpu), row_len, num_slots, group_tokens=group_tokens,
                         active=table.to(gpu)[:, 3])
    torch.cuda.synchronize()
    masked = [s if 0 < s < num_slots and int(active[s]) > 0 else 0 for s in row_slot.tolist()]
    check_plan(plan.tok.cpu().numpy(), plan.groups.cpu().numpy(), plan.meta.cpu().numpy(), masked, seq_lens.tolist(),
               row_len, num_slots, group_tokens=group_tokens)


CASES = [
    # dtype, rows, M, K, N, ranks, max_rank, k_splits, seed
    (torch.bfloat16, 8, 5, 64, 32, [2, 3, 4], 4, None, 10),
    (torch.float32, 8, 5, 64, 32, [2, 3, 4], 4, None, 11),
    (torch.float16, 8, 5, 64, 32, [2, 3, 4], 4, None, 12),
    (torch.bfloat16, 256, 1, 4096, 4096, [8, 16, 32, 64], 64, None, 13),
    (torch.bfloat16, 256, 1, 14336, 4096, [8, 16, 32, 64], 64, None, 14),
    (torch.bfloat16, 64, 1, 4096, 14336, [8, 16, 32, 64], 64, None, 15),
    (torch.bfloat16, 4, 300, 512, 1024, [16, 32], 64, None, 16),
    (torch.bfloat16, 33, 7, 1024, 768, [1, 7, 9, 15, 17, 33, 63], 64, 3, 17),
    (torch.float32, 33, 7, 768, 3072, [4, 8, 16], 16, 4, 18),
    (torch.float32, 6, 128, 3072, 768, [4, 8, 8, 16, 16], 16, None, 19),
    (torch.bfloat16, 16, 3, 4104, 1000, [80, 128], 128, 2, 20),
    (torch.bfloat16, 300, 1, 256, 256, [16] * 5, 16, 1, 21),
    # >= 512 shrink workgroups at 64-rank passes (the wide short shrink) and
    # >= 1536 expand workgroups at 4 planes (32-rank staged blocks)
    (torch.bfloat16, 2048, 1, 1024, 3072, [8, 16, 32, 64, 8, 16, 32, 64], 64, 4, 22),
    # the wide short shrink with two 64-rank passes (ranks up to 128)
    (torch.bfloat16, 2048, 1, 1024, 512, [80, 128, 8, 64, 33], 128, 4, 23),
    # 16 K splits: the expand sums 16 planes
    (torch.bfloat16, 24, 2, 4096, 768, [8, 64, 32], 64, 16, 24),
    # fp16 at the decode shapes, and on the wide short shrink with 32-rank expand blocks
    (torch.float16, 256, 1, 4096, 4096, [8, 16, 32, 64], 64, None, 25),
    (torch.float16, 2048, 1, 1024, 3072, [8, 16, 32, 64, 8, 16, 32, 64], 64, 4, 26),
]


@pytest.mark.parametrize("dtype,rows,M,K,N,ranks,max_rank,k_splits,seed", CASES)
def test_lora_apply_matches_oracle(gpu, dtype, rows, M, K, N, ranks, max_rank, k_splits, seed):
    _announce(test="lora_apply", dtype=dtype, rows=rows, M=M, K=K, N=N, ranks=ranks, k_splits=k_splits)
    g = torch.Generator().manual_seed(seed)
    adapters = _adapters(g, ranks, K, N)
    ids = list(adapters) + ["__base__"]
    cache = make_cache(adapters, {"m": (K, N)}, len(adapters), max_rank, gpu, dtype)
    pick = torch.randint(0, len(ids), (rows,), generator=g).tolist()
    adapter_ids = [ids[i] for i in pick]
    row_slot = cache.ensure_resident(adapter_ids)
    seq_lens = torch.randint(0, M + 2, (rows,), generator=g, dtype=torch.int32)
    x = torch.randn(rows, M, K, generator=g).to(dtype)
    base = torch.randn(rows, M, N, generator=g).to(dtype)
    A, B, rk, sc = oracle_slot_tensors(cache, adapters, "m", dtype)
    expect = reference_forward(x, base, seq_lens, row_slot.cpu(), A, B, rk, sc)
    # untouched rows (base adapter, padding) are bit-identical to the base output
    untouched = torch.ones(rows, M, dtype=torch.bool)
    for b, aid in enumerate(adapter_ids):
        if aid != "__base__":
            untouched[b, : min(int(seq_lens[b]), M)] = False
    for group_tokens in (16, 64):
        y = base.to(gpu)
        plan = sgmv.SgmvPlan(row_slot, seq_lens.to(gpu), M, cache.num_slots, group_tokens=group_tokens)
        sgmv.lora_apply(x.to(gpu).view(-1, K), y.view(-1, N), cache, "m", plan, k_splits=k_splits)
        got = y.cpu()
        torch.testing.assert_close(got, expect, **tol_for(dtype))
        assert torch.equal(got[untouched], base[untouched])


@pytest.mark.parametrize("dtype,rows,M,K,N,ranks,max_rank,k_splits,seed", CASES)
def test_lora_fused_matches_oracle(gpu, dtype, rows, M, K, N, ranks, max_rank, k_splits, seed):
    _announce(test="lora_fused", dtype=dtype, rows=rows, M=M, K=K, N=N, ranks=ranks)
    g = torch.Generator().manual_seed(seed)
    adapters = _adapters(g, ranks, K, N)
    ids = list(adapters) + ["__base__"]
    cache = make_cache(adapters, {"m": (K, N)}, len(adapters), max_rank, gpu, dtype)
    pick = torch.randint(0, len(ids), (rows,), generator=g).tolist()
    adapter_ids = [ids[i] for i in pick]
    row_slot = cache.ensure_resident(adapter_ids)
    seq_lens = torch.randint(0, M + 2, (rows,), generator=g, dtype=torch.int32)
    x = torch.randn(rows, M, K, generator=g).to(dtype)
    base = torch.randn(rows, M, N, generator=g).to(dtype)
    if cache.rank8_cap > sgmv.FUSED_MAX_RANK:
        plan = sgmv.SgmvPlan(row_slot, seq_lens.to(gpu), M, cache.num_slots)
        with pytest.raises(ValueError, match="ranks up to"):
            sgmv.lora_fused(x.to(gpu).view(-1, K), base.to(gpu).view(-1, N), cache, "m", plan)
        return
    A, B, rk, sc = oracle_slot_tensors(cache, adapters, "m", dtype)
    expect = reference_forward(x, base, seq_lens, row_slot.cpu(), A, B, rk, sc)
    untouched = torch.ones(rows, M, dtype=torch.bool)
    for b, aid in enumerate(adapter_ids):
        if aid != "__base__":
            untouched[b, : min(int(seq_lens[b]), M)] = False
    for group_tokens in (16, 64):
        plan = sgmv.SgmvPlan(row_slot, seq_lens.to(gpu), M, cache.num_slots, group_tokens=group_tokens)
        for slices in (None, 1, 3):
            y = base.to(gpu)
            sgmv.lora_fused(x.to(gpu).view(-1, K), y.view(-1, N), cache, "m", plan, slices=slices)
            got = y.cpu()
            torch.testing.assert_close(got, expect, **tol_for(dtype))
            assert torch.equal(got[untouched], base[untouched])


def test_lora_fused_bitwise_reproducible_and_triton_order(gpu):
    """Two fused runs agree bit for bit; the Triton epilogue order matches its oracle rounding."""
    _announce(test="lora_fused_reproducible")
    g = torch.Generator().manual_seed(31)
    K, N, rows = 2048, 3072, 512
    adapters = _adapters(g, [16, 32, 64], K, N)
    cache = make_cache(adapters, {"m": (K, N)}, 3, 64, gpu, torch.bfloat16)
    ids = list(adapters)
    adapter_ids = [ids[i % 3] for i in range(rows)]
    row_slot = cache.ensure_resident(adapter_ids)
    seq = torch.ones(rows, dtype=torch.int32, device=gpu)
    plan = sgmv.SgmvPlan(row_slot, seq, 1, cache.num_slots, group_tokens=16)
    x = torch.randn(rows, K, generator=g).to(torch.bfloat16).to(gpu)
    base = torch.randn(rows, N, generator=g).to(torch.bfloat16).to(gpu)
    y1, y2 = base.clone(), base.clone()
    sgmv.lora_fused(x, y1, cache, "m", plan, slices=2)
    sgmv.lora_fused(x, y2, cache, "m", plan, slices=2)
    assert torch.equal(y1, y2)
    # with the Triton order the delta is T(acc * scale): compare with the fallback
    # result within bf16 tolerance (the two orders differ by rounding only)
    y3 = base.clone()
    sgmv.lora_fused(x, y3, cache, "m", plan, slices=2, epilogue=1)
    torch.testing.assert_close(y3.float(), y1.float(), rtol=2e-2, atol=1e-2)


@pytest.mark.parametrize("dtype,group_tokens,n_mod", [(torch.bfloat16, 16, 3), (torch.bfloat16, 64, 3),
                                                     (torch.float32, 64, 3), (torch.float16, 16, 4)])
def test_stacked_fused_equals_separate(gpu, dtype, group_tokens, n_mod):
    """pl_lora_fused_stacked over q/k/v-like modules == one pl_lora_fused per module, bit for bit, and the oracle."""
    _announce(test="stacked_fused", dtype=dtype, group_tokens=group_tokens, n_mod=n_mod)
    g = torch.Generator().manual_seed(61)
    K, rows, M = 1024, 6, 90
    shapes = {"q": (K, 1024), "k": (K, 256), "v": (K, 136), "u": (K, 2056)}
    shapes = dict(list(shapes.items())[:n_mod])
    adapters = {}
    for i, r in enumerate([8, 24, 64]):
        adapters[f"s{i}"] = {m: peft_layer(g, fi, fo, r, 2.0 * r) for m, (fi, fo) in shapes.items() if not (i == 1 and m == "k")}
    cache = make_cache(adapters, shapes, 3, 64, gpu, dtype)
    ids = list(adapters) + ["__base__"]
    row_slot = cache.ensure_resident([ids[i % 4] for i in range(rows)])
    seq_lens = torch.tensor([90, 17, 64, 0, 33, 81], dtype=torch.int32)
    plan = sgmv.SgmvPlan(row_slot, seq_lens.to(gpu), M, cache.num_slots, group_tokens=group_tokens)
    x = torch.randn(rows, M, K, generator=g).to(dtype)
    base = {m: torch.randn(rows, M, fo, generator=g).to(dtype) for m, (fi, fo) in shapes.items()}
    xg = x.to(gpu).view(-1, K)
    for slices in (None, 1, 3):
        sep = {}
        for m in shapes:
            y = base[m].to(gpu).view(rows * M, -1)
            sgmv.lora_fused(xg, y, cache, m, plan, slices=slices)
            sep[m] = y
        ys = [base[m].to(gpu).view(rows * M, -1) for m in shapes]
        sgmv.lora_fused_stacked(xg, ys, cache, list(shapes), plan, slices=slices)
        for m, y in zip(shapes, ys):
            assert torch.equal(y, sep[m]), (m, slices)
    for m in shapes:
        A, B, rk, sc = oracle_slot_tensors(cache, adapters, m, dtype)
        expect = reference_forward(x, base[m], seq_lens, row_slot.cpu(), A, B, rk, sc)
        torch.testing.assert_close(sep[m].cpu().view(rows, M, -1), expect, **tol_for(dtype))
    with pytest.raises(ValueError, match="modules with one y each"):
        sgmv.lora_fused_stacked(xg, ys[:2], cache, list(shapes), plan)
    with pytest.raises(ValueError, match="must be"):  # a later module's output of the wrong width
        sgmv.lora_fused_stacked(xg, [ys[0], ys[1][:, :8].contiguous(), *ys[2:]], cache, list(shapes), plan)


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
@pytest.mark.parametrize("K,N,ranks", [(37, 30, [1, 3, 5]), (101, 75, [17, 40, 33])])
def test_rows_kernels_match_oracle(gpu, dtype, K, N, ranks):
    """K, N not multiples of the 16-byte chunk; the second shape spans several
    16-row tiles and 64-byte blocks of the arena's A and B."""
    _announce(test="rows", dtype=dtype, K=K, N=N, ranks=ranks)
    g = torch.Generator().manual_seed(30)
    rows, M = 5, 9
    adapters = _adapters(g, ranks, K, N)
    cache = make_cache(adapters, {"m": (K, N)}, 3, max(ranks), gpu, dtype, tiled=False)
    ids = ["a000", "__base__", "a001", "a002", "a001"]
    row_slot = cache.ensure_resident(ids)
    seq_lens = torch.tensor([9, 9, 0, 4, 11], dtype=torch.int32)
    x = torch.randn(rows, M, K, generator=g).to(dtype)
    base = torch.randn(rows, M, N, generator=g).to(dtype)
    y = base.to(gpu)
    sgmv.lora_apply_rows(x.to(gpu).view(-1, K), y.view(-1, N), cache, "m", row_slot, seq_lens.to(gpu), M)
    A, B, rk, sc = oracle_slot_tensors(cache, adapters, "m", dtype)
    expect = reference_forward(x, base, seq_lens, row_slot.cpu(), A, B, rk, sc)
    torch.testing.assert_close(y.cpu(), expect, **tol_for(dtype))


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32, torch.float16])
@pytest.mark.parametrize("stack_num", [1, 2])
def test_reference_layout_ops_match_oracle(gpu, dtype, stack_num):
    _announce(test="ref_ops", dtype=dtype, stack_num=stack_num)
    g = torch.Generator().manual_seed(40 + stack_num)
    Bt, M, K, N, S, R = 6, 10, 96, 80, 4, 8
    x = torch.randn(Bt, M, K, generator=g).to(dtype)
    wa = (torch.randn(S, K, R * stack_num, generator=g) * 0.05).to(dtype)
    wb = (torch.randn(S, R, N, generator=g) * 0.05).to(dtype)
    ranks = torch.tensor([0, 3, 8, 5], dtype=torch.int32)
    scal = torch.tensor([0.0, 1.5, 2.0, 3.0], dtype=torch.float32)
    seq = torch.tensor([10, 0, 7, 12, 3, 10], dtype=torch.int32)
    widx = torch.tensor([1, 2, 0, 3, 2, 1], dtype=torch.int64)
    tmp = sgmv.sgmv_lora_a_fwd(x.to(gpu), wa.to(gpu), seq.to(gpu), widx.to(gpu), ranks.to(gpu), stack_num)
    exp_tmp, valid = sgmv_shrink_reference(x, wa, seq, widx, ranks, stack_num)
    torch.testing.assert_close(tmp.cpu()[valid], exp_tmp[valid], **tol_for(dtype))
    # expand over the oracle's intermediate (zeros outside the valid region)
    base = torch.randn(Bt, M, N, generator=g).to(dtype)
    xb = exp_tmp[:, :, :R].contiguous()
    out = sgmv.sgmv_lora_b_fwd(xb.to(gpu), wb.to(gpu), seq.to(gpu), widx.to(gpu), ranks.to(gpu), scal.to(gpu), base.to(gpu))
    expect = sgmv_expand_reference(xb, wb, seq, widx, ranks, scal, base)
    torch.testing.assert_close(out.cpu(), expect, **tol_for(dtype))


def test_isolated_sgmv_config_bf16(gpu):
    """T=4096 tokens, K=N=4096, 16 slots + base, ranks cycling {0,4,8,16}, Dirichlet segments."""
    _announce(test="isolated_sgmv_4096")
    from bench import isolated_sgmv_workload

    wl = isolated_sgmv_workload(gpu, seed=1002)
    sgmv.lora_apply(wl.x, wl.y, wl.cache, "op", wl.plan)
    torch.cuda.synchronize()
    A, B, rk, sc = oracle_slot_tensors(wl.cache, wl.adapters, "op", torch.bfloat16)
    A, B, rk, sc = A.to(gpu), B.to(gpu), rk.to(gpu), sc.to(gpu)
    expect = reference_forward(
        wl.x.view(-1, 1, 4096), wl.base.view(-1, 1, 4096), wl.seq_lens, wl.row_slot, A, B, rk, sc
    ).view(-1, 4096)
    torch.testing.assert_close(wl.y, expect, rtol=2e-2, atol=1e-2)
    # tokens of rank-0 slots are untouched
    zero = (rk[wl.row_slot.long()] == 0).cpu()
    assert torch.equal(wl.y.cpu()[zero], wl.base.cpu()[zero])
    np.testing.assert_array_equal(np.bincount(wl.row_slot.cpu().numpy(), minlength=17).sum(), 4096)


def test_prefill_config_stacked_fused_bf16(gpu):
    """Prefill size: 32 rows x 1024, lengths U[512,1024], 8 adapters (4 x r16, 4 x r32), q/k/v of a
    4096-wide model in one stacked fused launch, every token against the oracle."""
    _announce(test="prefill_config_stacked_fused")
    g = torch.Generator().manual_seed(1004)
    K, B, S = 4096, 32, 1024
    shapes = {"q": (K, 4096), "k": (K, 1024), "v": (K, 1024)}
    adapters = {f"p{i}": {m: peft_layer(g, fi, fo, 16 if i < 4 else 32, 2.0 * (16 if i < 4 else 32))
                          for m, (fi, fo) in shapes.items()} for i in range(8)}
    cache = make_cache(adapters, shapes, 8, 32, gpu, torch.bfloat16)
    row_slot = cache.ensure_resident([f"p{i // 4}" for i in range(B)])
    seq_lens = torch.randint(512, S + 1, (B,), generator=g, dtype=torch.int32)
    plan = sgmv.SgmvPlan(row_slot, seq_lens.to(gpu), S, cache.num_slots, distinct_slots=8)
    assert plan.group_tokens == 64 and sgmv.fused_ok(plan, cache, K)
    gg = torch.Generator(device=gpu).manual_seed(1004)
    x = torch.randn(B * S, K, generator=gg, device=gpu).to(torch.bfloat16)
    base = {m: torch.randn(B * S, fo, generator=gg, device=gpu).to(torch.bfloat16) for m, (fi, fo) in shapes.items()}
    ys = [base[m].clone() for m in shapes]
    sgmv.lora_fused_stacked(x, ys, cache, list(shapes), plan)
    torch.cuda.synchronize()
    for m, y in zip(shapes, ys):
        A, Bm, rk, sc = (t.to(gpu) for t in oracle_slot_tensors(cache, adapters, m, torch.bfloat16))
        expect = reference_forward(x.view(B, S, K), base[m].view(B, S, -1), seq_lens.to(gpu), row_slot, A, Bm, rk, sc)
        torch.testing.assert_close(y.view(B, S, -1), expect, rtol=2e-2, atol=1e-2)
        pad = torch.arange(S)[None, :] >= seq_lens[:, None]  # padding tokens keep the base output
        assert torch.equal(y.view(B, S, -1)[pad.to(gpu)], base[m].view(B, S, -1)[pad.to(gpu)])


def test_decode_config_stacked_split_bf16(gpu):
    """Decode size: 256 rows of one token, 64 adapters of ranks {8,16,32,64}, Zipf(1.1) choice with 10%
    base rows; every module of a Llama-3-8B layer as the decode step launches it: q/k/v through one
    stacked shrink and one stacked expand, o (4096 -> 4096) alone, gate/up (4096 -> 14336 each) stacked,
    and down (K=14336, more K splits) alone, every row against the oracle at the plain tolerance."""
    _announce(test="decode_config_stacked_split")
    from bench import zipf_ids

    g = torch.Generator().manual_seed(1003)
    rng = np.random.default_rng(1003)
    shapes = {"q": (4096, 4096), "k": (4096, 1024), "v": (4096, 1024), "o": (4096, 4096), "gate": (4096, 14336),
              "up": (4096, 14336), "down": (14336, 4096)}
    names = [f"d{i:02d}" for i in range(64)]
    ranks = {n: int(rng.choice([8, 16, 32, 64])) for n in names}
    adapters = {n: {m: peft_layer(g, fi, fo, ranks[n], 2.0 * ranks[n]) for m, (fi, fo) in shapes.items()} for n in names}
    cache = make_cache(adapters, shapes, 64, 64, gpu, torch.bfloat16)
    ids = zipf_ids(rng, 256, 64, 1.1, 0.1, names)
    row_slot = cache.ensure_resident(ids)
    distinct = len({a for a in ids if a != "__base__"})
    seq = torch.ones(256, dtype=torch.int32, device=gpu)
    plan = sgmv.SgmvPlan(row_slot, seq, 1, cache.num_slots, distinct_slots=distinct)
    assert plan.group_tokens == 16 and not sgmv.fused_ok(plan, cache, 4096)
    gg = torch.Generator(device=gpu).manual_seed(1003)
    xs = {m: torch.randn(256, fi, generator=gg, device=gpu).to(torch.bfloat16) for m, (fi, fo) in shapes.items()}
    for m in ("k", "v"):
        xs[m] = xs["q"]
    xs["up"] = xs["gate"]
    base = {m: torch.randn(256, fo, generator=gg, device=gpu).to(torch.bfloat16) for m, (fi, fo) in shapes.items()}
    ys = {m: base[m].clone() for m in shapes}
    for run in (["q", "k", "v"], ["gate", "up"]):
        results = sgmv.lora_shrink_stacked(xs[run[0]], cache, run, plan)
        sgmv.lora_expand_stacked(results, [ys[m] for m in run], cache, run)
    for m in ("o", "down"):
        res = sgmv.lora_shrink(xs[m], cache, m, plan)
        sgmv.lora_expand(res, ys[m], cache, m)
    torch.cuda.synchronize()
    for m, (fi, fo) in shapes.items():
        A, Bm, rk, sc = (t.to(gpu) for t in oracle_slot_tensors(cache, adapters, m, torch.bfloat16))
        expect = reference_forward(xs[m].view(256, 1, fi), base[m].view(256, 1, fo), seq, row_slot, A, Bm, rk, sc)
        torch.testing.assert_close(ys[m].view(256, 1, fo), expect, rtol=2e-2, atol=1e-2, msg=lambda s, m=m: f"{m}: {s}")
        untouched = (row_slot == 0)
        assert torch.equal(ys[m][untouched], base[m][untouched])


def _small_case(gpu, dtype=torch.bfloat16, rows=40, M=3, K=1024, N=512, ranks=(4, 16, 33, 64), seed=50):
    g = torch.Generator().manual_seed(seed)
    adapters = _adapters(g, list(ranks), K, N)
    ids = list(adapters) + ["__base__"]
    cache = make_cache(adapters, {"m": (K, N)}, len(adapters), 64, gpu, dtype)
    adapter_ids = [ids[i] for i in torch.randint(0, len(ids), (rows,), generator=g).tolist()]
    row_slot = cache.ensure_resident(adapter_ids)
    seq_lens = torch.randint(0, M + 1, (rows,), generator=g, dtype=torch.int32)
    x = torch.randn(rows, M, K, generator=g).to(dtype)
    base = torch.randn(rows, M, N, generator=g).to(dtype)
    return adapters, cache, row_slot, seq_lens, x, base


def test_split_k_bitwise_reproducible(gpu):
    _announce(test="reproducible")
    adapters, cache, row_slot, seq_lens, x, base = _small_case(gpu)
    M, K, N = x.shape[1], x.shape[2], base.shape[2]
    plan = sgmv.SgmvPlan(row_slot, seq_lens.to(gpu), M, cache.num_slots, group_tokens=16)
    outs = []
    for _ in range(3):
        y = base.to(gpu)
        sgmv.lora_apply(x.to(gpu).view(-1, K), y.view(-1, N), cache, "m", plan, k_splits=4)
        outs.append(y.cpu())
    assert torch.equal(outs[0], outs[1]) and torch.equal(outs[0], outs[2])
    A, B, rk, sc = oracle_slot_tensors(cache, adapters, "m", torch.bfloat16)
    expect = reference_forward(x, base, seq_lens, row_slot.cpu(), A, B, rk, sc)
    torch.testing.assert_close(outs[0], expect, **tol_for(torch.bfloat16))


def test_separate_shrink_expand_equal_fused(gpu):
    """pl_sgmv_shrink + pl_sgmv_expand (planes from pl_shrink_planes) == pl_lora_apply, bit for bit."""
    _announce(test="separate_vs_fused")
    from bench import SgmvLaunch

    _, cache, row_slot, seq_lens, x, base = _small_case(gpu, seed=51)
    M, K, N = x.shape[1], x.shape[2], base.shape[2]
    for splits, group_tokens in ((1, 64), (2, 16), (5, 64), (3, 16)):
        plan = sgmv.SgmvPlan(row_slot, seq_lens.to(gpu), M, cache.num_slots, group_tokens=group_tokens)
        y1 = base.to(gpu)
        sgmv.lora_apply(x.to(gpu).view(-1, K), y1.view(-1, N), cache, "m", plan, k_splits=splits)
        y2 = base.to(gpu)
        launch = SgmvLaunch(x.to(gpu).view(-1, K), y2.view(-1, N), cache, "m", plan, k_splits=splits)
        launch.shrink()
        launch.expand()
        torch.cuda.synchronize()
        assert torch.equal(y1.cpu(), y2.cpu()), (splits, group_tokens)


def test_triton_epilogue_order(gpu):
    """PL_EPI_TRITON: y = T(T(acc * scale) + y) over T(x @ A) (sgmv.py:130-134, :268-275)."""
    _announce(test="triton_epilogue")
    from oracle.lora import dense_slot_tensors
    from polylora_amd import _native

    adapters, cache, row_slot, seq_lens, x, base = _small_case(gpu, seed=52)
    M, K, N = x.shape[1], x.shape[2], base.shape[2]
    plan = sgmv.SgmvPlan(row_slot, seq_lens.to(gpu), M, cache.num_slots)
    y = base.to(gpu)
    sgmv.lora_apply(x.to(gpu).view(-1, K), y.view(-1, N), cache, "m", plan, epilogue=_native.PL_EPI_TRITON)
    A, B, rk, sc = oracle_slot_tensors(cache, adapters, "m", torch.bfloat16)
    tmp, _ = sgmv_shrink_reference(x, A, seq_lens, row_slot.cpu(), rk)
    expect = sgmv_expand_reference(tmp, B, seq_lens, row_slot.cpu(), rk, sc, base)
    torch.testing.assert_close(y.cpu(), expect, **tol_for(torch.bfloat16))


def test_lora_apply_graph_replays(gpu):
    """Plan + two modules captured in a HIP graph; every replay equals the eager result bit for bit."""
    _announce(test="graph_replay")
    g = torch.Generator().manual_seed(53)
    K, N, rows = 1024, 768, 48
    shapes = {"q": (K, N), "o": (N, K)}
    adapters = {f"a{i}": {m: peft_layer(g, fi, fo, r, 2.0 * r) for m, (fi, fo) in shapes.items()} for i, r in enumerate([8, 16, 64])}
    cache = make_cache(adapters, shapes, 3, 64, gpu, torch.bfloat16)
    ids = list(adapters) + ["__base__"]
    row_slot = cache.ensure_resident([ids[i] for i in torch.randint(0, 4, (rows,), generator=g).tolist()])
    seq_lens = torch.ones(rows, dtype=torch.int32, device=gpu)
    x = torch.randn(rows, K, generator=g).to(torch.bfloat16).to(gpu)
    y0 = torch.randn(rows, N, generator=g).to(torch.bfloat16).to(gpu)
    z0 = torch.randn(rows, K, generator=g).to(torch.bfloat16).to(gpu)
    y, z = y0.clone(), z0.clone()

    def step():
        y.copy_(y0)
        z.copy_(z0)
        plan = sgmv.SgmvPlan(row_slot, seq_lens, 1, cache.num_slots)
        sgmv.lora_apply(x, y, cache, "q", plan)
        sgmv.lora_apply(y, z, cache, "o", plan)

    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        step()
    torch.cuda.current_stream().wait_stream(s)
    torch.cuda.synchronize()
    want_y, want_z = y.clone(), z.clone()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        step()
    for i in range(4):
        y.fill_(float(i))  # eager work between replays
        z.zero_()
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        assert torch.equal(y, want_y) and torch.equal(z, want_z), i


@pytest.mark.parametrize("group_tokens", [16, 64])
def test_stacked_shrink_equals_separate(gpu, group_tokens):
    """pl_sgmv_shrink_stacked over q/k/v-like modules == one pl_sgmv_shrink per module, bit for bit."""
    _announce(test="stacked_shrink", group_tokens=group_tokens)
    g = torch.Generator().manual_seed(60)
    K, rows = 512, 70
    shapes = {"q": (K, 512), "k": (K, 128), "v": (K, 136)}
    adapters = {}
    for i, r in enumerate([8, 24, 64]):
        adapters[f"s{i}"] = {m: peft_layer(g, fi, fo, r, 2.0 * r) for m, (fi, fo) in shapes.items() if not (i == 1 and m == "k")}
    cache = make_cache(adapters, shapes, 3, 64, gpu, torch.bfloat16)
    ids = list(adapters) + ["__base__"]
    row_slot = cache.ensure_resident([ids[i] for i in torch.randint(0, 4, (rows,), generator=g).tolist()])
    seq = torch.ones(rows, dtype=torch.int32, device=gpu)
    plan = sgmv.SgmvPlan(row_slot, seq, 1, cache.num_slots, group_tokens=group_tokens)
    x = torch.randn(rows, K, generator=g).to(torch.bfloat16).to(gpu)
    base = {m: torch.randn(rows, fo, generator=g).to(torch.bfloat16).to(gpu) for m, (fi, fo) in shapes.items()}
    # separate
    sep = {}
    for m in shapes:
        y = base[m].clone()
        res = sgmv.lora_shrink(x, cache, m, plan)
        sgmv.lora_expand(res, y, cache, m)
        sep[m] = y
    # stacked
    results = sgmv.lora_shrink_stacked(x, cache, list(shapes), plan)
    for m, res in zip(shapes, results):
        y = base[m].clone()
        sgmv.lora_expand(res, y, cache, m)
        assert torch.equal(y, sep[m]), m
    # one stacked expand over all three modules
    ys = [base[m].clone() for m in shapes]
    sgmv.lora_expand_stacked(results, ys, cache, list(shapes))
    for m, y in zip(shapes, ys):
        assert torch.equal(y, sep[m]), m
    # results of two different shrinks cannot share one expand (position 0 is
    # rewritten by the second shrink, so pair it with position 1's result)
    other = sgmv.lora_shrink(x, cache, "k", sgmv.SgmvPlan(row_slot, seq, 1, cache.num_slots, group_tokens=group_tokens))
    with pytest.raises(ValueError, match="one stacked shrink"):
        sgmv.lora_expand_stacked([results[1], other], [ys[1], ys[1].clone()], cache, ["k", "k"])
    # a later shrink on position 0 invalidates the first stacked result only
    sgmv.lora_shrink(x, cache, "q", plan)
    assert not results[0].valid and results[1].valid and results[2].valid
    with pytest.raises(RuntimeError, match="overwritten"):
        sgmv.lora_expand(results[0], base["q"].clone(), cache, "q")
    for m in shapes:
        A, B, rk, sc = oracle_slot_tensors(cache, adapters, m, torch.bfloat16)
        expect = reference_forward(x.cpu().view(rows, 1, K), base[m].cpu().view(rows, 1, -1), seq.cpu(), row_slot.cpu(), A, B, rk, sc)
        torch.testing.assert_close(sep[m].cpu(), expect.view(rows, -1), **tol_for(torch.bfloat16))
