"""Seeded random shapes through every kernel path, against the oracle.

Each case draws a dtype, a batch (rows x positions with ragged lengths, some
rows of length 0, some on the base adapter), K and N (whole 16-byte chunks,
mostly not multiples of the tile sizes), and adapters of random ranks up to a
random max_rank (some lacking the module, so their rows stay untouched).  It
then runs the split shrink + expand (16- and 64-token groups, the split count
drawn too), the fused kernel (where its rank limit allows), the one-launch
decode path (bit for bit against the split pair on the same plan and split
count), the row kernels, and the operator API's sgmv_lora_a_fwd /
sgmv_lora_b_fwd on the reference slot layout.  Further cases run 2..4 sibling
modules through the stacked launches, and the operator API alone with its
stack_num, index types, out-of-range indices and kept-part rebuilds.  Every
output is checked against the oracle at the dtype's tolerance (tests/_util.py:
CountedParity for outputs that add into a base, the plain tolerance for the
intermediate).

Reference: the fallback of layers.py:112-134 (reference_forward), the
operator signatures of sgmv.py:141-175 and :278-328.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

from oracle.lora import reference_forward, sgmv_expand_reference, sgmv_shrink_reference
from polylora_amd import refop_cache, sgmv
from tests._util import CountedParity, make_cache, oracle_slot_tensors, peft_layer, tol_for

pytestmark = pytest.mark.gpu

_DTYPES = (torch.bfloat16, torch.float16, torch.float32)


def _announce(**kw):
    print("case:", ", ".join(f"{k}={v}" for k, v in kw.items()), flush=True)


def _draw(seed: int) -> dict:
    r = np.random.default_rng(1000 + seed)
    dtype = _DTYPES[int(r.integers(3))]
    e = 4 if dtype == torch.float32 else 8  # elements per 16 bytes
    M = int(r.choice([1, 1, 1, 2, 3, 17, 64]))
    max_rank = int(r.choice([8, 16, 32, 64]))
    n_ad = int(r.integers(1, 13))
    ranks = [int(v) for v in r.integers(0, max_rank + 1, n_ad)]
    ranks[-1] = max_rank
    tokens = int(r.choice([2048, 2048, 8192]))  # at most, over rows x positions
    return dict(dtype=dtype, K=e * int(r.integers(1, 513)), N=e * int(r.integers(1, 513)), M=M,
                rows=int(r.integers(1, max(2, tokens // M))), ranks=ranks, max_rank=max_rank,
                base_frac=float(r.uniform(0.0, 0.3)), k_splits=int(r.choice([1, 2, 3, 4, 8])))


@pytest.mark.parametrize("seed", range(48))
def test_random_shapes_every_path_against_the_oracle(gpu, seed):
    c = _draw(seed)
    dtype, K, N, M, rows = c["dtype"], c["K"], c["N"], c["M"], c["rows"]
    _announce(test="sweep", seed=seed, **{k: v for k, v in c.items() if k != "dtype"}, dtype=dtype)
    g = torch.Generator().manual_seed(seed)
    adapters = {}
    for i, rk in enumerate(c["ranks"]):
        # rank 0: the adapter lacks the module (another module keeps it loadable)
        adapters[f"a{i:02d}"] = ({"m": peft_layer(g, K, N, rk, 2.0 * rk)} if rk else
                                 {"other": peft_layer(g, 8, 8, 2, 4.0)})
    cache = make_cache(adapters, {"m": (K, N), "other": (8, 8)}, len(adapters), c["max_rank"], gpu, dtype)
    names = list(adapters)
    pick = torch.randint(0, len(names), (rows,), generator=g).tolist()
    on_base = (torch.rand(rows, generator=g) < c["base_frac"]).tolist()
    adapter_ids = ["__base__" if b else names[i] for i, b in zip(pick, on_base)]
    row_slot = cache.ensure_resident(adapter_ids)
    seq = torch.randint(0, M + 2, (rows,), generator=g, dtype=torch.int32)
    x = torch.randn(rows, M, K, generator=g).to(dtype)
    base = torch.randn(rows, M, N, generator=g).to(dtype)
    A, B, rk, sc = oracle_slot_tensors(cache, adapters, "m", dtype)
    slots = row_slot.cpu()
    want = reference_forward(x, base, seq, slots, A, B, rk, sc)
    untouched = torch.ones(rows, M, dtype=torch.bool)
    for b in range(rows):
        if int(rk[int(slots[b])]) > 0:
            untouched[b, : min(int(seq[b]), M)] = False
    dx, dseq = x.to(gpu).view(-1, K), seq.to(gpu)
    parity = CountedParity(dtype, f"sweep seed {seed}")

    def check(y: torch.Tensor, path: str) -> None:
        got = y.cpu().view(rows, M, N)
        parity.check(got, want, base, f" [{path}]")
        assert torch.equal(got[untouched], base[untouched]), f"{path}: untouched rows were written"

    # split shrink + expand, both group sizes, the drawn split count
    for gt in (16, 64):
        plan = sgmv.SgmvPlan(row_slot, dseq, M, cache.num_slots, group_tokens=gt)
        _announce(path="split", group_tokens=gt)
        y = base.to(gpu).view(-1, N)
        sgmv.lora_apply(dx, y, cache, "m", plan, k_splits=c["k_splits"])
        check(y, f"split gt{gt}")
        if cache.rank8_cap <= sgmv.FUSED_MAX_RANK:
            _announce(path="fused", group_tokens=gt)
            y = base.to(gpu).view(-1, N)
            sgmv.lora_fused(dx, y, cache, "m", plan)
            check(y, f"fused gt{gt}")
        if sgmv.decode_ok(plan):
            _announce(path="decode", group_tokens=gt)
            pair = base.to(gpu).view(-1, N)
            res = sgmv.lora_shrink_stacked(dx, cache, ["m"], plan, k_splits=c["k_splits"])
            sgmv.lora_expand_stacked(res, [pair], cache, ["m"])
            y = base.to(gpu).view(-1, N)
            sgmv.lora_decode_stacked(dx, [y], cache, ["m"], plan, k_splits=c["k_splits"])
            torch.cuda.synchronize()
            assert torch.equal(y, pair), "decode launch differs from the split pair"
            assert not sgmv.decode_waits_timed_out(gpu)
            check(y, f"decode gt{gt}")
    _announce(path="rows")
    y = base.to(gpu).view(-1, N)
    sgmv.lora_apply_rows(dx, y, cache, "m", row_slot, dseq, M)
    check(y, "rows")

    # the operator API on the reference slot layout (slot 0 the base adapter, rank 0)
    _announce(path="operator")
    refop_cache.configure()
    try:
        dA, dB, drk, dsc, dslots = (t.to(gpu) for t in (A, B, rk, sc, slots))
        exp_tmp, valid = sgmv_shrink_reference(x, A, seq, slots, rk)
        for call in range(2):  # the second call runs on the kept parts
            tmp = sgmv.sgmv_lora_a_fwd(x.to(gpu), dA, dseq, dslots, drk).cpu()
            torch.testing.assert_close(tmp[valid], exp_tmp[valid], **tol_for(dtype))
        exp_out = sgmv_expand_reference(exp_tmp, B, seq, slots, rk, sc, base)
        for call in range(2):
            out = sgmv.sgmv_lora_b_fwd(exp_tmp.to(gpu), dB, dseq, dslots, drk, dsc, base.to(gpu)).cpu()
            parity.check(out, exp_out, base, " [operator b]")
            assert torch.equal(out[untouched], base[untouched]), "operator b: untouched rows were written"
    finally:
        refop_cache.configure()
    parity.finish()


@pytest.mark.parametrize("seed", range(16))
def test_random_sibling_modules_in_one_launch_against_the_oracle(gpu, seed):
    """2..4 sibling modules fed the same x (different N, and adapters that have only some of them) through
    the stacked launches: fused, split shrink + expand, and the decode launch (bit for bit against the
    stacked split pair); each module's output against the oracle."""
    r = np.random.default_rng(5000 + seed)
    dtype = _DTYPES[int(r.integers(3))]
    e = 4 if dtype == torch.float32 else 8
    n_mod = int(r.integers(2, 5))
    K = e * int(r.integers(1, 513))
    outs = [e * int(r.integers(1, 513)) for _ in range(n_mod)]
    M = int(r.choice([1, 1, 2, 9]))
    rows = int(r.integers(1, max(2, 2048 // M)))
    max_rank = int(r.choice([16, 32, 64]))
    n_ad = int(r.integers(1, 9))
    k_splits = int(r.choice([1, 2, 4, 8]))
    mods = [f"m{i}" for i in range(n_mod)]
    _announce(test="sweep_stacked", seed=seed, dtype=dtype, K=K, outs=outs, M=M, rows=rows, max_rank=max_rank,
              adapters=n_ad, k_splits=k_splits)
    g = torch.Generator().manual_seed(seed)
    adapters = {}
    for i in range(n_ad):
        layers = {}
        for m, n in zip(mods, outs):
            rk = int(r.integers(0, max_rank + 1))
            if rk:
                layers[m] = peft_layer(g, K, n, rk, 2.0 * rk)
        adapters[f"a{i:02d}"] = layers or {"other": peft_layer(g, 8, 8, 2, 4.0)}
    shapes = dict({m: (K, n) for m, n in zip(mods, outs)}, other=(8, 8))
    cache = make_cache(adapters, shapes, len(adapters), max_rank, gpu, dtype)
    names = list(adapters) + ["__base__"]
    ids = [names[i] for i in torch.randint(0, len(names), (rows,), generator=g).tolist()]
    row_slot = cache.ensure_resident(ids)
    seq = torch.randint(0, M + 2, (rows,), generator=g, dtype=torch.int32)
    x = torch.randn(rows, M, K, generator=g).to(dtype)
    bases = [torch.randn(rows, M, n, generator=g).to(dtype) for n in outs]
    slots = row_slot.cpu()
    wants, untouched = [], []
    for m, b0 in zip(mods, bases):
        A, B, rk, sc = oracle_slot_tensors(cache, adapters, m, dtype)
        wants.append(reference_forward(x, b0, seq, slots, A, B, rk, sc))
        u = torch.ones(rows, M, dtype=torch.bool)
        for b in range(rows):
            if int(rk[int(slots[b])]) > 0:
                u[b, : min(int(seq[b]), M)] = False
        untouched.append(u)
    dx, dseq = x.to(gpu).view(-1, K), seq.to(gpu)
    parity = CountedParity(dtype, f"stacked sweep seed {seed}")

    def check(ys, path):
        for m, y, w, b0, u in zip(mods, ys, wants, bases, untouched):
            got = y.cpu().view(rows, M, -1)
            parity.check(got, w, b0, f" [{path} {m}]")
            assert torch.equal(got[u], b0[u]), f"{path} {m}: untouched rows were written"

    for gt in (16, 64):
        plan = sgmv.SgmvPlan(row_slot, dseq, M, cache.num_slots, group_tokens=gt)
        _announce(path="stacked split", group_tokens=gt)
        pair = [b.to(gpu).view(-1, b.shape[-1]) for b in bases]
        res = sgmv.lora_shrink_stacked(dx, cache, mods, plan, k_splits=k_splits)
        sgmv.lora_expand_stacked(res, pair, cache, mods)
        check(pair, f"split gt{gt}")
        if cache.rank8_cap <= sgmv.FUSED_MAX_RANK:
            _announce(path="stacked fused", group_tokens=gt)
            ys = [b.to(gpu).view(-1, b.shape[-1]) for b in bases]
            sgmv.lora_fused_stacked(dx, ys, cache, mods, plan)
            check(ys, f"fused gt{gt}")
        if sgmv.decode_ok(plan):
            _announce(path="stacked decode", group_tokens=gt)
            ys = [b.to(gpu).view(-1, b.shape[-1]) for b in bases]
            sgmv.lora_decode_stacked(dx, ys, cache, mods, plan, k_splits=k_splits)
            torch.cuda.synchronize()
            for m, a, b in zip(mods, ys, pair):
                assert torch.equal(a, b), f"decode launch differs from the split pair ({m})"
            assert not sgmv.decode_waits_timed_out(gpu)
    parity.finish()


@pytest.mark.parametrize("seed", range(24))
def test_random_operator_calls_against_the_oracle(gpu, seed):
    """The reference operator API (sgmv_lora_a_fwd / sgmv_lora_b_fwd) on seeded random reference-layout
    tensors: stack_num 1..3, int32 or int64 indices (some out of range, which the kernels skip), rows whose
    seq_len exceeds M, rank caps up to 96 (above 64 the row kernels run), base_output given or not.  Each
    call is made twice (the second on the kept parts), then again after an in-place write to the weights
    (which must rebuild what was kept); every result against the oracle."""
    r = np.random.default_rng(6000 + seed)
    dtype = _DTYPES[int(r.integers(3))]
    e = 4 if dtype == torch.float32 else 8
    stack = int(r.integers(1, 4))
    R = int(r.choice([4, 8, 16, 32, 64, 96 // stack]))  # R * stack above 64: the row kernels
    S = int(r.integers(2, 20))
    M = int(r.choice([1, 1, 4, 33]))
    Bt = int(r.integers(1, max(2, 1536 // M)))
    K, N = e * int(r.integers(1, 385)), e * int(r.integers(1, 385))
    idx_dtype = (torch.int32, torch.int64)[int(r.integers(2))]
    with_base = bool(r.integers(2))
    _announce(test="sweep_operator", seed=seed, dtype=dtype, stack=stack, R=R, S=S, M=M, Bt=Bt, K=K, N=N,
              idx=idx_dtype, with_base=with_base)
    g = torch.Generator().manual_seed(seed)
    x = torch.randn(Bt, M, K, generator=g).to(dtype)
    wa = (torch.randn(S, K, R * stack, generator=g) * 0.05).to(dtype)
    wb = (torch.randn(S, R, N, generator=g) * 0.05).to(dtype)
    ranks = torch.randint(0, R + 1, (S,), generator=g, dtype=torch.int32)
    ranks[0] = 0
    scal = torch.rand(S, generator=g) * 4
    seq = torch.randint(0, M + 3, (Bt,), generator=g, dtype=torch.int32)
    widx = torch.randint(-1, S + 1, (Bt,), generator=g).to(idx_dtype)  # -1 and S: out of range, skipped
    ok = (widx >= 0) & (widx < S)
    base = torch.randn(Bt, M, N, generator=g).to(dtype)
    dx, dwa, dwb, dranks, dscal, dseq, dwidx = (t.to(gpu) for t in (x, wa, wb, ranks, scal, seq, widx))
    tol = tol_for(dtype)
    refop_cache.configure()
    try:
        for phase in range(2):
            if phase == 1:  # an in-place write, as the reference cache's slot loads make
                wa[1:] *= 0.5
                wb[1:] *= 2.0
                dwa.mul_(torch.tensor([1.0] + [0.5] * (S - 1), dtype=dtype, device=gpu).view(S, 1, 1))
                dwb.mul_(torch.tensor([1.0] + [2.0] * (S - 1), dtype=dtype, device=gpu).view(S, 1, 1))
                torch.testing.assert_close(dwa.cpu(), wa, rtol=0, atol=0)
            # the oracle takes the rows whose index is in range; the kernels leave the others untouched
            exp_tmp, valid = sgmv_shrink_reference(x[ok], wa, seq[ok], widx[ok], ranks, stack)
            for call in range(2):
                tmp = sgmv.sgmv_lora_a_fwd(dx, dwa, dseq, dwidx, dranks, stack).cpu()
                torch.testing.assert_close(tmp[ok][valid], exp_tmp[valid], **tol)
            xb = torch.zeros(Bt, M, R, dtype=dtype)
            xb[ok] = exp_tmp[:, :, :R]
            start = base if with_base else torch.zeros_like(base)
            exp_out = start.clone()
            exp_out[ok] = sgmv_expand_reference(xb[ok], wb, seq[ok], widx[ok], ranks, scal, start[ok])
            for call in range(2):
                out = sgmv.sgmv_lora_b_fwd(xb.to(gpu), dwb, dseq, dwidx, dranks, dscal,
                                           base.to(gpu) if with_base else None).cpu()
                torch.testing.assert_close(out, exp_out, **tol)
                assert torch.equal(out[~ok], start[~ok])
    finally:
        refop_cache.configure()
