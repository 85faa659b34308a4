"""Pins the oracle (CPU restatement of the reference) before the GPU tests compare against it.

Each oracle function is checked against something that does not share its
code: fp64 brute-force loops on tiny inputs, the textbook LoRA closed form
y = W x + b + (alpha / r) B A x, invariants of the reference's fallback
(layers.py:112-134), and the assertions of the reference's own tests.  Each
check is shown to catch a planted mistake (a dropped scale, a transposed
operand, an off-by-one slice, a wrong slot), planted on the CPU in a mutated
copy of the oracle.
"""

from __future__ import annotations

import itertools

import numpy as np
import pytest
import torch

from oracle import lora, plan, slots

# --------------------------------------------------------------------------- helpers


def _brute_lora(x, base, seq_lens, widx, A, B, ranks, scales):
    """fp64 element loops: out[b,m,n] = base + scale * sum_j (sum_k x[b,m,k] A[s,k,j]) B[s,j,n]."""
    rows, M, K = x.shape
    N = base.shape[2]
    out = base.double().clone()
    for b in range(rows):
        s = int(widx[b])
        r = int(ranks[s])
        L = min(max(int(seq_lens[b]), 0), M)
        for m in range(L):
            for n in range(N):
                acc = 0.0
                for j in range(r):
                    t = sum(float(x[b, m, k]) * float(A[s, k, j]) for k in range(K))
                    acc += t * float(B[s, j, n])
                out[b, m, n] += float(scales[s]) * acc
    return out


def _random_bank(gen, slots_n, K, N, R, ranks, dtype=torch.float32, noise_beyond_rank=True):
    A = torch.randn(slots_n, K, R, generator=gen, dtype=torch.float64)
    B = torch.randn(slots_n, R, N, generator=gen, dtype=torch.float64)
    if not noise_beyond_rank:
        for s, r in enumerate(ranks):
            A[s, :, r:] = 0
            B[s, r:, :] = 0
    rk = torch.tensor(ranks, dtype=torch.int32)
    sc = torch.tensor([0.0 if r == 0 else 2.0 / max(r, 1) * 3 for r in ranks], dtype=torch.float32)
    return A.to(dtype), B.to(dtype), rk, sc


# --------------------------------------------------------------------------- reference_forward


@pytest.mark.parametrize("seed", [0, 1, 2])
def test_reference_forward_matches_brute_force_fp32(seed):
    g = torch.Generator().manual_seed(seed)
    rows, M, K, N, R = 5, 3, 6, 4, 4
    ranks = [0, 1, 3, 4]
    A, B, rk, sc = _random_bank(g, 4, K, N, R, ranks)
    x = torch.randn(rows, M, K, generator=g)
    base = torch.randn(rows, M, N, generator=g)
    seq = torch.tensor([3, 0, 2, 5, 1], dtype=torch.int32)  # 5 > M exercises the slice clamp
    widx = torch.tensor([1, 2, 0, 3, 2])
    got = lora.reference_forward(x, base, seq, widx, A, B, rk, sc)
    want = _brute_lora(x, base, seq, widx, A, B, rk, sc)
    torch.testing.assert_close(got.double(), want, rtol=1e-5, atol=1e-5)


def test_reference_forward_closed_form_textbook_lora():
    """PEFT's y = W x + b + (alpha/r) * lora_B(lora_A(x)) with dropout 0 (tiny Linear)."""
    g = torch.Generator().manual_seed(5)
    K, N, r, alpha = 7, 5, 3, 9.0
    lin = torch.nn.Linear(K, N)
    lora_A = torch.randn(r, K, generator=g)
    lora_B = torch.randn(N, r, generator=g)
    x = torch.randn(2, 4, K, generator=g)
    with torch.no_grad():
        base = lin(x)
        textbook = base + (alpha / r) * torch.nn.functional.linear(torch.nn.functional.linear(x, lora_A), lora_B)
    a_t, b_t, rank, scale = lora.store_layout(lora_A, lora_B, alpha)
    A = torch.zeros(2, K, 4)
    B = torch.zeros(2, 4, N)
    A[1, :, :rank] = a_t
    B[1, :rank] = b_t
    rk = torch.tensor([0, rank], dtype=torch.int32)
    sc = torch.tensor([0.0, scale])
    got = lora.reference_forward(x, base, torch.tensor([4, 4]), torch.tensor([1, 1]), A, B, rk, sc)
    torch.testing.assert_close(got, textbook, rtol=1e-5, atol=1e-5)
    assert scale == 3.0  # 9 / 3: the non-power-of-two scale of the reference's second test


def test_reference_forward_invariants():
    g = torch.Generator().manual_seed(7)
    rows, M, K, N, R = 6, 4, 8, 5, 4
    A, B, rk, sc = _random_bank(g, 3, K, N, R, [0, 2, 4])
    x = torch.randn(rows, M, K, generator=g)
    base = torch.randn(rows, M, N, generator=g)
    seq = torch.tensor([4, 2, 0, 3, 4, 1], dtype=torch.int32)
    widx = torch.tensor([0, 1, 2, 2, 1, 0])
    out = lora.reference_forward(x, base, seq, widx, A, B, rk, sc)
    # base-slot rows, zero-length rows and padding tokens are bitwise base
    untouched = torch.ones(rows, M, dtype=torch.bool)
    for b in range(rows):
        if int(rk[int(widx[b])]) > 0:
            untouched[b, : int(seq[b])] = False
    assert torch.equal(out[untouched], base[untouched])
    assert not torch.equal(out[~untouched], base[~untouched])
    # entries beyond each slot's rank are never read
    A2, B2 = A.clone(), B.clone()
    A2[1, :, 2:] = 1e6
    B2[1, 2:, :] = -1e6
    assert torch.equal(lora.reference_forward(x, base, seq, widx, A2, B2, rk, sc), out)
    # linear in B: delta(2B) = 2 delta(B)
    d1 = lora.reference_forward(x, base, seq, widx, A, B, rk, sc) - base
    d2 = lora.reference_forward(x, base, seq, widx, A, 2 * B, rk, sc) - base
    torch.testing.assert_close(d2, 2 * d1, rtol=1e-5, atol=1e-6)
    # and linear in the scale
    d3 = lora.reference_forward(x, base, seq, widx, A, B, rk, 0.5 * sc) - base
    torch.testing.assert_close(d3, 0.5 * d1, rtol=1e-5, atol=1e-6)


def test_reference_forward_bf16_close_to_exact():
    """bf16 result within the bf16 tolerance of the fp64 truth, including rank 1 (strided column)."""
    g = torch.Generator().manual_seed(9)
    rows, M, K, N, R = 4, 3, 256, 64, 16
    A, B, rk, sc = _random_bank(g, 4, K, N, R, [0, 1, 7, 16])
    A, B = (A * 0.05).bfloat16(), (B * 0.05).bfloat16()
    x = torch.randn(rows, M, K, generator=g).bfloat16()
    base = torch.randn(rows, M, N, generator=g).bfloat16()
    seq = torch.tensor([3, 3, 2, 3], dtype=torch.int32)
    widx = torch.tensor([1, 2, 3, 1])
    got = lora.reference_forward(x, base, seq, widx, A, B, rk, sc)
    exact = lora.reference_forward(x.double(), base.double(), seq, widx, A.double(), B.double(), rk, sc)
    torch.testing.assert_close(got.double(), exact, rtol=2e-2, atol=1e-2)


def _planted_forwards():
    """Mutated copies of reference_forward, each with one plausible mistake."""

    def no_scale(x, base, seq, widx, A, B, rk, sc):
        return lora.reference_forward(x, base, seq, widx, A, B, rk, torch.ones_like(sc))

    def transposed_b(x, base, seq, widx, A, B, rk, sc):
        # B read as [N, R] instead of [R, N] (square shapes so it runs)
        return lora.reference_forward(x, base, seq, widx, A, B.transpose(1, 2).contiguous(), rk, sc)

    def off_by_one(x, base, seq, widx, A, B, rk, sc):
        return lora.reference_forward(x, base, seq - 1, widx, A, B, rk, sc)

    def wrong_slot(x, base, seq, widx, A, B, rk, sc):
        return lora.reference_forward(x, base, seq, (widx + 1) % A.shape[0], A, B, rk, sc)

    def rank_plus_one(x, base, seq, widx, A, B, rk, sc):
        return lora.reference_forward(x, base, seq, widx, A, B, torch.clamp(rk + 1, max=A.shape[2]), sc)

    return [no_scale, transposed_b, off_by_one, wrong_slot, rank_plus_one]


@pytest.mark.parametrize("mutant", _planted_forwards(), ids=lambda f: f.__name__)
def test_brute_force_check_catches_planted_mistakes(mutant):
    g = torch.Generator().manual_seed(11)
    rows, M, K, R = 4, 3, 5, 4
    N = R  # square B so a transposed read still runs
    A, B, rk, sc = _random_bank(g, 3, K, N, R, [0, 2, 3])
    x = torch.randn(rows, M, K, generator=g)
    base = torch.randn(rows, M, N, generator=g)
    seq = torch.tensor([3, 2, 3, 1], dtype=torch.int32)
    widx = torch.tensor([1, 2, 2, 1])
    want = _brute_lora(x, base, seq, widx, A, B, rk, sc)
    got = mutant(x, base, seq, widx, A, B, rk, sc)
    assert not torch.allclose(got.double(), want, rtol=1e-5, atol=1e-5)


# --------------------------------------------------------------------------- input shaping


def test_prepare_batched_inputs_branches():
    widx = torch.tensor([3, 1, 2])
    seq = torch.tensor([5, 2, 7], dtype=torch.int32)
    # (i) one row per batch row: 2-D becomes [B, 1, K]; seq_lens unclamped
    x = torch.randn(3, 8)
    x3, b3, s, w = lora.prepare_batched_inputs(x, x[:, :4], widx, seq)
    assert x3.shape == (3, 1, 8) and b3.shape == (3, 1, 4)
    assert torch.equal(s, seq) and torch.equal(w, widx)
    # >3-D input is flattened to [B, -1, K]
    x4 = torch.randn(3, 2, 2, 8)
    assert lora.prepare_batched_inputs(x4, x4[..., :4], widx, seq)[0].shape == (3, 4, 8)
    # (ii) shared batch-1 tensor: row 0's adapter, min(seq_lens[0], M)
    xs = torch.randn(1, 4, 8)
    _, _, s, w = lora.prepare_batched_inputs(xs, xs[..., :4], widx, seq)
    assert s.tolist() == [4] and w.tolist() == [3]
    # (iii) flattened [B*S, K]: clamp to S
    xf = torch.randn(3 * 6, 8)
    x3, b3, s, w = lora.prepare_batched_inputs(xf, xf[:, :4], widx, seq)
    assert x3.shape == (3, 6, 8) and s.tolist() == [5, 2, 6]
    # anything else raises the reference's ValueError
    with pytest.raises(ValueError, match="batch size does not match"):
        lora.prepare_batched_inputs(torch.randn(4, 8), torch.randn(4, 4), widx, seq)
    with pytest.raises(ValueError, match="expects a batched tensor"):
        lora.as_3d(torch.randn(8))


def test_decode_mask_length_longer_than_row():
    """Decode: seq_len = past + 1 = 513 while the layer sees one token; the fallback slices to 1."""
    g = torch.Generator().manual_seed(3)
    A, B, rk, sc = _random_bank(g, 2, 6, 4, 2, [0, 2])
    x = torch.randn(2, 1, 6, generator=g)
    base = torch.randn(2, 1, 4, generator=g)
    seq = torch.tensor([513, 513], dtype=torch.int32)
    widx = torch.tensor([1, 1])
    got = lora.reference_forward(x, base, seq, widx, A, B, rk, sc)
    want = lora.reference_forward(x, base, torch.tensor([1, 1]), widx, A, B, rk, sc)
    assert torch.equal(got, want)


# --------------------------------------------------------------------------- operator semantics


def test_sgmv_operator_references_match_brute_force():
    g = torch.Generator().manual_seed(21)
    Bt, M, K, S, R, N = 3, 4, 5, 3, 3, 6
    x = torch.randn(Bt, M, K, generator=g)
    wa = torch.randn(S, K, R * 2, generator=g)
    wb = torch.randn(S, R, N, generator=g)
    ranks = torch.tensor([0, 2, 3], dtype=torch.int32)
    scal = torch.tensor([0.0, 1.5, 0.25])
    seq = torch.tensor([4, 1, 9], dtype=torch.int32)
    widx = torch.tensor([1, 2, 0])
    for stack in (1, 2):
        out, valid = lora.sgmv_shrink_reference(x, wa, seq, widx, ranks, stack)
        for b, m, n in itertools.product(range(Bt), range(M), range(R * 2)):
            s = int(widx[b])
            ok = m < min(int(seq[b]), M) and n < int(ranks[s]) * stack
            assert bool(valid[b, m, n]) == ok
            if ok:
                want = sum(float(x[b, m, k]) * float(wa[s, k, n]) for k in range(K))
                assert abs(float(out[b, m, n]) - want) < 1e-4
    tmp = torch.randn(Bt, M, R, generator=g)
    base = torch.randn(Bt, M, N, generator=g)
    got = lora.sgmv_expand_reference(tmp, wb, seq, widx, ranks, scal, base)
    for b, m, n in itertools.product(range(Bt), range(M), range(N)):
        s = int(widx[b])
        want = float(base[b, m, n])
        if m < min(int(seq[b]), M) and int(ranks[s]) > 0:
            want += float(scal[s]) * sum(float(tmp[b, m, j]) * float(wb[s, j, n]) for j in range(int(ranks[s])))
        assert abs(float(got[b, m, n]) - want) < 1e-4


def test_right_padding_predicate():
    mask = torch.tensor([[1, 1, 0], [1, 1, 1], [0, 0, 0]])
    assert lora.right_padded(mask, mask.sum(-1))
    assert not lora.right_padded(torch.tensor([[1, 0, 1]]), torch.tensor([2]))
    assert not lora.right_padded(torch.tensor([[0, 1, 1]]), torch.tensor([2]))


def test_store_layout_closed_form():
    lora_A = torch.arange(6.0).reshape(2, 3)  # [r=2, in=3]
    lora_B = torch.arange(8.0).reshape(4, 2)  # [out=4, r=2]
    a, b, r, s = lora.store_layout(lora_A, lora_B, 8)
    assert a.shape == (3, 2) and b.shape == (2, 4) and r == 2 and s == 4.0
    assert torch.equal(a, lora_A.t()) and torch.equal(b, lora_B.t())
    assert a.is_contiguous() and b.is_contiguous()


# --------------------------------------------------------------------------- plan


def _plan_from_expected(row_slot, seq_lens, row_len, num_slots):
    expect = plan.expected_tokens(row_slot, seq_lens, row_len, num_slots)
    tok, groups = [], []
    for slot in sorted(expect):
        toks = expect[slot]
        for q in range(0, len(toks), plan.GROUP_TOKENS):
            chunk = toks[q : q + plan.GROUP_TOKENS]
            groups.append((slot, len(tok), len(chunk), 0))
            tok.extend(chunk)
    n = len(groups)
    placed = np.zeros((plan.positions(n), 4), dtype=np.int64)
    for gi, rec in enumerate(groups):
        placed[plan.group_position(gi, n)] = rec
    meta = np.array([n, len(tok), plan.GROUP_TOKENS, plan.positions(n)])
    return np.array(tok, dtype=np.int64), placed, meta, np.array(groups, dtype=np.int64).reshape(-1, 4)


@pytest.mark.parametrize("n", list(range(0, 70)) + [252, 1001])
def test_group_position_is_a_balanced_chunked_bijection(n):
    """Placement of the slot-major groups: chunk x of 8 contiguous, balanced chunks at positions = x mod 8."""
    pos = [plan.group_position(g, n) for g in range(n)]
    assert len(set(pos)) == n and all(0 <= p < plan.positions(n) for p in pos)
    assert plan.positions(n) % 8 == 0 and plan.positions(n) - n < 8
    sizes = []
    for x in range(8):
        members = [g for g, p in enumerate(pos) if p % 8 == x]
        # the groups one XCD gets are a contiguous run, stored in order at x, x+8, x+16, ...
        assert members == list(range(members[0], members[0] + len(members))) if members else True
        assert [pos[g] for g in members] == [x + 8 * i for i in range(len(members))]
        sizes.append(len(members))
    assert max(sizes) - min(sizes) <= 1
    # chunks follow the slot-major order: chunk x ends where chunk x+1 starts
    starts = [min((g for g, p in enumerate(pos) if p % 8 == x), default=None) for x in range(8)]
    nonempty = [v for v in starts if v is not None]
    assert nonempty == sorted(nonempty)


def test_expected_tokens_brute_force():
    rs = [2, 0, -1, 5, 2, 1]
    sl = [3, 4, 2, 1, 9, -1]
    got = plan.expected_tokens(rs, sl, 4, 5)
    assert got == {2: [0, 1, 2, 16, 17, 18, 19]}  # slot 5 is out of range, slot 0 is base, len -1 is empty


def test_check_plan_accepts_valid_and_rejects_planted():
    rng = np.random.default_rng(0)
    row_slot = rng.integers(-1, 8, size=40).tolist()
    seq_lens = rng.integers(-1, 80, size=40).tolist()
    tok, groups, meta, slot_major = _plan_from_expected(row_slot, seq_lens, 70, 7)
    plan.check_plan(tok, groups, meta, row_slot, seq_lens, 70, 7)
    assert int(meta[0]) > 8
    with pytest.raises(AssertionError):  # the records left in slot-major order, not placed per XCD
        plan.check_plan(tok, slot_major, meta, row_slot, seq_lens, 70, 7)
    bad_tok = tok.copy()
    bad_tok[3] += 1  # a token moved
    with pytest.raises(AssertionError):
        plan.check_plan(bad_tok, groups, meta, row_slot, seq_lens, 70, 7)
    bad_groups = groups.copy()
    bad_groups[0, 2] -= 1  # a group one token short
    with pytest.raises(AssertionError):
        plan.check_plan(tok, bad_groups, meta, row_slot, seq_lens, 70, 7)
    bad_meta = meta.copy()
    bad_meta[1] += 1
    with pytest.raises(AssertionError):
        plan.check_plan(tok, groups, bad_meta, row_slot, seq_lens, 70, 7)
    # capacity past the last position holds empty records
    padded = np.concatenate([groups, np.zeros((3, 4), dtype=groups.dtype)])
    plan.check_plan(tok, padded, meta, row_slot, seq_lens, 70, 7)
    padded[-1] = (1, 0, 1, 0)  # a stale record past the end
    with pytest.raises(AssertionError):
        plan.check_plan(tok, padded, meta, row_slot, seq_lens, 70, 7)


# --------------------------------------------------------------------------- slot bookkeeping


def test_slot_model_reference_test_assertions():
    known = {"a", "b", "c"}
    m = slots.SlotCacheModel(1)
    assert m.ensure_resident(["a"], known) == [1] and m.slot_to_adapter[1] == "a"
    assert m.ensure_resident(["b"], known) == [1] and m.slot_to_adapter[1] == "b"
    assert m.ensure_resident(["a"], known) == [1] and m.slot_to_adapter[1] == "a"
    assert m.ensure_resident(["__base__", "a"], known) == [0, 1]
    assert m.adapter_to_slot["__base__"] == 0
    with pytest.raises(RuntimeError, match="more adapters than GPU cache capacity"):
        m.ensure_resident(["a", "b"], known)
    with pytest.raises(KeyError, match="Unknown LoRA adapter"):
        m.ensure_resident(["zzz"], known)


def test_slot_model_lowest_free_then_lru():
    known = {f"x{i}" for i in range(6)}
    m = slots.SlotCacheModel(3)
    assert m.ensure_resident(["x2", "x0", "x1"], known) == [3, 1, 2]  # sorted load order, lowest free slot
    m.ensure_resident(["x1"], known)  # x1 becomes most recent
    # LRU order is now x0/x2 (set order of the first call) then x1; x3 evicts the oldest of them
    oldest = next(iter(m.lru))
    m.ensure_resident(["x3"], known)
    assert oldest not in m.adapter_to_slot and "x3" in m.adapter_to_slot and "x1" in m.adapter_to_slot
    # needed ids are never evicted
    m2 = slots.SlotCacheModel(2)
    m2.ensure_resident(["x0", "x1"], known)
    m2.ensure_resident(["x1", "x2"], known)
    assert "x1" in m2.adapter_to_slot and "x0" not in m2.adapter_to_slot
