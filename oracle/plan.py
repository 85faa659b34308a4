"""Expected adapter-major grouping of a forward's tokens (test infrastructure).

Token semantics follow the fallback's slicing x[b, :seq_len] (layers.py:127)
and the clamps of layers.py:91-108: row b contributes tokens b*M + m for
m < min(max(seq_len_b, 0), M), unless its slot is the base slot 0 (rank 0 in
every module, cache.py:32-34).  Grouping into runs of at most 64 tokens per
slot is this library's own schedule (the reference tiles per row,
sgmv.py:29-61), so only its invariants are checked, not an order, except
the placement of the group records: the slot-major group list is cut into 8
contiguous chunks, one per XCD, and the i-th group of chunk x is stored at
position 8*i + x (kernels deal position p to XCD p % 8).
"""

from __future__ import annotations

import numpy as np

GROUP_TOKENS = 64  # default group size; check_plan takes the plan's own
XCDS = 8  # kernels give the group at position p to XCD p % 8


def chunk_lo(x: int, n_groups: int) -> int:
    """First slot-major group of XCD chunk x: the n groups are cut into 8 contiguous chunks."""
    return (x * n_groups) // XCDS


def group_position(gi: int, n_groups: int) -> int:
    """Position of slot-major group gi: the i-th group of chunk x sits at 8*i + x."""
    x = max(c for c in range(XCDS) if chunk_lo(c, n_groups) <= gi)
    return (gi - chunk_lo(x, n_groups)) * XCDS + x


def positions(n_groups: int) -> int:
    """Positions a plan of n groups spans (meta[3]): 8 * ceil(n / 8)."""
    return -(-n_groups // XCDS) * XCDS


def expected_tokens(row_slot, seq_lens, row_len: int, num_slots: int) -> dict[int, list[int]]:
    per_slot: dict[int, list[int]] = {}
    for b, (slot, length) in enumerate(zip(list(row_slot), list(seq_lens))):
        slot, length = int(slot), min(max(int(length), 0), row_len)
        if slot <= 0 or slot >= num_slots or length == 0:
            continue
        per_slot.setdefault(slot, []).extend(b * row_len + m for m in range(length))
    return per_slot


def check_plan(tok: np.ndarray, groups: np.ndarray, meta: np.ndarray, row_slot, seq_lens, row_len: int, num_slots: int,
               group_tokens: int = GROUP_TOKENS) -> None:
    """Assert a device plan is a valid grouping of exactly the expected tokens."""
    expect = expected_tokens(row_slot, seq_lens, row_len, num_slots)
    n_tokens = sum(len(v) for v in expect.values())
    n_groups = sum(-(-len(v) // group_tokens) for v in expect.values())
    assert int(meta[0]) == n_groups, (int(meta[0]), n_groups)
    assert int(meta[1]) == n_tokens, (int(meta[1]), n_tokens)
    assert int(meta[2]) == group_tokens, (int(meta[2]), group_tokens)
    assert int(meta[3]) == positions(n_groups), (int(meta[3]), positions(n_groups))
    assert len(groups) >= positions(n_groups)
    seen: dict[int, list[int]] = {}
    covered = np.zeros(n_tokens, dtype=np.int64)
    used = set()
    prev_slot, next_start = 0, 0
    for gi in range(n_groups):  # slot-major order, read through the placement
        p = group_position(gi, n_groups)
        used.add(p)
        slot, start, length, _ = (int(v) for v in groups[p])
        assert 0 < slot < num_slots
        assert 1 <= length <= group_tokens
        assert slot >= prev_slot and start == next_start, (gi, p, slot, start)
        prev_slot, next_start = slot, start + length
        covered[start : start + length] += 1
        seen.setdefault(slot, []).extend(int(t) for t in tok[start : start + length])
    assert (covered == 1).all(), "groups must tile the sorted token list exactly once"
    for p in range(len(groups)):  # every other position: an empty group
        if p not in used:
            assert int(groups[p][0]) == 0 and int(groups[p][2]) == 0, (p, groups[p])
    assert set(seen) == set(expect)
    for slot, toks in expect.items():
        assert sorted(seen[slot]) == sorted(toks), f"slot {slot} token set differs"
    # groups of one slot: all full except possibly one
    for slot in expect:
        lens = sorted((int(groups[p][2]) for p in used if int(groups[p][0]) == slot), reverse=True)
        assert all(v == group_tokens for v in lens[:-1])
