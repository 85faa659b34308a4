"""Expected adapter-major grouping of a forward's tokens (test infrastructure).

Token semantics follow the fallback's slicing x[b, :seq_len] (layers.py:127)
and the clamps of layers.py:91-108: row b contributes tokens b*M + m for
m < min(max(seq_len_b, 0), M), unless its slot is the base slot 0 (rank 0 in
every module, cache.py:32-34).  Grouping into runs of at most 64 tokens per
slot is this build's own schedule (the reference tiles per row,
sgmv.py:29-61), so only its invariants are checked, not an order.
"""

from __future__ import annotations

import numpy as np

GROUP_TOKENS = 64  # default group size; check_plan takes the plan's own


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
    seen: dict[int, list[int]] = {}
    covered = np.zeros(n_tokens, dtype=np.int64)
    for g in range(n_groups):
        slot, start, length, _ = (int(v) for v in groups[g])
        assert 0 < slot < num_slots
        assert 1 <= length <= group_tokens
        assert 0 <= start and start + length <= n_tokens
        covered[start : start + length] += 1
        seen.setdefault(slot, []).extend(int(t) for t in tok[start : start + length])
    assert (covered == 1).all(), "groups must tile the sorted token list exactly once"
    for g in range(n_groups, len(groups)):  # the rest of the capacity: empty groups
        assert int(groups[g][0]) == 0 and int(groups[g][2]) == 0, (g, groups[g])
    assert set(seen) == set(expect)
    for slot, toks in expect.items():
        assert sorted(seen[slot]) == sorted(toks), f"slot {slot} token set differs"
    # groups of one slot: all full except possibly one
    for slot in expect:
        lens = sorted((int(groups[g][2]) for g in range(n_groups) if int(groups[g][0]) == slot), reverse=True)
        assert all(v == group_tokens for v in lens[:-1])
