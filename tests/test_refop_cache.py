"""Host logic of the operator API's kept parts (polylora_amd.refop_cache): when a plan or a weights part is
reused, rebuilt in place, packed lazily, or not kept at all.  CPU tensors stand in for device tensors (the
cache only reads their identity and version counters and allocates its buffers on their device)."""

from __future__ import annotations

import gc

import torch

from polylora_amd import _native, refop_cache

CPU = torch.device("cpu")
USED = _native.PL_REF_PACK_USED | _native.PL_REF_KEEP_PACKED
ALL = _native.PL_REF_PACK_ALL | _native.PL_REF_KEEP_PACKED


def _cache(max_bytes=1 << 20, max_plans=16):
    refop_cache.configure(max_bytes=max_bytes, max_plans=max_plans)
    return refop_cache.CACHE


def _part(c, w, r, s=None, stream=0, nbytes=4096, which=0):
    """(buffer, flags, epoch) of a weights-part lookup; the buffer's address comes back with it."""
    buf, ptr, flags, epoch = c.weights_part(CPU, stream, which, w, r, s, 1, (64, 16), nbytes, 256)
    assert ptr == buf.data_ptr()
    return buf, flags, epoch


def _plan(c, *args):
    buf, ptr, build = c.plan(CPU, 0, *args)
    assert ptr == buf.data_ptr()
    return buf, build


def test_weights_part_packs_used_then_all_then_nothing_and_rebuilds_on_a_write():
    c = _cache()
    w, r = torch.zeros(5, 64, 16), torch.ones(5, dtype=torch.int32)
    buf, f, e = _part(c, w, r)
    assert (f, e) == (USED, 1) and buf.numel() == 4096 and buf.data_ptr() % 256 == 0
    buf.fill_(1)
    b2, f, e = _part(c, w, r)
    assert b2.data_ptr() == buf.data_ptr() and (f, e) == (ALL, 2)
    assert _part(c, w, r)[1:] == (0, 0)
    assert _part(c, w[:], r)[1:] == (0, 0)  # a view of the same storage is the same tensor
    w.add_(1)  # in-place write: version counter moves
    b3, f, e = _part(c, w, r)
    assert b3.data_ptr() == buf.data_ptr() and (f, e) == (USED, 1)
    assert int(buf[:256].sum()) == 0 and bool((buf[256:] == 1).all()), "only the marks are cleared"
    _part(c, w, r)
    r[0] = 3
    assert _part(c, w, r)[1] == USED
    s = torch.ones(5)
    assert _part(c, w, r, s, which=1)[1] == USED  # the expand's part is its own entry
    s.mul_(2)
    assert _part(c, w, r, s, which=1)[1] == USED
    assert c.stats["pack_used"] == 5 and c.stats["pack_all"] == 2 and c.stats["weights_hits"] == 2


def test_weights_parts_are_per_stream_and_identity():
    c = _cache()
    w, r = torch.zeros(5, 64, 16), torch.ones(5, dtype=torch.int32)
    a = _part(c, w, r, stream=1)[0]
    b = _part(c, w, r, stream=2)[0]
    assert a.data_ptr() != b.data_ptr() and len(c.weights) == 2
    w2 = w.clone()
    assert _part(c, w2, r)[1] == USED and len(c.weights) == 3


def test_tensors_without_version_counter_and_oversized_parts_are_not_kept():
    c = _cache(max_bytes=3000)
    w, r = torch.zeros(5, 64, 16), torch.ones(5, dtype=torch.int32)
    assert _part(c, w, r, nbytes=4096)[1:] == (_native.PL_REF_PACK_USED, 0)  # beyond the budget
    c = _cache()
    with torch.inference_mode():
        wi = torch.zeros(5, 64, 16)
    for _ in range(2):
        assert _part(c, wi, r)[1:] == (_native.PL_REF_PACK_USED, 0)
    assert not c.weights and c.stats["uncached"] == 2
    c = _cache(max_bytes=0)
    assert _part(c, w, r)[1:] == (_native.PL_REF_PACK_USED, 0)


def test_budget_evicts_least_recently_used_and_dead_tensors_drop_their_entry():
    c = _cache(max_bytes=10000)
    r = torch.ones(5, dtype=torch.int32)
    ws = [torch.zeros(5, 64, 16) for _ in range(3)]
    _part(c, ws[0], r)
    _part(c, ws[1], r)
    _part(c, ws[0], r)  # ws[0] is now the most recent
    _part(c, ws[2], r)  # 3 x 4096 > 10000: ws[1]'s entry goes
    keys = list(c.weights)
    assert len(keys) == 2 and c.bytes[CPU] == 8192
    assert _part(c, ws[1], r)[1] == USED  # rebuilt from scratch
    del ws[2]
    gc.collect()
    _part(c, ws[0], r)  # the next call drops the dead tensor's entry
    assert len(c.weights) == 2 and c.bytes[CPU] == 8192


def test_plan_entries_are_reused_rebuilt_in_place_and_bounded():
    c = _cache(max_plans=2)
    seq, idx = torch.ones(8, dtype=torch.int32), torch.zeros(8, dtype=torch.int32)
    p, build = _plan(c, 8, 1, 4, seq, idx, 1024)
    assert build and p.numel() == 1024
    p2, build = _plan(c, 8, 1, 4, seq, idx, 1024)
    assert not build and p2.data_ptr() == p.data_ptr()
    idx[3] = 2
    p3, build = _plan(c, 8, 1, 4, seq, idx, 1024)
    assert build and p3.data_ptr() == p.data_ptr()
    assert _plan(c, 8, 2, 4, seq, idx, 1024)[1], "another row length is another plan"
    assert _plan(c, 8, 1, 4, seq.clone(), idx, 1024)[1]  # a third entry: the oldest goes
    assert len(c.plans) == 2 and _plan(c, 8, 1, 4, seq, idx, 1024)[1]
    with torch.inference_mode():
        si = torch.ones(8, dtype=torch.int32)
    assert _plan(c, 8, 1, 4, si, idx, 1024)[1] and _plan(c, 8, 1, 4, si, idx, 1024)[1]


def test_marks_bytes():
    assert refop_cache.marks_bytes(1) == 256 and refop_cache.marks_bytes(64) == 256
    assert refop_cache.marks_bytes(65) == 512
    refop_cache.configure()


def test_scratch_is_one_aligned_buffer_per_stream_grown_on_demand():
    c = _cache()
    p = c.scratch(CPU, 0, 1000)
    assert p % 256 == 0
    assert c.scratch(CPU, 0, 1000) == p and c.scratch(CPU, 0, 10) == p  # reused while it is large enough
    q = c.scratch(CPU, 7, 1000)  # another stream: its own buffer
    assert q != p and c.scratch(CPU, 7, 500) == q
    grown = c.scratch(CPU, 0, 1500)  # past its size: replaced by one at least twice as large
    assert grown % 256 == 0 and c._scratch[(CPU, 0)][1] == 2000
    assert c.scratch(CPU, 0, 2000) == grown
    refop_cache.clear()
    assert not c._scratch


def test_parts_made_under_inference_mode_are_rebuilt_outside_it():
    """A weights part first made inside torch.inference_mode is cleared in place (its pack marks) when its
    tensors change outside that mode: its buffer is an ordinary tensor."""
    c = _cache()
    w, r = torch.zeros(5, 64, 16), torch.ones(5, dtype=torch.int32)
    with torch.inference_mode():
        buf, f, e = _part(c, w, r)
        assert (f, e) == (USED, 1) and not buf.is_inference()
        c.scratch(CPU, 0, 1000)
        assert not c._scratch[(CPU, 0)][2].is_inference()
    w.add_(1)  # a write the version counter sees
    buf[:256].fill_(3)  # marks left by the earlier packing
    buf2, f, e = _part(c, w, r)
    assert buf2.data_ptr() == buf.data_ptr() and (f, e) == (USED, 1) and not buf2[:256].any()


def _steady(c, w, r, **kw):
    """Lookups until the weights part needs nothing more (packed used, then all, then kept)."""
    flags = None
    for _ in range(3):
        buf, flags, _ = _part(c, w, r, **kw)
    assert flags == 0
    return buf


def test_identity_memo_never_serves_a_dropped_entry_or_another_tensor():
    """The lookups' identity-keyed front memos: a kept part is served again without its full key, but
    never after clear()/configure(), after the budget dropped it, after its tensor died and a new one
    took its id(), or after the storage under the same tensor object changed."""
    c = _cache(max_bytes=3 * 4096)
    w, r = torch.zeros(5, 64, 16), torch.ones(5, dtype=torch.int32)
    buf = _steady(c, w, r)
    hits = c.stats["weights_hits"]
    assert _part(c, w, r)[1] == 0 and c.stats["weights_hits"] == hits + 1  # served again, nothing to build
    refop_cache.clear()
    assert _part(c, w, r)[1] == USED  # a fresh entry: packs again
    # the budget holds 3 parts of 4096 bytes: a fourth drops the oldest
    _steady(c, w, r)
    others = [(torch.zeros(5, 64, 16), torch.ones(5, dtype=torch.int32)) for _ in range(3)]
    for wo, ro in others:
        _part(c, wo, ro)
    assert _part(c, w, r)[1] == USED  # dropped by the budget: built again
    # a new tensor that reuses a dead one's id() is never taken for it
    c = _cache()
    w2 = torch.zeros(5, 64, 16)
    _steady(c, w2, r)
    ident = id(w2)
    del w2
    gc.collect()
    for _ in range(50):
        w3 = torch.zeros(5, 64, 16)
        if id(w3) == ident:
            break
    assert _part(c, w3, r)[1] == USED
    # the storage under one tensor object changed without a version bump (.data): not served
    w4 = torch.zeros(5, 64, 16)
    _steady(c, w4, r)
    w4.data = torch.zeros(5, 64, 16)
    assert _part(c, w4, r)[1] == USED
    # plans: served from the memo while their tensors stand, rebuilt after an in-place write
    c = _cache()
    s, i = torch.ones(4, dtype=torch.int32), torch.zeros(4, dtype=torch.int32)
    assert _plan(c, 4, 1, 5, s, i, 4096)[1] and not _plan(c, 4, 1, 5, s, i, 4096)[1]
    i[0] = 2
    assert _plan(c, 4, 1, 5, s, i, 4096)[1]
    refop_cache.clear()
    assert _plan(c, 4, 1, 5, s, i, 4096)[1]
    del buf
