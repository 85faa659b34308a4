"""pl_lora_apply_noalloc (plan and shrink planes in the library's static scratch) against the entry points it
combines, pl_plan_build + pl_lora_apply with caller-allocated buffers, through the C ABI.

Two calls in a row per case, the second on a smaller batch (the scratch keeps the first call's
contents); each must equal the existing entry points' result bit for bit and match the oracle.
"""

from __future__ import annotations

import pytest
import torch

from oracle.lora import reference_forward
from polylora_amd import _native
from tests._util import CountedParity, make_cache, oracle_slot_tensors, peft_layer, tol_for

pytestmark = pytest.mark.gpu

K, N = 512, 384


def _existing(lib, dt, x, y, cache, row_slot, seq, rows, row_len, group_tokens, k_splits, stream):
    """pl_plan_build + pl_lora_apply with torch-allocated plan and workspace."""
    dev = x.device
    K, N = int(x.shape[1]), int(y.shape[1])
    cap = int(lib.pl_plan_group_capacity(rows, row_len, cache.num_slots, group_tokens))
    T = max(1, rows * row_len)
    tok = torch.empty(T, dtype=torch.int32, device=dev)
    groups = torch.empty((max(1, cap), 4), dtype=torch.int32, device=dev)
    meta = torch.empty(4, dtype=torch.int32, device=dev)
    _native.check(lib.pl_plan_build(row_slot.data_ptr(), seq.data_ptr(), rows, row_len, cache.num_slots,
                                    group_tokens, tok.data_ptr(), groups.data_ptr(), meta.data_ptr(), max(1, cap),
                                    stream), "pl_plan_build")
    ldt = cache.rank8_cap
    nbytes = int(lib.pl_shrink_workspace_bytes(dt, K, k_splits, group_tokens, T, ldt))
    ws = torch.empty(nbytes, dtype=torch.uint8, device=dev)
    _native.check(lib.pl_lora_apply(dt, x.data_ptr(), x.stride(0), K, y.data_ptr(), y.stride(0), N,
                                    cache.arena.data_ptr(), cache.table.data_ptr(), len(cache.module_index), 0,
                                    tok.data_ptr(), groups.data_ptr(), meta.data_ptr(), max(1, cap), group_tokens,
                                    ws.data_ptr(), nbytes, ldt, T, k_splits, _native.PL_EPI_FALLBACK, stream),
                  "pl_lora_apply")
    torch.cuda.synchronize()


# (rows, row_len) of two calls in a row, the second smaller: decode-like rows, and prefill-shaped rows longer
# than 16 tokens (the plan places their tokens with one wave per row)
CALLS = [((40, 16), (9, 5)), ((4, 300), (3, 120))]


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16, torch.float32])
@pytest.mark.parametrize("group_tokens,k_splits", [(16, 4), (64, 2)])
@pytest.mark.parametrize("calls", CALLS)
def test_noalloc_equals_plan_build_plus_lora_apply(gpu, dtype, group_tokens, k_splits, calls):
    print(f"case: noalloc dtype={dtype} group_tokens={group_tokens} k_splits={k_splits} calls={calls}", flush=True)
    lib = _native.load()
    dt = _native.dtype_code(dtype)
    g = torch.Generator().manual_seed(31)
    adapters = {f"n{i}": {"m": peft_layer(g, K, N, r, 2.0 * r)} for i, r in enumerate([4, 8, 16, 12])}
    cache = make_cache(adapters, {"m": (K, N)}, 5, 16, gpu, dtype)
    ids_pool = ["__base__", *adapters]
    stream = _native.current_stream_handle(gpu)
    for rows, row_len in calls:
        ids = [ids_pool[int(i)] for i in torch.randint(0, len(ids_pool), (rows,), generator=g)]
        row_slot = cache.ensure_resident(ids)
        seq_cpu = torch.randint(0, row_len + 3, (rows,), generator=g, dtype=torch.int32)
        seq = seq_cpu.to(gpu)
        x_cpu = torch.randn(rows * row_len, K, generator=g).to(dtype)
        base_cpu = torch.randn(rows * row_len, N, generator=g).to(dtype)
        x = x_cpu.to(gpu)
        y_new = base_cpu.to(gpu)
        y_old = base_cpu.to(gpu)
        torch.cuda.synchronize()
        st = lib.pl_lora_apply_noalloc(dt, x.data_ptr(), x.stride(0), K, y_new.data_ptr(), y_new.stride(0), N,
                                       cache.arena.data_ptr(), cache.table.data_ptr(), len(cache.module_index), 0,
                                       row_slot.data_ptr(), seq.data_ptr(), rows, row_len, cache.num_slots,
                                       group_tokens, cache.rank8_cap, k_splits, _native.PL_EPI_FALLBACK, stream)
        _native.check(st, "pl_lora_apply_noalloc")
        torch.cuda.synchronize()
        _existing(lib, dt, x, y_old, cache, row_slot, seq, rows, row_len, group_tokens, k_splits, stream)
        assert torch.equal(y_new, y_old), (rows, row_len)
        A, B, rk, sc = oracle_slot_tensors(cache, adapters, "m", dtype)
        want = reference_forward(x_cpu.view(rows, row_len, K), base_cpu.view(rows, row_len, N), seq_cpu,
                                 row_slot.cpu().long(), A, B, rk, sc)
        torch.testing.assert_close(y_new.cpu().view(rows, row_len, N), want, **tol_for(dtype))


def test_noalloc_rejects_a_batch_beyond_its_scratch(gpu):
    print("case: noalloc limit", flush=True)
    lib = _native.load()
    g = torch.Generator().manual_seed(32)
    cache = make_cache({"z": {"m": peft_layer(g, K, N, 8, 16.0)}}, {"m": (K, N)}, 1, 64, gpu, torch.bfloat16)
    rows, row_len = 4096, 64  # 262144 tokens: far beyond 32 MiB of planes
    x = torch.empty(8, K, dtype=torch.bfloat16, device=gpu)  # never read: the size check fails first
    st = lib.pl_lora_apply_noalloc(_native.PL_BF16, x.data_ptr(), K, K, x.data_ptr(), K, N, cache.arena.data_ptr(),
                                   cache.table.data_ptr(), 1, 0, x.data_ptr(), x.data_ptr(), rows, row_len,
                                   cache.num_slots, 64, cache.rank8_cap, 8, 0, _native.current_stream_handle(gpu))
    assert st == 4  # PL_ERR_LIMIT
    assert b"static scratch" in lib.pl_last_error()


def _noalloc_need(lib, dt, rows, row_len, num_slots, group_tokens, ldt, k_splits):
    """Scratch bytes a pl_lora_apply_noalloc call needs (the formula its declaration states)."""
    a256 = lambda v: (v + 255) // 256 * 256  # noqa: E731
    T = max(1, rows * row_len)
    cap = int(lib.pl_plan_group_capacity(rows, row_len, num_slots, group_tokens))
    return 256 + a256(16 * cap) + a256(4 * T) + int(lib.pl_shrink_workspace_bytes(dt, K, k_splits, group_tokens, T, ldt))


def test_noalloc_just_under_its_scratch_limit(gpu):
    """The largest batch of 64-token rows whose plan and planes fit the static scratch: bit for bit equal
    to pl_plan_build + pl_lora_apply, then a smaller call, then one more row is refused."""
    print("case: noalloc near the limit", flush=True)
    lib = _native.load()
    dt, gt, ks, row_len = _native.PL_BF16, 64, 2, 64
    g = torch.Generator().manual_seed(33)
    adapters = {f"n{i}": {"m": peft_layer(g, K, N, r, 2.0 * r)} for i, r in enumerate([4, 8, 16])}
    cache = make_cache(adapters, {"m": (K, N)}, 3, 16, gpu, torch.bfloat16)
    limit = _native.PL_NOALLOC_SCRATCH_BYTES
    need = lambda r: _noalloc_need(lib, dt, r, row_len, cache.num_slots, gt, cache.rank8_cap, ks)  # noqa: E731
    lo, hi = 1, 1 << 16
    assert need(lo) <= limit < need(hi)
    while hi - lo > 1:
        mid = (lo + hi) // 2
        lo, hi = (mid, hi) if need(mid) <= limit else (lo, mid)
    rows = lo
    assert need(rows) <= limit < need(rows + 1) and need(rows) > limit - (1 << 20)
    stream = _native.current_stream_handle(gpu)
    gd = torch.Generator(device=gpu).manual_seed(33)
    ids_pool = ["__base__", *adapters]
    for r in (rows, rows // 3):
        ids = [ids_pool[int(i)] for i in torch.randint(0, len(ids_pool), (r,), generator=g)]
        row_slot = cache.ensure_resident(ids)
        seq = torch.randint(0, row_len + 3, (r,), generator=g, dtype=torch.int32).to(gpu)
        x = torch.randn(r * row_len, K, generator=gd, device=gpu).bfloat16()
        y_new = torch.randn(r * row_len, N, generator=gd, device=gpu).bfloat16()
        y_old = y_new.clone()
        torch.cuda.synchronize()
        _native.check(lib.pl_lora_apply_noalloc(dt, x.data_ptr(), K, K, y_new.data_ptr(), N, N, cache.arena.data_ptr(),
                                                cache.table.data_ptr(), 1, 0, row_slot.data_ptr(), seq.data_ptr(), r,
                                                row_len, cache.num_slots, gt, cache.rank8_cap, ks,
                                                _native.PL_EPI_FALLBACK, stream), "pl_lora_apply_noalloc")
        torch.cuda.synchronize()
        _existing(lib, dt, x, y_old, cache, row_slot, seq, r, row_len, gt, ks, stream)
        assert torch.equal(y_new, y_old), r
        del x, y_new, y_old
    x = torch.empty(8, K, dtype=torch.bfloat16, device=gpu)  # never read: the size check fails first
    st = lib.pl_lora_apply_noalloc(dt, x.data_ptr(), K, K, x.data_ptr(), N, N, cache.arena.data_ptr(),
                                   cache.table.data_ptr(), 1, 0, x.data_ptr(), x.data_ptr(), rows + 1, row_len,
                                   cache.num_slots, gt, cache.rank8_cap, ks, 0, stream)
    assert st == _native.PL_ERR_LIMIT


@pytest.mark.parametrize("seed", range(16))
def test_noalloc_random_shapes_equal_the_existing_entry_points(gpu, seed):
    """Seeded random dtype, K, N, ranks, batch geometry, group size and split count, two calls in a row (the
    second smaller), each bit for bit against pl_plan_build + pl_lora_apply and within tolerance of the oracle."""
    import numpy as np

    r = np.random.default_rng(9000 + seed)
    dtype = (torch.bfloat16, torch.float16, torch.float32)[int(r.integers(3))]
    e = 4 if dtype == torch.float32 else 8
    k, n = e * int(r.integers(1, 257)), e * int(r.integers(1, 257))
    max_rank = int(r.choice([8, 16, 32, 64]))
    ranks = [int(v) for v in r.integers(1, max_rank + 1, int(r.integers(1, 9)))]
    group_tokens = int(r.choice([16, 64]))
    k_splits = int(r.choice([1, 2, 3, 4, 8]))
    print(f"case: noalloc sweep seed={seed} dtype={dtype} K={k} N={n} ranks={ranks} group_tokens={group_tokens} "
          f"k_splits={k_splits}", flush=True)
    lib = _native.load()
    dt = _native.dtype_code(dtype)
    g = torch.Generator().manual_seed(seed)
    adapters = {f"n{i}": {"m": peft_layer(g, k, n, rk, 2.0 * rk)} for i, rk in enumerate(ranks)}
    cache = make_cache(adapters, {"m": (k, n)}, len(adapters), max_rank, gpu, dtype)
    ids_pool = ["__base__", *adapters]
    stream = _native.current_stream_handle(gpu)
    parity = CountedParity(dtype, f"noalloc sweep seed {seed}")
    row_len = int(r.choice([1, 1, 3, 40]))
    rows = int(r.integers(2, max(3, 2048 // row_len)))
    for rows_i in (rows, max(1, rows // 3)):
        ids = [ids_pool[int(i)] for i in r.integers(0, len(ids_pool), rows_i)]
        row_slot = cache.ensure_resident(ids)
        seq_cpu = torch.randint(0, row_len + 2, (rows_i,), generator=g, dtype=torch.int32)
        seq = seq_cpu.to(gpu)
        x_cpu = torch.randn(rows_i * row_len, k, generator=g).to(dtype)
        base_cpu = torch.randn(rows_i * row_len, n, generator=g).to(dtype)
        x, y_new, y_old = x_cpu.to(gpu), base_cpu.to(gpu), base_cpu.to(gpu)
        torch.cuda.synchronize()
        st = lib.pl_lora_apply_noalloc(dt, x.data_ptr(), x.stride(0), k, y_new.data_ptr(), y_new.stride(0), n,
                                       cache.arena.data_ptr(), cache.table.data_ptr(), len(cache.module_index), 0,
                                       row_slot.data_ptr(), seq.data_ptr(), rows_i, row_len, cache.num_slots,
                                       group_tokens, cache.rank8_cap, k_splits, _native.PL_EPI_FALLBACK, stream)
        _native.check(st, "pl_lora_apply_noalloc")
        torch.cuda.synchronize()
        _existing(lib, dt, x, y_old, cache, row_slot, seq, rows_i, row_len, group_tokens, k_splits, stream)
        assert torch.equal(y_new, y_old), (rows_i, row_len)
        A, B, rk, sc = oracle_slot_tensors(cache, adapters, "m", dtype)
        want = reference_forward(x_cpu.view(rows_i, row_len, k), base_cpu.view(rows_i, row_len, n), seq_cpu,
                                 row_slot.cpu().long(), A, B, rk, sc)
        parity.check(y_new.cpu().view(rows_i, row_len, n), want, base_cpu.view(rows_i, row_len, n))
    parity.finish()
