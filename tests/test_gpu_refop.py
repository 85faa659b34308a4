"""The reference-layout operator API (sgmv_lora_a_fwd / sgmv_lora_b_fwd, sgmv.py:141-175, :278-328).

Both entry points have an MFMA path (weights repacked into the slot arena's
block layout in a workspace, a device plan, then the tiled shrink or expand,
or for long adapter segments a phase of the fused kernel) and the row
kernels for shapes that path does not take.  Each is checked against
the oracle's restatement of the operators (oracle.lora.sgmv_shrink_reference
/ sgmv_expand_reference), and the two paths against each other.
"""

from __future__ import annotations

import ctypes

import numpy as np
import pytest
import torch

from oracle.lora import sgmv_expand_reference, sgmv_shrink_reference
from polylora_amd import _native, refop_cache, sgmv
from tests._util import tol_for

pytestmark = pytest.mark.gpu


def _announce(**kw):
    print("case:", ", ".join(f"{k}={v}" for k, v in kw.items()), flush=True)


def _workspace(lib, x, which, B, M, K, n, num_adapters):
    """One 256-byte aligned workspace of pl_sgmv_ref_workspace_bytes bytes, or (None, 0) when the MFMA path
    declines the shape."""
    nbytes = int(lib.pl_sgmv_ref_workspace_bytes(_native.dtype_code(x.dtype), which, B, M, K, n, num_adapters))
    if nbytes <= 0:
        return None, 0
    buf = torch.empty(nbytes + 256, dtype=torch.uint8, device=x.device)
    pad = (-buf.data_ptr()) % 256
    return buf[pad : pad + nbytes], nbytes


def _call_a(x, w, seq, widx, ranks, stack_num, *, mfma: bool):
    """pl_sgmv_lora_a_ref through the C-ABI, with (MFMA path) or without (row kernels) a workspace."""
    lib = _native.load()
    B, M, K = x.shape
    n_max = w.shape[2]
    out = torch.full((B, M, n_max), 7.0, device=x.device, dtype=x.dtype)  # untouched entries stay 7
    ws, nbytes = _workspace(lib, x, 0, B, M, K, n_max, w.shape[0]) if mfma else (None, 0)
    if mfma:
        assert ws is not None, "the MFMA path declined this shape"
    _native.check(lib.pl_sgmv_lora_a_ref(_native.dtype_code(x.dtype), x.data_ptr(), B, M, K, w.data_ptr(), *w.stride(),
                                         w.shape[0], n_max, seq.data_ptr(), widx.data_ptr(), ranks.data_ptr(),
                                         stack_num, out.data_ptr(), 0 if ws is None else ws.data_ptr(), nbytes,
                                         torch.cuda.current_stream().cuda_stream), "pl_sgmv_lora_a_ref")
    return out


def _call_b(x, w, seq, widx, ranks, scal, base, *, mfma: bool):
    lib = _native.load()
    B, M, k_max = x.shape
    N = w.shape[2]
    out = base.clone()
    ws, nbytes = _workspace(lib, x, 1, B, M, k_max, N, w.shape[0]) if mfma else (None, 0)
    if mfma:
        assert ws is not None, "the MFMA path declined this shape"
    _native.check(lib.pl_sgmv_lora_b_ref(_native.dtype_code(x.dtype), x.data_ptr(), B, M, k_max, w.data_ptr(),
                                         *w.stride(), w.shape[0], N, seq.data_ptr(), widx.data_ptr(),
                                         ranks.data_ptr(), scal.data_ptr(), out.data_ptr(),
                                         0 if ws is None else ws.data_ptr(), nbytes,
                                         torch.cuda.current_stream().cuda_stream), "pl_sgmv_lora_b_ref")
    return out


def _case(g, Bt, M, K, N, S, R, stack_num, dtype, gpu):
    x = torch.randn(Bt, M, K, generator=g).to(dtype)
    wa = (torch.randn(S, K, R * stack_num, generator=g) * 0.05).to(dtype)
    wb = (torch.randn(S, R, N, generator=g) * 0.05).to(dtype)
    ranks = torch.randint(0, R + 1, (S,), generator=g, dtype=torch.int32)
    ranks[0] = 0
    ranks[-1] = R
    scal = torch.rand(S, generator=g) * 4
    seq = torch.randint(0, M + 3, (Bt,), generator=g, dtype=torch.int32)  # some beyond M
    widx = torch.randint(0, S, (Bt,), generator=g, dtype=torch.int32)
    dev = [t.to(gpu) for t in (x, wa, wb, ranks, scal, seq, widx)]
    return (x, wa, wb, ranks, scal, seq, widx), dev


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16, torch.float32])
@pytest.mark.parametrize("stack_num", [1, 2])
# the first three take the split kernels (few tokens per adapter); the last two have long adapter
# segments and take the fused kernel's shrink and expand phases (16- and 64-token groups)
@pytest.mark.parametrize("Bt,M,K,N,S,R", [(6, 10, 96, 80, 4, 8), (9, 70, 256, 136, 5, 32), (40, 1, 512, 64, 7, 16),
                                          (24, 96, 256, 136, 5, 32), (40, 256, 128, 64, 4, 16)])
def test_mfma_and_row_paths_match_the_oracle(gpu, dtype, stack_num, Bt, M, K, N, S, R):
    _announce(test="refop_paths", dtype=dtype, stack_num=stack_num, shape=(Bt, M, K, N, S, R))
    g = torch.Generator().manual_seed(Bt * 7 + stack_num)
    (x, wa, wb, ranks, scal, seq, widx), (dx, dwa, dwb, dranks, dscal, dseq, dwidx) = _case(
        g, Bt, M, K, N, S, R, stack_num, dtype, gpu)
    exp_tmp, valid = sgmv_shrink_reference(x, wa, seq, widx, ranks, stack_num)
    outs = {}
    for mfma in (True, False):
        tmp = _call_a(dx, dwa, dseq, dwidx, dranks, stack_num, mfma=mfma).cpu()
        torch.testing.assert_close(tmp[valid], exp_tmp[valid], **tol_for(dtype))
        assert bool((tmp[~valid] == 7).all()), "entries outside the defined region were written"
        outs[mfma] = tmp
    torch.testing.assert_close(outs[True][valid], outs[False][valid], **tol_for(dtype))
    # expand over the oracle's intermediate
    base = torch.randn(Bt, M, N, generator=g).to(dtype)
    xb = exp_tmp[:, :, :R].contiguous()
    expect = sgmv_expand_reference(xb, wb, seq, widx, ranks, scal, base)
    for mfma in (True, False):
        out = _call_b(xb.to(gpu), dwb, dseq, dwidx, dranks, dscal, base.to(gpu), mfma=mfma).cpu()
        torch.testing.assert_close(out, expect, **tol_for(dtype))
        untouched = (ranks[widx.long()] == 0) | (seq <= 0)
        assert torch.equal(out[untouched], base[untouched])


def test_unaligned_shapes_take_the_row_kernels(gpu):
    """K = 97, N = 75: no 16-byte chunks, so the MFMA path declines and the row kernels answer."""
    _announce(test="refop_unaligned")
    lib = _native.load()
    assert int(lib.pl_sgmv_ref_workspace_bytes(_native.PL_BF16, 0, 4, 3, 97, 8, 3)) == 0
    assert int(lib.pl_sgmv_ref_workspace_bytes(_native.PL_BF16, 1, 4, 3, 8, 75, 3)) == 0
    assert int(lib.pl_sgmv_ref_workspace_bytes(_native.PL_BF16, 0, 4, 3, 96, 72, 3)) == 0  # rank above 64
    g = torch.Generator().manual_seed(5)
    (x, wa, wb, ranks, scal, seq, widx), (dx, dwa, dwb, dranks, dscal, dseq, dwidx) = _case(
        g, 4, 3, 97, 75, 3, 8, 1, torch.bfloat16, gpu)
    tmp = sgmv.sgmv_lora_a_fwd(dx, dwa, dseq, dwidx, dranks).cpu()
    exp_tmp, valid = sgmv_shrink_reference(x, wa, seq, widx, ranks)
    torch.testing.assert_close(tmp[valid], exp_tmp[valid], **tol_for(torch.bfloat16))
    base = torch.randn(4, 3, 75, generator=g).bfloat16()
    out = sgmv.sgmv_lora_b_fwd(exp_tmp.to(gpu), dwb, dseq, dwidx, dranks, dscal, base.to(gpu)).cpu()
    torch.testing.assert_close(out, sgmv_expand_reference(exp_tmp, wb, seq, widx, ranks, scal, base),
                               **tol_for(torch.bfloat16))


def test_decode_rows_and_out_of_range_indices(gpu):
    """M = 1 rows with seq_len 513 (a KV mask's length) act as min(seq_len, M) = 1; indices -1 and S are skipped."""
    _announce(test="refop_decode_rows")
    g = torch.Generator().manual_seed(9)
    Bt, K, N, S, R = 64, 1024, 512, 6, 16
    x = torch.randn(Bt, 1, K, generator=g).bfloat16()
    wa = (torch.randn(S, K, R, generator=g) * 0.05).bfloat16()
    wb = (torch.randn(S, R, N, generator=g) * 0.05).bfloat16()
    ranks = torch.tensor([0, 4, 8, 16, 12, 16], dtype=torch.int32)
    scal = torch.tensor([0.0, 8.0, 4.0, 2.0, 2.5, 2.0])
    seq = torch.full((Bt,), 513, dtype=torch.int32)
    widx = torch.randint(0, S, (Bt,), generator=g, dtype=torch.int32)
    widx[3], widx[10] = -1, S
    ok = (widx >= 0) & (widx < S)
    tmp = _call_a(x.to(gpu), wa.to(gpu), seq.to(gpu), widx.to(gpu), ranks.to(gpu), 1, mfma=True).cpu()
    exp_tmp, valid = sgmv_shrink_reference(x[ok], wa, seq[ok], widx[ok], ranks)
    torch.testing.assert_close(tmp[ok][valid], exp_tmp[valid], **tol_for(torch.bfloat16))
    assert bool((tmp[~ok] == 7).all())
    base = torch.randn(Bt, 1, N, generator=g).bfloat16()
    xb = torch.zeros(Bt, 1, R, dtype=torch.bfloat16)
    xb[ok] = exp_tmp
    out = _call_b(xb.to(gpu), wb.to(gpu), seq.to(gpu), widx.to(gpu), ranks.to(gpu), scal.to(gpu), base.to(gpu),
                  mfma=True).cpu()
    expect = base.clone()
    expect[ok] = sgmv_expand_reference(exp_tmp, wb, seq[ok], widx[ok], ranks, scal, base[ok])
    torch.testing.assert_close(out, expect, **tol_for(torch.bfloat16))
    assert torch.equal(out[~ok], base[~ok])


def test_isolated_op_shapes_through_the_operator_api(gpu):
    """4096 rows of one token, K = N = 4096, 17 adapters of ranks {0,4,8,16}, Dirichlet segments: the
    isolated op's shapes in the reference's own layout, shrink then expand, against the oracle."""
    _announce(test="refop_isolated_4096")
    from bench import _dirichlet_segments

    rng = np.random.default_rng(1002)
    g = torch.Generator().manual_seed(1002)
    T, K, N, S, R = 4096, 4096, 4096, 17, 16
    ranks = torch.tensor([[0, 4, 8, 16][s % 4] for s in range(S)], dtype=torch.int32)
    scal = torch.tensor([32.0 / r if r else 0.0 for r in ranks.tolist()])
    wa = (torch.randn(S, K, R, generator=g) * 0.02).bfloat16()
    wb = (torch.randn(S, R, N, generator=g) * 0.02).bfloat16()
    seg = _dirichlet_segments(rng, T, S)
    widx = torch.tensor(np.repeat(np.arange(S), seg), dtype=torch.int32)
    seq = torch.ones(T, dtype=torch.int32)
    x = torch.randn(T, 1, K, generator=g).bfloat16()
    base = torch.randn(T, 1, N, generator=g).bfloat16()
    dev = {k: v.to(gpu) for k, v in dict(x=x, wa=wa, wb=wb, ranks=ranks, scal=scal, seq=seq, widx=widx).items()}
    tmp = sgmv.sgmv_lora_a_fwd(dev["x"], dev["wa"], dev["seq"], dev["widx"], dev["ranks"])
    out = sgmv.sgmv_lora_b_fwd(tmp[:, :, :R].contiguous(), dev["wb"], dev["seq"], dev["widx"], dev["ranks"],
                               dev["scal"], base.to(gpu))
    exp_tmp, valid = sgmv_shrink_reference(x, wa, seq, widx, ranks)
    got_tmp = tmp.cpu()
    torch.testing.assert_close(got_tmp[valid], exp_tmp[valid], **tol_for(torch.bfloat16))
    # the expand checked on the intermediate it was given (invalid entries zeroed for the oracle)
    xb = torch.where(valid, got_tmp, torch.zeros((), dtype=torch.bfloat16))[:, :, :R].contiguous()
    expect = sgmv_expand_reference(xb, wb, seq, widx, ranks, scal, base)
    torch.testing.assert_close(out.cpu(), expect, rtol=2e-2, atol=1e-2)
    zero = ranks[widx.long()] == 0
    assert torch.equal(out.cpu()[zero], base[zero])


@pytest.mark.parametrize("Bt,M", [(3000, 1), (1600, 64)])
def test_more_adapters_than_plan_threads(gpu, Bt, M):
    """1500 adapters: the slot table and the plan's slot counts span more entries than the plan
    workgroup has threads.  3000 one-token rows take the split kernels; 1600 rows of 64 tokens (at
    least 64 per adapter) take the fused kernel's phases.  Rank-0 adapters and indices -1 and S are
    skipped."""
    _announce(test="refop_many_adapters", Bt=Bt, M=M)
    g = torch.Generator().manual_seed(Bt + M)
    K, N, S, R = 128, 64, 1500, 8
    x = torch.randn(Bt, M, K, generator=g).bfloat16()
    wa = (torch.randn(S, K, R, generator=g) * 0.05).bfloat16()
    wb = (torch.randn(S, R, N, generator=g) * 0.05).bfloat16()
    ranks = torch.randint(1, R + 1, (S,), generator=g, dtype=torch.int32)
    ranks[::7] = 0
    scal = torch.rand(S, generator=g) * 4
    seq = torch.randint(0, M + 2, (Bt,), generator=g, dtype=torch.int32)
    widx = torch.randint(0, S, (Bt,), generator=g, dtype=torch.int32)
    widx[5], widx[17] = -1, S
    ok = (widx >= 0) & (widx < S)
    d = {k: v.to(gpu) for k, v in dict(x=x, wa=wa, wb=wb, ranks=ranks, scal=scal, seq=seq, widx=widx).items()}
    tmp = _call_a(d["x"], d["wa"], d["seq"], d["widx"], d["ranks"], 1, mfma=True).cpu()
    exp_tmp, valid = sgmv_shrink_reference(x[ok], wa, seq[ok], widx[ok], ranks)
    torch.testing.assert_close(tmp[ok][valid], exp_tmp[valid], **tol_for(torch.bfloat16))
    assert bool((tmp[ok][~valid] == 7).all()) and bool((tmp[~ok] == 7).all())
    base = torch.randn(Bt, M, N, generator=g).bfloat16()
    xb = torch.zeros(Bt, M, R, dtype=torch.bfloat16)
    xb[ok] = exp_tmp
    out = _call_b(xb.to(gpu), d["wb"], d["seq"], d["widx"], d["ranks"], d["scal"], base.to(gpu), mfma=True).cpu()
    expect = base.clone()
    expect[ok] = sgmv_expand_reference(exp_tmp, wb, seq[ok], widx[ok], ranks, scal, base[ok])
    torch.testing.assert_close(out, expect, **tol_for(torch.bfloat16))
    assert torch.equal(out[~ok], base[~ok])


def test_workspace_errors_are_reported(gpu):
    """A workspace below the size the call needs, or misaligned, is an error, not a silent fallback."""
    _announce(test="refop_ws_errors")
    lib = _native.load()
    x = torch.randn(4, 2, 64, device=gpu).bfloat16()
    w = torch.randn(3, 64, 8, device=gpu).bfloat16()
    seq = torch.full((4,), 2, dtype=torch.int32, device=gpu)
    widx = torch.tensor([0, 1, 2, 1], dtype=torch.int32, device=gpu)
    ranks = torch.tensor([2, 4, 8], dtype=torch.int32, device=gpu)
    out = torch.empty(4, 2, 8, device=gpu).bfloat16()
    need = int(lib.pl_sgmv_ref_workspace_bytes(_native.PL_BF16, 0, 4, 2, 64, 8, 3))
    assert need > 0
    ws = torch.empty(need + 512, dtype=torch.uint8, device=gpu)
    base = ws.data_ptr() + (-ws.data_ptr()) % 256
    s = torch.cuda.current_stream().cuda_stream
    args = (_native.PL_BF16, x.data_ptr(), 4, 2, 64, w.data_ptr(), *w.stride(), 3, 8, seq.data_ptr(),
            widx.data_ptr(), ranks.data_ptr(), 1, out.data_ptr())
    assert lib.pl_sgmv_lora_a_ref(*args, ctypes.c_void_p(base), need - 256, s) == _native.PL_ERR_ARG
    assert b"workspace" in lib.pl_last_error()
    assert lib.pl_sgmv_lora_a_ref(*args, ctypes.c_void_p(base + 16), need, s) == _native.PL_ERR_ARG
    assert lib.pl_sgmv_lora_a_ref(*args, ctypes.c_void_p(base), need, s) == 0
    torch.cuda.synchronize()


def _fresh_cache():
    refop_cache.configure()
    for k in refop_cache.CACHE.stats:
        refop_cache.CACHE.stats[k] = 0


def _valid(seq, widx, ranks, M, n_max, stack_num=1):
    """Mask of the shrink output the operator defines: m < min(seq_len, M), n < rank * stack_num."""
    B = seq.shape[0]
    ok = (widx >= 0) & (widx < ranks.shape[0])
    r = torch.where(ok, ranks[widx.clamp(0, ranks.shape[0] - 1).long()], torch.zeros_like(widx)) * stack_num
    m = torch.arange(M).view(1, M, 1)
    n = torch.arange(n_max).view(1, 1, n_max)
    return (m < seq.clamp(max=M).view(B, 1, 1)) & (n < r.view(B, 1, 1))


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
@pytest.mark.parametrize("Bt,M,K,N,S,R", [(40, 1, 512, 256, 9, 16), (24, 96, 256, 136, 5, 32)])
def test_kept_parts_equal_a_fresh_workspace_call(gpu, dtype, Bt, M, K, N, S, R):
    """sgmv_lora_a_fwd / sgmv_lora_b_fwd keep the plan and the repacked weights across calls.  The first
    call packs only the adapters its rows use, the second the rest, later calls launch no repack, and
    one plan serves the shrink and the expand.  Every call equals the C-ABI call with a fresh single
    workspace bit for bit, also for a batch whose rows use only adapters the first batch did not; then
    in-place writes to an adapter's weights, to a rank and to the adapter index are seen."""
    _announce(test="refop_kept_parts", dtype=dtype, shape=(Bt, M, K, N, S, R))
    _fresh_cache()
    st = refop_cache.CACHE.stats
    g = torch.Generator().manual_seed(Bt + K)
    _, (dx, dwa, dwb, dranks, dscal, dseq, _) = _case(g, Bt, M, K, N, S, R, 1, dtype, gpu)
    dranks[1:] = torch.randint(1, R + 1, (S - 1,), generator=g, dtype=torch.int32).to(gpu)
    half = S // 2 + 1
    idx = {1: (torch.arange(Bt) % half).to(torch.int32).to(gpu),
           2: (half + torch.arange(Bt) % (S - half)).to(torch.int32).to(gpu)}
    base = torch.randn(Bt, M, N, generator=g).to(dtype).to(gpu)

    def check(w_idx, step):
        want_a = _call_a(dx, dwa, dseq, w_idx, dranks, 1, mfma=True)
        got_a = sgmv.sgmv_lora_a_fwd(dx, dwa, dseq, w_idx, dranks)
        valid = _valid(dseq.cpu(), w_idx.cpu(), dranks.cpu(), M, R).to(gpu)
        assert torch.equal(got_a[valid], want_a[valid]), step
        want_b = _call_b(want_a, dwb, dseq, w_idx, dranks, dscal, base, mfma=True)
        got_b = sgmv.sgmv_lora_b_fwd(want_a, dwb, dseq, w_idx, dranks, dscal, base.clone())
        assert torch.equal(got_b, want_b), step

    for step, which in enumerate([1, 1, 2, 2, 1]):
        check(idx[which], step)
    torch.cuda.synchronize()
    assert (st["pack_used"], st["pack_all"], st["weights_hits"]) == (2, 2, 6), st
    assert (st["plan_builds"], st["plan_hits"]) == (2, 8), st
    dwa[1].mul_(2.0)  # adapter 1 (used by batch 1) changes in place
    check(idx[1], "weights written")
    assert st["pack_used"] == 3 and st["weights_hits"] == 7, st  # the shrink's part repacked, the expand's kept
    dranks[2] = max(1, int(dranks[2]) // 2)
    check(idx[1], "rank written")
    assert st["pack_used"] == 5, st
    idx[1][0] = S - 1
    check(idx[1], "index written")
    assert st["plan_builds"] == 3, st
    torch.cuda.synchronize()


def test_tensors_without_version_counter_are_not_kept(gpu):
    _announce(test="refop_inference_tensors")
    _fresh_cache()
    g = torch.Generator().manual_seed(31)
    _, (dx, dwa, dwb, dranks, dscal, dseq, dwidx) = _case(g, 16, 1, 256, 128, 5, 16, 1, torch.bfloat16, gpu)
    with torch.inference_mode():
        wi, idx_i = dwa.clone(), dwidx.clone()
    for _ in range(2):
        want = _call_a(dx, dwa, dseq, dwidx, dranks, 1, mfma=True)
        got = sgmv.sgmv_lora_a_fwd(dx, wi, dseq, idx_i, dranks)
        valid = _valid(dseq.cpu(), dwidx.cpu(), dranks.cpu(), 1, 16).to(gpu)
        assert torch.equal(got[valid], want[valid])
    st = refop_cache.CACHE.stats
    assert st["uncached"] == 2 and st["plan_hits"] == 0 and st["plan_builds"] == 2, st
    assert not refop_cache.CACHE.weights


def test_kept_weights_die_with_their_tensor(gpu):
    import gc

    _announce(test="refop_dead_weights")
    _fresh_cache()
    g = torch.Generator().manual_seed(32)
    _, (dx, dwa, dwb, dranks, dscal, dseq, dwidx) = _case(g, 16, 1, 256, 128, 5, 16, 1, torch.bfloat16, gpu)
    w = dwa.clone()
    sgmv.sgmv_lora_a_fwd(dx, w, dseq, dwidx, dranks)
    assert len(refop_cache.CACHE.weights) == 1 and refop_cache.CACHE.bytes[dx.device] > 0
    del w
    gc.collect()
    sgmv.sgmv_lora_a_fwd(dx, dwa, dseq, dwidx, dranks)  # the next call drops the dead entry
    assert len(refop_cache.CACHE.weights) == 1
    torch.cuda.synchronize()


@pytest.mark.parametrize("K", [512, 4096])
def test_operator_api_in_a_graph_replays(gpu, K):
    """Shrink then expand captured in a HIP graph (every part taken for the captured call, nothing kept):
    each replay, with eager work between replays, equals the eager result bit for bit.  32 rows take the
    split shrink with its in-launch finish: one K split at K = 512, four at 4096 (each replay's plan build
    zeroes the finish counters)."""
    _announce(test="refop_graph", K=K)
    _fresh_cache()
    g = torch.Generator().manual_seed(33)
    _, (dx, dwa, dwb, dranks, dscal, dseq, dwidx) = _case(g, 32, 1, K, 256, 6, 16, 1, torch.bfloat16, gpu)
    base = torch.randn(32, 1, 256, generator=g).bfloat16().to(gpu)
    out = torch.empty_like(base)
    tmp = torch.zeros(32, 1, 16, dtype=torch.bfloat16, device=gpu)

    def step():
        tmp.copy_(sgmv.sgmv_lora_a_fwd(dx, dwa, dseq, dwidx, dranks))
        out.copy_(base)
        sgmv.sgmv_lora_b_fwd(tmp, dwb, dseq, dwidx, dranks, dscal, out)

    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        step()
    torch.cuda.current_stream().wait_stream(s)
    torch.cuda.synchronize()
    valid = _valid(dseq.cpu(), dwidx.cpu(), dranks.cpu(), 1, 16).to(gpu)
    want_tmp, want = tmp.clone(), out.clone()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        step()
    for i in range(3):
        out.fill_(float(i))
        tmp.zero_()
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        assert torch.equal(tmp[valid], want_tmp[valid]) and torch.equal(out, want), i


def test_part_entry_points_reject_bad_flags(gpu):
    """The part-based entry points refuse unknown flags, PL_REF_KEEP_PACKED without an epoch, and parts
    below their sizes."""
    _announce(test="refop_part_errors")
    lib = _native.load()
    x = torch.randn(4, 2, 64, device=gpu).bfloat16()
    w = torch.randn(3, 64, 8, device=gpu).bfloat16()
    seq = torch.full((4,), 2, dtype=torch.int32, device=gpu)
    widx = torch.tensor([0, 1, 2, 1], dtype=torch.int32, device=gpu)
    ranks = torch.tensor([2, 4, 8], dtype=torch.int32, device=gpu)
    out = torch.empty(4, 2, 8, device=gpu).bfloat16()
    sizes = [int(lib.pl_sgmv_ref_part_bytes(_native.PL_BF16, 0, 4, 2, 64, 8, 3, p)) for p in range(3)]
    assert all(n > 0 for n in sizes)
    bufs = [torch.zeros(n + 256, dtype=torch.uint8, device=gpu) for n in sizes]
    ptrs = [b.data_ptr() + (-b.data_ptr()) % 256 for b in bufs]
    s = torch.cuda.current_stream().cuda_stream
    args = (_native.PL_BF16, x.data_ptr(), 4, 2, 64, w.data_ptr(), *w.stride(), 3, 8, seq.data_ptr(),
            widx.data_ptr(), ranks.data_ptr(), 1, out.data_ptr())

    def call(flags, epoch, shrink=0):
        return lib.pl_sgmv_lora_a_ref_parts(*args, ptrs[0], sizes[0], ptrs[1], sizes[1] - shrink, ptrs[2], sizes[2],
                                            flags, epoch, s)

    assert call(16, 0) == _native.PL_ERR_ARG
    assert call(_native.PL_REF_PACK_USED | _native.PL_REF_KEEP_PACKED, 0) == _native.PL_ERR_ARG
    assert call(_native.PL_REF_BUILD_PLAN | _native.PL_REF_PACK_USED, 0, shrink=256) == _native.PL_ERR_ARG
    assert b"parts" in lib.pl_last_error()
    assert call(_native.PL_REF_BUILD_PLAN | _native.PL_REF_PACK_ALL | _native.PL_REF_KEEP_PACKED, 1) == 0
    torch.cuda.synchronize()


@pytest.mark.parametrize("dtype", [torch.float16])
def test_kept_parts_with_int64_indices_and_stacked_columns(gpu, dtype):
    """The reference passes int64 index and length tensors and may stack modules along n (stack_num 2): the
    parts are kept by the caller's own tensors (not the int32 copies made per call), and every call still
    equals a fresh-workspace call bit for bit."""
    _announce(test="refop_kept_int64_stack2", dtype=dtype)
    _fresh_cache()
    st = refop_cache.CACHE.stats
    g = torch.Generator().manual_seed(34)
    Bt, M, K, N, S, R = 48, 1, 512, 256, 6, 16
    _, (dx, dwa, dwb, dranks, dscal, dseq, dwidx) = _case(g, Bt, M, K, N, S, R, 2, dtype, gpu)
    widx64, seq64 = dwidx.long(), dseq.long()
    for step in range(3):
        want = _call_a(dx, dwa, dseq, dwidx, dranks, 2, mfma=True)
        got = sgmv.sgmv_lora_a_fwd(dx, dwa, seq64, widx64, dranks, stack_num=2)
        valid = _valid(dseq.cpu(), dwidx.cpu(), dranks.cpu(), M, 2 * R, stack_num=2).to(gpu)
        assert torch.equal(got[valid], want[valid]), step
    torch.cuda.synchronize()
    assert (st["plan_builds"], st["plan_hits"]) == (1, 2), st
    assert (st["pack_used"], st["pack_all"], st["weights_hits"]) == (1, 1, 1), st


@pytest.mark.parametrize("dtype,Bt,K,R,stack_num,S", [
    (torch.bfloat16, 256, 4096, 64, 1, 17),  # 4 K splits, up to 64 ranks
    (torch.float16, 200, 14336, 16, 1, 9),  # 8 K splits, 64-byte plane rows shared by neighbouring groups
    (torch.float32, 96, 4096, 8, 2, 6),  # fp32, two stacked columns per rank
    (torch.bfloat16, 2048, 4096, 32, 2, 40),  # ~170 groups, 64 columns
    (torch.bfloat16, 130, 1000, 24, 1, 7),  # one K split: every workgroup is its tile's last; K ends mid-step
    (torch.float16, 300, 2048, 64, 1, 12),  # 2 K splits, two rank passes
    (torch.float32, 77, 3000, 40, 1, 5),  # 3 K splits, the last one short; fp32 at 40 ranks
    # 64-token groups (8192 tokens, ~41 per adapter: too few for the fused kernel): the split shrink with
    # its planes summed by a second launch
    (torch.bfloat16, 8192, 2048, 16, 1, 200),
])
def test_split_shrink_finishes_inside_its_launch(gpu, dtype, Bt, K, R, stack_num, S):
    """Short adapter segments take the split shrink; with 16-token groups its last K split of each tile writes
    the intermediate in the same launch on counters kept in the plan part.  Three calls with a kept plan (the
    counters must be back at zero after each launch) and new x each time, every one against the oracle, and
    equal bit for bit to the single-workspace entry (which builds the plan, and zeroes the counters, on every
    call)."""
    _announce(test="refop_split_finish", dtype=dtype, Bt=Bt, K=K, R=R, stack_num=stack_num, S=S)
    g = torch.Generator().manual_seed(Bt + K + R)
    M = 1
    wa = (torch.randn(S, K, R * stack_num, generator=g) * 0.05).to(dtype)
    ranks = torch.randint(0, R + 1, (S,), generator=g, dtype=torch.int32)
    ranks[0], ranks[-1] = 0, R
    seq = (torch.rand(Bt, generator=g) > 0.05).to(torch.int32)  # a few rows of length 0
    widx = torch.randint(0, S, (Bt,), generator=g, dtype=torch.int32)
    dwa, dranks, dseq, dwidx = (t.to(gpu) for t in (wa, ranks, seq, widx))
    refop_cache.configure()
    try:
        for call in range(3):
            x = torch.randn(Bt, M, K, generator=g).to(dtype)
            exp, valid = sgmv_shrink_reference(x, wa, seq, widx, ranks, stack_num)
            dx = x.to(gpu)
            got = sgmv.sgmv_lora_a_fwd(dx, dwa, dseq, dwidx, dranks, stack_num).cpu()
            torch.testing.assert_close(got[valid], exp[valid], **tol_for(dtype))
            fresh = _call_a(dx, dwa, dseq, dwidx, dranks, stack_num, mfma=True).cpu()
            assert torch.equal(fresh[valid], got[valid]), call
            assert bool((fresh[~valid] == 7).all()), "entries outside the defined region were written"
        st = refop_cache.CACHE.stats
        assert (st["plan_builds"], st["plan_hits"]) == (1, 2), st
    finally:
        refop_cache.configure()
