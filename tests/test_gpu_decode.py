"""The one-launch decode path (pl_lora_decode_stacked): shrink and expand with the hand-off inside the launch.

Reference: the pair of Triton kernels MultiLoraLinear runs per wrapped Linear
(src/polylora/layers.py:42-58 -> sgmv.py:141-175 and :278-328).  The launch
must give exactly what pl_sgmv_shrink_stacked followed by
pl_sgmv_expand_stacked give on the same plan and workspace geometry (bit for
bit: the same sums in the same order), and so the oracle's result within the
dtype's tolerance; the hand-off counters must be back at zero after every
launch, with the timed-out-wait status word still 0.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

from oracle.lora import reference_forward
from polylora_amd import sgmv
from tests._util import make_cache, oracle_slot_tensors, peft_layer, tol_for
from tests.test_gpu_model import _announce

pytestmark = pytest.mark.gpu


def _counters_clear(device):
    for key, c in sgmv._COUNTERS.items():
        if c.buf is not None:
            torch.cuda.synchronize(device)
            assert int(c.buf[0]) == 0, "a hand-off wait ran out of polls"
            assert int(c.buf.abs().sum()) == 0, "hand-off counters left non-zero"


def _split_pair(x, ys, cache, mods, plan, k_splits=None):
    res = sgmv.lora_shrink_stacked(x, cache, mods, plan, k_splits=k_splits)
    sgmv.lora_expand_stacked(res, ys, cache, mods)
    return ys


CASES = [
    # dtype, rows, K, outs, ranks, max_rank, k_splits, seed
    (torch.bfloat16, 40, 1024, [512], [4, 16, 33, 64, 0], 64, None, 70),
    (torch.bfloat16, 70, 512, [512, 128, 136], [8, 24, 64, 0], 64, 2, 71),
    (torch.float16, 64, 1024, [768, 256], [8, 16, 32], 32, 3, 72),
    (torch.float32, 33, 768, [3072], [4, 8, 16], 16, 4, 73),
    # 16 K splits (16-plane expand) and two 64-rank passes (ranks up to 128)
    (torch.bfloat16, 24, 4096, [768], [8, 64, 32], 64, 16, 74),
    (torch.bfloat16, 2048, 1024, [512], [80, 128, 8, 64, 33], 128, 4, 75),
    # >= 1536 expand workgroups at 4 planes (32-rank staged blocks)
    (torch.bfloat16, 2048, 1024, [3072], [8, 16, 32, 64, 8, 16, 32, 64], 64, 4, 76),
]


@pytest.mark.parametrize("dtype,rows,K,outs,ranks,max_rank,k_splits,seed", CASES)
def test_decode_launch_equals_split_pair_and_oracle(gpu, dtype, rows, K, outs, ranks, max_rank, k_splits, seed):
    _announce(test="decode_launch", dtype=dtype, rows=rows, K=K, outs=outs, ranks=ranks, k_splits=k_splits)
    g = torch.Generator().manual_seed(seed)
    mods = [f"m{i}" for i in range(len(outs))]
    shapes = {m: (K, n) for m, n in zip(mods, outs)}
    # rank 0: the adapter lacks the modules (its rows are untouched)
    adapters = {f"a{i}": ({m: peft_layer(g, K, n, r, 2.0 * r) for m, (_, n) in shapes.items()} if r else
                          {"other": peft_layer(g, 8, 8, 2, 4.0)})
                for i, r in enumerate(ranks)}
    shapes_all = dict(shapes, other=(8, 8))
    cache = make_cache(adapters, shapes_all, len(adapters), max_rank, gpu, dtype)
    ids = list(adapters) + ["__base__"]
    adapter_ids = [ids[i] for i in torch.randint(0, len(ids), (rows,), generator=g).tolist()]
    row_slot = cache.ensure_resident(adapter_ids)
    seq = torch.ones(rows, dtype=torch.int32, device=gpu)
    plan = sgmv.SgmvPlan(row_slot, seq, 1, cache.num_slots, group_tokens=16)
    x = torch.randn(rows, K, generator=g).to(dtype).to(gpu)
    base = [torch.randn(rows, n, generator=g).to(dtype).to(gpu) for n in outs]
    want = _split_pair(x, [b.clone() for b in base], cache, mods, plan, k_splits)
    for rep in range(3):
        got = sgmv.lora_decode_stacked(x, [b.clone() for b in base], cache, mods, plan, k_splits=k_splits)
        torch.cuda.synchronize()
        for m, a, b in zip(mods, got, want):
            assert torch.equal(a, b), (m, rep)
    _counters_clear(gpu)
    untouched = torch.tensor([cache.ranks[mods[0]][int(s)] == 0 for s in row_slot.tolist()])
    for m, y, b0 in zip(mods, got, base):
        A, B, rk, sc = oracle_slot_tensors(cache, adapters, m, dtype)
        expect = reference_forward(x.cpu().view(rows, 1, K), b0.cpu().view(rows, 1, -1), seq.cpu(), row_slot.cpu(),
                                   A, B, rk, sc).view(rows, -1)
        torch.testing.assert_close(y.cpu(), expect, **tol_for(dtype))
        assert torch.equal(y.cpu()[untouched], b0.cpu()[untouched])


def test_timed_out_waits_are_reported_and_clearing_restores_the_counters(gpu, monkeypatch):
    """Waits forced to give up after one poll (a spin limit of 1, set from the host: every wave still
    ends) set the status word and can leave counters above zero; decode_waits_timed_out reports them and
    zeroes the counter set, after which launches with the normal limit equal the split pair bit for bit."""
    _announce(test="decode_timeout_clear")
    g = torch.Generator().manual_seed(77)
    K, outs, ranks = 1024, [512, 256], [8, 16, 32, 64]
    mods = ["m0", "m1"]
    shapes = {m: (K, n) for m, n in zip(mods, outs)}
    adapters = {f"a{i}": {m: peft_layer(g, K, n, r, 2.0 * r) for m, (_, n) in shapes.items()} for i, r in enumerate(ranks)}
    cache = make_cache(adapters, shapes, len(adapters), 64, gpu, torch.bfloat16)
    ids = [list(adapters)[i] for i in torch.randint(0, len(adapters), (256,), generator=g).tolist()]
    row_slot = cache.ensure_resident(ids)
    plan = sgmv.SgmvPlan(row_slot, torch.ones(256, dtype=torch.int32, device=gpu), 1, cache.num_slots, group_tokens=16)
    x = torch.randn(256, K, generator=g).to(torch.bfloat16).to(gpu)
    base = [torch.randn(256, n, generator=g).to(torch.bfloat16).to(gpu) for n in outs]
    want = _split_pair(x, [b.clone() for b in base], cache, mods, plan)
    torch.cuda.synchronize()
    assert not sgmv.decode_waits_timed_out(gpu)
    limit = sgmv.DECODE_SPIN_LIMIT
    monkeypatch.setattr(sgmv, "DECODE_SPIN_LIMIT", 1)
    for _ in range(3):
        sgmv.lora_decode_stacked(x, [b.clone() for b in base], cache, mods, plan)
    monkeypatch.setattr(sgmv, "DECODE_SPIN_LIMIT", limit)
    # the expand workgroups resident at the start poll once, long before every shrink has arrived
    assert sgmv.decode_waits_timed_out(gpu)
    _counters_clear(gpu)  # status word and every counter back at zero
    for rep in range(3):
        got = sgmv.lora_decode_stacked(x, [b.clone() for b in base], cache, mods, plan)
        torch.cuda.synchronize()
        for m, a, b in zip(mods, got, want):
            assert torch.equal(a, b), (m, rep)
    _counters_clear(gpu)
    assert not sgmv.decode_waits_timed_out(gpu)


def test_decode_config_layer_repeated_launches(gpu):
    """The decode configuration's layer (256 rows, 64 adapters of ranks {8,16,32,64}, Zipf(1.1) with 10% base
    rows): q/k/v, o, gate/up and down each as one launch, 30 times over, every launch bitwise equal to the
    split pair and the counters clear after each; then every module against the oracle."""
    _announce(test="decode_config_repeated")
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
    seq = torch.ones(256, dtype=torch.int32, device=gpu)
    plan = sgmv.SgmvPlan(row_slot, seq, 1, cache.num_slots, distinct_slots=len(set(ids) - {"__base__"}))
    assert sgmv.decode_ok(plan)
    gg = torch.Generator(device=gpu).manual_seed(1003)
    runs = [["q", "k", "v"], ["o"], ["gate", "up"], ["down"]]
    xs = {r[0]: torch.randn(256, shapes[r[0]][0], generator=gg, device=gpu).to(torch.bfloat16) for r in runs}
    base = {m: torch.randn(256, fo, generator=gg, device=gpu).to(torch.bfloat16) for m, (fi, fo) in shapes.items()}
    want = {}
    for r in runs:
        for m, y in zip(r, _split_pair(xs[r[0]], [base[m].clone() for m in r], cache, r, plan)):
            want[m] = y
    torch.cuda.synchronize()
    outs = {m: torch.empty_like(base[m]) for m in shapes}
    for rep in range(30):
        for r in runs:
            ys = [outs[m].copy_(base[m]) for m in r]
            sgmv.lora_decode_stacked(xs[r[0]], ys, cache, r, plan)
        torch.cuda.synchronize()
        for m in shapes:
            assert torch.equal(outs[m], want[m]), (m, rep)
        _counters_clear(gpu)
    assert not sgmv.decode_waits_timed_out(gpu)
    for r in runs:
        for m in r:
            fi, fo = shapes[m]
            A, Bm, rk, sc = (t.to(gpu) for t in oracle_slot_tensors(cache, adapters, m, torch.bfloat16))
            expect = reference_forward(xs[r[0]].view(256, 1, fi), base[m].view(256, 1, fo), seq, row_slot, A, Bm, rk, sc)
            torch.testing.assert_close(outs[m].view(256, 1, fo), expect, rtol=2e-2, atol=1e-2)


def test_decode_launch_graph_replays(gpu):
    """Two decode launches (stacked and single) captured in a HIP graph: every replay, with eager work between
    replays, equals the eager result bit for bit, and the counters are clear after each."""
    _announce(test="decode_graph")
    g = torch.Generator().manual_seed(77)
    K, rows = 1024, 48
    shapes = {"q": (K, 768), "k": (K, 256), "o": (768, K)}
    adapters = {f"a{i}": {m: peft_layer(g, fi, fo, r, 2.0 * r) for m, (fi, fo) in shapes.items()}
                for i, r in enumerate([8, 16, 64])}
    cache = make_cache(adapters, shapes, 3, 64, gpu, torch.bfloat16)
    ids = list(adapters) + ["__base__"]
    row_slot = cache.ensure_resident([ids[i] for i in torch.randint(0, 4, (rows,), generator=g).tolist()])
    seq = torch.ones(rows, dtype=torch.int32, device=gpu)
    x = torch.randn(rows, K, generator=g).to(torch.bfloat16).to(gpu)
    q0 = torch.randn(rows, 768, generator=g).to(torch.bfloat16).to(gpu)
    k0 = torch.randn(rows, 256, generator=g).to(torch.bfloat16).to(gpu)
    z0 = torch.randn(rows, K, generator=g).to(torch.bfloat16).to(gpu)
    q, k, z = q0.clone(), k0.clone(), z0.clone()

    def step():
        q.copy_(q0)
        k.copy_(k0)
        z.copy_(z0)
        plan = sgmv.SgmvPlan(row_slot, seq, 1, cache.num_slots)
        sgmv.lora_decode_stacked(x, [q, k], cache, ["q", "k"], plan)
        sgmv.lora_decode_stacked(q, [z], cache, ["o"], plan)

    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        step()
    torch.cuda.current_stream().wait_stream(s)
    torch.cuda.synchronize()
    want = [t.clone() for t in (q, k, z)]
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        step()
    for i in range(4):
        q.fill_(float(i))  # eager work between replays
        z.zero_()
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        assert all(torch.equal(a, b) for a, b in zip((q, k, z), want)), i
        _counters_clear(gpu)


def test_decode_launch_rejects_long_group_plans(gpu):
    g = torch.Generator().manual_seed(78)
    adapters = {"a": {"m": peft_layer(g, 256, 256, 8, 16.0)}}
    cache = make_cache(adapters, {"m": (256, 256)}, 1, 8, gpu, torch.bfloat16)
    row_slot = cache.ensure_resident(["a"] * 4)
    plan = sgmv.SgmvPlan(row_slot, torch.full((4,), 100, dtype=torch.int32, device=gpu), 100, cache.num_slots,
                         group_tokens=64)
    x = torch.zeros(400, 256, dtype=torch.bfloat16, device=gpu)
    with pytest.raises(ValueError, match="16-token groups"):
        sgmv.lora_decode_stacked(x, [torch.zeros_like(x)], cache, ["m"], plan)
