"""Two streams at once: the per-stream state of the operator API and of the decode launch.

The operator API keeps its plan and weights parts per (device, stream) and one
scratch buffer per stream (polylora_amd/refop_cache.py); the decode launch
uses the stream's shrink workspaces and hand-off counters (polylora_amd/sgmv.py).
Calls issued on two streams that run concurrently must therefore give, bit for
bit, what the same calls give one after the other on one stream.  Both
streams keep the default priority.

Reference: the operator calls of layers.py:42-58 (sgmv.py:141-175, :278-328).
"""

from __future__ import annotations

import pytest
import torch

from oracle.lora import sgmv_shrink_reference
from polylora_amd import refop_cache, sgmv
from tests._util import make_cache, peft_layer, tol_for

pytestmark = pytest.mark.gpu


def _announce(**kw):
    print("case:", ", ".join(f"{k}={v}" for k, v in kw.items()), flush=True)


def test_operator_api_on_two_concurrent_streams(gpu):
    _announce(test="streams_operator")
    g = torch.Generator().manual_seed(91)
    Bt, M, K, N, S, R = 256, 1, 2048, 1024, 9, 32
    dtype = torch.bfloat16
    wa = (torch.randn(S, K, R, generator=g) * 0.05).to(dtype).to(gpu)
    wb = (torch.randn(S, R, N, generator=g) * 0.05).to(dtype).to(gpu)
    ranks = torch.randint(1, R + 1, (S,), generator=g, dtype=torch.int32)
    ranks[0] = 0
    scal = (torch.rand(S, generator=g) * 4).to(gpu)
    seq = torch.ones(Bt, dtype=torch.int32)
    widx = torch.randint(0, S, (Bt,), generator=g, dtype=torch.int32)
    xs = [torch.randn(Bt, M, K, generator=g).to(dtype).to(gpu) for _ in range(2)]
    bases = [torch.randn(Bt, M, N, generator=g).to(dtype).to(gpu) for _ in range(2)]
    dranks, dseq, dwidx = ranks.to(gpu), seq.to(gpu), widx.to(gpu)
    _, valid = sgmv_shrink_reference(xs[0].cpu(), wa.cpu(), seq, widx, ranks)

    def pair(i):
        tmp = sgmv.sgmv_lora_a_fwd(xs[i], wa, dseq, dwidx, dranks)
        out = sgmv.sgmv_lora_b_fwd(tmp, wb, dseq, dwidx, dranks, scal, bases[i].clone())
        return tmp, out

    refop_cache.configure()
    try:
        want = [pair(i) for i in range(2)]
        torch.cuda.synchronize()
        want = [(t.cpu(), o.cpu()) for t, o in want]
        exp, _ = sgmv_shrink_reference(xs[0].cpu(), wa.cpu(), seq, widx, ranks)
        torch.testing.assert_close(want[0][0][valid], exp[valid], **tol_for(dtype))
        streams = [torch.cuda.Stream(), torch.cuda.Stream()]
        got = [[], []]
        for rnd in range(6):
            for i, s in enumerate(streams):
                with torch.cuda.stream(s):
                    got[i].append(pair(i))
        torch.cuda.synchronize()
        for i in range(2):
            for rnd, (t, o) in enumerate(got[i]):
                assert torch.equal(t.cpu()[valid], want[i][0][valid]), (i, rnd)
                assert torch.equal(o.cpu(), want[i][1]), (i, rnd)
        st = refop_cache.CACHE.stats
        assert st["plan_builds"] == 3 and st["uncached"] == 0, st  # one plan per stream
    finally:
        refop_cache.configure()


def test_decode_launch_on_two_concurrent_streams(gpu):
    _announce(test="streams_decode")
    g = torch.Generator().manual_seed(92)
    K, outs, ranks = 2048, [1024, 512], [8, 16, 32, 64, 64]
    mods = ["m0", "m1"]
    shapes = {m: (K, n) for m, n in zip(mods, outs)}
    adapters = {f"a{i}": {m: peft_layer(g, K, n, r, 2.0 * r) for m, (_, n) in shapes.items()}
                for i, r in enumerate(ranks)}
    dtype = torch.bfloat16
    cache = make_cache(adapters, shapes, len(adapters), 64, gpu, dtype)
    names = list(adapters) + ["__base__"]
    rows = 256
    ids = [names[i] for i in torch.randint(0, len(names), (rows,), generator=g).tolist()]
    row_slot = cache.ensure_resident(ids)
    plan = sgmv.SgmvPlan(row_slot, torch.ones(rows, dtype=torch.int32, device=gpu), 1, cache.num_slots,
                         group_tokens=16)
    xs = [torch.randn(rows, K, generator=g).to(dtype).to(gpu) for _ in range(2)]
    bases = [[torch.randn(rows, n, generator=g).to(dtype).to(gpu) for n in outs] for _ in range(2)]

    def run(i):
        return sgmv.lora_decode_stacked(xs[i], [b.clone() for b in bases[i]], cache, mods, plan)

    want = [[y.cpu() for y in run(i)] for i in range(2)]
    streams = [torch.cuda.Stream(), torch.cuda.Stream()]
    got = [[], []]
    for rnd in range(6):
        for i, s in enumerate(streams):
            with torch.cuda.stream(s):
                got[i].append(run(i))
    torch.cuda.synchronize()
    assert not sgmv.decode_waits_timed_out(gpu)
    for i in range(2):
        for rnd, ys in enumerate(got[i]):
            for m, y, w in zip(mods, ys, want[i]):
                assert torch.equal(y.cpu(), w), (i, rnd, m)
