"""bench.py --reduce-profile: rocprofv3 CSVs of a --launch-profile run -> labelled per-launch figures."""

from __future__ import annotations

import csv
import json

import pytest

import bench

TRACE_COLS = ["Kind", "Agent_Id", "Queue_Id", "Dispatch_Id", "Kernel_Name", "Start_Timestamp", "End_Timestamp",
              "Workgroup_Size_X", "Workgroup_Size_Y", "Workgroup_Size_Z", "Grid_Size_X", "Grid_Size_Y", "Grid_Size_Z"]
PMC_COLS = ["Dispatch_Id", "Kernel_Name", "Grid_Size", "Workgroup_Size", "Counter_Name", "Counter_Value"]

SEQ = [{"label": "q/k/v stacked shrink", "part": "shrink", "bytes": 1000},
       {"label": "q/k/v stacked expand", "part": "expand", "bytes": 3000},
       {"label": "o fused", "part": "fused", "bytes": 8000}]
KERNELS = ["void pl_shrink_short<__hip_bfloat16>(pl_args)", "void pl_expand_short<__hip_bfloat16, 2>(pl_args)",
           "void pl_lora_fused_tile<__hip_bfloat16, false>(pl_fused_args)"]
DUR_NS = [10_000, 30_000, 40_000]


def _write(path, cols, rows):
    with open(path, "w", newline="") as fh:
        w = csv.DictWriter(fh, fieldnames=cols)
        w.writeheader()
        for r in rows:
            w.writerow(r)


def _trace_rows(passes, swap_at=None):
    rows, did, t = [], 1, 0
    for name in ("void pl_plan_kernel(int const*)", "at::native::elementwise_kernel<128, 4>"):
        rows.append(dict(Kind="KERNEL_DISPATCH", Agent_Id=1, Queue_Id=1, Dispatch_Id=did, Kernel_Name=name,
                         Start_Timestamp=t, End_Timestamp=t + 5000, Workgroup_Size_X=1024, Workgroup_Size_Y=1,
                         Workgroup_Size_Z=1, Grid_Size_X=1024, Grid_Size_Y=1, Grid_Size_Z=1))
        did, t = did + 1, t + 10_000
    for p in range(passes):
        for i, (k, d) in enumerate(zip(KERNELS, DUR_NS)):
            if swap_at == (p, i):
                k = KERNELS[(i + 1) % 3]
            rows.append(dict(Kind="KERNEL_DISPATCH", Agent_Id=1, Queue_Id=1, Dispatch_Id=did, Kernel_Name=k,
                             Start_Timestamp=t, End_Timestamp=t + d + 1000 * p, Workgroup_Size_X=256,
                             Workgroup_Size_Y=1, Workgroup_Size_Z=1, Grid_Size_X=256 * (i + 1) * 64, Grid_Size_Y=1,
                             Grid_Size_Z=1))
            did, t = did + 1, t + 100_000
    return rows


def _pmc_rows(counter, passes, per_kernel):
    rows = [dict(Dispatch_Id=1, Kernel_Name="__amd_rocclr_copyBuffer", Grid_Size=1, Workgroup_Size=1,
                 Counter_Name=counter, Counter_Value=per_kernel["copy"])]
    did = 2
    for _ in range(passes):
        for i, k in enumerate(KERNELS):
            # two rows for one dispatch (the reducer sums them)
            for half in (0.5, 0.5):
                rows.append(dict(Dispatch_Id=did, Kernel_Name=k, Grid_Size=256, Workgroup_Size=256,
                                 Counter_Name=counter, Counter_Value=per_kernel[i] * half))
            did += 1
    return rows


def _args(tmp_path, **kw):
    ns = dict(manifest=str(tmp_path / "m.json"), trace=str(tmp_path / "t.csv"), fetch=None, write=None,
              copy_fetch=None, copy_write=None, copy_bytes=1 << 20, reduce_json=str(tmp_path / "r.json"))
    ns.update(kw)
    return type("A", (), ns)


def _manifest(tmp_path, warmup=1, passes=2):
    (tmp_path / "m.json").write_text(json.dumps({"workload": "synthetic", "kind": "decode", "warmup": warmup,
                                                 "passes": passes, "plan_builds": 1, "event_ms_per_pass": 0.09,
                                                 "sequence": SEQ}))


def test_kernel_base_name():
    assert bench.kernel_base_name(KERNELS[1]) == "pl_expand_short"
    assert bench.kernel_base_name("pl_plan_kernel") == "pl_plan_kernel"


def test_reduce_labels_by_position_and_drops_warmup(tmp_path, capsys):
    _manifest(tmp_path)
    _write(tmp_path / "t.csv", TRACE_COLS, _trace_rows(3))
    fetch = _pmc_rows("FETCH_SIZE", 3, {"copy": 512, 0: 2.0, 1: 1.0, 2: 4.0})  # copy reads 1 MiB, FETCH says half
    write = _pmc_rows("WRITE_SIZE", 3, {"copy": 1024, 0: 0.5, 1: 2.0, 2: 3.0})
    _write(tmp_path / "f.csv", PMC_COLS, fetch)
    _write(tmp_path / "w.csv", PMC_COLS, write)
    args = _args(tmp_path, fetch=str(tmp_path / "f.csv"), write=str(tmp_path / "w.csv"),
                 copy_fetch=str(tmp_path / "f.csv"), copy_write=str(tmp_path / "w.csv"))
    assert bench.reduce_profile(args) == 0
    text = capsys.readouterr().out
    rep = json.loads((tmp_path / "r.json").read_text())
    assert rep["fetch_scale"] == pytest.approx(2.0) and rep["write_scale"] == pytest.approx(1.0)
    lab = rep["labels"]
    # passes 1 and 2 (pass 0 is warm-up): durations d + 1000 p ns
    assert lab["q/k/v stacked shrink"]["avg_us"] == pytest.approx(11.5)
    assert lab["o fused"]["avg_us"] == pytest.approx(41.5)
    assert lab["o fused"]["kernels"] == ["pl_lora_fused_tile"]
    assert lab["q/k/v stacked expand"]["traffic_bytes_per_launch"] == pytest.approx(1024 * (1.0 * 2 + 2.0))
    assert rep["kernels"]["pl_shrink_short"]["traffic_bytes_per_launch"] == pytest.approx(1024 * (2.0 * 2 + 0.5))
    assert rep["pass_us"] == pytest.approx(11.5 + 31.5 + 41.5)
    assert rep["pass_bytes"] == 12000
    assert "pl_plan_kernel: 1 dispatches" in text and "| o fused | pl_lora_fused_tile | 1 | 192 |" in text


def test_reduce_rejects_a_pass_whose_kernels_differ(tmp_path):
    _manifest(tmp_path)
    _write(tmp_path / "t.csv", TRACE_COLS, _trace_rows(3, swap_at=(2, 1)))
    with pytest.raises(ValueError, match="where the first pass had"):
        bench.reduce_profile(_args(tmp_path))


def test_reduce_rejects_too_few_dispatches(tmp_path):
    _manifest(tmp_path, passes=5)
    _write(tmp_path / "t.csv", TRACE_COLS, _trace_rows(3))
    with pytest.raises(ValueError, match="the manifest needs 18"):
        bench.reduce_profile(_args(tmp_path))


def test_reduce_graph_trace_splits_bursts_and_compares_steps(tmp_path, capsys):
    """bench.py --reduce-graph-trace: base and LoRA timed bursts, per-kernel time per step."""
    rows, t, did = [], 0, 1

    def burst(kernels, reps):
        nonlocal t, did
        for _ in range(reps):
            for name, dur in kernels:
                rows.append(dict(Kind="KERNEL_DISPATCH", Agent_Id=1, Queue_Id=1, Dispatch_Id=did, Kernel_Name=name,
                                 Start_Timestamp=t, End_Timestamp=t + dur, Workgroup_Size_X=256, Workgroup_Size_Y=1,
                                 Workgroup_Size_Z=1, Grid_Size_X=256, Grid_Size_Y=1, Grid_Size_Z=1))
                did, t = did + 1, t + dur + 1000
        t += 300_000_000  # the pause between bursts

    base = [("Cijk_gemm(args)", 50_000), ("attn_fwd(args)", 100_000)]
    lora = [("Cijk_gemm(args)", 50_000), ("void pl_shrink_short<__hip_bfloat16, 4>(pl_shrink_args)", 10_000),
            ("void pl_expand_short<__hip_bfloat16, 4, 32>(pl_expand_args)", 12_000), ("attn_fwd(args)", 100_000)]
    burst(base, 2)
    burst(base, 5)
    burst(lora, 2)
    burst(lora, 5)
    _write(tmp_path / "t.csv", TRACE_COLS, rows)
    assert bench.main(["--reduce-graph-trace", "--trace", str(tmp_path / "t.csv"), "--profile-passes", "5"]) == 0
    out = capsys.readouterr().out
    assert "| pl_shrink_short | 0.0 | 10.0 | +10.0 | 0 / 1 |" in out
    assert "| pl_expand_short | 0.0 | 12.0 | +12.0 | 0 / 1 |" in out
    assert "| attn_fwd | 100.0 | 100.0 | +0.0 | 1 / 1 |" in out
    assert "base: " in out and "2 kernels." in out and "4 kernels." in out
    # a trace without the four bursts is refused
    _write(tmp_path / "short.csv", TRACE_COLS, rows[:4])
    assert bench.main(["--reduce-graph-trace", "--trace", str(tmp_path / "short.csv"), "--profile-passes", "5"]) == 1
