"""Host logic without a GPU: config, PEFT parsing, CPU/disk tiers, slot cache, C-ABI surface.

The reference's tests (tests/test_polylora_peft.py) compare against PEFT,
which is not installed; their assertions on slots, ranks, scales, errors and
cache tiers are restated here on fixtures this suite writes in PEFT's file
layout.  The slot cache runs on a CPU device here (its uploads become host
copies), so the packed arena and the slot table can be checked byte for byte
against the reference-layout tensors of the oracle.
"""

from __future__ import annotations

import ctypes
import re
import shutil
import subprocess
from pathlib import Path

import numpy as np
import pytest
import torch

from oracle.lora import dense_slot_tensors
from oracle.slots import SlotCacheModel
from polylora_amd import PolyLoraConfig, PolyLoraModel, _native
from polylora_amd.cache import GpuAdapterCache, ModuleSpec, SlotLayout, tile_rows, untile_rows
from polylora_amd.context import LoraBatchContext, assert_right_padded, get_lora_context, use_lora_context
from polylora_amd.store import CpuAdapterStore, CpuLayerWeights, DiskAdapterCache
from tests import _peft

ROOT = Path(__file__).resolve().parents[1]
TARGETS = ["query_proj", "key_proj", "value_proj", "dense"]


# --------------------------------------------------------------------------- config


def test_config_validation_messages():
    with pytest.raises(ValueError, match="max_gpu_adapters must be at least 1"):
        PolyLoraConfig(max_gpu_adapters=0, max_rank=4)
    with pytest.raises(ValueError, match="max_cpu_adapters must be at least max_gpu_adapters"):
        PolyLoraConfig(max_gpu_adapters=3, max_rank=4, max_cpu_adapters=2)
    with pytest.raises(ValueError, match="max_disk_adapters must be at least 1"):
        PolyLoraConfig(max_gpu_adapters=1, max_rank=4, disk_cache_dir="/tmp/x", max_disk_adapters=0)
    with pytest.raises(ValueError, match="disk_cache_dir must be set"):
        PolyLoraConfig(max_gpu_adapters=1, max_rank=4, max_disk_adapters=2)
    with pytest.raises(ValueError, match="max_rank must be at least 1"):
        PolyLoraConfig(max_gpu_adapters=1, max_rank=0)
    with pytest.raises(ValueError, match="target_modules must not be empty"):
        PolyLoraConfig(max_gpu_adapters=1, max_rank=4, target_modules=[])
    cfg = PolyLoraConfig(max_gpu_adapters=2, max_rank=8)
    assert cfg.base_adapter_id == "__base__" and cfg.enforce_right_padding and cfg.use_triton_kernels
    from polylora_amd import CustomLoraConfig, CustomPeftModel

    assert CustomLoraConfig is PolyLoraConfig and CustomPeftModel is PolyLoraModel


# --------------------------------------------------------------------------- store: PEFT parsing


def _shapes():
    return {"enc.q_proj": (6, 4), "enc.v_proj": (6, 5)}


def test_peft_state_dict_layout_and_scale():
    g = torch.Generator().manual_seed(0)
    w = _peft.make_lora_weights(g, _shapes(), rank=3)
    store = CpuAdapterStore()
    for name in (None, "ad"):
        store.add_adapter_from_peft_state_dict(
            f"x{name}", _peft.state_dict(w, name), list(_shapes()), lora_alpha=9, peft_adapter_name=name or "default"
        )
        layers = store.adapters[f"x{name}"].layers
        for mod, (a, b) in w.items():
            assert torch.equal(layers[mod].A, a.t()) and torch.equal(layers[mod].B, b.t())
            assert layers[mod].rank == 3 and layers[mod].scale == 3.0


def test_peft_rejects_outside_module_set_and_incomplete_pair():
    g = torch.Generator().manual_seed(1)
    w = _peft.make_lora_weights(g, _shapes(), rank=2)
    store = CpuAdapterStore()
    with pytest.raises(ValueError, match="outside the configured module set"):
        store.add_adapter_from_peft_state_dict("a", _peft.state_dict(w, "a"), ["enc.v_proj"], 4, "a")
    sd = {k: v for k, v in _peft.state_dict(w, "a").items() if ".lora_B." not in k}
    with pytest.raises(ValueError, match="incomplete LoRA weights"):
        store.add_adapter_from_peft_state_dict("a", sd, list(_shapes()), 4, "a")
    with pytest.raises(ValueError, match="reserved for base-only rows"):
        store.add_adapter("__base__", {"m": CpuLayerWeights(torch.zeros(2, 1), torch.zeros(1, 2), 1, 1.0)})
    with pytest.raises(ValueError, match="at least one target layer"):
        store.add_adapter("e", {})


def test_sparse_adapter_missing_modules_are_rank_zero():
    g = torch.Generator().manual_seed(2)
    w = _peft.make_lora_weights(g, _shapes(), rank=2, modules=["enc.v_proj"])
    store = CpuAdapterStore()
    store.add_adapter_from_peft_state_dict("s", _peft.state_dict(w, "s"), list(_shapes()), 4, "s")
    cache = _cpu_cache(store, _shapes(), 1, 2)
    cache.ensure_resident(["s"])
    slot = cache.adapter_to_slot["s"]
    assert int(cache.ranks["enc.q_proj"][slot]) == 0 and float(cache.scales["enc.q_proj"][slot]) == 0.0
    assert int(cache.ranks["enc.v_proj"][slot]) == 2 and float(cache.scales["enc.v_proj"][slot]) == 2.0


@pytest.mark.parametrize("fmt", ["safetensors", "bin"])
def test_load_from_disk_formats(tmp_path, fmt):
    g = torch.Generator().manual_seed(3)
    w = _peft.make_lora_weights(g, _shapes(), rank=4)
    path = _peft.write_adapter_dir(tmp_path / "ad", w, 4, 8, fmt=fmt)
    store = CpuAdapterStore()
    store.load_adapter_from_disk("a", path, list(_shapes()))
    for mod, (a, b) in w.items():
        assert torch.equal(store.adapters["a"].layers[mod].A, a.t())
        assert store.adapters["a"].layers[mod].scale == 2.0


@pytest.mark.parametrize(
    "extra,msg",
    [
        ({"peft_type": "IA3"}, "Unsupported PEFT adapter type"),
        ({"use_dora": True}, "DoRA adapters are not supported"),
        ({"use_rslora": True}, "RS-LoRA adapters are not supported"),
        ({"lora_bias": True}, "LoRA bias is not supported"),
        ({"lora_dropout": 0.1}, "LoRA dropout is not supported"),
    ],
)
def test_peft_config_validation(tmp_path, extra, msg):
    g = torch.Generator().manual_seed(4)
    w = _peft.make_lora_weights(g, _shapes(), rank=2)
    path = _peft.write_adapter_dir(tmp_path / "ad", w, 2, 4, extra_config=extra)
    with pytest.raises(ValueError, match=msg):
        CpuAdapterStore().load_adapter_from_disk("a", path, list(_shapes()))


def test_cpu_lru_and_disk_reload(tmp_path):
    """tests/test_polylora_peft.py:484-550: a CPU miss reloads from the disk cache."""
    g = torch.Generator().manual_seed(5)
    disk = DiskAdapterCache(tmp_path / "disk", 2)
    store = CpuAdapterStore(max_adapters=1, disk_cache=disk, module_names=list(_shapes()))
    ws = {}
    for aid in ("a", "b"):
        ws[aid] = _peft.make_lora_weights(g, _shapes(), rank=2)
        store.load_adapter_from_disk(aid, _peft.write_adapter_dir(tmp_path / f"src_{aid}", ws[aid], 2, 4, fmt="bin"), list(_shapes()))
    assert "a" not in store.adapters and "a" in store
    got = store.get("a")
    assert "a" in store.adapters and "b" not in store.adapters
    assert torch.equal(got.layers["enc.q_proj"].A, ws["a"]["enc.q_proj"][0].t())


def test_disk_cache_evicts_oldest_directory(tmp_path):
    """tests/test_polylora_peft.py:553-609."""
    g = torch.Generator().manual_seed(6)
    disk = DiskAdapterCache(tmp_path / "disk", 2)
    store = CpuAdapterStore(max_adapters=1, disk_cache=disk, module_names=list(_shapes()))
    src = {}
    for aid in ("a", "b", "c"):
        src[aid] = _peft.write_adapter_dir(tmp_path / f"src_{aid}", _peft.make_lora_weights(g, _shapes(), 2), 2, 4)
        store.load_adapter_from_disk(aid, src[aid], list(_shapes()))
    assert "a" not in store
    assert list(disk.entries) == ["b", "c"]
    dirs = [p for p in (tmp_path / "disk").iterdir() if p.is_dir()]
    assert len(dirs) == 2 and all(p != src["a"] for p in dirs)
    # the manifest survives a restart
    again = DiskAdapterCache(tmp_path / "disk", 2)
    assert list(again.entries) == ["b", "c"]
    assert not [p for p in (tmp_path / "disk").iterdir() if p.name.endswith(".tmp")]


def test_disk_cache_manifest_write_is_all_or_nothing(tmp_path, monkeypatch):
    """A write that dies before the rename leaves the previous manifest whole."""
    g = torch.Generator().manual_seed(7)
    disk = DiskAdapterCache(tmp_path / "disk", 3)
    src = _peft.write_adapter_dir(tmp_path / "src_a", _peft.make_lora_weights(g, _shapes(), 2), 2, 4)
    disk.add_adapter("a", src)
    before = (tmp_path / "disk" / "manifest.json").read_text()

    def die(*_a, **_k):
        raise OSError("killed mid-write")

    monkeypatch.setattr("polylora_amd.store.os.replace", die)
    with pytest.raises(OSError, match="killed mid-write"):
        disk.add_adapter("b", src)
    monkeypatch.undo()
    assert (tmp_path / "disk" / "manifest.json").read_text() == before
    assert list(DiskAdapterCache(tmp_path / "disk", 3).entries) == ["a"]


def test_cpu_store_never_evicts_gpu_resident():
    store = CpuAdapterStore(max_adapters=1)
    lw = {"m": CpuLayerWeights(torch.zeros(2, 1), torch.zeros(1, 2), 1, 1.0)}
    store.add_adapter("a", lw)
    store.set_eviction_exclusions({"a"})
    with pytest.raises(RuntimeError, match="No evictable CPU LoRA adapter"):
        store.add_adapter("b", lw)


# --------------------------------------------------------------------------- GPU slot cache (CPU device)


def _cpu_cache(store, shapes, max_gpu, max_rank, dtype=torch.float32):
    cfg = PolyLoraConfig(max_gpu_adapters=max_gpu, max_rank=max_rank)
    specs = [ModuleSpec(n, i, o) for n, (i, o) in shapes.items()]
    return GpuAdapterCache(store, specs, cfg, torch.device("cpu"), dtype)


def _store_with(ws: dict, alphas: dict) -> CpuAdapterStore:
    store = CpuAdapterStore()
    for aid, w in ws.items():
        store.add_adapter_from_peft_state_dict(aid, _peft.state_dict(w), sorted({m for m in w}), alphas[aid])
    return store


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_slot_arena_matches_reference_layout_bit_exact(dtype):
    g = torch.Generator().manual_seed(7)
    shapes = {"l0.q": (24, 16), "l0.o": (16, 40), "l1.q": (24, 16)}
    ranks = {"a": 3, "b": 8, "c": 5}
    ws = {aid: _peft.make_lora_weights(g, shapes, r, modules=None if aid != "c" else ["l0.o"]) for aid, r in ranks.items()}
    store = _store_with(ws, {"a": 6, "b": 4, "c": 5})
    cache = _cpu_cache(store, shapes, 3, 8, dtype)
    slots_ = cache.ensure_resident(["c", "__base__", "a", "b", "a"])
    assert slots_.dtype == torch.int32
    assert slots_.tolist() == [3, 0, 1, 2, 1]  # sorted load order into the lowest free slots
    for mod, (fin, fout) in shapes.items():
        per_slot = [None] + [
            None if mod not in ws[cache.slot_to_adapter[s]] else (*ws[cache.slot_to_adapter[s]][mod], {"a": 6, "b": 4, "c": 5}[cache.slot_to_adapter[s]])
            for s in range(1, 4)
        ]
        A, B, rk, sc = dense_slot_tensors(per_slot, fin, fout, 8, dtype)
        assert torch.equal(cache.A[mod], A)
        assert torch.equal(cache.B[mod], B)
        assert torch.equal(cache.ranks[mod], rk)
        assert torch.equal(cache.scales[mod], sc)
    # base slot 0: rank 0 and scale 0 in every module (tests/test_polylora_peft.py:323-326)
    assert cache.adapter_to_slot["__base__"] == 0
    assert all(int(cache.ranks[m][0]) == 0 and float(cache.scales[m][0]) == 0.0 for m in shapes)


def test_slot_cache_matches_slot_model_under_churn():
    """Same slot trace as the restated bookkeeping for a long random id sequence."""
    g = torch.Generator().manual_seed(8)
    rng = np.random.default_rng(8)
    shapes = {"m": (8, 8)}
    ids = [f"ad{i:02d}" for i in range(12)]
    ws = {aid: _peft.make_lora_weights(g, shapes, 1 + i % 4) for i, aid in enumerate(ids)}
    store = _store_with(ws, {aid: 2.0 for aid in ids})
    cache = _cpu_cache(store, shapes, 4, 4)
    model = SlotCacheModel(4)
    for step in range(60):
        batch = [ids[int(i)] if rng.random() > 0.2 else "__base__" for i in rng.integers(0, 12, size=5)]
        distinct = {a for a in batch if a != "__base__"}
        if len(distinct) > 4:
            with pytest.raises(RuntimeError, match="more adapters than GPU cache capacity"):
                cache.ensure_resident(batch)
            continue
        got = cache.ensure_resident(batch).tolist()
        want = model.ensure_resident(batch, set(ids))
        assert got == want, step
        assert cache.slot_to_adapter == model.slot_to_adapter
        assert list(cache.lru) == list(model.lru)
        for s, aid in enumerate(cache.slot_to_adapter):
            want_rank = 0 if s == 0 or aid is None else ws[aid]["m"][0].shape[0]
            assert int(cache.ranks["m"][s]) == want_rank


def test_slot_reload_cycle_and_errors():
    g = torch.Generator().manual_seed(9)
    shapes = {"m": (8, 8)}
    ws = {aid: _peft.make_lora_weights(g, shapes, 2) for aid in ("a", "b")}
    cache = _cpu_cache(_store_with(ws, {"a": 4, "b": 4}), shapes, 1, 2)
    for aid in ("a", "b", "a"):
        cache.ensure_resident([aid])
        assert cache.slot_to_adapter[1] == aid
        assert torch.equal(cache.A["m"][1], ws[aid]["m"][0].t())
    with pytest.raises(KeyError, match="Unknown LoRA adapter"):
        cache.ensure_resident(["nope"])
    with pytest.raises(RuntimeError, match="more adapters than GPU cache capacity"):
        cache.ensure_resident(["a", "b"])
    big = {"m": (torch.zeros(3, 8), torch.zeros(8, 3))}
    store = _store_with({"r3": big}, {"r3": 3})
    with pytest.raises(ValueError, match="exceeds max_rank"):
        _cpu_cache(store, shapes, 1, 2).ensure_resident(["r3"])


def test_pack_adapter_layout():
    shapes = {"x": (16, 24), "y": (8, 8)}
    a = torch.arange(3 * 16, dtype=torch.float32).reshape(3, 16)
    b = torch.arange(24 * 3, dtype=torch.float32).reshape(24, 3)
    store = CpuAdapterStore()
    store.add_adapter("p", {"x": CpuLayerWeights(a.t().contiguous(), b.t().contiguous(), 3, 1.5)})
    layout = SlotLayout([ModuleSpec(n, i, o) for n, (i, o) in shapes.items()], torch.bfloat16, 6)
    packed = store.adapters["p"].image_for(layout)
    rows = packed.rows
    assert rows[0, 0] == 3 and rows[0, 2] == 8 and rows.view(np.float32)[0, 1] == np.float32(1.5)
    a_off, b_off = int(rows.view(np.int64)[0, 2]), int(rows.view(np.int64)[0, 3])
    assert a_off % 256 == 0 and b_off % 256 == 0
    img = packed.data
    A = img[a_off : a_off + 3 * 16 * 2].view(torch.bfloat16).view(3, 16)
    B = img[b_off : b_off + 24 * 8 * 2].view(torch.bfloat16).view(24, 8)
    assert torch.equal(A, a.bfloat16()) and torch.equal(B[:, :3], b.bfloat16())
    assert torch.equal(B[:, 3:], torch.zeros(24, 5, dtype=torch.bfloat16))  # rank padding is zero
    assert rows[1].tolist() == [0] * 8  # module without weights: rank 0, scale 0
    assert layout.rank8_cap == 8


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
@pytest.mark.parametrize("R,C", [(3, 16), (20, 72), (40, 33 * 8), (16, 64), (1, 1000), (64, 8)])
def test_tile_rows_block_layout(dtype, R, C):
    """The arena's MFMA-block layout: a round trip, and the position of every element."""
    m = torch.randn(R, C).to(dtype)
    flat = tile_rows(m)
    assert flat.shape == (R * C,)
    assert torch.equal(untile_rows(flat, R, C), m)
    w = 64 // m.element_size()
    # element (i, c) sits at 16t*C + s*rt*W + (i % 16)*wb + (c - sW): walk the
    # tiles and blocks in storage order and compare slices of the flat image
    pos = 0
    for t in range(0, R, 16):
        rt = min(16, R - t)
        for c0 in range(0, C, w):
            wb = min(w, C - c0)
            assert torch.equal(flat[pos : pos + rt * wb].view(rt, wb), m[t : t + rt, c0 : c0 + wb]), (t, c0)
            pos += rt * wb
    assert pos == R * C
    if C <= w:
        assert torch.equal(flat.view(R, C), m)  # narrow matrices stay row-major


def test_pack_adapter_block_layout_round_trip():
    """Packed A and B of ranks and widths that use several tiles and blocks read back exactly."""
    g = torch.Generator().manual_seed(11)
    shapes = {"a": (72, 40), "b": (4104, 1000)}
    store = CpuAdapterStore()
    ws = {}
    for name, (fin, fout) in shapes.items():
        r = 20 if name == "a" else 40
        A = torch.randn(fin, r, generator=g)
        B = torch.randn(r, fout, generator=g)
        ws[name] = (A, B, r)
    store.add_adapter("p", {n: CpuLayerWeights(A, B, r, 0.5) for n, (A, B, r) in ws.items()})
    layout = SlotLayout([ModuleSpec(n, i, o) for n, (i, o) in shapes.items()], torch.bfloat16, 40)
    packed = store.adapters["p"].image_for(layout)
    for i, (name, (fin, fout)) in enumerate(shapes.items()):
        A, B, r = ws[name]
        r8 = (r + 7) // 8 * 8
        a_off, b_off = int(packed.rows.view(np.int64)[i, 2]), int(packed.rows.view(np.int64)[i, 3])
        a_img = packed.data[a_off : a_off + r * fin * 2].view(torch.bfloat16)
        b_img = packed.data[b_off : b_off + fout * r8 * 2].view(torch.bfloat16)
        assert torch.equal(untile_rows(a_img, r, fin), A.t().bfloat16())
        b_rows = untile_rows(b_img, fout, r8)
        assert torch.equal(b_rows[:, :r], B.t().bfloat16())
        assert not b_rows[:, r:].any()  # rank padding is zero


def test_shrink_result_ownership():
    """A shrink result stays valid until a later shrink takes over its workspace."""
    from polylora_amd import sgmv

    class _Ws:
        owner = None

    ws0, ws1 = _Ws(), _Ws()
    batch = sgmv._ShrinkBatch(2, None)
    a = sgmv.ShrinkResult(ws0, None, 4, 16, 8, None, 64, batch, 0)
    b = sgmv.ShrinkResult(ws1, None, 4, 16, 8, None, 64, batch, 1)
    assert a.valid and b.valid and a.batch is b.batch and (a.index, b.index) == (0, 1)
    c = sgmv.ShrinkResult(ws0, None, 4, 16, 8, None, 64)
    assert c.valid and not a.valid and b.valid and c.batch is None


# --------------------------------------------------------------------------- context and model wrapper


def test_context_var_protocol():
    assert get_lora_context() is None
    ctx = LoraBatchContext(["a"], torch.tensor([1], dtype=torch.int32), torch.tensor([3], dtype=torch.int32))
    with use_lora_context(ctx):
        assert get_lora_context() is ctx
    assert get_lora_context() is None


def test_assert_right_padded():
    mask = torch.tensor([[1, 1, 0], [1, 1, 1]])
    assert_right_padded(mask, mask.sum(-1))
    with pytest.raises(ValueError, match="right-padded attention_mask"):
        bad = torch.tensor([[0, 1, 1]])
        assert_right_padded(bad, bad.sum(-1))
    with pytest.raises(ValueError, match="2D batch mask"):
        assert_right_padded(torch.ones(2, 2, 2), torch.tensor([2, 2]))


def test_model_wrapping_and_cpu_lora_refuses():
    model = _peft.tiny_deberta(0)
    pm = PolyLoraModel(model, PolyLoraConfig(max_gpu_adapters=2, max_rank=3, target_modules=TARGETS))
    names = pm.target_module_names
    assert len(names) == 6  # q, k, v, attention.output.dense, intermediate.dense, output.dense
    assert all(type(pm.base_model.get_submodule(n)).__name__ == "MultiLoraLinear" for n in names)
    ids = torch.tensor([[1, 5, 6, 2]])
    with torch.inference_mode():
        base = pm(input_ids=ids).last_hidden_state  # no adapter_ids: plain base model
    assert base.shape == (1, 4, 32)
    g = torch.Generator().manual_seed(0)
    w = _peft.make_lora_weights(g, {sp.name: (sp.in_features, sp.out_features) for sp in pm.module_specs}, 2)
    pm.adapter_store.add_adapter_from_peft_state_dict("a", _peft.state_dict(w, "a"), names, 4, "a")
    with pytest.raises(RuntimeError, match="only on a ROCm GPU"):
        with torch.inference_mode():
            pm(input_ids=ids, adapter_ids=["a"])
    with pytest.raises(ValueError, match="adapter_ids length must match batch size"):
        pm(input_ids=ids, adapter_ids=["a", "a"])
    with pytest.raises(ValueError, match="No nn.Linear modules matched"):
        PolyLoraModel(_peft.tiny_deberta(0), PolyLoraConfig(max_gpu_adapters=1, max_rank=2, target_modules=["nothing"]))


# --------------------------------------------------------------------------- C-ABI surface


def _header_functions() -> list[str]:
    text = (ROOT / "include" / "polylora_hip.h").read_text()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"^\s*(?:const\s+)?[a-z_0-9]+\s*\*?\s*(pl_[a-z_0-9]+)\s*\(", text, flags=re.M)))


def test_library_exports_every_declared_symbol():
    lib = ctypes.CDLL(str(_native.LIB_PATH))
    declared = _header_functions()
    assert len(declared) >= 12
    for name in declared:
        assert hasattr(lib, name), name
    assert set(declared) == set(_native.EXPORTED_SYMBOLS)


@pytest.mark.parametrize("compiler,std,suffix", [("gcc", "c99", "c"), ("g++", "c++17", "cpp")])
def test_header_compiles_as_c_and_cpp_and_links(tmp_path, compiler, std, suffix):
    """A C (cgo, FFI) or C++ client: a program that includes the public header, takes the address of every
    declared entry point and links against the library compiles warning-free under -pedantic and runs."""
    if shutil.which(compiler) is None:
        pytest.skip(f"{compiler} is not installed")
    names = _header_functions()
    src = tmp_path / f"client.{suffix}"
    src.write_text(
        '#include "polylora_hip.h"\n#include <stdio.h>\n'
        "int main(void) {\n  void (*fns[])(void) = {\n"
        + "".join(f"    (void (*)(void))&{n},\n" for n in names)
        + '  };\n  printf("%d %d\\n", pl_version(), (int)(sizeof(fns) / sizeof(fns[0])));\n  return 0;\n}\n')
    exe = tmp_path / "client"
    lib_dir = _native.LIB_PATH.parent
    subprocess.run([compiler, f"-std={std}", "-Wall", "-Wextra", "-pedantic", "-Werror", f"-I{ROOT / 'include'}",
                    str(src), "-o", str(exe), f"-L{lib_dir}", "-lpolylora_hip", f"-Wl,-rpath,{lib_dir}"],
                   check=True, capture_output=True, text=True)
    out = subprocess.run([str(exe)], check=True, capture_output=True, text=True).stdout.split()
    assert out == [str(_native.load().pl_version()), str(len(names))]


def test_library_host_side_errors_without_gpu():
    """Argument checks run before any HIP call, so they are testable on the CPU."""
    lib = _native.load()
    assert lib.pl_version() >= 100
    # at most ceil(tokens / G) + slots - 1 groups, rounded up to whole XCD rounds of 8 positions
    assert lib.pl_plan_group_capacity(256, 1, 65, 64) == 72  # 4 + 64 = 68 -> 72
    assert lib.pl_plan_group_capacity(256, 1, 65, 16) == 80  # 16 + 64
    assert lib.pl_plan_group_capacity(32, 1024, 9, 64) == 520  # 512 + 8
    assert lib.pl_plan_group_capacity(4096, 1, 17, 16) == 272  # 256 + 16
    # split planes: whole wave steps (16-token groups: 64 elements of a
    # 2-byte type per wave step, 32 of fp32; 64-token groups: 64 and 32), four
    # waves per split, at most the requested count and at most 16
    assert lib.pl_shrink_planes(_native.PL_BF16, 4096, 8, 64) == 8
    assert lib.pl_shrink_planes(_native.PL_BF16, 4096, 100, 64) == 16
    assert lib.pl_shrink_planes(_native.PL_BF16, 4096, 100, 16) == 16  # capped at 16 planes
    assert lib.pl_shrink_planes(_native.PL_BF16, 4096, 4, 16) == 4
    assert lib.pl_shrink_planes(_native.PL_BF16, 4096, 2, 16) == 2
    assert lib.pl_shrink_planes(_native.PL_BF16, 14336, 100, 16) == 14
    assert lib.pl_shrink_planes(_native.PL_BF16, 65536, 100, 16) == 16
    assert lib.pl_shrink_planes(_native.PL_F32, 4096, 100, 16) == 16
    assert lib.pl_shrink_planes(_native.PL_BF16, 100, 16, 16) == 1  # one 64-element step covers a split
    assert lib.pl_shrink_planes(_native.PL_BF16, 14336, 16, 64) == 14
    assert lib.pl_shrink_planes(_native.PL_F32, 768, 4, 64) == 3
    assert lib.pl_shrink_planes(_native.PL_BF16, 32, 1, 16) == 1
    assert lib.pl_shrink_planes(_native.PL_BF16, 4096, 4, 32) == 0  # only 16 or 64
    # workspace: fp32 planes [planes][rows][ldt]
    assert lib.pl_shrink_workspace_bytes(_native.PL_BF16, 4096, 1, 64, 100, 16) == 100 * 16 * 4
    assert lib.pl_shrink_workspace_bytes(_native.PL_BF16, 4096, 8, 64, 100, 16) == 8 * 100 * 16 * 4
    assert lib.pl_shrink_workspace_bytes(_native.PL_F32, 768, 4, 64, 10, 8) == 3 * 10 * 8 * 4
    fake = ctypes.c_void_p(64)  # never dereferenced: the size check fails first
    assert lib.pl_plan_build(fake, fake, 4, 1, 5000, 64, fake, fake, fake, 100, None) == 4  # PL_ERR_LIMIT
    assert b"exceed the maximum" in lib.pl_last_error()
    st = lib.pl_sgmv_shrink(7, None, 0, 0, None, None, 1, 0, None, None, None, 1, 64, None, 0, 8, 1, 1, None)
    assert st == 1 and b"dtype" in lib.pl_last_error()
    with pytest.raises(RuntimeError, match="dtype"):
        _native.check(st, "pl_sgmv_shrink")
    # the no-alloc entry point refuses a call beyond its static scratch before any HIP call
    st = lib.pl_lora_apply_noalloc(_native.PL_BF16, fake, 4096, 4096, fake, 4096, 4096, fake, fake, 1, 0, fake,
                                   fake, 8192, 64, 17, 16, 64, 8, 0, None)
    assert st == 4 and b"needs" in lib.pl_last_error() and b"static scratch" in lib.pl_last_error()
    st = lib.pl_lora_apply_noalloc(_native.PL_BF16, fake, 4096, 4096, fake, 4096, 4096, fake, fake, 1, 0, fake,
                                   fake, 4, 1, 17, 32, 64, 8, 0, None)
    assert st == 1 and b"bad sizes" in lib.pl_last_error()
    # a grid counts its work-items in 32 bits: 2^32 mask elements at 256 per workgroup do not fit
    st = lib.pl_check_right_padded(fake, 0, 65536, 65536, fake, fake, None)
    assert st == 4 and b"too large" in lib.pl_last_error()


def test_no_cpu_fallback_in_product_ops():
    from polylora_amd import sgmv

    x = torch.randn(2, 3, 4)
    with pytest.raises(RuntimeError, match="no CPU fallback"):
        sgmv.sgmv_lora_a_fwd(x, torch.randn(2, 4, 2), torch.tensor([3, 3]), torch.tensor([0, 1]), torch.tensor([0, 2]))


def test_group_size_choice():
    from polylora_amd import sgmv

    short, long_ = _native.PL_GROUP_TOKENS_SHORT, _native.PL_GROUP_TOKENS_LONG
    assert sgmv.choose_group_tokens(256, 47) == short  # decode: a few rows per adapter
    assert sgmv.choose_group_tokens(4096, 16) == short  # below the long-group batch size
    assert sgmv.choose_group_tokens(32 * 1024, 8) == long_  # prefill: long segments
    assert sgmv.choose_group_tokens(32 * 1024, None) == long_
    assert sgmv.choose_group_tokens(32 * 1024, 2048) == short  # many adapters, short segments
    assert sgmv.choose_k_splits(80, 4096, torch.bfloat16) == 4
    assert sgmv.choose_k_splits(4096, 4096, torch.bfloat16) == 1  # groups alone fill the GPU


def test_cache_moved_under_inference_mode_still_loads_outside_it():
    """A cache whose arena and table were (re)allocated inside torch.inference_mode (a first forward there moves
    it) loads adapters outside that mode: they are ordinary tensors, written with in-place copies."""
    g = torch.Generator().manual_seed(40)
    w = _peft.make_lora_weights(g, _shapes(), rank=2)
    store = CpuAdapterStore()
    store.add_adapter_from_peft_state_dict("a", _peft.state_dict(w), list(_shapes()), 4)
    cache = _cpu_cache(store, _shapes(), 1, 2)
    with torch.inference_mode():
        cache.to(torch.device("cpu"), torch.bfloat16)
    assert not cache.arena.is_inference() and not cache.table.is_inference()
    cache.ensure_resident(["a"])
    slot = cache.adapter_to_slot["a"]
    assert int(cache.ranks["enc.q_proj"][slot]) == 2
    for mod, (a, b) in w.items():
        assert torch.equal(cache.A[mod][slot, :, :2], a.t().to(torch.bfloat16))


@pytest.mark.skipif(torch.cuda.is_available(), reason="fake device pointers: run only where no GPU can be reached")
def test_decode_launch_refuses_bad_arguments_before_any_launch():
    """pl_lora_decode_stacked checks its plan geometry, workspaces, hand-off counters and spin limit on the
    host and returns PL_ERR_ARG with a message before any HIP call; each call below breaks one rule."""
    import ctypes

    lib = _native.load()
    fake = [ctypes.c_void_p(4096 * (i + 1)) for i in range(8)]  # 16-byte aligned, never dereferenced
    dt, K, n, cap, rows, ldt, splits = _native.PL_BF16, 1024, 2, 40, 256, 64, 4
    ws_bytes = int(lib.pl_shrink_workspace_bytes(dt, K, splits, 16, rows, ldt))
    ints = int(lib.pl_decode_counter_ints(cap, n))
    assert ws_bytes > 0 and ints > 0

    def call(gt=16, ldt_=ldt, ws=(fake[5], fake[6]), counters=fake[7], counter_ints=ints, spin=1 << 16):
        mods = (ctypes.c_int32 * n)(0, 1)
        wsp = (ctypes.c_void_p * n)(*ws)
        yp = (ctypes.c_void_p * n)(fake[3], fake[4])
        ldy = (ctypes.c_int64 * n)(512, 512)
        nn = (ctypes.c_int32 * n)(512, 512)
        return lib.pl_lora_decode_stacked(dt, fake[0], K, K, fake[1], fake[2], 2, n, mods, wsp, fake[1], fake[2],
                                          fake[1], cap, gt, ws_bytes, ldt_, rows, splits, yp, ldy, nn,
                                          _native.PL_EPI_FALLBACK, counters, counter_ints, spin, None)

    cases = [
        (dict(gt=64), b"16-token groups"),
        (dict(ldt_=40), b"multiple of 32"),
        (dict(ws=(fake[5], fake[5])), b"its own workspace"),
        (dict(counters=None), b"null or misaligned hand-off counters"),
        (dict(counters=ctypes.c_void_p(4096 * 8 + 2)), b"null or misaligned hand-off counters"),
        (dict(counter_ints=ints - 1), b"needed"),
        (dict(spin=0), b"spin_limit"),
    ]
    for kw, msg in cases:
        st = call(**kw)
        assert st == 1, (kw, st, lib.pl_last_error())
        assert msg in lib.pl_last_error(), (kw, lib.pl_last_error())


def test_operator_part_sizes_depend_only_on_what_their_keys_hold():
    """The kept operator parts are looked up by keys that leave some sizes out, so their byte counts must not
    depend on those: the weights part depends on the weights' shape and dtype only (not on the batch), and
    the plan part on the batch geometry and adapter count only (not on K, n, dtype or which call), so one
    plan serves the shrink and the expand of every Linear of a forward.  Shapes the MFMA path declines
    (ranks above 64, K or N not whole 16-byte chunks) report 0 bytes."""
    lib = _native.load()

    def size(dt, which, B, M, K, n, S, part):
        return int(lib.pl_sgmv_ref_part_bytes(dt, which, B, M, K, n, S, part))

    bf, f32 = _native.PL_BF16, _native.PL_F32
    for which, (K, n) in ((0, (4096, 64)), (1, (64, 4096)), (0, (14336, 16)), (1, (32, 1024))):
        w = {size(dt, which, B, M, K, n, 65, 1) for dt in (bf,) for B, M in ((1, 1), (256, 1), (32, 1024), (8192, 1), (7, 33))}
        assert len(w) == 1 and w.pop() > 0, (which, K, n)
    for B, M, S in ((256, 1, 65), (32, 1024, 9), (4096, 1, 17), (3, 7, 2)):
        p = {size(dt, which, B, M, K, n, S, 0) for dt in (bf, f32) for which, (K, n) in
             ((0, (4096, 64)), (1, (64, 4096)), (0, (1024, 8)), (1, (16, 768)))}
        assert len(p) == 1 and p.pop() > 0, (B, M, S)
    assert size(bf, 0, 256, 1, 4096, 128, 65, 0) == 0  # n_max above 64: the row kernels
    assert size(bf, 0, 256, 1, 4100, 64, 65, 1) == 0  # K not whole 16-byte chunks
    assert size(bf, 1, 256, 1, 64, 1001, 65, 0) == 0  # N not whole 16-byte chunks
    # the expand reads the caller's intermediate directly: no scratch; the shrink's split planes need some
    assert size(bf, 1, 256, 1, 64, 1000, 65, 2) == 0 and size(bf, 0, 256, 1, 4096, 64, 65, 2) > 0
