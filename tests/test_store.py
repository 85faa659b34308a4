"""The host store's single copy of an adapter: slot images packed straight from PEFT tensors and files.

Reference behaviour kept (store.py:160-436, cache.py:119-150): the same
errors at the same moments, ``CpuLayerWeights`` views with A = lora_A^T,
B = lora_B^T and scale = alpha / r.  New here: once the GPU cache binds its
slot layout, an adapter is held only as its packed image; the safetensors
reader maps the file instead of materializing a state dict.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

from polylora_amd.cache import GpuAdapterCache, ModuleSpec
from polylora_amd.config import PolyLoraConfig
from polylora_amd.slot_image import ImageBuilder, SlotLayout, untile_rows
from polylora_amd.store import CpuAdapterStore, CpuLayerWeights, read_safetensors
from tests import _peft

SHAPES = {"enc.q_proj": (24, 16), "enc.v_proj": (16, 40), "dec.o_proj": (40, 24)}


def _specs():
    return [ModuleSpec(n, i, o) for n, (i, o) in SHAPES.items()]


def _bound(dtype=torch.bfloat16, max_rank=8, max_gpu=2):
    store = CpuAdapterStore(module_names=list(SHAPES))
    cache = GpuAdapterCache(store, _specs(), PolyLoraConfig(max_gpu_adapters=max_gpu, max_rank=max_rank),
                            torch.device("cpu"), dtype)
    return store, cache


def _weights(seed, rank, modules=None):
    return _peft.make_lora_weights(torch.Generator().manual_seed(seed), SHAPES, rank, modules=modules)


@pytest.mark.parametrize("dtype,src", [(torch.bfloat16, torch.bfloat16), (torch.float32, torch.float32),
                                       (torch.float32, torch.bfloat16)])
def test_bound_store_holds_only_the_packed_image(dtype, src):
    store, cache = _bound(dtype)
    w = {m: (a.to(src), b.to(src)) for m, (a, b) in _weights(0, 5).items()}
    store.add_adapter_from_peft_state_dict("a", _peft.state_dict(w), list(SHAPES), lora_alpha=10)
    ad = store.adapters["a"]
    assert ad.image is not None and ad._modules is None  # packing is exact: no PEFT tensors kept beside the image
    for mod, (a, b) in w.items():
        lw = ad.layers[mod]
        assert lw.rank == 5 and lw.scale == 2.0
        assert torch.equal(lw.A, a.t().to(dtype)) and torch.equal(lw.B, b.t().to(dtype))
    # the same bytes as packing the unbound store's copy of the adapter for this layout
    free = CpuAdapterStore()
    free.add_adapter_from_peft_state_dict("a", _peft.state_dict(w), list(SHAPES), lora_alpha=10)
    ref = free.adapters["a"].image_for(cache.layout)
    assert torch.equal(ref.data, ad.image.data) and np.array_equal(ref.rows, ad.image.rows)
    # and the slot holds exactly that image
    cache.ensure_resident(["a"])
    slot = cache.adapter_to_slot["a"]
    base = cache.slot_offset(slot)
    assert torch.equal(cache.arena[base : base + ad.image.nbytes], ad.image.data[: ad.image.nbytes])


def test_image_parts_are_peft_tensors_in_block_layout():
    store, cache = _bound(torch.float32)
    w = _weights(1, 3, modules=["enc.v_proj"])
    store.add_adapter_from_peft_state_dict("s", _peft.state_dict(w), list(SHAPES), lora_alpha=6)
    img = store.adapters["s"].image
    assert img.entry("enc.q_proj") is None and img.entry("dec.o_proj") is None
    rank, scale, r8, a_off, b_off = img.entry("enc.v_proj")
    assert (rank, scale, r8) == (3, 2.0, 8) and a_off % 256 == 0 and b_off % 256 == 0
    a, b = w["enc.v_proj"]
    fin, fout = SHAPES["enc.v_proj"]
    A = untile_rows(img.data[a_off : a_off + rank * fin * 4].view(torch.float32), rank, fin)
    B = untile_rows(img.data[b_off : b_off + fout * r8 * 4].view(torch.float32), fout, r8)
    assert torch.equal(A, a) and torch.equal(B[:, :3], b) and not B[:, 3:].any()


def test_read_safetensors_matches_the_library(tmp_path):
    from safetensors.torch import load_file, save_file

    g = torch.Generator().manual_seed(2)
    tensors = {
        "w.f32": torch.randn(3, 5, generator=g),
        "w.bf16": torch.randn(7, 2, generator=g).bfloat16(),
        "w.f16": torch.randn(1, 9, generator=g).half(),
        "w.odd": torch.randn(3, generator=g).bfloat16(),
        "w.f64": torch.randn(2, 2, generator=g).double(),
    }
    path = tmp_path / "t.safetensors"
    save_file(tensors, str(path), metadata={"format": "pt"})
    mine, lib = read_safetensors(path), load_file(str(path))
    assert set(mine) == set(lib)
    for k, v in lib.items():
        assert mine[k].dtype == v.dtype and torch.equal(mine[k], v), k


@pytest.mark.parametrize("fmt", ["safetensors", "bin"])
@pytest.mark.parametrize("src", [torch.bfloat16, torch.float32])
def test_disk_load_packs_straight_into_the_image(tmp_path, fmt, src):
    w = {m: (a.to(src), b.to(src)) for m, (a, b) in _weights(3, 4).items()}
    path = _peft.write_adapter_dir(tmp_path / "ad", w, 4, 8, fmt=fmt)
    store, cache = _bound()
    store.load_adapter_from_disk("d", path, list(SHAPES))
    ad = store.adapters["d"]
    # bf16 files into a bf16 layout: only the image; fp32 files: their fp32 copy stays too
    assert (ad._modules is None) == (src == torch.bfloat16)
    for mod, (a, b) in w.items():
        assert torch.equal(ad.layers[mod].A, a.t()) and torch.equal(ad.layers[mod].B, b.t())
    free = CpuAdapterStore()
    free.add_adapter_from_peft_state_dict("d", _peft.state_dict(w), list(SHAPES), lora_alpha=8)
    assert torch.equal(free.adapters["d"].image_for(cache.layout).data, ad.image.data)
    assert ad.config["lora_alpha"] == 8


def test_rank_above_the_cap_fails_at_the_slot_load_as_the_reference():
    store, cache = _bound(max_rank=2)
    store.add_adapter_from_peft_state_dict("big", _peft.state_dict(_weights(4, 3)), list(SHAPES), lora_alpha=3)
    assert "big" in store.adapters  # accepted by the store (store.py:221-255 has no rank cap)
    with pytest.raises(ValueError, match="rank 3 exceeds max_rank 2"):
        cache.ensure_resident(["big"])
    assert "big" not in cache.adapter_to_slot


def test_add_adapter_keeps_reference_layout_views_until_bound():
    a, b = torch.randn(16, 2), torch.randn(2, 24)  # stored layout: A = lora_A^T [in, r], B = lora_B^T [r, out]
    store = CpuAdapterStore()
    store.add_adapter("x", {"dec.o_proj": CpuLayerWeights(a, b, 2, 0.5)})
    lw = store.adapters["x"].layers["dec.o_proj"]
    assert torch.equal(lw.A, a) and torch.equal(lw.B, b) and lw.rank == 2 and lw.scale == 0.5
    assert list(store.adapters["x"].layers) == ["dec.o_proj"] and "enc.q_proj" not in store.adapters["x"].layers


def test_add_adapter_image_adopts_a_packed_image():
    store, cache = _bound()
    layout = cache.layout
    builder = ImageBuilder(layout, {"enc.q_proj": (4, 1.5)})
    builder.put("enc.q_proj", torch.ones(4, 24), torch.full((16, 4), 2.0))
    store.add_adapter_image("img", builder.finish())
    ad = store.adapters["img"]
    assert ad.module_ranks() == {"enc.q_proj": (4, 1.5)}
    assert torch.equal(ad.layers["enc.q_proj"].B, torch.full((4, 16), 2.0, dtype=torch.bfloat16))
    cache.ensure_resident(["img"])
    assert int(cache.ranks["enc.q_proj"][cache.adapter_to_slot["img"]]) == 4
    other = SlotLayout(_specs(), torch.float32, 8)
    foreign = ImageBuilder(other, {"enc.q_proj": (4, 1.0)})
    foreign.put("enc.q_proj", torch.ones(4, 24), torch.ones(16, 4))
    with pytest.raises(ValueError, match="image layout does not match"):
        store.add_adapter_image("bad", foreign.finish())
    with pytest.raises(ValueError, match="at least one target layer"):
        store.add_adapter_image("empty", ImageBuilder(layout, {}).finish())


def test_dtype_change_repacks_resident_adapters():
    store, cache = _bound(torch.float32)
    w = _weights(5, 3)
    store.add_adapter_from_peft_state_dict("r", _peft.state_dict(w), list(SHAPES), lora_alpha=3)
    cache.ensure_resident(["r"])
    cache.to(torch.device("cpu"), torch.bfloat16)
    assert store.adapters["r"].image.layout.dtype == torch.bfloat16
    for mod, (a, b) in w.items():
        assert torch.equal(store.adapters["r"].layers[mod].A, a.t().bfloat16())
    assert torch.equal(cache.A["enc.q_proj"][cache.adapter_to_slot["r"], :, :3], w["enc.q_proj"][0].t().bfloat16())


def test_source_dtype_kept_when_packing_rounds_and_a_later_dtype_packs_from_it():
    """fp32 PEFT tensors into a bf16-bound store keep their fp32 copy (the reference holds the source dtype and
    converts at every slot load, store.py:240-241, cache.py:139): after the cache moves to fp32, the adapter's
    slot image and its CpuLayerWeights are the fp32 values exactly, for adapters added before and after."""
    store, cache = _bound(torch.bfloat16)
    w = _weights(3, 4)
    store.add_adapter_from_peft_state_dict("early", _peft.state_dict(w), list(SHAPES), lora_alpha=8)
    ad = store.adapters["early"]
    assert ad.image.layout.dtype == torch.bfloat16 and ad._modules is not None
    for mod, (a, b) in w.items():
        assert ad.layers[mod].A.dtype == torch.float32 and torch.equal(ad.layers[mod].A, a.t())
    cache.ensure_resident(["early"])
    cache.to(torch.device("cpu"), torch.float32)
    w2 = _weights(4, 3)
    store.add_adapter_from_peft_state_dict("late", _peft.state_dict(w2), list(SHAPES), lora_alpha=6)
    assert store.adapters["late"]._modules is None  # fp32 into fp32: exact, nothing kept beside the image
    for aid, ws in (("early", w), ("late", w2)):
        img = store.image(store.adapters[aid], cache.layout)
        assert img.layout.dtype == torch.float32
        for mod, (a, b) in ws.items():
            got_a, got_b, _ = img.lora_tensors(mod)
            assert torch.equal(got_a, a) and torch.equal(got_b, b), (aid, mod)
    # the resident adapter was rewritten into the fp32 arena from its fp32 source
    slot = cache.adapter_to_slot["early"]
    img = store.adapters["early"].image
    off = cache.slot_offset(slot)
    assert torch.equal(cache.arena[off : off + img.nbytes], img.data[: img.nbytes])


def test_reference_layout_slot_tensors_refuse_writes():
    """cache.A[m] / cache.B[m] hold the reference layout (cache.py:43-56) as copies of the arena: reads work, and
    every write into them or a view of them raises instead of being lost."""
    store, cache = _bound(torch.float32)
    w = _weights(0, 4)
    store.add_adapter_from_peft_state_dict("a", _peft.state_dict(w), list(SHAPES), lora_alpha=8)
    cache.ensure_resident(["a"])
    slot = cache.adapter_to_slot["a"]
    for mod, (a, b) in w.items():
        A, B = cache.A[mod], cache.B[mod]
        assert torch.equal(A[slot, :, :4], a.t()) and torch.equal(B[slot, :4, :], b.t())
        assert not A[slot, :, 4:].any() and not A[0].any()
    A = cache.A["enc.q_proj"]
    writes = [lambda: A[slot, :, :2].zero_(), lambda: A.copy_(torch.zeros_like(A)), lambda: A.__setitem__(slot, 0.0),
              lambda: torch.add(A, 1, out=A), lambda: A[slot].add_(1), lambda: A.view(-1).fill_(0),
              lambda: A.__iadd__(1)]
    for write in writes:
        with pytest.raises(RuntimeError, match="would not reach the kernels"):
            write()
    c = A.clone()
    c.add_(1)  # a copy is an ordinary tensor
    assert type(c) is torch.Tensor and type(A * 2) is torch.Tensor
    assert torch.equal(cache.A["enc.q_proj"], A)  # nothing was written
