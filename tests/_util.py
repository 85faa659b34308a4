"""Shared test helpers: synthetic PEFT adapters, caches and the matching oracle tensors."""

from __future__ import annotations

import torch

from oracle.lora import dense_slot_tensors
from polylora_amd.cache import GpuAdapterCache, ModuleSpec
from polylora_amd.config import PolyLoraConfig
from polylora_amd.store import CpuAdapterStore, CpuLayerWeights

BF16_TOL = dict(rtol=2e-2, atol=1e-2)
FP32_TOL = dict(rtol=1e-5, atol=1e-5)


def tol_for(dtype: torch.dtype) -> dict:
    return FP32_TOL if dtype == torch.float32 else BF16_TOL


_MANTISSA_BITS = {torch.bfloat16: 7, torch.float16: 10, torch.float32: 23}
EXEMPT_FRACTION = 1e-5  # at most this share of the checked elements may take the cancellation exemption


def ulp_of(v: torch.Tensor, dtype: torch.dtype) -> torch.Tensor:
    """One unit in the last place of `dtype` at |v| (0 where v is 0), as fp32."""
    v = v.float().abs()
    _, e = torch.frexp(v)  # v = m * 2**e, m in [0.5, 1)
    ulp = torch.ldexp(torch.ones_like(v), (e - 1 - _MANTISSA_BITS[dtype]).to(torch.int32))
    return torch.where(v > 0, ulp, torch.zeros_like(v))


class CountedParity:
    """Plain tolerance on every element, with a counted, capped exemption for cancellations.

    Each output element of a wrapped Linear is T(base + delta).  The kernels'
    fp32 sums of x·A run in another order than the oracle's matmul, so the
    rounded intermediate T(x·A) (layers.py:127) can land one bf16 step apart,
    and delta then one ulp of |delta| apart; the epilogue itself rounds
    T(acc), T(T(acc)·T(scale)) and T(y + d) exactly as the oracle does.  Where
    base and delta cancel, one ulp of the operands is far more than rtol of
    the result (an output of 0.09 from operands near 2 is 0.0156 off).

    An element passes when |got - want| <= atol + rtol·|want|.  An element
    that fails that is *exempt* only when (i) |got - want| is at most one ulp
    of the model dtype at max(|base|, |want - base|) and (ii) |want| is less
    than half that maximum (a cancellation).  Exempt elements are counted over
    the whole test, printed, and the test fails when they exceed
    EXEMPT_FRACTION of the elements checked.  Any other miss fails at once.
    """

    def __init__(self, dtype: torch.dtype, label: str = "") -> None:
        self.dtype, self.label = dtype, label
        self.tol = tol_for(dtype)
        self.checked = 0
        self.exempt = 0
        self.worst = 0.0

    def check(self, got: torch.Tensor, want: torch.Tensor, base: torch.Tensor, where: str = "") -> None:
        got, want, base = got.float(), want.float(), base.float()
        err = (got - want).abs()
        plain = err <= self.tol["atol"] + self.tol["rtol"] * want.abs()
        self.checked += err.numel()
        if bool(plain.all()):
            return
        big = torch.maximum(base.abs(), (want - base).abs())
        exempt = ~plain & (err <= ulp_of(big, self.dtype)) & (want.abs() < 0.5 * big)
        bad = ~plain & ~exempt
        if bool(bad.any()):
            i = int(torch.argmax(torch.where(bad, err, torch.zeros_like(err)).flatten()))
            raise AssertionError(
                f"{self.label}{where}: {int(bad.sum())} / {err.numel()} elements beyond rtol {self.tol['rtol']} / atol "
                f"{self.tol['atol']}; worst at flat index {i}: got {got.flatten()[i].item():.6g}, want "
                f"{want.flatten()[i].item():.6g}, base {base.flatten()[i].item():.6g}")
        self.exempt += int(exempt.sum())
        self.worst = max(self.worst, float(err[exempt].max()))

    def finish(self) -> None:
        limit = EXEMPT_FRACTION * self.checked
        print(f"parity {self.label}: {self.checked} elements at rtol {self.tol['rtol']} / atol {self.tol['atol']}, "
              f"{self.exempt} exempt (cancellation, <= 1 ulp of the operands; limit {limit:.1f}), worst exempt error "
              f"{self.worst:.4g}", flush=True)
        assert self.exempt <= limit, f"{self.label}: {self.exempt} exempt elements, limit {limit:.1f}"


def peft_layer(gen: torch.Generator, fin: int, fout: int, rank: int, alpha: float, std: float = 0.02):
    """PEFT-layout weights: lora_A [rank, in], lora_B [out, rank] ~ N(0, std)."""
    a = torch.randn(rank, fin, generator=gen) * std
    b = torch.randn(fout, rank, generator=gen) * std
    return a, b, float(alpha)


def make_store(adapters: dict, base_id: str = "__base__") -> CpuAdapterStore:
    """adapters: id -> {module: (lora_A, lora_B, alpha)} -> a CpuAdapterStore."""
    store = CpuAdapterStore(base_id)
    for aid, layers in adapters.items():
        store.add_adapter(
            aid,
            {
                m: CpuLayerWeights(A=a.t().contiguous(), B=b.t().contiguous(), rank=a.shape[0], scale=alpha / a.shape[0])
                for m, (a, b, alpha) in layers.items()
            },
        )
    return store


def make_cache(adapters: dict, module_shapes: dict, max_gpu_adapters: int, max_rank: int, device, dtype, tiled=True):
    config = PolyLoraConfig(max_gpu_adapters=max_gpu_adapters, max_rank=max_rank, use_triton_kernels=tiled)
    specs = [ModuleSpec(n, fin, fout) for n, (fin, fout) in module_shapes.items()]
    return GpuAdapterCache(make_store(adapters), specs, config, device, dtype)


def oracle_slot_tensors(cache: GpuAdapterCache, adapters: dict, module: str, dtype: torch.dtype):
    """Reference-layout dense tensors following the cache's current slot assignment."""
    spec = cache.module_specs[module]
    per_slot = [None]
    for slot in range(1, cache.num_slots):
        aid = cache.slot_to_adapter[slot]
        per_slot.append(None if aid is None else adapters[aid].get(module))
    return dense_slot_tensors(per_slot, spec.in_features, spec.out_features, cache.config.max_rank, dtype)
