"""Per-forward LoRA batch context (src/polylora/context.py:11-45).

The context travels through a ContextVar exactly like the reference, so the
wrapped Linear layers keep the ``nn.Linear.forward(x)`` signature.  It also
carries the per-forward device plans (built once per distinct layer shape by
``sgmv.SgmvPlan`` and shared by every wrapped Linear of the forward), which
replace the per-layer host schedule of sgmv.py:29-61.
"""

from __future__ import annotations

from contextlib import contextmanager
from contextvars import ContextVar
from dataclasses import dataclass, field
from typing import Iterator

import torch


@dataclass(frozen=True)
class LoraBatchContext:
    adapter_ids: list[str]
    # int32 [B] row -> GPU slot (slot 0 = base adapter); the reference uses int64
    weight_indices: torch.Tensor
    # int32 [B] valid length per row (attention_mask.sum(-1) or the full length)
    seq_lens: torch.Tensor
    attention_mask: torch.Tensor | None = None
    # (rows, row_len) -> SgmvPlan, filled lazily by the first layer of that shape
    plans: dict = field(default_factory=dict, compare=False, repr=False)
    # shrinks computed ahead for sibling Linears fed the same input, and the
    # run of consecutive calls on one input used to learn such siblings
    stack: dict = field(default_factory=dict, compare=False, repr=False)


_CURRENT_LORA_CONTEXT: ContextVar[LoraBatchContext | None] = ContextVar(
    "polylora_current_lora_context", default=None
)


def get_lora_context() -> LoraBatchContext | None:
    return _CURRENT_LORA_CONTEXT.get()


@contextmanager
def use_lora_context(ctx: LoraBatchContext | None) -> Iterator[None]:
    token = _CURRENT_LORA_CONTEXT.set(ctx)
    try:
        yield
    finally:
        _CURRENT_LORA_CONTEXT.reset(token)


_PAD_ERROR = "Custom multi-LoRA runtime currently requires right-padded attention_mask"


def assert_right_padded(attention_mask: torch.Tensor, seq_lens: torch.Tensor) -> None:
    """Raise ValueError unless every row of the mask is ones then zeros (context.py:37-45).

    Synchronous: reads the comparison result on the host.  PolyLoraModel uses
    :class:`RightPaddingCheck` for device masks so the forward is not stalled.
    """
    if attention_mask.dim() != 2:
        raise ValueError("attention_mask must be a 2D batch mask")
    _, max_len = attention_mask.shape
    positions = torch.arange(max_len, device=attention_mask.device).expand_as(attention_mask)
    expected = positions < seq_lens.to(attention_mask.device)[:, None]
    if not torch.equal(attention_mask.bool(), expected):
        raise ValueError(_PAD_ERROR)


class RightPaddingCheck:
    """Right-padding check of a device mask whose verdict is read later.

    A HIP kernel compares the mask with ``s < seq_lens[b]`` and sets a device
    flag, which is copied to pinned host memory behind an event; ``raise_if_bad``
    waits for that event only (not for the rest of the forward) and raises the
    reference's ValueError.
    """

    def __init__(self, attention_mask: torch.Tensor, seq_lens: torch.Tensor) -> None:
        from . import _native

        if attention_mask.dim() != 2:
            raise ValueError("attention_mask must be a 2D batch mask")
        lib = _native.load()
        mask = attention_mask.contiguous()
        code = _native.MASK_DTYPE_CODES.get(mask.dtype)
        if code is None:
            mask = mask.to(torch.int32)
            code = _native.MASK_DTYPE_CODES[torch.int32]
        device = mask.device
        flag = torch.zeros(1, dtype=torch.int32, device=device)
        stream = torch.cuda.current_stream(device)
        B, S = mask.shape
        _native.check(
            lib.pl_check_right_padded(
                mask.data_ptr(), code, B, S, seq_lens.data_ptr(), flag.data_ptr(), stream.cuda_stream
            ),
            "pl_check_right_padded",
        )
        self._host = torch.empty(1, dtype=torch.int32, pin_memory=True)
        self._host.copy_(flag, non_blocking=True)
        self._event = torch.cuda.Event()
        self._event.record(stream)
        self._keep = (mask, flag)

    def raise_if_bad(self) -> None:
        self._event.synchronize()
        if int(self._host[0]) != 0:
            raise ValueError(_PAD_ERROR)
