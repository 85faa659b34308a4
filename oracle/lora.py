"""CPU restatement of the reference LoRA math and operator semantics (test infrastructure).

All functions are device-agnostic torch; tests run them on CPU tensors (or,
for same-process comparisons, on the GPU tensors of the run) as the expected values.
"""

from __future__ import annotations

import torch


def reference_forward(
    x: torch.Tensor,
    base: torch.Tensor,
    seq_lens: torch.Tensor,
    weight_indices: torch.Tensor,
    A: torch.Tensor,
    B: torch.Tensor,
    ranks: torch.Tensor,
    scales: torch.Tensor,
) -> torch.Tensor:
    """Per-row LoRA of MultiLoraLinear._reference_forward (layers.py:112-134).

    x [rows, M, K], base [rows, M, N]; A [slots, K, R] (lora_A^T per slot),
    B [slots, R, N] (lora_B^T), ranks int [slots], scales fp32 [slots].
    Same op order and rounding points as the reference (layers.py:127-128):
    t = T(x @ A[:, :r]); d = T(t @ B[:r]); d = T(d * T(scale)); out = T(out + d)
    on a clone of base, where T rounds to the model dtype.

    Each product is computed as an fp32 matmul of the model-dtype values and
    then rounded once to the model dtype, i.e. a model-dtype GEMM with fp32
    accumulation, which is what the reference's torch matmul does on the GPU
    for bf16/fp16.  For fp32 it is the reference op itself.  torch's CPU
    bf16 matmul is deliberately not used: for a single strided column
    (A[:, :1] of a [K, R] slot) it returns results off by more than 2 where
    the exact product is below 1, so it cannot restate the GPU semantics.
    """
    out = base.clone()
    dtype = out.dtype
    lengths = [int(v) for v in seq_lens.detach().cpu().tolist()]
    slots = [int(v) for v in weight_indices.detach().cpu().tolist()]
    for row, slot in enumerate(slots):
        rank = int(ranks[slot].item())
        length = min(max(lengths[row], 0), x.shape[1])
        if rank == 0 or length == 0:
            continue
        t = _gemm(x[row, :length], A[slot, :, :rank], dtype)
        delta = _gemm(t, B[slot, :rank, :], dtype)
        out[row, :length] += delta * scales[slot].to(dtype=dtype)
    return out


def _gemm(a: torch.Tensor, b: torch.Tensor, dtype: torch.dtype) -> torch.Tensor:
    """a @ b of model-dtype operands: fp32 (or fp64) accumulation, one rounding to `dtype`."""
    if dtype in (torch.float32, torch.float64):
        return a.matmul(b)
    return a.float().matmul(b.float()).to(dtype)


def as_3d(x: torch.Tensor) -> torch.Tensor:
    """layers.py:72-80."""
    if x.dim() == 2:
        return x.unsqueeze(1)
    if x.dim() == 3:
        return x
    if x.dim() > 3:
        return x.reshape(x.shape[0], -1, x.shape[-1])
    raise ValueError("MultiLoraLinear expects a batched tensor")


def prepare_batched_inputs(x, base, weight_indices, seq_lens):
    """The three input-shape branches of layers.py:82-110."""
    batch = weight_indices.shape[0]
    if x.shape[0] == batch:
        return as_3d(x).contiguous(), as_3d(base).contiguous(), seq_lens, weight_indices
    if x.dim() == 3 and x.shape[0] == 1:
        return x.contiguous(), base.contiguous(), torch.clamp(seq_lens[:1], max=x.shape[1]), weight_indices[:1]
    if x.dim() == 2 and x.shape[0] % batch == 0:
        seq_len = x.shape[0] // batch
        return (
            x.reshape(batch, seq_len, x.shape[-1]).contiguous(),
            base.reshape(batch, seq_len, base.shape[-1]).contiguous(),
            torch.clamp(seq_lens, max=seq_len),
            weight_indices,
        )
    raise ValueError("LoRA batch context batch size does not match layer input batch size")


def sgmv_shrink_reference(x, weights, seq_lens, weight_indices, ranks, stack_num=1):
    """Defined outputs of the shrink operator (sgmv.py:63-175).

    Returns (out, valid): out[b, m, n] = x-dtype(fp32 sum_k x[b,m,k] * w[w_b,k,n])
    where valid[b, m, n] is True (m < min(seq_len_b, M), n < rank*stack_num);
    other entries are undefined in the reference (torch.empty) and are zero here.
    """
    Bt, M, K = x.shape
    n_max = weights.shape[2]
    out = torch.zeros((Bt, M, n_max), dtype=x.dtype)
    valid = torch.zeros((Bt, M, n_max), dtype=torch.bool)
    for b in range(Bt):
        slot = int(weight_indices[b])
        rows = min(max(int(seq_lens[b]), 0), M)
        cols = min(int(ranks[slot]) * stack_num, n_max)
        if rows == 0 or cols == 0:
            continue
        acc = x[b, :rows].float() @ weights[slot, :, :cols].float()
        out[b, :rows, :cols] = acc.to(x.dtype)
        valid[b, :rows, :cols] = True
    return out, valid


def sgmv_expand_reference(x, weights, seq_lens, weight_indices, ranks, scalings, base):
    """Fused expand of sgmv.py:178-328: y = T(T(scale * fp32(x[:, :k] @ w[:k])) + y)."""
    out = base.clone()
    Bt, M, k_max = x.shape
    for b in range(Bt):
        slot = int(weight_indices[b])
        rows = min(max(int(seq_lens[b]), 0), M)
        k = min(k_max, int(ranks[slot]))
        if rows == 0 or k <= 0:
            continue
        acc = x[b, :rows, :k].float() @ weights[slot, :k, :].float()
        acc = acc * float(scalings[slot])
        out[b, :rows] = acc.to(out.dtype) + out[b, :rows]
    return out


def right_padded(attention_mask: torch.Tensor, seq_lens: torch.Tensor) -> bool:
    """context.py:37-45 as a predicate: each row is ones then zeros, seq_len ones."""
    _, max_len = attention_mask.shape
    positions = torch.arange(max_len).expand_as(attention_mask)
    return bool(torch.equal(attention_mask.bool().cpu(), positions < seq_lens.cpu()[:, None]))


def store_layout(lora_A: torch.Tensor, lora_B: torch.Tensor, lora_alpha: float):
    """store.py:240-253: PEFT lora_A [r, in], lora_B [out, r] -> (A^T, B^T, rank, alpha/rank)."""
    rank = int(lora_A.shape[0])
    return lora_A.t().contiguous(), lora_B.t().contiguous(), rank, float(lora_alpha) / rank


def dense_slot_tensors(adapters_per_slot, in_features, out_features, max_rank, dtype):
    """Reference slot tensors of cache.py:43-58 for one module.

    adapters_per_slot[s] is None (empty / base) or (lora_A [r, in], lora_B [out, r], alpha).
    """
    slots = len(adapters_per_slot)
    A = torch.zeros(slots, in_features, max_rank, dtype=dtype)
    B = torch.zeros(slots, max_rank, out_features, dtype=dtype)
    ranks = torch.zeros(slots, dtype=torch.int32)
    scales = torch.zeros(slots, dtype=torch.float32)
    for s, item in enumerate(adapters_per_slot):
        if item is None:
            continue
        a_t, b_t, rank, scale = store_layout(*item)
        A[s, :, :rank] = a_t.to(dtype)
        B[s, :rank, :] = b_t.to(dtype)
        ranks[s] = rank
        scales[s] = scale
    return A, B, ranks, scales
