"""MultiLoraLinear — drop-in wrapper of nn.Linear (src/polylora/layers.py:18-134).

forward(x) = base_layer(x), then, when a LoRA batch context is active, the
HIP SGMV shrink + expand adds ``scale * (x @ A^T) @ B^T`` in place into the
base output for every row whose slot has rank > 0 in this module, over the
first ``min(seq_len, M)`` tokens of the row.  Rank-0 rows and padding tokens
keep the base output bit for bit.  On the tiled path, layers with many
tokens run the shrink on a side stream concurrently with the base GEMM (it
needs only x); the expand joins back on the caller's stream.

Where the reference picks Triton or its torch fallback (layers.py:42-58,
:64-70), this layer always runs HIP kernels: the MFMA-tiled ones when
``config.use_triton_kernels`` is True, the row-based ones otherwise.  A CPU
input with an active LoRA context raises.
"""

from __future__ import annotations

import torch
from torch import nn

from . import _native, sgmv
from .cache import GpuAdapterCache
from .context import LoraBatchContext, get_lora_context


# Layers with at least this many tokens run the shrink on a side stream while
# the base GEMM computes.  Measured on MI355X: in decode (a few hundred
# tokens) the concurrent shrink slows the memory-bound base GEMM and the
# cross-stream joins cost more than the overlap saves, so small layers run
# the shrink and expand back to back on the caller's stream.
OVERLAP_MIN_TOKENS = 2048


def _version_of(x: torch.Tensor):
    """In-place modification counter of x, or None for inference tensors (they keep none)."""
    if x.is_inference():
        return None
    return x._version


def _siblings(cache: GpuAdapterCache, run: tuple, element_size: int):
    """The wrapped Linears of a sibling run, or None when one is missing or has an output width
    that is not whole 16-byte chunks (x itself is checked by the caller); memoized per cache."""
    memo = cache.__dict__.setdefault("_run_siblings", {})
    key = (run, element_size, len(cache.wrapped))
    hit = memo.get(key, False)
    if hit is False:
        mods = [cache.wrapped.get(name) for name in run]
        chunk = 16 // element_size
        ok = all(m is not None and m.out_features % chunk == 0 for m in mods)
        hit = memo[key] = mods if ok else None
    return hit


class MultiLoraLinear(nn.Module):
    def __init__(self, base_layer: nn.Linear, module_name: str, cache: GpuAdapterCache) -> None:
        super().__init__()
        self.base_layer = base_layer
        self.module_name = module_name
        self.cache = cache
        self._n_out = base_layer.out_features  # read on every call; the submodule lookup is slower
        cache.wrapped[module_name] = self

    @property
    def in_features(self) -> int:
        return self.base_layer.in_features

    @property
    def out_features(self) -> int:
        return self.base_layer.out_features

    def forward(self, x: torch.Tensor) -> torch.Tensor:
        lora_ctx = get_lora_context()
        if lora_ctx is None:
            return self.base_layer(x)
        stack = lora_ctx.stack
        stack["calls"] = stack.get("calls", 0) + 1  # wrapped calls under this context so far
        if x.is_cuda and self.cache.config.use_triton_kernels:
            out = self._tiled_forward(x, lora_ctx)
            if out is not None:
                return out
        base = self.base_layer(x)
        original_shape = base.shape
        x_3d, base_3d, seq_lens, weight_indices = self._prepare_batched_inputs(x, base, lora_ctx)
        out = self._hip_forward(x_3d, base_3d, seq_lens, weight_indices, lora_ctx)
        return out.reshape(original_shape)

    def _tiled_forward(self, x: torch.Tensor, lora_ctx: LoraBatchContext) -> torch.Tensor | None:
        """Tiled path: shrink (shared with sibling Linears when it can be), base GEMM, expand.

        Returns None when the shapes do not suit the tiled kernels; the caller
        then takes the sequential path (row kernels).
        """
        cache = self.cache
        x_3d, seq_lens, weight_indices, reshape = self._batched_view(x, lora_ctx)
        rows, row_len, in_features = x_3d.shape
        if rows * row_len == 0 or x.dtype != cache.dtype:
            return None
        x2 = x_3d.reshape(rows * row_len, in_features)
        if not sgmv.tiled_shapes_ok(x2, self._n_out):
            return None
        plan = self._plan(lora_ctx, rows, row_len, seq_lens, weight_indices)
        main = sgmv._stream(x.device)  # handle of the caller's stream
        fused = sgmv.fused_ok(plan, cache, in_features)
        run_out = self._run_forward(x, x2, plan, lora_ctx, reshape, main, fused)
        if run_out is not None:
            return run_out
        if not fused and rows * row_len < OVERLAP_MIN_TOKENS and cache.decode_handoff and sgmv.decode_ok(plan):
            # decode-sized batches: base GEMM, then shrink and expand in one launch
            self._observe_call(x, _version_of(x), lora_ctx.stack)
            base = self.base_layer(x)
            base_3d = reshape(base)
            y2 = base_3d.view(rows * row_len, base_3d.shape[-1])
            sgmv.lora_decode_stacked(x2, [y2], cache, [self.module_name], plan, stream=main)
            return base_3d.reshape(base.shape)
        if fused:
            # long adapter segments: base GEMM, then one fused shrink+expand launch
            self._observe_call(x, _version_of(x), lora_ctx.stack)
            base = self.base_layer(x)
            base_3d = reshape(base)
            y2 = base_3d.view(rows * row_len, base_3d.shape[-1])
            if y2.shape[1] == self._n_out and y2.dtype == cache.dtype and y2.data_ptr() % 16 == 0:
                # x2 passed tiled_shapes_ok and y2 is the fresh contiguous base output
                sgmv._fused_launch(x2, y2, cache, self.module_name, plan, _native.PL_EPI_FALLBACK, None, main)
            else:
                sgmv.lora_fused(x2, y2, cache, self.module_name, plan, stream=main)  # checks and raises
            return base_3d.reshape(base.shape)
        if rows * row_len >= OVERLAP_MIN_TOKENS:
            main_s = torch.cuda.current_stream(x.device)
            side = sgmv.side_stream(x.device)
            side.wait_stream(main_s)  # x is ready, and every earlier expand has read the side workspaces
            with torch.cuda.stream(side):
                shrunk = self._shrink(x, x2, plan, lora_ctx, side.cuda_stream)
            base = self.base_layer(x)
            main_s.wait_stream(side)
        else:
            shrunk = self._shrink(x, x2, plan, lora_ctx, main)
            base = self.base_layer(x)
        base_3d = reshape(base)
        sgmv.lora_expand(shrunk, base_3d.view(rows * row_len, base_3d.shape[-1]), cache, self.module_name,
                         stream=main)
        return base_3d.reshape(base.shape)

    def _run_forward(self, x, x2, plan, lora_ctx: LoraBatchContext, reshape, main: int, fused: bool):
        """Whole outputs for a run of sibling Linears, or None to take the single-module path.

        Siblings are wrapped Linears that the model calls back to back on the
        very same input tensor (q/k/v, gate/up), learned from the call order of
        a forward.  The first of a run computes every sibling's base output
        and then the LoRA deltas of all of them, in one stacked fused launch
        for long adapter segments or else one stacked shrink and one stacked
        expand, and keeps the siblings' finished outputs; a sibling then returns its kept output when its own
        call brings the same input tensor, unmodified (same version counter;
        inference-mode tensors keep none, so for them object identity alone),
        for the same plan, and is the very next wrapped call (the i-th sibling
        the i-th call after the first); any other call drops what was kept.
        Under inference mode an in-place edit of x by a plain tensor op between
        two sibling calls is not seen; models that do that set
        ``cache.stack_siblings = False``.  A base output is a function of x and the weights
        only, so computing it at the first sibling's call gives the value the
        sibling's own call would.  Only without autograd: the LoRA path is for
        inference.
        """
        if torch.is_grad_enabled() and (x.requires_grad or self.base_layer.weight.requires_grad):
            return None
        stack = lora_ctx.stack
        outputs = stack.setdefault("outputs", {})
        version = _version_of(x)
        kept = outputs.pop(self.module_name, None)
        if kept is not None:
            kx, kversion, kplan, kcall, out = kept
            if kx is x and kversion == version and kplan is plan and kcall == stack["calls"]:
                self._observe_call(x, version, stack)
                return out
        outputs.clear()  # a run interrupted by another call keeps nothing
        cache = self.cache
        run = cache.stacked_runs.get((self.module_name, tuple(x.shape))) if cache.stack_siblings else None
        if run is None or len(run) < 2:
            return None
        siblings = _siblings(cache, run, x2.element_size())
        if siblings is None:
            return None
        self._observe_call(x, version, stack)
        tokens = x2.shape[0]
        done = fused  # the outputs are complete after the launches below
        if fused:
            # long adapter segments: every sibling's base GEMM, then one fused
            # launch for all of them
            bases = [m.base_layer(x) for m in siblings]
            outs = [reshape(b) for b in bases]
            sgmv.lora_fused_stacked(x2, [o.view(tokens, o.shape[-1]) for o in outs], cache, list(run), plan,
                                    stream=main)
        elif tokens >= OVERLAP_MIN_TOKENS:
            main_s = torch.cuda.current_stream(x.device)
            side = sgmv.side_stream(x.device)
            side.wait_stream(main_s)
            with torch.cuda.stream(side):
                results = sgmv.lora_shrink_stacked(x2, cache, list(run), plan, stream=side.cuda_stream)
            bases = [m.base_layer(x) for m in siblings]
            main_s.wait_stream(side)
        elif cache.decode_handoff and sgmv.decode_ok(plan):
            # decode-sized batches: every sibling's base GEMM, then one launch
            # for all of their shrinks and expands
            bases = [m.base_layer(x) for m in siblings]
            outs = [reshape(b) for b in bases]
            sgmv.lora_decode_stacked(x2, [o.view(tokens, o.shape[-1]) for o in outs], cache, list(run), plan,
                                     stream=main)
            done = True
        else:
            results = sgmv.lora_shrink_stacked(x2, cache, list(run), plan, stream=main)
            bases = [m.base_layer(x) for m in siblings]
        if not done:
            outs = [reshape(b) for b in bases]
            sgmv.lora_expand_stacked(results, [o.view(tokens, o.shape[-1]) for o in outs], cache, list(run),
                                     stream=main)
        finished = [o.reshape(b.shape) for o, b in zip(outs, bases)]
        # sibling i is valid only as the i-th wrapped call after this one
        calls = stack["calls"]
        for i, (name, out) in enumerate(zip(run[1:], finished[1:]), start=1):
            outputs[name] = (x, version, plan, calls + i, out)
        return finished[0]

    def _shrink(self, x: torch.Tensor, x2: torch.Tensor, plan, lora_ctx: LoraBatchContext, stream: int):
        """This module's shrink result: computed ahead by a sibling, stacked with siblings, or alone.

        Siblings are wrapped Linears that the model calls back to back on the
        very same input tensor (q/k/v, gate/up).  The first forward learns them
        from the call sequence; later forwards let the first of them shrink for
        all in one launch.  A precomputed result is used only if this call's
        input is that same tensor object, unmodified (same version counter;
        inference-mode tensors keep none, so for them object identity alone),
        with the same plan, as the very next wrapped call, and its workspace
        still holds it; otherwise the module computes its own.
        """
        stack = lora_ctx.stack
        shared = stack.setdefault("shared", {})
        hit = shared.pop(self.module_name, None)
        version = _version_of(x)
        self._observe_call(x, version, stack)
        if hit is not None:
            hx, hversion, hcall, res = hit
            if hx is x and hversion == version and hcall == stack["calls"] and res.plan is plan and res.valid:
                return res
        shared.clear()  # a run interrupted by another call keeps nothing
        run = self.cache.stacked_runs.get((self.module_name, tuple(x.shape))) if self.cache.stack_siblings else None
        if run is not None and len(run) > 1:
            results = sgmv.lora_shrink_stacked(x2, self.cache, list(run), plan, stream=stream)
            calls = stack["calls"]
            for i, (name, res) in enumerate(zip(run[1:], results[1:]), start=1):
                shared[name] = (x, version, calls + i, res)
            return results[0]
        return sgmv.lora_shrink(x2, self.cache, self.module_name, plan, stream=stream)

    def _observe_call(self, x: torch.Tensor, version, stack: dict) -> None:
        """Extend the current run of calls on one input tensor, recording it as a sibling set."""
        run = stack.get("run")
        if (
            run is not None
            and stack.get("run_x") is x
            and stack.get("run_version") == version
            and self.module_name not in run
            and len(run) < sgmv.MAX_STACKED_MODULES
        ):
            run.append(self.module_name)
            self.cache.stacked_runs[(run[0], tuple(x.shape))] = tuple(run)
        else:
            stack["run"], stack["run_x"], stack["run_version"] = [self.module_name], x, version

    def _plan(self, lora_ctx: LoraBatchContext, rows: int, row_len: int, seq_lens, weight_indices):
        key = (rows, row_len)
        plan = lora_ctx.plans.get(key)
        if plan is None:
            cache = self.cache
            distinct = len({a for a in lora_ctx.adapter_ids if a != cache.config.base_adapter_id})
            plan = sgmv.SgmvPlan(weight_indices, seq_lens, row_len, cache.num_slots, distinct_slots=distinct)
            lora_ctx.plans[key] = plan
        return plan

    def _batched_view(self, x: torch.Tensor, lora_ctx: LoraBatchContext):
        """_prepare_batched_inputs for x alone, plus the function that shapes the base output the same way."""
        batch = lora_ctx.weight_indices.shape[0]
        if x.shape[0] == batch:
            return self._as_3d(x).contiguous(), lora_ctx.seq_lens, lora_ctx.weight_indices, lambda t: self._as_3d(t).contiguous()
        if x.dim() == 3 and x.shape[0] == 1:
            return x.contiguous(), lora_ctx.seq_lens[:1], lora_ctx.weight_indices[:1], lambda t: t.contiguous()
        if x.dim() == 2 and x.shape[0] % batch == 0:
            seq_len = x.shape[0] // batch
            return (
                x.reshape(batch, seq_len, x.shape[-1]).contiguous(),
                lora_ctx.seq_lens,
                lora_ctx.weight_indices,
                lambda t: t.reshape(batch, seq_len, t.shape[-1]).contiguous(),
            )
        raise ValueError("LoRA batch context batch size does not match layer input batch size")

    @staticmethod
    def _as_3d(x: torch.Tensor) -> torch.Tensor:
        if x.dim() == 2:
            return x.unsqueeze(1)
        if x.dim() == 3:
            return x
        if x.dim() > 3:
            return x.reshape(x.shape[0], -1, x.shape[-1])
        raise ValueError("MultiLoraLinear expects a batched tensor")

    def _prepare_batched_inputs(self, x: torch.Tensor, base: torch.Tensor, lora_ctx: LoraBatchContext):
        """The three input shapes of layers.py:82-110.

        Row lengths are returned unclamped; the plan (and the row kernels) use
        min(seq_len, M), which is what the reference's slicing x[b, :seq_len]
        and its explicit clamps compute.
        """
        batch = lora_ctx.weight_indices.shape[0]
        if x.shape[0] == batch:
            # (i) one row per context row: [B, K], [B, M, K] or [B, ..., K]
            return (self._as_3d(x).contiguous(), self._as_3d(base).contiguous(), lora_ctx.seq_lens, lora_ctx.weight_indices)
        if x.dim() == 3 and x.shape[0] == 1:
            # (ii) a shared batch-1 tensor (e.g. DeBERTa relative position
            # embeddings): row 0's adapter over its first min(seq_len, M) rows
            return (x.contiguous(), base.contiguous(), lora_ctx.seq_lens[:1], lora_ctx.weight_indices[:1])
        if x.dim() == 2 and x.shape[0] % batch == 0:
            # (iii) flattened [B*S, K]
            seq_len = x.shape[0] // batch
            return (
                x.reshape(batch, seq_len, x.shape[-1]).contiguous(),
                base.reshape(batch, seq_len, base.shape[-1]).contiguous(),
                lora_ctx.seq_lens,
                lora_ctx.weight_indices,
            )
        raise ValueError("LoRA batch context batch size does not match layer input batch size")

    def _hip_forward(
        self,
        x: torch.Tensor,
        base: torch.Tensor,
        seq_lens: torch.Tensor,
        weight_indices: torch.Tensor,
        lora_ctx: LoraBatchContext,
    ) -> torch.Tensor:
        if not x.is_cuda:
            raise RuntimeError(
                "MultiLoraLinear: the LoRA path of polylora_amd runs only on a ROCm GPU "
                "(HIP kernels); move the model and inputs to a GPU device"
            )
        cache = self.cache
        if x.dtype != cache.dtype or base.dtype != cache.dtype:
            raise TypeError(
                f"MultiLoraLinear {self.module_name!r}: input {x.dtype} / output {base.dtype} "
                f"must match the adapter cache dtype {cache.dtype}"
            )
        rows, row_len, in_features = x.shape
        if rows * row_len == 0:
            return base
        x2 = x.view(rows * row_len, in_features)
        y2 = base.view(rows * row_len, base.shape[-1])
        if cache.config.use_triton_kernels:
            plan = self._plan(lora_ctx, rows, row_len, seq_lens, weight_indices)
            sgmv.lora_apply(x2, y2, cache, self.module_name, plan)
        else:
            sgmv.lora_apply_rows(x2, y2, cache, self.module_name, weight_indices, seq_lens, row_len)
        return base
