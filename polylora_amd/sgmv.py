"""SGMV operators on the gfx950 HIP library (replaces src/polylora/sgmv.py).

Two levels:

* ``sgmv_lora_a_fwd`` / ``sgmv_lora_b_fwd`` keep the reference operator
  signatures and tensor layouts (sgmv.py:141-175, :278-328): weights
  ``[adapters, K, N]``, per-row ``seq_lens`` / ``weight_indices`` /
  ``lora_ranks`` (/ ``scalings``).  With a workspace from torch's caching
  allocator they run the MFMA path (weights repacked on the device, device
  plan, tiled shrink or expand); shapes that path does not take run the
  row-based HIP kernels.
* ``SgmvPlan`` + ``lora_apply`` are what ``MultiLoraLinear`` uses: one device
  plan per forward (no host sync) and the MFMA-tiled shrink/expand over the
  packed slot arena of ``GpuAdapterCache``.

There is no CPU path: CPU tensors raise.
"""

from __future__ import annotations

import ctypes
import threading

import torch

from . import _native, refop_cache

__all__ = ["SgmvPlan", "lora_apply", "lora_apply_rows", "lora_shrink", "lora_expand", "sgmv_lora_a_fwd",
           "sgmv_lora_b_fwd", "choose_k_splits", "choose_group_tokens", "side_stream", "lora_shrink_stacked",
           "lora_fused", "fused_ok", "choose_slices", "lora_expand_stacked", "lora_decode_stacked", "decode_ok",
           "decode_waits_timed_out"]


def _stream(device: torch.device) -> int:
    """Handle of the current stream of `device` (one C call, no Stream object)."""
    idx = device.index if device.index is not None else torch.cuda.current_device()
    return torch._C._cuda_getCurrentRawStream(idx)


def _require_gpu(t: torch.Tensor, what: str) -> None:
    if not t.is_cuda:
        raise RuntimeError(
            f"{what}: polylora_amd runs LoRA math only on a ROCm GPU through its HIP library; "
            "got a CPU tensor (there is no CPU fallback)"
        )


def _i32(t: torch.Tensor) -> torch.Tensor:
    if t.dtype is torch.int32 and t.is_contiguous():
        return t
    return t.to(torch.int32).contiguous()


_LONG_GROUP_MIN_TOKENS = 8192


def choose_group_tokens(tokens: int, distinct_slots: int | None) -> int:
    """Plan group size: 64-token groups only for large batches of long adapter segments.

    16-token groups give one workgroup per 16-row tile, the most parallel
    launch; 64-token groups let the shrink read each adapter's A once per 64
    tokens, which pays once a batch has enough tokens (prefill) to fill the
    GPU with 64-token groups anyway.
    """
    if tokens < _LONG_GROUP_MIN_TOKENS:
        return _native.PL_GROUP_TOKENS_SHORT
    if distinct_slots is not None and tokens <= 32 * max(1, distinct_slots):
        return _native.PL_GROUP_TOKENS_SHORT
    return _native.PL_GROUP_TOKENS_LONG


class SgmvPlan:
    """Adapter-major token groups for one (rows, row_len) layer shape of a forward.

    Built on the device by ``pl_plan_build`` from the int32 row -> slot map and
    per-row lengths; every wrapped Linear of the forward with this shape reuses
    it.  Buffers: ``tok`` [rows*row_len] sorted token indices, ``groups``
    [group_cap, 4] (slot, start, len, 0), ``meta`` [4] (num_groups,
    num_tokens, group_tokens, positions in use).  ``distinct_slots`` (the number of different
    adapters in the batch, known on the host) picks the group size; without
    it the plan uses 64-token groups.
    """

    __slots__ = ("rows", "row_len", "num_slots", "group_tokens", "tokens_cap", "group_cap", "tok", "groups", "meta",
                 "row_slot", "seq_lens", "distinct_slots", "launch_args", "launch_args_c", "active", "_build")

    def __init__(self, row_slot: torch.Tensor, seq_lens: torch.Tensor, row_len: int, num_slots: int,
                 distinct_slots: int | None = None, group_tokens: int | None = None,
                 active: torch.Tensor | None = None) -> None:
        """``active`` (optional, int32 [num_slots], any stride, e.g. ``cache.ranks[module]``): rows whose
        slot reads <= 0 there are left out, so a plan that serves one module spends no group
        positions (and no XCD share) on slots without weights for it."""
        _require_gpu(row_slot, "SgmvPlan")
        if active is not None and (active.dtype != torch.int32 or active.dim() != 1 or active.numel() < num_slots
                                   or active.device != row_slot.device):
            raise ValueError("active must be an int32 vector of num_slots entries on the row map's device")
        lib = _native.load()
        row_slot = _i32(row_slot)
        seq_lens = _i32(seq_lens)
        rows = int(row_slot.numel())
        if int(seq_lens.numel()) != rows:
            raise ValueError("row_slot and seq_lens must have the same length")
        self.rows, self.row_len, self.num_slots = rows, int(row_len), int(num_slots)
        self.tokens_cap = rows * self.row_len
        self.distinct_slots = distinct_slots
        if group_tokens is None:
            group_tokens = choose_group_tokens(self.tokens_cap, distinct_slots)
        if group_tokens not in (_native.PL_GROUP_TOKENS_SHORT, _native.PL_GROUP_TOKENS_LONG):
            raise ValueError(f"group_tokens must be 16 or 64, not {group_tokens}")
        self.group_tokens = int(group_tokens)
        self.group_cap = int(lib.pl_plan_group_capacity(rows, self.row_len, self.num_slots, self.group_tokens))
        dev = row_slot.device
        self.tok = torch.empty(max(1, self.tokens_cap), dtype=torch.int32, device=dev)
        self.groups = torch.empty((max(1, self.group_cap), 4), dtype=torch.int32, device=dev)
        self.meta = torch.empty(4, dtype=torch.int32, device=dev)
        # the plan's arguments of the fused entry points, in their order
        self.launch_args = (self.tok.data_ptr(), self.groups.data_ptr(), self.meta.data_ptr(), max(1, self.group_cap),
                            self.group_tokens)
        self.launch_args_c = (ctypes.c_void_p(self.launch_args[0]), ctypes.c_void_p(self.launch_args[1]),
                              ctypes.c_void_p(self.launch_args[2]), ctypes.c_int64(self.launch_args[3]),
                              ctypes.c_int32(self.launch_args[4]))
        self.row_slot, self.seq_lens, self.active = row_slot, seq_lens, active
        out = (self.tok.data_ptr(), self.groups.data_ptr(), self.meta.data_ptr(), max(1, self.group_cap))
        if active is None:
            self._build = (lib.pl_plan_build, "pl_plan_build",
                           (row_slot.data_ptr(), seq_lens.data_ptr(), rows, self.row_len, self.num_slots,
                            self.group_tokens, *out))
        else:
            self._build = (lib.pl_plan_build_active, "pl_plan_build_active",
                           (row_slot.data_ptr(), seq_lens.data_ptr(), rows, self.row_len, self.num_slots,
                            active.data_ptr(), active.stride(0), self.group_tokens, *out))
        self.rebuild(_stream(dev))

    def rebuild(self, stream: int | None = None) -> None:
        """Build the plan again into the same buffers from the current contents of its row -> slot map,
        lengths and active vector (on the current stream, or `stream`); nothing is allocated."""
        fn, what, args = self._build
        _native.check(fn(*args, _stream(self.tok.device) if stream is None else stream), what)


class _Workspace:
    """fp32 shrink planes for one (device, stream), grown on demand.

    The shrink writes every entry the expand reads, so the buffer is never
    cleared.  Buffers are only ever replaced by larger ones, and replaced
    buffers stay allocated for the life of the process, so a HIP graph that
    recorded a launch keeps a valid pointer.
    """

    def __init__(self, device: torch.device) -> None:
        self.device = device
        self.buf: torch.Tensor | None = None
        self.retired: list[torch.Tensor] = []
        self.owner: object | None = None  # the ShrinkResult whose planes the buffer holds

    def get(self, nbytes: int) -> torch.Tensor:
        nbytes = max(256, (nbytes + 255) // 256 * 256)
        if self.buf is None or self.buf.numel() < nbytes:
            if self.buf is not None:
                self.retired.append(self.buf)
                nbytes = max(nbytes, 2 * self.buf.numel())
            self.buf = torch.empty(nbytes, dtype=torch.uint8, device=self.device)
        return self.buf


_WORKSPACES: dict[tuple[int, int, int], _Workspace] = {}


def _workspace(device: torch.device, stream: int, position: int = 0) -> _Workspace:
    """Workspace `position` of (device, stream); a stacked shrink writes module i to position i."""
    key = (device.index if device.index is not None else torch.cuda.current_device(), stream, position)
    ws = _WORKSPACES.get(key)
    if ws is None:
        ws = _WORKSPACES[key] = _Workspace(device)
    return ws


# K elements per shrink split, and the active shrink workgroups to aim for.
# Measured on MI355X (bf16, K=4096/14336): more splits feed the shrink more
# workgroups, but every expand workgroup re-reads every split's partial sums,
# so about one split per 1024 of K balances the two kernels.  At most 8
# splits: the expand holds one register set per split, and with 9..16 it runs
# half as many waves per SIMD (decode down_proj, K = 14336: 14 splits 22.7 us
# for the pair, 8 splits 21.9 us).
_K_PER_SPLIT = 1024
_TARGET_SHRINK_BLOCKS = 2048
_MAX_K_SPLITS = 8


def choose_k_splits(group_cap: int, K: int, dtype: torch.dtype) -> int:
    """K splits of the shrink: about one per 1024 of K (at most 8), fewer when the group count alone fills the GPU."""
    by_k = min(_MAX_K_SPLITS, max(1, -(-K // _K_PER_SPLIT)))
    by_groups = max(1, -(-_TARGET_SHRINK_BLOCKS // max(1, group_cap)))
    return min(by_k, by_groups)


def _tiled_ok(x: torch.Tensor, y: torch.Tensor) -> bool:
    """Unit column stride, 16-byte aligned base pointers, and K, N and both row strides whole 16-byte chunks."""
    xs, ys = x.stride(), y.stride()
    chunk = 16 // x.element_size()  # elements per 16 bytes
    return (
        xs[1] == 1
        and ys[1] == 1
        and (x.shape[1] | y.shape[1] | xs[0] | ys[0]) % chunk == 0
        and (x.data_ptr() | y.data_ptr()) % 16 == 0
    )


def _check_operands(x: torch.Tensor, y: torch.Tensor, cache, module_name: str, tokens: int) -> None:
    """Shapes, dtypes and devices the kernels assume; a mismatch would read outside the arena."""
    spec = cache.module_specs.get(module_name)
    if spec is None:
        raise KeyError(f"module {module_name!r} is not in the adapter cache")
    xs, ys = x.shape, y.shape
    if len(xs) != 2 or len(ys) != 2:
        raise ValueError("x and y must be 2-D [tokens, features]")
    if xs[0] != tokens or ys[0] != tokens:
        raise ValueError(f"x / y have {xs[0]} / {ys[0]} token rows; the plan covers {tokens}")
    if xs[1] != spec.in_features or ys[1] != spec.out_features:
        raise ValueError(
            f"module {module_name!r} is {spec.in_features} -> {spec.out_features}, "
            f"got x [.., {x.shape[1]}] and y [.., {y.shape[1]}]"
        )
    if x.dtype != cache.dtype or y.dtype != cache.dtype:
        raise TypeError(f"x {x.dtype} / y {y.dtype} must match the adapter cache dtype {cache.dtype}")
    if x.device != cache.device or y.device != cache.device:
        raise ValueError(f"x / y must be on the adapter cache device {cache.device}")


def lora_apply(
    x: torch.Tensor,
    y: torch.Tensor,
    cache,
    module_name: str,
    plan: SgmvPlan,
    *,
    epilogue: int = _native.PL_EPI_FALLBACK,
    k_splits: int | None = None,
) -> torch.Tensor:
    """y[t] += scale * (x[t] @ A^T) @ B^T for every planned token t, in place.

    x: [rows*row_len, in_features], y: [rows*row_len, out_features], both of
    the cache's dtype, on the cache's device.  Long adapter segments go to
    the fused kernel (lora_fused) unless k_splits asks for the split pair;
    x / y that do not meet the tiled path's alignment go to the row-based HIP
    kernels.
    """
    _require_gpu(x, "lora_apply")
    _check_operands(x, y, cache, module_name, plan.tokens_cap)
    if not _tiled_ok(x, y):
        return lora_apply_rows(x, y, cache, module_name, plan.row_slot, plan.seq_lens, plan.row_len, epilogue=epilogue)
    if k_splits is None and fused_ok(plan, cache, int(x.shape[1])):
        # operands checked above; fused_ok guarantees the rank limit
        _fused_launch(x, y, cache, module_name, plan, epilogue, None, _stream(x.device))
        return y
    lib = _native.load()
    dt = _native.dtype_code(x.dtype)
    K = int(x.shape[1])
    N = int(y.shape[1])
    ldt = cache.rank8_cap
    stream = _stream(x.device)
    rows = max(1, plan.tokens_cap)
    group_cap = max(1, plan.group_cap)
    splits, _, nbytes = _shrink_geometry(lib, dt, K, x.dtype, plan, rows, ldt, k_splits)
    ws = _workspace(x.device, stream)
    buf = ws.get(nbytes)
    ws.owner = None  # planes of an earlier separate shrink on this workspace are gone
    status = lib.pl_lora_apply(
        dt,
        x.data_ptr(),
        x.stride(0),
        K,
        y.data_ptr(),
        y.stride(0),
        N,
        cache.arena.data_ptr(),
        cache.table.data_ptr(),
        len(cache.module_index),
        cache.module_index[module_name],
        plan.tok.data_ptr(),
        plan.groups.data_ptr(),
        plan.meta.data_ptr(),
        group_cap,
        plan.group_tokens,
        buf.data_ptr(),
        buf.numel(),
        ldt,
        rows,
        splits,
        epilogue,
        stream,
    )
    _native.check(status, "pl_lora_apply")
    return y


class ShrinkResult:
    """Where a shrink left its partial sums: a workspace of the stream it ran on.

    ``valid`` turns False once a later shrink has reused that workspace.
    ``batch`` identifies the stacked shrink this result came from (its
    workspace pointer array) and ``index`` its position in it.
    """

    __slots__ = ("ws", "buf", "planes", "rows", "ldt", "plan", "K", "batch", "index")

    def __init__(self, ws, buf, planes, rows, ldt, plan, K, batch=None, index=0) -> None:
        self.ws, self.buf, self.planes, self.rows, self.ldt, self.plan, self.K = ws, buf, planes, rows, ldt, plan, K
        self.batch, self.index = batch, index
        ws.owner = self

    @property
    def valid(self) -> bool:
        return self.ws.owner is self


class _ShrinkBatch:
    """The modules of one stacked shrink: their count and workspace pointers as passed to the kernel."""

    __slots__ = ("n", "ptrs")

    def __init__(self, n: int, ptrs) -> None:
        self.n, self.ptrs = n, ptrs


MAX_STACKED_MODULES = _native.PL_MAX_STACKED_MODULES

_SIDE_STREAMS: dict[int, torch.cuda.Stream] = {}


def side_stream(device: torch.device) -> torch.cuda.Stream:
    """The per-device stream shrinks run on while the base GEMM runs on the current stream (default priority)."""
    idx = device.index if device.index is not None else torch.cuda.current_device()
    st = _SIDE_STREAMS.get(idx)
    if st is None:
        st = _SIDE_STREAMS[idx] = torch.cuda.Stream(device=torch.device("cuda", idx))
    return st


def tiled_shapes_ok(x: torch.Tensor, out_features: int) -> bool:
    """Whether x [tokens, K] and a fresh contiguous output of out_features columns suit the tiled kernels."""
    chunk = 4 if x.dtype == torch.float32 else 8
    return (
        x.is_cuda
        and x.dim() == 2
        and x.stride(1) == 1
        and x.shape[1] % chunk == 0
        and out_features % chunk == 0
        and (x.stride(0) * x.element_size()) % 16 == 0
        and x.data_ptr() % 16 == 0
    )


_GEOMETRY: dict[tuple, tuple[int, int, int]] = {}


def _shrink_geometry(lib, dt: int, K: int, dtype: torch.dtype, plan: SgmvPlan, rows: int, ldt: int,
                     k_splits: int | None) -> tuple[int, int, int]:
    """(k_splits, planes, workspace bytes) of a shrink, computed once per shape."""
    key = (dt, K, plan.group_cap, plan.group_tokens, rows, ldt, k_splits)
    geo = _GEOMETRY.get(key)
    if geo is None:
        splits = k_splits if k_splits is not None else choose_k_splits(plan.group_cap, K, dtype)
        planes = int(lib.pl_shrink_planes(dt, K, splits, plan.group_tokens))
        nbytes = int(lib.pl_shrink_workspace_bytes(dt, K, splits, plan.group_tokens, rows, ldt))
        geo = _GEOMETRY[key] = (splits, planes, nbytes)
    return geo


def lora_shrink(x: torch.Tensor, cache, module_name: str, plan: SgmvPlan, *, k_splits: int | None = None,
                stream: int | None = None) -> ShrinkResult:
    """Launch the shrink of one wrapped Linear on the current stream; the expand reads the result later."""
    return lora_shrink_stacked(x, cache, [module_name], plan, k_splits=k_splits, stream=stream)[0]


def _module_set(cache, module_names) -> tuple:
    """(specs, ctypes int32 array of table columns) of a module list, built once per cache and list."""
    sets = cache.__dict__.setdefault("_module_sets", {})
    key = tuple(module_names)
    hit = sets.get(key)
    if hit is not None:
        return hit
    specs = []
    for name in module_names:
        spec = cache.module_specs.get(name)
        if spec is None:
            raise KeyError(f"module {name!r} is not in the adapter cache")
        specs.append(spec)
    cols = (ctypes.c_int32 * len(specs))(*(cache.module_index[name] for name in module_names))
    sets[key] = (specs, cols)
    return specs, cols


def _fused_set(cache, module_names) -> tuple:
    """_module_set plus the output-pointer, row-stride and column-count arrays of one stacked fused launch.

    The arrays are reused call after call by the calling thread (the pointers
    and strides are rewritten before each launch, which reads them when it is
    enqueued); another thread gets its own, since the library call runs
    without the GIL.
    """
    sets = cache.__dict__.setdefault("_fused_sets", {})
    key = (tuple(module_names), threading.get_ident())
    hit = sets.get(key)
    if hit is None:
        specs, cols = _module_set(cache, module_names)
        n = len(specs)
        cnt = (ctypes.c_int32 * n)(*(spec.out_features for spec in specs))
        hit = sets[key] = (specs, cols, ((ctypes.c_void_p * n)(), (ctypes.c_int64 * n)(), cnt))
    return hit


_WS_SETS: dict = {}


def _workspace_set(device: torch.device, stream: int, n: int, nbytes: int) -> tuple:
    """(workspaces, buffers, ctypes pointer array) of positions 0..n-1 of (device, stream)."""
    key = (device.index if device.index is not None else torch.cuda.current_device(), stream, n)
    hit = _WS_SETS.get(key)
    if hit is None:
        wss = [_workspace(device, stream, i) for i in range(n)]
        hit = [wss, None, None]
        _WS_SETS[key] = hit
    wss = hit[0]
    bufs = [ws.get(nbytes) for ws in wss]
    if hit[1] is None or any(b is not c for b, c in zip(bufs, hit[1])):
        hit[1] = bufs
        hit[2] = (ctypes.c_void_p * n)(*(b.data_ptr() for b in bufs))
    return wss, hit[1], hit[2]


def lora_shrink_stacked(x: torch.Tensor, cache, module_names: list, plan: SgmvPlan, *,
                        k_splits: int | None = None, stream: int | None = None) -> list:
    """One shrink launch for wrapped Linears that read the same x (pl_sgmv_shrink_stacked).

    Module i's partial sums go to workspace position i of the current stream.
    `stream` is that stream's handle when the caller already has it.
    """
    _require_gpu(x, "lora_shrink")
    n = len(module_names)
    if not 1 <= n <= _native.PL_MAX_STACKED_MODULES:
        raise ValueError(f"a shrink serves 1..{_native.PL_MAX_STACKED_MODULES} modules, got {n}")
    specs, modules = _module_set(cache, module_names)
    K = int(x.shape[1]) if x.dim() == 2 else -1
    if x.dim() != 2 or x.shape[0] != plan.tokens_cap or any(sp.in_features != K for sp in specs):
        raise ValueError(f"x must be [{plan.tokens_cap}, in_features] for every module, got {list(x.shape)}")
    if x.dtype != cache.dtype or x.device != cache.device:
        raise TypeError(f"x {x.dtype} on {x.device} must match the adapter cache ({cache.dtype} on {cache.device})")
    lib = _native.load()
    dt = _native.dtype_code(x.dtype)
    ldt = cache.rank8_cap
    if stream is None:
        stream = _stream(x.device)
    rows = max(1, plan.tokens_cap)
    splits, planes, nbytes = _shrink_geometry(lib, dt, K, x.dtype, plan, rows, ldt, k_splits)
    wss, bufs, ptrs = _workspace_set(x.device, stream, n, nbytes)
    _native.check(
        lib.pl_sgmv_shrink_stacked(
            dt, x.data_ptr(), x.stride(0), K, cache.arena.data_ptr(), cache.table.data_ptr(), len(cache.module_index),
            n, modules, ptrs, plan.tok.data_ptr(), plan.groups.data_ptr(), plan.meta.data_ptr(),
            max(1, plan.group_cap), plan.group_tokens, min(b.numel() for b in bufs), ldt, rows, splits, stream,
        ),
        "pl_sgmv_shrink_stacked",
    )
    batch = _ShrinkBatch(n, ptrs)
    return [ShrinkResult(ws, b, planes, rows, ldt, plan, K, batch, i) for i, (ws, b) in enumerate(zip(wss, bufs))]


def lora_expand(res: ShrinkResult, y: torch.Tensor, cache, module_name: str, *,
                epilogue: int = _native.PL_EPI_FALLBACK, stream: int | None = None) -> torch.Tensor:
    """Launch the expand on the current stream (handle `stream` if given), ordered after the shrink."""
    _require_gpu(y, "lora_expand")
    spec = cache.module_specs[module_name]
    plan = res.plan
    if y.dim() != 2 or y.shape[0] != plan.tokens_cap or y.shape[1] != spec.out_features:
        raise ValueError(f"y must be [{plan.tokens_cap}, {spec.out_features}], got {list(y.shape)}")
    if y.dtype != cache.dtype or y.device != cache.device:
        raise TypeError(f"y {y.dtype} on {y.device} must match the adapter cache ({cache.dtype} on {cache.device})")
    if not res.valid:
        raise RuntimeError("the shrink result was overwritten by a later shrink on the same workspace")
    lib = _native.load()
    _native.check(
        lib.pl_sgmv_expand(
            _native.dtype_code(y.dtype), res.buf.data_ptr(), res.ldt, res.rows, res.planes, cache.arena.data_ptr(),
            cache.table.data_ptr(), len(cache.module_index), cache.module_index[module_name], plan.tok.data_ptr(),
            plan.groups.data_ptr(), plan.meta.data_ptr(), max(1, plan.group_cap), plan.group_tokens, y.data_ptr(),
            y.stride(0), int(y.shape[1]), epilogue, _stream(y.device) if stream is None else stream,
        ),
        "pl_sgmv_expand",
    )
    return y


FUSED_MAX_RANK = 64


def choose_slices(plan: SgmvPlan, out_features: int) -> int:
    """Column slices per 16-token tile of the fused kernel.

    Every slice recomputes its tile's shrink, which costs more than the extra
    workgroups gain as soon as the tiles alone give about one workgroup per
    CU (measured on MI355X at 256 and 2048 tiles: one slice is fastest), so
    slices are added only below 128 tiles, and never below 1024 columns each.
    """
    tiles = max(1, plan.tokens_cap // 16)
    want = max(1, 256 // tiles)
    most = max(1, out_features // 1024)
    return max(1, min(want, most, 4))


# Largest in_features the fused kernel takes on the forward path.  Measured
# on MI355X (Llama-3-8B prefill shapes): at K = 14336 (down_proj) one fused
# launch per layer beats the split shrink/expand pair in the forward's launch
# sequence; longer reductions are untried and keep the split pair.
FUSED_MAX_K = 16384


def fused_ok(plan: SgmvPlan, cache, in_features: int) -> bool:
    """Whether the fused kernel suits a plan and module: ranks within its limit, full 16-token tiles.

    The fused kernel reads each adapter's A and B once per 16-token tile, so it
    wants tiles that are full (long adapter segments, known from the plan's
    distinct-adapter count); with a few tokens per adapter (decode) the split
    shrink/expand spreads the weights over many more workgroups.
    """
    distinct = plan.distinct_slots
    if cache.rank8_cap > FUSED_MAX_RANK or distinct is None or in_features > FUSED_MAX_K:
        return False
    return plan.tokens_cap >= 64 * max(1, distinct) and plan.tokens_cap >= 1024


def lora_fused(
    x: torch.Tensor,
    y: torch.Tensor,
    cache,
    module_name: str,
    plan: SgmvPlan,
    *,
    epilogue: int = _native.PL_EPI_FALLBACK,
    slices: int | None = None,
    stream: int | None = None,
) -> torch.Tensor:
    """y[t] += scale * (x[t] @ A^T) @ B^T for every planned token t, in place, in one launch (pl_lora_fused).

    Same operands as lora_apply; needs the tiled path's alignment and slot
    ranks up to FUSED_MAX_RANK.
    """
    _require_gpu(x, "lora_fused")
    _check_operands(x, y, cache, module_name, plan.tokens_cap)
    if not _tiled_ok(x, y):
        raise ValueError("lora_fused needs 16-byte aligned rows and K, N multiples of 16 bytes")
    if cache.rank8_cap > FUSED_MAX_RANK:
        raise ValueError(f"lora_fused takes ranks up to {FUSED_MAX_RANK}; the cache holds up to {cache.rank8_cap}")
    _fused_launch(x, y, cache, module_name, plan, epilogue, slices, _stream(x.device) if stream is None else stream)
    return y


def _cache_args(cache, module_name: str) -> tuple:
    """(arena, table, module count, table column, rank capacity) of a module as pl_lora_fused takes them.

    The arena and table are allocated once with the cache, so the tuple is
    built once per cache and module.
    """
    args = cache.__dict__.setdefault("_launch_args", {})
    hit = args.get(module_name)
    if hit is None:
        hit = args[module_name] = (cache.arena.data_ptr(), cache.table.data_ptr(), len(cache.module_index),
                                   cache.module_index[module_name], cache.rank8_cap)
    return hit


def _cache_args_c(cache, module_name: str) -> tuple:
    """_cache_args as ctypes objects, built once per cache and module.

    Kept in the same memo as _cache_args, which the cache drops whenever it
    allocates a new arena and table (GpuAdapterCache.to), so neither form
    can outlive the memory it points at.
    """
    args = cache.__dict__.setdefault("_launch_args", {})
    key = ("ctypes", module_name)
    hit = args.get(key)
    if hit is None:
        arena, table, n_modules, column, ldt = _cache_args(cache, module_name)
        hit = args[key] = (ctypes.c_void_p(arena), ctypes.c_void_p(table), ctypes.c_int32(n_modules),
                           ctypes.c_int32(column), ctypes.c_int32(ldt))
    return hit


def _fused_launch(x, y, cache, module_name: str, plan: SgmvPlan, epilogue: int, slices, stream: int) -> None:
    """pl_lora_fused on operands the caller has checked.

    The wrapped Linear's hot call: the cache's and the plan's arguments are
    ctypes objects built once (per cache and module, per plan), and the
    entry point is called without per-argument conversion.
    """
    N = y.shape[1]
    c32 = _native.c32
    rc = _native.raw("pl_lora_fused")(
        c32(_native.dtype_code(x.dtype)), ctypes.c_void_p(x.data_ptr()), ctypes.c_int64(x.stride(0)),
        c32(x.shape[1]), ctypes.c_void_p(y.data_ptr()), ctypes.c_int64(y.stride(0)), c32(N),
        *_cache_args_c(cache, module_name), *plan.launch_args_c,
        c32(choose_slices(plan, N) if slices is None else slices), c32(epilogue), ctypes.c_void_p(stream))
    if rc:
        _native.check(rc, "pl_lora_fused")


def lora_fused_stacked(
    x: torch.Tensor,
    ys: list,
    cache,
    module_names: list,
    plan: SgmvPlan,
    *,
    epilogue: int = _native.PL_EPI_FALLBACK,
    slices: int | None = None,
    stream: int | None = None,
) -> list:
    """lora_fused for sibling Linears fed the same x, in one launch (pl_lora_fused_stacked): ys[i] in place.

    A tile's modules run side by side on one XCD, so x comes from HBM once.
    """
    _require_gpu(x, "lora_fused_stacked")
    n = len(module_names)
    if not 1 <= n <= _native.PL_MAX_STACKED_MODULES or len(ys) != n:
        raise ValueError(f"a fused launch serves 1..{_native.PL_MAX_STACKED_MODULES} modules with one y each")
    # x and the first output in full, the others against the first
    _check_operands(x, ys[0], cache, module_names[0], plan.tokens_cap)
    if not _tiled_ok(x, ys[0]):
        raise ValueError("lora_fused needs 16-byte aligned rows and K, N multiples of 16 bytes")
    specs, mods, arrays = _fused_set(cache, module_names)
    chunk = 16 // x.element_size()
    for y, spec in zip(ys[1:], specs[1:]):
        if spec.in_features != x.shape[1]:
            raise ValueError(f"module {spec.name!r} takes {spec.in_features} inputs; x has {x.shape[1]}")
        shape, st = y.shape, y.stride()
        if len(shape) != 2 or shape[0] != plan.tokens_cap or shape[1] != spec.out_features:
            raise ValueError(f"y of {spec.name!r} must be [{plan.tokens_cap}, {spec.out_features}], got {list(shape)}")
        if y.dtype != cache.dtype or y.device != cache.device:
            raise TypeError(f"y {y.dtype} on {y.device} must match the adapter cache ({cache.dtype} on {cache.device})")
        if st[1] != 1 or (shape[1] | st[0]) % chunk or y.data_ptr() % 16:
            raise ValueError("lora_fused needs 16-byte aligned rows and K, N multiples of 16 bytes")
    if cache.rank8_cap > FUSED_MAX_RANK:
        raise ValueError(f"lora_fused takes ranks up to {FUSED_MAX_RANK}; the cache holds up to {cache.rank8_cap}")
    yp, ldy, nn_ = arrays
    for i, y in enumerate(ys):
        yp[i] = y.data_ptr()
        ldy[i] = y.stride(0)
    n_slices = slices if slices is not None else choose_slices(plan, min(spec.out_features for spec in specs))
    arena, table, n_mod, _, ldt = _cache_args(cache, module_names[0])
    _native.check(
        _native.load().pl_lora_fused_stacked(
            _native.dtype_code(x.dtype), x.data_ptr(), x.stride(0), x.shape[1], n, mods, yp, ldy, nn_,
            arena, table, n_mod, ldt, *plan.launch_args, n_slices, epilogue,
            _stream(x.device) if stream is None else stream,
        ),
        "pl_lora_fused_stacked",
    )
    return ys


def lora_expand_stacked(results: list, ys: list, cache, module_names: list, *,
                        epilogue: int = _native.PL_EPI_FALLBACK, stream: int | None = None) -> list:
    """One expand launch for sibling Linears (pl_sgmv_expand_stacked): results[i] -> ys[i] in place.

    results are the ShrinkResults of one stacked shrink (same plan, K split
    and workspace geometry); the stream must be ordered after that shrink and
    after every ys[i]'s producer.
    """
    n = len(module_names)
    if not 1 <= n <= _native.PL_MAX_STACKED_MODULES or len(results) != n or len(ys) != n:
        raise ValueError(f"an expand serves 1..{_native.PL_MAX_STACKED_MODULES} modules with one result and one y each")
    plan = results[0].plan
    for res, y, name in zip(results, ys, module_names):
        _require_gpu(y, "lora_expand_stacked")
        spec = cache.module_specs[name]
        if res.plan is not plan or res.planes != results[0].planes or res.rows != results[0].rows:
            raise ValueError("stacked expand results must come from one stacked shrink")
        if y.dim() != 2 or y.shape[0] != plan.tokens_cap or y.shape[1] != spec.out_features:
            raise ValueError(f"y must be [{plan.tokens_cap}, {spec.out_features}], got {list(y.shape)}")
        if y.dtype != cache.dtype or y.device != cache.device:
            raise TypeError(f"y {y.dtype} on {y.device} must match the adapter cache ({cache.dtype} on {cache.device})")
        if not res.valid:
            raise RuntimeError("the shrink result was overwritten by a later shrink on the same workspace")
    lib = _native.load()
    r0 = results[0]
    batch = r0.batch
    if batch is not None and batch.n == n and all(r.batch is batch and r.index == i for i, r in enumerate(results)):
        ws = batch.ptrs  # the shrink's own pointer array, in the same order
    else:
        ws = (ctypes.c_void_p * n)(*(r.buf.data_ptr() for r in results))
    _, mods = _module_set(cache, module_names)
    yp = (ctypes.c_void_p * n)(*(y.data_ptr() for y in ys))
    ldy = (ctypes.c_int64 * n)(*(y.stride(0) for y in ys))
    nn_ = (ctypes.c_int32 * n)(*(int(y.shape[1]) for y in ys))
    _native.check(
        lib.pl_sgmv_expand_stacked(
            _native.dtype_code(ys[0].dtype), ws, r0.ldt, r0.rows, r0.planes, cache.arena.data_ptr(),
            cache.table.data_ptr(), len(cache.module_index), n, mods, plan.tok.data_ptr(), plan.groups.data_ptr(),
            plan.meta.data_ptr(), max(1, plan.group_cap), plan.group_tokens, yp, ldy, nn_, epilogue,
            _stream(ys[0].device) if stream is None else stream,
        ),
        "pl_sgmv_expand_stacked",
    )
    return ys


class _HandoffCounters:
    """Zeroed int32 hand-off counters of pl_lora_decode_stacked for one (device, stream), grown on demand.

    Every launch whose waits all end in time leaves them zero (each counter's
    last reader resets it), so they are cleared only when allocated, on the
    current stream, which must be the stream the launches run on, and by
    decode_waits_timed_out after a wait ran out; replaced buffers stay
    allocated for the life of the process, so a HIP graph that recorded a
    launch keeps a valid pointer.  Word 0 is the status a timed-out wait sets
    to 1.
    """

    def __init__(self, device: torch.device) -> None:
        self.device = device
        self.buf: torch.Tensor | None = None
        self.retired: list[torch.Tensor] = []

    def get(self, ints: int) -> torch.Tensor:
        if self.buf is None or self.buf.numel() < ints:
            if self.buf is not None:
                self.retired.append(self.buf)
                ints = max(ints, 2 * self.buf.numel())
            # cleared by a fill kernel on the current stream (the launch's stream),
            # which a HIP graph being captured records like any other kernel; an
            # ordinary tensor even under torch.inference_mode, so that
            # decode_waits_timed_out can clear it outside that mode
            with torch.inference_mode(False):
                self.buf = torch.empty(max(64, ints), dtype=torch.int32, device=self.device).zero_()
        return self.buf


_COUNTERS: dict[tuple[int, int], _HandoffCounters] = {}

# Polls of a hand-off counter before a waiting expand workgroup gives up (each
# poll is one memory round trip plus a short sleep: well under a second in all,
# against the tens of microseconds a launch's shrink takes).
DECODE_SPIN_LIMIT = 1 << 16


def handoff_counters(device: torch.device, stream: int) -> _HandoffCounters:
    key = (device.index if device.index is not None else torch.cuda.current_device(), stream)
    hit = _COUNTERS.get(key)
    if hit is None:
        hit = _COUNTERS[key] = _HandoffCounters(device)
    return hit


def decode_waits_timed_out(device: torch.device | None = None, clear: bool = True) -> bool:
    """Whether a pl_lora_decode_stacked wait on `device` (all devices when None) ran out of polls since the
    status words were last cleared: the results of that launch are then undefined.  Waits for the work
    queued so far on each counter set's device.  With `clear`, a counter set whose status word is set is
    zeroed whole (on the current stream) for the next launches: a shrink workgroup that arrived after a
    wait gave up can leave its counter above zero, and a later launch's waits would then end early.  A
    timed-out wait is not expected on a GPU this process has to itself: the limit is far above what a
    launch's shrink takes."""
    hit = False
    for (index, _), c in _COUNTERS.items():
        if c.buf is None or (device is not None and c.device != torch.device(device)):
            continue
        torch.cuda.synchronize(c.device)
        if int(c.buf[0]) != 0:
            hit = True
            if clear:
                c.buf.zero_()  # no launch is in flight on the device: every counter can be reset
    return hit


def decode_ok(plan: SgmvPlan) -> bool:
    """Whether a plan suits the one-launch decode path (pl_lora_decode_stacked): 16-token groups."""
    return plan.group_tokens == 16


def lora_decode_stacked(x: torch.Tensor, ys: list, cache, module_names: list, plan: SgmvPlan, *,
                        k_splits: int | None = None, epilogue: int = _native.PL_EPI_FALLBACK,
                        stream: int | None = None) -> list:
    """Shrink and expand of 1..4 sibling Linears fed the same x in ONE launch (pl_lora_decode_stacked).

    Adds each module's LoRA delta into ys[i] in place, bitwise equal to
    lora_shrink_stacked followed by lora_expand_stacked on the same stream:
    the expand workgroups of a group start on its partial sums as soon as
    every shrink workgroup of that group has stored them, inside the launch.
    For plans of 16-token groups (decode).  Uses the stream's shrink
    workspaces (positions 0..n-1) and its hand-off counters.
    """
    _require_gpu(x, "lora_decode_stacked")
    n = len(module_names)
    if not 1 <= n <= _native.PL_MAX_STACKED_MODULES or len(ys) != n:
        raise ValueError(f"a decode launch serves 1..{_native.PL_MAX_STACKED_MODULES} modules with one y each")
    if not decode_ok(plan):
        raise ValueError("lora_decode_stacked takes plans of 16-token groups")
    specs, mods, arrays = _fused_set(cache, module_names)
    K = int(x.shape[1]) if x.dim() == 2 else -1
    if x.dim() != 2 or x.shape[0] != plan.tokens_cap or any(sp.in_features != K for sp in specs):
        raise ValueError(f"x must be [{plan.tokens_cap}, in_features] for every module, got {list(x.shape)}")
    if x.dtype != cache.dtype or x.device != cache.device:
        raise TypeError(f"x {x.dtype} on {x.device} must match the adapter cache ({cache.dtype} on {cache.device})")
    for y, spec in zip(ys, specs):
        _require_gpu(y, "lora_decode_stacked")
        if y.dim() != 2 or y.shape[0] != plan.tokens_cap or y.shape[1] != spec.out_features:
            raise ValueError(f"y of {spec.name!r} must be [{plan.tokens_cap}, {spec.out_features}], got {list(y.shape)}")
        if y.dtype != cache.dtype or y.device != cache.device:
            raise TypeError(f"y {y.dtype} on {y.device} must match the adapter cache ({cache.dtype} on {cache.device})")
    lib = _native.load()
    dt = _native.dtype_code(x.dtype)
    ldt = -(-cache.rank8_cap // 32) * 32  # plane rows of whole 128-byte lines
    if stream is None:
        stream = _stream(x.device)
    rows = max(1, plan.tokens_cap)
    splits, planes, nbytes = _shrink_geometry(lib, dt, K, x.dtype, plan, rows, ldt, k_splits)
    wss, bufs, ptrs = _workspace_set(x.device, stream, n, nbytes)
    for ws in wss:
        ws.owner = None  # any earlier shrink's planes there are overwritten by this launch
    cap = max(1, plan.group_cap)
    need = int(lib.pl_decode_counter_ints(cap, n))
    counters = handoff_counters(x.device, stream).get(need)
    yp, ldy, nn_ = arrays
    for i, y in enumerate(ys):
        yp[i] = y.data_ptr()
        ldy[i] = y.stride(0)
    _native.check(
        lib.pl_lora_decode_stacked(
            dt, x.data_ptr(), x.stride(0), K, cache.arena.data_ptr(), cache.table.data_ptr(), len(cache.module_index),
            n, mods, ptrs, plan.tok.data_ptr(), plan.groups.data_ptr(), plan.meta.data_ptr(), cap, plan.group_tokens,
            min(b.numel() for b in bufs), ldt, rows, splits, yp, ldy, nn_, epilogue, counters.data_ptr(),
            counters.numel(), DECODE_SPIN_LIMIT, stream,
        ),
        "pl_lora_decode_stacked",
    )
    return ys


def lora_apply_rows(
    x: torch.Tensor,
    y: torch.Tensor,
    cache,
    module_name: str,
    row_slot: torch.Tensor,
    seq_lens: torch.Tensor,
    row_len: int,
    *,
    epilogue: int = _native.PL_EPI_FALLBACK,
) -> torch.Tensor:
    """Row-based HIP kernels on the slot arena: any K, N, stride or alignment."""
    _require_gpu(x, "lora_apply_rows")
    _check_operands(x, y, cache, module_name, int(row_slot.numel()) * int(row_len))
    if int(seq_lens.numel()) != int(row_slot.numel()):
        raise ValueError("row_slot and seq_lens must have the same length")
    lib = _native.load()
    if x.stride(-1) != 1:
        x = x.contiguous()
    y_work = y if y.stride(-1) == 1 else y.contiguous()
    rows = int(row_slot.numel())
    T = rows * int(row_len)
    ldt = max(1, cache.config.max_rank)
    tmp = torch.empty(max(1, T * ldt), dtype=torch.float32, device=x.device)
    row_slot = _i32(row_slot)
    seq_lens = _i32(seq_lens)
    _native.check(
        lib.pl_lora_apply_rows(
            _native.dtype_code(x.dtype),
            x.data_ptr(),
            x.stride(0),
            int(x.shape[1]),
            y_work.data_ptr(),
            y_work.stride(0),
            int(y_work.shape[1]),
            cache.arena.data_ptr(),
            cache.table.data_ptr(),
            cache.num_slots,
            len(cache.module_index),
            cache.module_index[module_name],
            row_slot.data_ptr(),
            seq_lens.data_ptr(),
            rows,
            int(row_len),
            tmp.data_ptr(),
            ldt,
            epilogue,
            _stream(x.device),
        ),
        "pl_lora_apply_rows",
    )
    if y_work is not y:
        y.copy_(y_work)
    return y


def _check_row_meta(B: int, num_adapters: int, seq_lens, weight_indices, lora_ranks, scalings=None,
                    device_index: int | None = None) -> None:
    """Per-row and per-adapter vectors must cover every row and adapter the kernels index, on the GPU of
    index `device_index` (compared as integers: no device objects on the per-call path)."""
    if device_index is not None:
        for name, t in (("seq_lens", seq_lens), ("weight_indices", weight_indices), ("lora_ranks", lora_ranks),
                        ("scalings", scalings)):
            if t is not None and t.get_device() != device_index:
                raise ValueError(f"{name} is on {t.device}; the kernels read it on cuda:{device_index}")
    if int(seq_lens.numel()) != B or int(weight_indices.numel()) != B:
        raise ValueError(f"seq_lens / weight_indices must have {B} entries")
    if int(lora_ranks.numel()) < num_adapters or (scalings is not None and int(scalings.numel()) < num_adapters):
        raise ValueError(f"lora_ranks / scalings must have an entry for each of the {num_adapters} adapters")


_REF_SIZES: dict = {}


def _ref_parts(lib, dt: int, stream: int, x: torch.Tensor, which: int, B: int, M: int, K: int, n: int,
               weights: torch.Tensor, seq_lens: torch.Tensor, weight_indices: torch.Tensor, lora_ranks: torch.Tensor,
               scalings: torch.Tensor | None, stack_num: int):
    """The parts of the operator API's MFMA path for this call, as the
    pl_sgmv_lora_*_ref_parts arguments (plan, plan bytes, weights, weights
    bytes, scratch, scratch bytes, flags, epoch) plus the tensors that must
    stay alive until the launch is enqueued, or None when that path does not
    take the shape (the row kernels then run).

    The plan and weights parts come from refop_cache (kept across calls,
    rebuilt when the tensors they depend on change) and the scratch is the
    stream's reused buffer, except while a HIP graph is being captured, when
    every part is taken for this call only.  Parts taken for one call come
    from torch's caching allocator, which hands a block to later work on the
    same stream only after this call's kernels.
    """
    num_adapters = int(weights.shape[0])
    skey = (dt, which, B, M, K, n, num_adapters)
    sizes = _REF_SIZES.get(skey)
    if sizes is None:
        sizes = tuple(int(lib.pl_sgmv_ref_part_bytes(dt, which, B, M, K, n, num_adapters, p)) for p in range(3))
        _REF_SIZES[skey] = sizes
    plan_bytes, weights_bytes, scratch_bytes = sizes
    if plan_bytes <= 0:
        return None
    device = x.device
    scratch, scratch_ptr = None, 0
    if torch._C._cuda_isCurrentStreamCapturing():  # torch.cuda.is_current_stream_capturing without its wrapper
        plan = refop_cache._aligned_buffer(plan_bytes, device)
        wpart = refop_cache._aligned_buffer(weights_bytes, device)
        plan_ptr, w_ptr = plan.data_ptr(), wpart.data_ptr()
        if scratch_bytes:
            scratch = refop_cache._aligned_buffer(scratch_bytes, device)
            scratch_ptr = scratch.data_ptr()
        flags, epoch = _native.PL_REF_BUILD_PLAN | _native.PL_REF_PACK_USED, 0
    else:
        if scratch_bytes:
            scratch_ptr = refop_cache.CACHE.scratch(device, stream, scratch_bytes)
        plan, plan_ptr, build = refop_cache.CACHE.plan(device, stream, B, M, num_adapters, seq_lens, weight_indices,
                                                       plan_bytes)
        wpart, w_ptr, flags, epoch = refop_cache.CACHE.weights_part(
            device, stream, which, weights, lora_ranks, scalings, stack_num, (K, n), weights_bytes,
            refop_cache.marks_bytes(num_adapters))
        if build:
            flags |= _native.PL_REF_BUILD_PLAN
    keep = (plan, wpart, scratch)
    return (plan_ptr, plan_bytes, w_ptr, weights_bytes, scratch_ptr, scratch_bytes, flags, epoch), keep


def sgmv_lora_a_fwd(
    x: torch.Tensor,  # (B, M, K)
    weights: torch.Tensor,  # (num_adapters, K, N_max)
    seq_lens: torch.Tensor,  # (B,)
    weight_indices: torch.Tensor,  # (B,)
    lora_ranks: torch.Tensor,  # (num_adapters,)
    stack_num: int = 1,
) -> torch.Tensor:
    """Shrink with the reference signature: out[b, m, n] = x[b, m] @ weights[w_b][:, n].

    Rows m >= seq_lens[b] and columns n >= ranks[w_b] * stack_num are left
    unwritten, like the reference's ``torch.empty`` output.
    """
    assert x.is_contiguous() and weights.is_contiguous()
    assert x.dim() == 3 and weights.dim() == 3
    B, M, K = x.shape
    _, Kw, N_max = weights.shape
    assert Kw == K, f"K mismatch: x={K}, weights={Kw}"
    output = x.new_empty((B, M, N_max))
    if B == 0 or M == 0 or N_max == 0:
        return output
    _require_gpu(x, "sgmv_lora_a_fwd")
    if weights.dtype != x.dtype:
        raise TypeError(f"weights dtype {weights.dtype} must match x dtype {x.dtype}")
    seq_lens_in, weight_indices_in, lora_ranks_in = seq_lens, weight_indices, lora_ranks
    seq_lens, weight_indices, lora_ranks = _i32(seq_lens), _i32(weight_indices), _i32(lora_ranks)
    dev = x.get_device()
    if weights.get_device() != dev:
        raise ValueError(f"weights are on {weights.device}, x on {x.device}")
    _check_row_meta(B, weights.shape[0], seq_lens, weight_indices, lora_ranks, device_index=dev)
    lib = _native.load()
    dt, stream, stack_num = _native.dtype_code(x.dtype), torch._C._cuda_getCurrentRawStream(dev), int(stack_num)
    head = (dt, x.data_ptr(), B, M, K, weights.data_ptr(), *weights.stride(), int(weights.shape[0]), N_max,
            seq_lens.data_ptr(), weight_indices.data_ptr(), lora_ranks.data_ptr(), stack_num, output.data_ptr())
    parts = _ref_parts(lib, dt, stream, x, 0, B, M, K, N_max, weights, seq_lens_in, weight_indices_in, lora_ranks_in,
                       None, stack_num)
    if parts is None:
        _native.check(lib.pl_sgmv_lora_a_ref(*head, 0, 0, stream), "pl_sgmv_lora_a_ref")
    else:
        _native.check(lib.pl_sgmv_lora_a_ref_parts(*head, *parts[0], stream), "pl_sgmv_lora_a_ref_parts")
    return output


def sgmv_lora_b_fwd(
    x: torch.Tensor,  # (B, M, K_max)
    weights: torch.Tensor,  # (num_adapters, K_max, N)
    seq_lens: torch.Tensor,  # (B,)
    weight_indices: torch.Tensor,  # (B,)
    lora_ranks: torch.Tensor,  # (num_adapters,)
    scalings: torch.Tensor,  # (num_adapters,) fp32
    base_output: torch.Tensor | None = None,  # (B, M, N) fused add target
) -> torch.Tensor:
    """Expand with the reference signature and fused add-back (sgmv.py:278-328)."""
    assert x.is_contiguous() and weights.is_contiguous()
    assert x.dim() == 3 and weights.dim() == 3
    B, M, K_max = x.shape
    _, Kw, N = weights.shape
    assert Kw == K_max, f"K mismatch: x={K_max}, weights={Kw}"
    if base_output is None:
        output = torch.zeros((B, M, N), device=x.device, dtype=x.dtype)
    else:
        assert base_output.shape == (B, M, N)
        output = base_output
    if B == 0 or M == 0 or N == 0:
        return output
    _require_gpu(x, "sgmv_lora_b_fwd")
    if weights.dtype != x.dtype or output.dtype != x.dtype:
        raise TypeError("x, weights and base_output must share one dtype")
    work = output if output.is_contiguous() else output.contiguous()
    seq_lens_in, weight_indices_in, lora_ranks_in, scalings_in = seq_lens, weight_indices, lora_ranks, scalings
    seq_lens, weight_indices, lora_ranks = _i32(seq_lens), _i32(weight_indices), _i32(lora_ranks)
    if not (scalings.dtype is torch.float32 and scalings.is_contiguous()):
        scalings = scalings.to(torch.float32).contiguous()
    dev = x.get_device()
    if weights.get_device() != dev or output.get_device() != dev:
        raise ValueError("x, weights and base_output must be on one device")
    _check_row_meta(B, weights.shape[0], seq_lens, weight_indices, lora_ranks, scalings, device_index=dev)
    lib = _native.load()
    dt, stream = _native.dtype_code(x.dtype), torch._C._cuda_getCurrentRawStream(dev)
    head = (dt, x.data_ptr(), B, M, K_max, weights.data_ptr(), *weights.stride(), int(weights.shape[0]), N,
            seq_lens.data_ptr(), weight_indices.data_ptr(), lora_ranks.data_ptr(), scalings.data_ptr(),
            work.data_ptr())
    parts = _ref_parts(lib, dt, stream, x, 1, B, M, K_max, N, weights, seq_lens_in, weight_indices_in, lora_ranks_in,
                       scalings_in, 1)
    if parts is None:
        _native.check(lib.pl_sgmv_lora_b_ref(*head, 0, 0, stream), "pl_sgmv_lora_b_ref")
    else:
        _native.check(lib.pl_sgmv_lora_b_ref_parts(*head, *parts[0], stream), "pl_sgmv_lora_b_ref_parts")
    if work is not output:
        output.copy_(work)
    return output
