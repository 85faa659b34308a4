"""ctypes binding of ``libpolylora_hip.so`` (declared in ``include/polylora_hip.h``).

The library is the only compute path of this package: when it is missing
every LoRA entry point raises instead of computing anything on the CPU.
torch is imported first so that the library binds to torch's HIP runtime.
"""

from __future__ import annotations

import ctypes
from ctypes import c_int32, c_int64, c_void_p
from pathlib import Path

import torch  # noqa: F401  (loads the HIP runtime the library must share)

LIB_PATH = Path(__file__).resolve().parent / "_lib" / "libpolylora_hip.so"

PL_F32, PL_BF16, PL_F16 = 0, 1, 2
PL_OK, PL_ERR_ARG, PL_ERR_ALIGN, PL_ERR_LAUNCH, PL_ERR_LIMIT = 0, 1, 2, 3, 4
PL_EPI_FALLBACK, PL_EPI_TRITON = 0, 1
PL_MAX_SLOTS = 4096
PL_GROUP_TOKENS_SHORT, PL_GROUP_TOKENS_LONG = 16, 64
PL_MAX_STACKED_MODULES = 4
PL_NOALLOC_SCRATCH_BYTES = 32 << 20
PL_REF_PART_PLAN, PL_REF_PART_WEIGHTS, PL_REF_PART_SCRATCH = 0, 1, 2
PL_REF_BUILD_PLAN, PL_REF_PACK_USED, PL_REF_PACK_ALL, PL_REF_KEEP_PACKED = 1, 2, 4, 8
SLOT_ENTRY_INT32S = 8  # sizeof(pl_slot_entry) / 4

DTYPE_CODES = {torch.float32: PL_F32, torch.bfloat16: PL_BF16, torch.float16: PL_F16}
MASK_DTYPE_CODES = {
    torch.int64: 0,
    torch.int32: 1,
    torch.uint8: 2,
    torch.bool: 2,
    torch.float32: 3,
    torch.bfloat16: 4,
    torch.float16: 5,
}

# name -> argument types; every function returns int32 unless listed in _RESTYPES
_SIGNATURES: dict[str, tuple] = {
    "pl_version": (),
    "pl_last_error": (),
    "pl_is_device_pointer": (c_void_p,),
    "pl_plan_group_capacity": (c_int32, c_int32, c_int32, c_int32),
    "pl_plan_build": (c_void_p, c_void_p, c_int32, c_int32, c_int32, c_int32, c_void_p, c_void_p, c_void_p, c_int64, c_void_p),
    "pl_plan_build_active": (c_void_p, c_void_p, c_int32, c_int32, c_int32, c_void_p, c_int64, c_int32, c_void_p,
                             c_void_p, c_void_p, c_int64, c_void_p),
    "pl_shrink_planes": (c_int32, c_int32, c_int32, c_int32),
    "pl_shrink_workspace_bytes": (c_int32, c_int32, c_int32, c_int32, c_int64, c_int32),
    "pl_sgmv_shrink": (
        c_int32, c_void_p, c_int64, c_int32, c_void_p, c_void_p, c_int32, c_int32, c_void_p, c_void_p,
        c_void_p, c_int64, c_int32, c_void_p, c_int64, c_int32, c_int64, c_int32, c_void_p,
    ),
    "pl_sgmv_shrink_stacked": (
        c_int32, c_void_p, c_int64, c_int32, c_void_p, c_void_p, c_int32, c_int32, c_void_p, c_void_p,
        c_void_p, c_void_p, c_void_p, c_int64, c_int32, c_int64, c_int32, c_int64, c_int32, c_void_p,
    ),
    "pl_sgmv_expand": (
        c_int32, c_void_p, c_int32, c_int64, c_int32, c_void_p, c_void_p, c_int32, c_int32, c_void_p,
        c_void_p, c_void_p, c_int64, c_int32, c_void_p, c_int64, c_int32, c_int32, c_void_p,
    ),
    "pl_sgmv_expand_stacked": (
        c_int32, c_void_p, c_int32, c_int64, c_int32, c_void_p, c_void_p, c_int32, c_int32, c_void_p,
        c_void_p, c_void_p, c_void_p, c_int64, c_int32, c_void_p, c_void_p, c_void_p, c_int32, c_void_p,
    ),
    "pl_lora_decode_stacked": (
        c_int32, c_void_p, c_int64, c_int32, c_void_p, c_void_p, c_int32, c_int32, c_void_p, c_void_p,
        c_void_p, c_void_p, c_void_p, c_int64, c_int32, c_int64, c_int32, c_int64, c_int32, c_void_p,
        c_void_p, c_void_p, c_int32, c_void_p, c_int64, c_int32, c_void_p,
    ),
    "pl_decode_counter_ints": (c_int64, c_int32),
    "pl_lora_apply": (
        c_int32, c_void_p, c_int64, c_int32, c_void_p, c_int64, c_int32, c_void_p, c_void_p, c_int32,
        c_int32, c_void_p, c_void_p, c_void_p, c_int64, c_int32, c_void_p, c_int64, c_int32, c_int64,
        c_int32, c_int32, c_void_p,
    ),
    "pl_lora_fused": (
        c_int32, c_void_p, c_int64, c_int32, c_void_p, c_int64, c_int32, c_void_p, c_void_p, c_int32,
        c_int32, c_int32, c_void_p, c_void_p, c_void_p, c_int64, c_int32, c_int32, c_int32, c_void_p,
    ),
    "pl_lora_fused_stacked": (
        c_int32, c_void_p, c_int64, c_int32, c_int32, c_void_p, c_void_p, c_void_p, c_void_p, c_void_p,
        c_void_p, c_int32, c_int32, c_void_p, c_void_p, c_void_p, c_int64, c_int32, c_int32, c_int32,
        c_void_p,
    ),
    "pl_lora_apply_rows": (
        c_int32, c_void_p, c_int64, c_int32, c_void_p, c_int64, c_int32, c_void_p, c_void_p, c_int32,
        c_int32, c_int32, c_void_p, c_void_p, c_int32, c_int32, c_void_p, c_int32, c_int32, c_void_p,
    ),
    "pl_sgmv_ref_workspace_bytes": (c_int32, c_int32, c_int32, c_int32, c_int32, c_int32, c_int32),
    "pl_sgmv_lora_a_ref": (
        c_int32, c_void_p, c_int32, c_int32, c_int32, c_void_p, c_int64, c_int64, c_int64, c_int32,
        c_int32, c_void_p, c_void_p, c_void_p, c_int32, c_void_p, c_void_p, c_int64, c_void_p,
    ),
    "pl_sgmv_lora_b_ref": (
        c_int32, c_void_p, c_int32, c_int32, c_int32, c_void_p, c_int64, c_int64, c_int64, c_int32,
        c_int32, c_void_p, c_void_p, c_void_p, c_void_p, c_void_p, c_void_p, c_int64, c_void_p,
    ),
    "pl_sgmv_ref_part_bytes": (c_int32, c_int32, c_int32, c_int32, c_int32, c_int32, c_int32, c_int32),
    "pl_sgmv_lora_a_ref_parts": (
        c_int32, c_void_p, c_int32, c_int32, c_int32, c_void_p, c_int64, c_int64, c_int64, c_int32,
        c_int32, c_void_p, c_void_p, c_void_p, c_int32, c_void_p, c_void_p, c_int64, c_void_p, c_int64,
        c_void_p, c_int64, c_int32, c_int32, c_void_p,
    ),
    "pl_sgmv_lora_b_ref_parts": (
        c_int32, c_void_p, c_int32, c_int32, c_int32, c_void_p, c_int64, c_int64, c_int64, c_int32,
        c_int32, c_void_p, c_void_p, c_void_p, c_void_p, c_void_p, c_void_p, c_int64, c_void_p, c_int64,
        c_void_p, c_int64, c_int32, c_int32, c_void_p,
    ),
    "pl_lora_apply_noalloc": (
        c_int32, c_void_p, c_int64, c_int32, c_void_p, c_int64, c_int32, c_void_p, c_void_p, c_int32,
        c_int32, c_void_p, c_void_p, c_int32, c_int32, c_int32, c_int32, c_int32, c_int32, c_int32, c_void_p,
    ),
    "pl_host_copy_async": (c_void_p, c_void_p, c_int64, c_void_p),
    "pl_host_alloc": (c_int64,),
    "pl_host_free": (c_void_p,),
    "pl_slot_upload": (c_void_p, c_void_p, c_int64, c_void_p, c_void_p, c_int64, c_void_p),
    "pl_check_right_padded": (c_void_p, c_int32, c_int32, c_int32, c_void_p, c_void_p, c_void_p),
}
_RESTYPES = {"pl_last_error": ctypes.c_char_p, "pl_plan_group_capacity": c_int64, "pl_shrink_workspace_bytes": c_int64,
             "pl_host_alloc": c_void_p, "pl_sgmv_ref_workspace_bytes": c_int64, "pl_decode_counter_ints": c_int64,
             "pl_sgmv_ref_part_bytes": c_int64}

EXPORTED_SYMBOLS = tuple(_SIGNATURES)

_lib = None
_checked_runtime = False


_raw: dict = {}


def raw(name: str):
    """Entry point `name` without ctypes argument conversion.

    Every argument must already be a ctypes object of the declared type
    (c_int32, c_int64, c_void_p); arguments that do not change between calls
    can then be built once and passed as they are, which saves the per-call
    conversion of the declared-argtypes binding.  Returns int32.
    """
    f = _raw.get(name)
    if f is None:
        f = load()[name]  # a separate function object with no argtypes
        f.restype = c_int32
        _raw[name] = f
    return f


_c32: dict = {}


def c32(v: int) -> ctypes.c_int32:
    """A shared c_int32 for a small constant argument (dtype codes, flags, counts)."""
    got = _c32.get(v)
    if got is None:
        got = _c32[v] = c_int32(v)
    return got


class NativeLibraryMissing(RuntimeError):
    """The HIP library has not been built (run ``python -m polylora_amd.build``)."""


def load() -> ctypes.CDLL:
    """Load the library once and attach argument types."""
    global _lib
    if _lib is not None:
        return _lib
    if not LIB_PATH.exists():
        raise NativeLibraryMissing(
            f"polylora_amd HIP library not found at {LIB_PATH}; build it with "
            "`python -m polylora_amd.build` (the LoRA path has no CPU fallback)"
        )
    lib = ctypes.CDLL(str(LIB_PATH))
    for name, argtypes in _SIGNATURES.items():
        fn = getattr(lib, name)
        fn.argtypes = list(argtypes)
        fn.restype = _RESTYPES.get(name, c_int32)
    _lib = lib
    return lib


def check(status: int, what: str) -> None:
    if status != 0:
        msg = load().pl_last_error().decode("utf-8", "replace")
        raise RuntimeError(f"{what} failed (status {status}): {msg}")


def check_runtime(tensor: torch.Tensor) -> None:
    """Verify once that a torch device pointer is a device pointer to the library."""
    global _checked_runtime
    if _checked_runtime:
        return
    res = load().pl_is_device_pointer(tensor.data_ptr())
    if res != 1:
        msg = load().pl_last_error().decode("utf-8", "replace")
        raise RuntimeError(
            "polylora_amd HIP library does not see torch's device memory "
            f"(pl_is_device_pointer={res}: {msg}); two HIP runtimes are loaded"
        )
    _checked_runtime = True


def dtype_code(dtype: torch.dtype) -> int:
    try:
        return DTYPE_CODES[dtype]
    except KeyError:
        raise TypeError(f"polylora_amd kernels support float32, bfloat16 and float16, not {dtype}") from None


def current_stream_handle(device: torch.device) -> int:
    idx = device.index if device.index is not None else torch.cuda.current_device()
    return torch._C._cuda_getCurrentRawStream(idx)
