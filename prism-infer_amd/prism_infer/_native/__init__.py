"""ctypes binding of libprism_mi355x.so (declared in include/prism_kv.h).

The library is loaded lazily on first use.  torch is imported first so that
the library binds to the HIP runtime torch already holds (it is linked
against torch/lib/libamdhip64.so).  A missing or unloadable library raises
``RuntimeError``: there is no fallback implementation.
"""

from __future__ import annotations

import ctypes
from pathlib import Path

import torch

LIB_NAME = "libprism_mi355x.so"
LIB_PATH = Path(__file__).resolve().parent / LIB_NAME

DTYPE_F32 = 0
DTYPE_BF16 = 1
DTYPE_F16 = 2
DTYPE_FP8_E4M3FN = 3

_TORCH_TO_CODE = {
    torch.float32: DTYPE_F32,
    torch.bfloat16: DTYPE_BF16,
    torch.float16: DTYPE_F16,
}
if hasattr(torch, "float8_e4m3fn"):
    _TORCH_TO_CODE[torch.float8_e4m3fn] = DTYPE_FP8_E4M3FN

# Every symbol include/prism_kv.h declares, with (restype, argtypes).
_I64P = ctypes.POINTER(ctypes.c_int64)
_VP = ctypes.c_void_p
_I = ctypes.c_int
_I64 = ctypes.c_int64
_F = ctypes.c_float
SIGNATURES: dict[str, tuple] = {
    "prism_abi_version": (_I, []),
    "prism_last_error": (ctypes.c_char_p, []),
    "prism_device_cu_count": (_I, []),
    "prism_preload": (_I, []),
    "prism_kv_store": (
        _I,
        [_VP, _VP, _I, _I64P, _I64P, _VP, _VP, _I, _VP, _VP, _VP, _I64, _I, _I, _I64, _VP],
    ),
    "prism_paged_decode_workspace_bytes": (_I64, [_I, _I, _I, _I, _I, _I, _I]),
    "prism_paged_decode_split_tokens": (_I, [_I, _I, _I, _I, _I, _I, _I]),
    "prism_paged_decode_kernel_family": (_I, [_I, _I, _I, _I, _I, _I, _I]),
    "prism_paged_decode_set_overrides": (_I, [_I, _I, _I]),
    "prism_paged_decode_get_overrides": (None, [ctypes.POINTER(ctypes.c_int)]),
    "prism_paged_decode_set_plan_wait_limit": (_I, [_I]),
    "prism_paged_decode_default_plan_wait_limit": (_I, []),
    "prism_paged_decode": (
        _I,
        [_VP, _I, _I64P, _VP, _VP, _I, _I64P, _I64P, _VP, _VP, _I64P, _I64P, _VP, _I64P, _VP, _VP, _VP,
         _I64P, _I, _I, _I, _I, _I, _I64, _I, _F, _VP, _I64, _VP],
    ),
    "prism_paged_decode_noalloc": (
        _I,
        [_VP, _I, _I64P, _VP, _VP, _I, _I64P, _I64P, _VP, _VP, _I64P, _I64P, _VP, _I64P, _VP, _VP, _VP,
         _I64P, _I, _I, _I, _I, _I, _I64, _I, _F, _VP],
    ),
    "prism_paged_decode_stage": (
        _I,
        [_I, _VP, _I, _I64P, _VP, _VP, _I, _I64P, _I64P, _VP, _VP, _I64P, _I64P, _VP, _I64P, _VP, _VP, _VP,
         _I64P, _I, _I, _I, _I, _I, _I64, _I, _F, _VP, _I64, _VP],
    ),
    "prism_compact_slots_workspace_bytes": (_I64, [_I64, _I64, _I64, _I64]),
    "prism_compact_slots": (_I, [_VP, _I64, _I64, _I64, _VP, _VP, _I64, _VP, _I64, _VP]),
    "prism_copy_blocks": (_I, [_VP, _VP, _I64, _I64, _I64, _I64, _I64, _I64, _I64P, _I64P, _I64, _VP]),
    "prism_device_copy": (_I, [_VP, _VP, _I64, _I, _VP]),
    "prism_paged_prefill": (
        _I,
        [_VP, _I, _I64P, _VP, _VP, _I, _I64P, _I64P, _VP, _VP, _I64P, _I64P, _VP, _I64P, _VP, _VP, _VP,
         _I64P, _I, _I, _I, _I, _I, _I, _I, _I, _F, _VP, _VP],
    ),
    "prism_debug_fp8_encode": (_I, [_VP, _VP, _I64, _VP]),
}

ABI_VERSION = 2

_LIB: ctypes.CDLL | None = None


def library_path() -> Path:
    return LIB_PATH


def is_built() -> bool:
    return LIB_PATH.exists()


def lib() -> ctypes.CDLL:
    """Load (once) and return the native library, or raise RuntimeError."""

    global _LIB
    if _LIB is not None:
        return _LIB
    if not LIB_PATH.exists():
        raise RuntimeError(
            f"{LIB_NAME} is not built ({LIB_PATH}); run `python prism-infer_amd/build_native.py` "
            "or __graft_entry__.build() -- the KV ops have no non-HIP fallback"
        )
    try:
        handle = ctypes.CDLL(str(LIB_PATH))
    except OSError as exc:
        raise RuntimeError(f"cannot load {LIB_PATH}: {exc}") from exc
    for name, (restype, argtypes) in SIGNATURES.items():
        fn = getattr(handle, name)
        fn.restype = restype
        fn.argtypes = argtypes
    version = handle.prism_abi_version()
    if version != ABI_VERSION:
        raise RuntimeError(f"{LIB_NAME} ABI version {version} != expected {ABI_VERSION}; rebuild it")
    _LIB = handle
    return handle


_PRELOADED: set[int] = set()


def device_lib(device: torch.device | None = None) -> ctypes.CDLL:
    """The library, with every kernel's code object loaded on ``device``.

    HIP otherwise loads a code object at its kernel's first launch, which
    stalls that call (28 ms for the decode kernels) and slows the launches
    right after it.  The GPU ops call this before their first launch on a
    device; the load runs once per device, and a failure raises here.
    """

    handle = lib()
    index = torch.cuda.current_device() if device is None or device.index is None else device.index
    if index in _PRELOADED:
        return handle
    with torch.cuda.device(index):
        status = handle.prism_preload()
    if status != 0:
        raise RuntimeError(f"prism_preload failed ({status}): {handle.prism_last_error().decode(errors='replace')}")
    _PRELOADED.add(index)
    return handle


def available() -> bool:
    """True when the library file exists and loads (no GPU work is done)."""

    try:
        lib()
    except RuntimeError:
        return False
    return True


def dtype_code(dtype: torch.dtype) -> int:
    try:
        return _TORCH_TO_CODE[dtype]
    except KeyError:
        raise ValueError(f"dtype {dtype} is not supported by the MI355X KV kernels") from None


def strides(tensor: torch.Tensor) -> ctypes.Array:
    values = tensor.stride()
    return (ctypes.c_int64 * len(values))(*values)


def int64s(*values: int) -> ctypes.Array:
    return (ctypes.c_int64 * len(values))(*values)


def stream_handle(device: torch.device) -> int:
    return torch.cuda.current_stream(device).cuda_stream


def check(status: int, what: str) -> None:
    """Raise for a non-zero status: ValueError for contract errors, RuntimeError otherwise."""

    if status == 0:
        return
    message = lib().prism_last_error().decode("utf-8", "replace")
    if status == -1:
        raise ValueError(f"{what}: {message}")
    raise RuntimeError(f"{what}: {message}")


__all__ = [
    "ABI_VERSION",
    "DTYPE_BF16",
    "DTYPE_F16",
    "DTYPE_F32",
    "DTYPE_FP8_E4M3FN",
    "LIB_NAME",
    "LIB_PATH",
    "SIGNATURES",
    "available",
    "check",
    "device_lib",
    "dtype_code",
    "int64s",
    "is_built",
    "lib",
    "library_path",
    "stream_handle",
    "strides",
]
