"""Paged decode attention on MI355X (hand-written gfx950 HIP kernels).

Drop-in for prism_infer/ops/paged_decode.py: same ``paged_decode_attention``
signature (:443-455), same validation order and messages (:187-372), same
kernel semantics (:83-180):

- q: [batch, num_heads, head_dim]; k_cache/v_cache: [num_blocks, block_size,
  num_kv_heads, head_dim]; optional per-token/per-head fp32 scales
  [num_blocks, block_size, num_kv_heads];
- block_tables: int32 [>= batch, max_blocks]; block ids < 0 are skipped;
- context_lens: int32 [>= batch]; max_context_len: int32 scalar tensor read on
  the device (graph replay follows updated values).  When it is omitted the
  reference derives ``context_lens.max()``, a bound no sequence's own length
  exceeds, so it clips nothing; a cached "no bound" scalar (2^31 - 1) gives
  the same attended tokens without the reduction launch;
- a sequence with no attended token returns zeros.

``block_n`` is validated as in the reference (positive power of two) but the
HIP kernel's tiling is its own (32-token MFMA tiles, split-K over long
contexts), so the value does not change results.  Split-K scratch is
allocated here from static shapes through torch's caching allocator.
"""

from __future__ import annotations

import torch

from prism_infer import _native

HAS_HIP_KERNELS = _native.available()
HAS_TRITON = HAS_HIP_KERNELS  # the reference's "kernel available" flag name

QUERY_TENSOR_RANK = 3
PAGED_KV_CACHE_RANK = 4
BLOCK_TABLE_TENSOR_RANK = 2
CONTEXT_LENGTH_VECTOR_RANK = 1
DEFAULT_PAGED_DECODE_BLOCK_N = 32
MAX_PAGED_DECODE_HEAD_DIM = 256


def _next_power_of_2(value: int) -> int:
    return 1 << (value - 1).bit_length()


def _validate_paged_decode_inputs(q, k_cache, v_cache, block_tables, context_lens, max_context_len, *,
                                  k_scale_cache=None, v_scale_cache=None,
                                  block_n: int = DEFAULT_PAGED_DECODE_BLOCK_N) -> bool:
    """Validate the public paged-decode contract; returns whether scales are used."""

    # contract (ValueError) first, then where the tensors live (RuntimeError)
    scaled_kv = _validate_paged_scale_pair(k_scale_cache, v_scale_cache)
    _validate_paged_query_cache_contract(q, k_cache, v_cache)
    _validate_paged_cache_dtypes(q, k_cache)
    if scaled_kv:
        _validate_paged_scale_cache(k_cache, k_scale_cache, v_scale_cache)
    _validate_paged_metadata(block_tables, context_lens, max_context_len)
    _validate_paged_geometry(q, k_cache, block_tables, context_lens, block_n)
    _validate_paged_decode_runtime(q)
    _validate_paged_device_tensors(q, k_cache, v_cache, block_tables, context_lens, max_context_len,
                                   k_scale_cache, v_scale_cache)
    return scaled_kv


def _validate_paged_decode_runtime(q: torch.Tensor) -> None:
    if not HAS_HIP_KERNELS:
        _native.lib()  # raises with the reason the library is unavailable
    if not q.is_cuda:
        raise RuntimeError("paged_decode_attention requires GPU tensors (there is no CPU fallback)")


def _validate_paged_scale_pair(k_scale_cache, v_scale_cache) -> bool:
    if (k_scale_cache is None) != (v_scale_cache is None):
        raise ValueError("K/V scale caches must be provided together")
    return k_scale_cache is not None


def _validate_paged_device_tensors(q, k_cache, v_cache, block_tables, context_lens, max_context_len,
                                   k_scale_cache, v_scale_cache) -> None:
    tensors = (q, k_cache, v_cache, block_tables, context_lens, max_context_len,
               *(t for t in (k_scale_cache, v_scale_cache) if t is not None))
    if not all(t.is_cuda for t in tensors):
        raise RuntimeError("paged_decode_attention requires all tensors on the GPU")
    if any(t.device != q.device for t in tensors[1:]):
        raise RuntimeError("paged_decode_attention requires all tensors on one device")


def _validate_paged_query_cache_contract(q, k_cache, v_cache) -> None:
    if q.ndim != QUERY_TENSOR_RANK:
        raise ValueError(f"q must be [batch, num_heads, head_dim], got {list(q.shape)}")
    if k_cache.ndim != PAGED_KV_CACHE_RANK or v_cache.ndim != PAGED_KV_CACHE_RANK:
        raise ValueError(
            "k_cache/v_cache must be [num_blocks, block_size, num_kv_heads, head_dim], "
            f"got {list(k_cache.shape)} and {list(v_cache.shape)}"
        )
    if k_cache.shape != v_cache.shape:
        raise ValueError(f"k_cache and v_cache shapes differ: {list(k_cache.shape)} vs {list(v_cache.shape)}")
    if k_cache.dtype != v_cache.dtype:
        raise ValueError(f"k_cache/v_cache dtype mismatch: {k_cache.dtype} vs {v_cache.dtype}")


def _validate_paged_cache_dtypes(q, k_cache) -> None:
    supported_query_dtypes = {torch.float16, torch.bfloat16, torch.float32}
    if q.dtype not in supported_query_dtypes:
        raise ValueError(f"unsupported paged decode query dtype: {q.dtype}")
    supported_cache_dtypes = set(supported_query_dtypes)
    if hasattr(torch, "float8_e4m3fn"):
        supported_cache_dtypes.add(torch.float8_e4m3fn)
    if k_cache.dtype not in supported_cache_dtypes:
        raise ValueError(f"unsupported paged decode cache dtype: {k_cache.dtype}")


def _validate_paged_scale_cache(k_cache, k_scale_cache, v_scale_cache) -> None:
    fp8_dtype = getattr(torch, "float8_e4m3fn", None)
    if fp8_dtype is None or k_cache.dtype != fp8_dtype:
        raise ValueError("token-head scales require FP8 E4M3FN K/V payload caches")
    expected = tuple(k_cache.shape[:-1])
    if k_scale_cache.shape != v_scale_cache.shape or tuple(k_scale_cache.shape) != expected:
        raise ValueError(
            "K/V scale cache shape must equal payload shape without head_dim: "
            f"expected={list(expected)}"
        )
    if k_scale_cache.dtype != torch.float32 or v_scale_cache.dtype != torch.float32:
        raise ValueError("K/V scale caches must use torch.float32")


def _validate_paged_metadata(block_tables, context_lens, max_context_len) -> None:
    if block_tables.ndim != BLOCK_TABLE_TENSOR_RANK:
        raise ValueError(f"block_tables must be [batch, max_blocks], got {list(block_tables.shape)}")
    if context_lens.ndim != CONTEXT_LENGTH_VECTOR_RANK:
        raise ValueError(f"context_lens must be [batch], got {list(context_lens.shape)}")
    if block_tables.dtype != torch.int32 or context_lens.dtype != torch.int32:
        raise ValueError(
            "block_tables/context_lens must use torch.int32, got "
            f"{block_tables.dtype}/{context_lens.dtype}"
        )
    if max_context_len.numel() != 1 or max_context_len.dtype != torch.int32:
        raise ValueError(
            "max_context_len must be one torch.int32 scalar tensor, got "
            f"shape={list(max_context_len.shape)} dtype={max_context_len.dtype}"
        )


def _validate_paged_geometry(q, k_cache, block_tables, context_lens, block_n) -> None:
    if block_n <= 0 or block_n & (block_n - 1):
        raise ValueError(f"block_n must be a positive power of two, got {block_n}")
    batch, num_heads, head_dim = q.shape
    _, page_block_size, num_kv_heads, cache_head_dim = k_cache.shape
    if page_block_size <= 0:
        raise ValueError("paged decode cache block size must be positive")
    if cache_head_dim != head_dim:
        raise ValueError(f"head_dim mismatch: q={head_dim}, cache={cache_head_dim}")
    if num_kv_heads <= 0:
        raise ValueError("paged decode cache must contain at least one KV head")
    if num_heads % num_kv_heads != 0:
        raise ValueError(f"num_heads must be divisible by num_kv_heads, got {num_heads} and {num_kv_heads}")
    if block_tables.shape[0] < batch or context_lens.shape[0] < batch:
        raise ValueError(
            "block_tables/context_lens batch must cover q batch, "
            f"got q={batch}, block_tables={block_tables.shape[0]}, context_lens={context_lens.shape[0]}"
        )
    if _next_power_of_2(head_dim) > MAX_PAGED_DECODE_HEAD_DIM:
        raise ValueError(f"paged_decode_attention supports head_dim <= {MAX_PAGED_DECODE_HEAD_DIM}, got {head_dim}")
    if k_cache.stride(-1) != 1:
        raise RuntimeError("paged_decode_attention requires a unit head_dim stride in the K/V caches")


def decode_workspace_bytes(q: torch.Tensor, k_cache: torch.Tensor, block_tables: torch.Tensor) -> int:
    """Split-K scratch bytes for this geometry (depends on static shapes only)."""

    batch, num_heads, head_dim = q.shape
    _, page_size, num_kv_heads, _ = k_cache.shape
    return int(_native.lib().prism_paged_decode_workspace_bytes(
        batch, num_heads, num_kv_heads, head_dim, page_size, block_tables.shape[1],
        _native.dtype_code(k_cache.dtype)))


# One decode workspace per (device, stream), reused across calls: besides the
# split-K partials it holds the streaming kernel's work plan together with
# the inputs the plan was computed from, so consecutive calls with the same
# metadata (every layer of a decode step) skip recomputing it.  Calls on one
# stream are ordered, so they may share it; other streams get their own.
# Under graph capture a fresh buffer from the graph's pool is used instead.
_WORKSPACES: dict[tuple[int, int], torch.Tensor] = {}


def decode_workspace(device: torch.device, nbytes: int) -> torch.Tensor:
    """The reused decode workspace of the current stream (at least ``nbytes``)."""

    if torch.cuda.is_current_stream_capturing():
        return torch.empty(max(nbytes, 1), dtype=torch.uint8, device=device)
    index = device.index if device.index is not None else torch.cuda.current_device()
    key = (index, torch.cuda.current_stream(device).cuda_stream)
    ws = _WORKSPACES.get(key)
    if ws is None or ws.numel() < nbytes:
        ws = torch.empty(max(nbytes, 1), dtype=torch.uint8, device=device)
        _WORKSPACES[key] = ws
    return ws


def _launch_paged_decode_attention(q, k_cache, v_cache, block_tables, context_lens, scale, max_context_len, *,
                                   k_scale_cache, v_scale_cache, scaled_kv, stage: int = 0,
                                   output: torch.Tensor | None = None,
                                   workspace: torch.Tensor | None = None) -> torch.Tensor:
    batch, num_heads, head_dim = q.shape
    num_blocks, page_size, num_kv_heads, _ = k_cache.shape
    lib = _native.device_lib(q.device)
    if output is None:
        output = torch.empty_like(q)
    ws_bytes = decode_workspace_bytes(q, k_cache, block_tables)
    if ws_bytes > 0 and (workspace is None or workspace.numel() < ws_bytes):
        workspace = decode_workspace(q.device, ws_bytes)
    zero3 = _native.int64s(0, 0, 0)
    with torch.cuda.device(q.device):
        status = lib.prism_paged_decode_stage(
            stage,
            q.data_ptr(), _native.dtype_code(q.dtype), _native.strides(q),
            k_cache.data_ptr(), v_cache.data_ptr(), _native.dtype_code(k_cache.dtype),
            _native.strides(k_cache), _native.strides(v_cache),
            k_scale_cache.data_ptr() if scaled_kv else None,
            v_scale_cache.data_ptr() if scaled_kv else None,
            _native.strides(k_scale_cache) if scaled_kv else zero3,
            _native.strides(v_scale_cache) if scaled_kv else zero3,
            block_tables.data_ptr(), _native.strides(block_tables),
            context_lens.data_ptr(), max_context_len.data_ptr(),
            output.data_ptr(), _native.strides(output),
            batch, num_heads, num_kv_heads, head_dim, page_size, num_blocks, block_tables.shape[1],
            float(scale),
            workspace.data_ptr() if ws_bytes > 0 else None, ws_bytes,
            _native.stream_handle(q.device),
        )
    _native.check(status, "paged_decode_attention")
    return output


_NO_BOUND: dict = {}


def _no_context_bound(context_lens: torch.Tensor) -> torch.Tensor:
    """The omitted ``max_context_len``: min(ctx[b], max(context_lens)) is
    ctx[b] for every sequence, so a scalar that bounds nothing attends the
    same tokens as the reference's ``context_lens.max()`` (`paged_decode.py:458-461`)
    and needs no reduction kernel per call.  Cached per device; while a graph
    is being captured and no scalar is cached yet, the reduction is captured
    instead (no allocation from the graph's pool is kept)."""

    if context_lens.numel() == 0:
        return context_lens.max()  # raises torch's error for an empty reduction, as the reference does
    dev = context_lens.device
    cached = _NO_BOUND.get(dev)
    if cached is not None:
        return cached
    if dev.type == "cuda" and torch.cuda.is_current_stream_capturing():
        return context_lens.max()
    cached = torch.full((1,), 2**31 - 1, dtype=torch.int32, device=dev)
    _NO_BOUND[dev] = cached
    return cached


def paged_decode_attention(
    q: torch.Tensor,
    k_cache: torch.Tensor,
    v_cache: torch.Tensor,
    block_tables: torch.Tensor,
    context_lens: torch.Tensor,
    scale: float,
    *,
    k_scale_cache: torch.Tensor | None = None,
    v_scale_cache: torch.Tensor | None = None,
    max_context_len: torch.Tensor | None = None,
    block_n: int = DEFAULT_PAGED_DECODE_BLOCK_N,
) -> torch.Tensor:
    """Single-query paged attention over (scaled-)FP8 or 16/32-bit KV pages."""

    if max_context_len is None:
        max_context_len = _no_context_bound(context_lens)
    scaled_kv = _validate_paged_decode_inputs(
        q, k_cache, v_cache, block_tables, context_lens, max_context_len,
        k_scale_cache=k_scale_cache, v_scale_cache=v_scale_cache, block_n=block_n,
    )
    return _launch_paged_decode_attention(
        q, k_cache, v_cache, block_tables, context_lens, scale, max_context_len,
        k_scale_cache=k_scale_cache, v_scale_cache=v_scale_cache, scaled_kv=scaled_kv,
    )


__all__ = [
    "DEFAULT_PAGED_DECODE_BLOCK_N",
    "HAS_HIP_KERNELS",
    "HAS_TRITON",
    "decode_workspace",
    "decode_workspace_bytes",
    "get_decode_overrides",
    "paged_decode_attention",
    "set_decode_overrides",
]


_PATH_CODES = {"auto": 0, "split": 1, "stream": 2}


def set_decode_overrides(path: str = "auto", split_tokens: int = 0, share: bool = True) -> None:
    """Force a decode kernel family for this process (tests, A/B runs).

    ``path``: "auto", "split" or "stream" (where the geometry allows it);
    ``split_tokens``: 0 for the automatic split-K size; ``share``: False treats
    every page as private (no device-side prefix-sharing analysis).  Results
    stay within the decode tolerance whatever is chosen.
    """

    if path not in _PATH_CODES:
        raise ValueError(f"path must be one of {sorted(_PATH_CODES)}, got {path!r}")
    _native.check(_native.lib().prism_paged_decode_set_overrides(_PATH_CODES[path], int(split_tokens), int(share)),
                  "set_decode_overrides")


def get_decode_overrides() -> tuple[str, int, bool]:
    import ctypes  # noqa: PLC0415

    out = (ctypes.c_int * 3)()
    _native.lib().prism_paged_decode_get_overrides(out)
    names = {v: k for k, v in _PATH_CODES.items()}
    return names[out[0]], int(out[1]), bool(out[2])
