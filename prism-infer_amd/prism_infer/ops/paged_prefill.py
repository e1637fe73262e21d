"""Paged prefill attention over scaled-FP8 pages on MI355X (HIP kernel).

Drop-in for ``paged_prefill_attention_reference``
(prism_infer/ops/paged_attention_reference.py:185-246), which
``Attention._forward_prefill_paged`` calls for chunked and prefix-hit
prefill (prism_infer/layers/attention.py:448-459):

- q: [total_q, num_heads, head_dim] packed by ``context.cu_seqlens_q``;
- k_cache/v_cache: [num_blocks, block_size, num_kv_heads, head_dim] holding
  each sequence's whole history, the chunk's own K/V included;
- ``context.context_lens[i]`` is sequence i's history length, so query token
  j of its chunk sits at position ``context_len - query_len + j`` and attends
  causally to keys ``0 .. context_len - query_len + j``;
- the result is the per-sequence outputs concatenated, in q's dtype.

The reference loops over sequences on the host (one ``.item()`` sync per
sequence) and gathers pages into dense tensors.  Here one kernel launch
reads the pages in place, with the metadata on the device, and the host
synchronises once at the end to raise the reference's errors: invalid
lengths, a block id past the cache, or a block table too short for the
context.  Under graph capture that check is skipped (invalid sequences then
leave their rows unspecified).

Differences a caller can see: K/V are dequantised in fp32 (payload times
scale applied to the fp32 scores and to the softmax weights, as the decode
kernels do) instead of in q's dtype, so results differ from the reference
by bf16 rounding of the dequantised cache (the GPU tests bound it).  The
kernel covers FP8 E4M3FN caches (scaled or unit-scale), head_dim 128, page
sizes that are multiples of 16, GQA groups of 1, 2, 4 or 8 and bf16/fp16
queries; other cases raise ``RuntimeError`` (no CPU fallback).
"""

from __future__ import annotations

import torch

from prism_infer import _native

HAS_HIP_KERNELS = _native.available()

MINIMUM_PAGED_CACHE_RANK = 3
PREFILL_HEAD_DIM = 128
_STATUS_OK = 2**31 - 1


def _validate_caches(k_cache, v_cache, k_scale_cache, v_scale_cache) -> bool:
    """The reference's gather and dequantisation contract (:31-38, :108-119)."""

    if k_cache.shape != v_cache.shape:
        raise ValueError("K/V cache shapes must match for paged gather")
    if k_cache.ndim < MINIMUM_PAGED_CACHE_RANK:
        raise ValueError(
            "paged K/V caches must contain block and page dimensions, "
            f"got shape={list(k_cache.shape)}"
        )
    if (k_scale_cache is None) != (v_scale_cache is None):
        raise ValueError("k_scale_cache and v_scale_cache must be provided together")
    if k_scale_cache is None:
        return False
    if k_cache.dtype != torch.float8_e4m3fn:
        raise ValueError("token-head scales require an FP8 payload tensor")
    for scales in (k_scale_cache, v_scale_cache):
        if tuple(scales.shape) != tuple(k_cache.shape[:-1]):
            raise ValueError(
                "scale shape must equal payload shape without head_dim: "
                f"payload={list(k_cache.shape)}, scales={list(scales.shape)}"
            )
        if scales.dtype != torch.float32:
            raise ValueError(f"token-head scales must use torch.float32, got {scales.dtype}")
    return True


def _validate_heads(num_heads: int, num_kv_heads: int) -> None:
    """``expand_gqa_kv``'s check (:133-139)."""

    if num_heads != num_kv_heads and (num_kv_heads <= 0 or num_heads % num_kv_heads):
        raise ValueError(
            "num_heads must be divisible by num_kv_heads, "
            f"got num_heads={num_heads}, num_kv_heads={num_kv_heads}"
        )


def _int32_device(t: torch.Tensor, device: torch.device) -> torch.Tensor:
    if t.device != device:
        raise RuntimeError(f"paged prefill metadata must be on {device}, got {t.device}")
    return t if t.dtype == torch.int32 else t.to(torch.int32)


def _raise_sequence_error(seq: int, cu_seqlens_q, context_lens, block_tables, num_blocks: int,
                          page_size: int) -> None:
    """Re-derive and raise the reference's error for sequence ``seq`` (:207-214, :46-62)."""

    query_len = int(cu_seqlens_q[seq + 1]) - int(cu_seqlens_q[seq])
    context_len = int(context_lens[seq])
    if query_len <= 0 or context_len < query_len:
        raise RuntimeError(f"invalid paged prefill lengths: query={query_len} context={context_len}")
    remaining = context_len
    for block_id in block_tables[seq].tolist():
        if remaining <= 0 or block_id < 0:
            break
        if block_id >= num_blocks:
            raise RuntimeError(
                "paged KV block id exceeds cache capacity: "
                f"block_id={block_id}, num_blocks={num_blocks}"
            )
        remaining -= min(page_size, remaining)
    raise RuntimeError(
        "invalid block table for paged KV reference: "
        f"context_len={context_len}, remaining={remaining}"
    )


def _launch_paged_prefill(q, k_cache, v_cache, context, *, num_heads, num_kv_heads, scale, k_scale_cache=None,
                          v_scale_cache=None):
    """Validate and enqueue the kernel; returns (out, status, cu_seqlens_q, batch) without synchronising."""

    if context.block_tables is None or context.context_lens is None or context.cu_seqlens_q is None:
        raise RuntimeError("paged prefill requires block_tables/context_lens/cu_seqlens_q")
    scaled = _validate_caches(k_cache, v_cache, k_scale_cache, v_scale_cache)
    _validate_heads(num_heads, num_kv_heads)
    if q.ndim != 3 or q.shape[1] != num_heads:
        raise ValueError(f"q must be [tokens, num_heads={num_heads}, head_dim], got {list(q.shape)}")
    if k_cache.ndim != 4 or k_cache.shape[2] != num_kv_heads or k_cache.shape[3] != q.shape[2]:
        raise ValueError(
            "K/V caches must be [num_blocks, block_size, num_kv_heads, head_dim] matching q, "
            f"got {list(k_cache.shape)}"
        )
    _native.lib()  # raises with the reason the library is unavailable
    tensors = [q, k_cache, v_cache] + ([k_scale_cache, v_scale_cache] if scaled else [])
    if not all(t.is_cuda for t in tensors) or any(t.device != q.device for t in tensors):
        raise RuntimeError("paged_prefill_attention runs on the GPU: q, caches and scales must share one CUDA device")
    lib = _native.device_lib(q.device)
    if k_cache.dtype != torch.float8_e4m3fn:
        raise RuntimeError(f"the HIP paged prefill kernel reads FP8 E4M3FN caches, got {k_cache.dtype}")
    if q.dtype not in (torch.bfloat16, torch.float16):
        raise RuntimeError(f"the HIP paged prefill kernel takes bf16 or float16 queries, got {q.dtype}")
    if q.shape[2] != PREFILL_HEAD_DIM:
        raise RuntimeError(f"the HIP paged prefill kernel covers head_dim {PREFILL_HEAD_DIM}, got {q.shape[2]}")

    device = q.device
    context_lens = _int32_device(context.context_lens, device)
    cu_seqlens_q = _int32_device(context.cu_seqlens_q, device)
    block_tables = _int32_device(context.block_tables, device)
    if block_tables.ndim != 2:
        raise ValueError(f"block_tables must be two-dimensional, got {list(block_tables.shape)}")
    batch = context_lens.numel()
    if cu_seqlens_q.numel() < batch + 1 or block_tables.shape[0] < batch:
        raise ValueError(
            f"cu_seqlens_q needs {batch + 1} entries and block_tables {batch} rows, "
            f"got {cu_seqlens_q.numel()} and {block_tables.shape[0]}"
        )
    if q.stride(2) != 1:
        q = q.contiguous()
    out = torch.empty(q.shape, dtype=q.dtype, device=device)
    status = torch.full((1,), _STATUS_OK, dtype=torch.int32, device=device)
    zero3 = _native.int64s(0, 0, 0)
    with torch.cuda.device(device):
        rc = lib.prism_paged_prefill(
            q.data_ptr(), _native.dtype_code(q.dtype), _native.strides(q),
            k_cache.data_ptr(), v_cache.data_ptr(), _native.dtype_code(k_cache.dtype),
            _native.strides(k_cache), _native.strides(v_cache),
            k_scale_cache.data_ptr() if scaled else None, v_scale_cache.data_ptr() if scaled else None,
            _native.strides(k_scale_cache) if scaled else zero3,
            _native.strides(v_scale_cache) if scaled else zero3,
            block_tables.data_ptr(), _native.strides(block_tables),
            context_lens.data_ptr(), cu_seqlens_q.data_ptr(),
            out.data_ptr(), _native.strides(out),
            batch, q.shape[0], num_heads, num_kv_heads, q.shape[2], k_cache.shape[1], k_cache.shape[0],
            block_tables.shape[1], float(scale), status.data_ptr(), _native.stream_handle(device),
        )
    _native.check(rc, "paged_prefill_attention")
    return out, status, (context_lens, cu_seqlens_q, block_tables), batch


def paged_prefill_attention(
    q: torch.Tensor,
    k_cache: torch.Tensor,
    v_cache: torch.Tensor,
    context,
    *,
    num_heads: int,
    num_kv_heads: int,
    scale: float,
    k_scale_cache: torch.Tensor | None = None,
    v_scale_cache: torch.Tensor | None = None,
) -> torch.Tensor:
    """Run chunked/prefix-hit prefill against already-written paged KV.

    ``context`` is any object with ``block_tables``, ``context_lens`` and
    ``cu_seqlens_q`` tensors (the reference's ``Context``).
    """

    out, status, (context_lens, cu_seqlens_q, block_tables), batch = _launch_paged_prefill(
        q, k_cache, v_cache, context, num_heads=num_heads, num_kv_heads=num_kv_heads, scale=scale,
        k_scale_cache=k_scale_cache, v_scale_cache=v_scale_cache)
    if batch == 0:
        return out[:0]
    if torch.cuda.is_current_stream_capturing():
        return out
    # one synchronisation: the status word and the packed rows' extent
    first_bad, row0, row1 = torch.cat([status, cu_seqlens_q[0:1], cu_seqlens_q[batch:batch + 1]]).tolist()
    if first_bad != _STATUS_OK:
        _raise_sequence_error(first_bad, cu_seqlens_q.cpu(), context_lens.cpu(), block_tables.cpu(),
                              k_cache.shape[0], k_cache.shape[1])
    return out[row0:row1]


__all__ = ["HAS_HIP_KERNELS", "paged_prefill_attention"]
