"""Page-level KV movement on the paged-cache layout (payload and scales together).

Host-side counterparts of the block operations of the reference's model
runner (prism_infer/engine/model_runner.py:908-1031), taking the caches as
arguments instead of reading them from a runner:

* :func:`copy_kv_blocks` -- copy-on-write of whole blocks
  (``ModelRunner.copy_kv_blocks``, :908-915);
* :func:`copy_kv_block_prefixes` -- the first ``num_rows`` rows of shared
  compact-prefix tail blocks (``copy_kv_block_prefixes``, :917-937);
* :func:`swap_blocks` -- whole blocks between the GPU cache and a pinned CPU
  cache (``swap_blocks``, :1001-1031).

Payload caches are ``[2, layers, blocks, block_size, kv_heads, head_dim]``;
token-head scale caches ``[2, layers, blocks, block_size, kv_heads]`` fp32.

On the device, a batch of block or row moves is one launch of the slot
compaction kernels (``compact_kv_slots``) per cache instead of one torch copy
per block: whole blocks move as slots of ``block_size * kv_heads * head_dim``
bytes, prefix rows as token slots.  Semantics differ from the reference's
in-order Python loop only for chained entries (a destination that is the
source of a later entry), which copy-on-write never produces: here all reads
precede all writes.  Swaps issue one strided DMA copy per block and cache
(``prism_copy_blocks``) and, like the reference, synchronise at the end.
"""

from __future__ import annotations

import math

import torch

from prism_infer import _native
from prism_infer.ops.kv_compaction import compact_kv_slots

PAYLOAD_CACHE_RANK = 6
SCALE_CACHE_RANK = 5


def _check_pair(kv_cache: torch.Tensor, scale_cache: torch.Tensor | None) -> None:
    if kv_cache.ndim != PAYLOAD_CACHE_RANK:
        raise ValueError(
            "KV cache must be [2, layers, blocks, block_size, kv_heads, head_dim], "
            f"got {list(kv_cache.shape)}"
        )
    if scale_cache is not None and tuple(scale_cache.shape) != tuple(kv_cache.shape[:-1]):
        raise ValueError(
            "KV scale cache shape must equal the payload shape without head_dim: "
            f"payload={list(kv_cache.shape)}, scales={list(scale_cache.shape)}"
        )


def _ids(values, device) -> torch.Tensor:
    return torch.tensor(list(values), dtype=torch.long, device=device)


def copy_kv_blocks(kv_cache: torch.Tensor, cow_pairs, scale_cache: torch.Tensor | None = None) -> None:
    """Copy complete source KV blocks into private destination blocks (payload and scales)."""

    _check_pair(kv_cache, scale_cache)
    pairs = [(int(s), int(d)) for s, d in cow_pairs]
    if not pairs:
        return
    num_blocks = kv_cache.shape[2]
    for s, d in pairs:
        if not (0 <= s < num_blocks and 0 <= d < num_blocks):
            raise ValueError(f"KV block ids must be in [0, {num_blocks}), got ({s}, {d})")
    src = _ids((s for s, _ in pairs), kv_cache.device)
    dst = _ids((d for _, d in pairs), kv_cache.device)
    kv, layers = kv_cache.shape[:2]
    compact_kv_slots(kv_cache.view(kv, layers, num_blocks, -1), src, dst)
    if scale_cache is not None:
        compact_kv_slots(scale_cache.view(kv, layers, num_blocks, -1), src, dst)


def copy_kv_block_prefixes(kv_cache: torch.Tensor, copies, scale_cache: torch.Tensor | None = None) -> None:
    """Copy only the first ``num_rows`` rows of each (source block, destination block)."""

    _check_pair(kv_cache, scale_cache)
    entries = [(int(s), int(d), int(n)) for s, d, n in copies]
    block_size = kv_cache.shape[3]
    num_blocks = kv_cache.shape[2]
    src_slots: list[int] = []
    dst_slots: list[int] = []
    for s, d, n in entries:
        if n <= 0 or n > block_size:
            raise ValueError(f"KV block-prefix rows must be in [1, {block_size}], got {n}")
        if not (0 <= s < num_blocks and 0 <= d < num_blocks):
            raise ValueError(f"KV block ids must be in [0, {num_blocks}), got ({s}, {d})")
        src_slots.extend(range(s * block_size, s * block_size + n))
        dst_slots.extend(range(d * block_size, d * block_size + n))
    if not src_slots:
        return
    src = _ids(src_slots, kv_cache.device)
    dst = _ids(dst_slots, kv_cache.device)
    kv, layers = kv_cache.shape[:2]
    slots = num_blocks * block_size
    compact_kv_slots(kv_cache.view(kv, layers, slots, *kv_cache.shape[4:]), src, dst)
    if scale_cache is not None:
        compact_kv_slots(scale_cache.view(kv, layers, slots, scale_cache.shape[4]), src, dst)


def _copy_blocks(dst: torch.Tensor, src: torch.Tensor, dst_ids: list[int], src_ids: list[int], stream) -> None:
    rows = src.shape[0] * src.shape[1]
    block_bytes = math.prod(src.shape[3:]) * src.element_size()
    status = _native.device_lib(dst.device).prism_copy_blocks(
        dst.data_ptr(), src.data_ptr(), rows, dst.shape[2] * block_bytes, src.shape[2] * block_bytes,
        block_bytes, dst.shape[2], src.shape[2], _native.int64s(*dst_ids), _native.int64s(*src_ids),
        len(dst_ids), stream,
    )
    _native.check(status, "swap_blocks")


def swap_blocks(gpu_cache: torch.Tensor, cpu_cache: torch.Tensor | None, swap_map, direction: str, *,
                gpu_scale_cache: torch.Tensor | None = None, cpu_scale_cache: torch.Tensor | None = None) -> None:
    """Copy KV blocks between GPU and pinned CPU storage in ``direction`` ("out": GPU to CPU)."""

    pairs = [(int(s), int(d)) for s, d in swap_map]
    if not pairs:
        return
    if direction not in ("out", "in"):
        raise ValueError(f"swap direction must be 'out' or 'in', got {direction!r}")
    if cpu_cache is None:
        raise RuntimeError("KV swap requested without an allocated CPU payload cache")
    if (gpu_scale_cache is None) != (cpu_scale_cache is None):
        raise RuntimeError("GPU/CPU scale caches must either both exist or both be absent")
    _check_pair(gpu_cache, gpu_scale_cache)
    _check_pair(cpu_cache, cpu_scale_cache)
    if not gpu_cache.is_cuda or cpu_cache.is_cuda:
        raise RuntimeError("swap_blocks moves between a GPU cache and a CPU cache")
    caches = [(gpu_cache, cpu_cache)]
    if gpu_scale_cache is not None:
        caches.append((gpu_scale_cache, cpu_scale_cache))
    for g, c in caches:
        if g.dtype != c.dtype or tuple(g.shape[:2]) != tuple(c.shape[:2]) or tuple(g.shape[3:]) != tuple(c.shape[3:]):
            raise ValueError(f"GPU/CPU caches differ in dtype or block layout: {list(g.shape)} vs {list(c.shape)}")
        if not g.is_contiguous() or not c.is_contiguous():
            raise RuntimeError("swap_blocks requires contiguous caches")
        if not c.is_pinned():
            raise RuntimeError("swap_blocks requires a pinned (page-locked) CPU cache")
    src_ids = [s for s, _ in pairs]
    dst_ids = [d for _, d in pairs]
    with torch.cuda.device(gpu_cache.device):
        stream = _native.stream_handle(gpu_cache.device)
        for g, c in caches:
            if direction == "out":
                _copy_blocks(c, g, dst_ids, src_ids, stream)
            else:
                _copy_blocks(g, c, dst_ids, src_ids, stream)
        torch.cuda.current_stream(gpu_cache.device).synchronize()


__all__ = ["copy_kv_block_prefixes", "copy_kv_blocks", "swap_blocks"]
