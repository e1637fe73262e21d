"""Paged KV slot compaction primitive (MI355X HIP kernels).

Drop-in for prism_infer/ops/kv_compaction.py: same ``compact_kv_slots``
signature (:93-97) and validation messages (:115-141).  The op only moves
physical slots; it does not choose which tokens are kept and does not touch
page tables.  Semantics (reference :110-112): for every row of ``cache``
([kv, layers, slots, ...]), destination slot ``dst[i]`` receives the bytes
source slot ``src[i]`` held before the call -- all reads precede all writes,
so overlapping in-place plans are safe.  Payload and scale caches are moved
by separate calls, exactly as the reference's caller does.

The native side first detects on the device whether any destination aliases
another entry's source; only then does it stage through the workspace (two
passes), otherwise it moves each slot once.  Every dtype goes through the
same byte-moving kernels on the GPU.  A CPU cache is compacted with torch
index ops over a byte view of the cache (the reference uses index ops for CPU
and non-FP8 caches, :105-112).
"""

from __future__ import annotations

import math

import torch

from prism_infer import _native

HAS_HIP_KERNELS = _native.available()
HAS_TRITON = HAS_HIP_KERNELS  # the reference's "kernel available" flag name

SUPPORTED_COMPACTION_CACHE_RANKS = (4, 5)
SLOT_INDEX_TENSOR_RANK = 1


def _validate_compaction_inputs(cache, source_slots, destination_slots) -> None:
    if cache.ndim not in SUPPORTED_COMPACTION_CACHE_RANKS:
        raise ValueError(
            "cache must be [kv, layers, slots, kv_heads] or "
            "[kv, layers, slots, kv_heads, head_dim], "
            f"got {list(cache.shape)}"
        )
    if source_slots.ndim != SLOT_INDEX_TENSOR_RANK or destination_slots.ndim != SLOT_INDEX_TENSOR_RANK:
        raise ValueError("source/destination slots must be 1D")
    if source_slots.numel() == 0:
        raise ValueError("KV compaction requires at least one retained slot")
    if source_slots.shape != destination_slots.shape:
        raise ValueError(
            "source/destination slot shapes must match: "
            f"{list(source_slots.shape)} vs {list(destination_slots.shape)}"
        )
    if source_slots.dtype != torch.long or destination_slots.dtype != torch.long:
        raise ValueError("source/destination slots must use torch.long")
    if source_slots.device != cache.device or destination_slots.device != cache.device:
        raise RuntimeError("cache and slot tensors must share one device")


def _validate_device_layout(cache, source_slots, destination_slots) -> None:
    if not HAS_HIP_KERNELS:
        _native.lib()  # raises with the reason
    if not cache.is_contiguous():
        raise RuntimeError("MI355X KV compaction requires contiguous cache")
    if not source_slots.is_contiguous() or not destination_slots.is_contiguous():
        raise RuntimeError("MI355X KV compaction requires contiguous slot tensors")


def _compact_cpu(cache: torch.Tensor, source_slots: torch.Tensor, destination_slots: torch.Tensor) -> None:
    """Host caches: gather every source slot, then scatter to the destinations.

    The cache is seen as [rows, slots, bytes] so every dtype (FP8 payload,
    fp32 scales, NaN bit patterns) moves exactly.  The gather completes before
    the scatter starts, so overlapping plans read what the sources held before
    the call.  Out-of-range slots raise from index_select, as the reference's
    index ops do."""

    if not cache.is_contiguous():
        raise RuntimeError("KV compaction requires a contiguous cache")
    rows = cache.shape[0] * cache.shape[1]
    as_bytes = cache.view(torch.uint8).view(rows, cache.shape[2], -1)
    gathered = as_bytes.index_select(1, source_slots)
    as_bytes.index_copy_(1, destination_slots, gathered)


def compaction_workspace_bytes(cache: torch.Tensor, retained: int) -> int:
    rows = cache.shape[0] * cache.shape[1]
    vec_bytes = math.prod(cache.shape[3:]) * cache.element_size()
    return int(_native.lib().prism_compact_slots_workspace_bytes(rows, cache.shape[2], vec_bytes, retained))


def compact_kv_slots(
    cache: torch.Tensor,
    source_slots: torch.Tensor,
    destination_slots: torch.Tensor,
) -> None:
    """Move retained slots to their destination slots, in place, reads before writes.

    cache: payload [kv, layers, slots, kv_heads, head_dim] or token-head
        scales [kv, layers, slots, kv_heads]
    source_slots/destination_slots: int64 [retained_tokens]
    """

    _validate_compaction_inputs(cache, source_slots, destination_slots)
    if not cache.is_cuda:
        _compact_cpu(cache, source_slots, destination_slots)
        return
    _validate_device_layout(cache, source_slots, destination_slots)
    rows = cache.shape[0] * cache.shape[1]
    num_slots = cache.shape[2]
    vec_bytes = math.prod(cache.shape[3:]) * cache.element_size()
    retained = source_slots.numel()
    lib = _native.device_lib(cache.device)
    ws_bytes = compaction_workspace_bytes(cache, retained)
    workspace = torch.empty(ws_bytes, dtype=torch.uint8, device=cache.device)
    with torch.cuda.device(cache.device):
        status = lib.prism_compact_slots(
            cache.data_ptr(), rows, num_slots, vec_bytes,
            source_slots.data_ptr(), destination_slots.data_ptr(), retained,
            workspace.data_ptr(), ws_bytes, _native.stream_handle(cache.device),
        )
    _native.check(status, "compact_kv_slots")


__all__ = ["HAS_HIP_KERNELS", "HAS_TRITON", "compact_kv_slots", "compaction_workspace_bytes"]
