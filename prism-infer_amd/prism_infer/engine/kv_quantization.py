"""Scaled-FP8 KV format: the numeric constants and the byte arithmetic of pages.

The public names and values are the ones callers of
prism_infer/engine/kv_quantization.py (:9-13, :33-107) import: an E4M3FN payload
whose largest finite magnitude is 448, one fp32 scale per (token, kv head)
equal to ``max(amax|row| / 448, 1e-6)``, and a scale tensor whose shape is the
payload's without its trailing ``head_dim`` axis.

Byte accounting, for one layer and one token:

    payload = 2 (K and V) * kv_heads * head_dim * itemsize(payload dtype)
    scales  = 2 (K and V) * kv_heads * 4            (only for scaled caches)

which for 8 kv heads of 128 dims in E4M3FN is 2048 + 64 = 2112 bytes. A block
multiplies that by ``page_size * num_layers``.
"""

from __future__ import annotations

import math
from typing import NamedTuple, Optional, Sequence

import torch

# E4M3FN has no infinities; its largest finite code 0x7E is 1.75 * 2**8.
FP8_E4M3FN_MAX = 448.0
FP8_E4M3FN_MIN = -448.0
# Scales never fall below this, so an all-zero row still divides safely.
PER_TOKEN_HEAD_SCALE_FLOOR = 1.0e-6
KV_SCALE_DTYPE = torch.float32
# K and V are stored as two independent tensors of identical layout.
KV_COMPONENT_COUNT = 2

_SCALE_ITEMSIZE = 4  # bytes of one KV_SCALE_DTYPE element


class KVStorageBytes(NamedTuple):
    """Bytes held by KV storage, split into quantized payload and fp32 scales."""

    payload: int
    scales: int

    @property
    def total(self) -> int:
        return self.payload + self.scales


def _is_count(x) -> bool:
    # bool is an int subclass; a True/False dimension is a caller mistake.
    return type(x) is int or (isinstance(x, int) and not isinstance(x, bool))


def _require_counts(named: dict) -> None:
    for key in named:
        v = named[key]
        if not _is_count(v) or v < 1:
            raise ValueError(f"{key}: expected an int >= 1, received {v!r}")


def scale_cache_shape(payload_shape: Sequence[int]) -> tuple[int, ...]:
    """Shape of the fp32 scale tensor that goes with a KV payload tensor.

    A payload is either flat ``[slots, kv_heads, head_dim]`` or paged
    ``[blocks, page_size, kv_heads, head_dim]``; one scale covers one head_dim
    row, so the answer drops the last axis.
    """

    dims = tuple(payload_shape)
    if not 3 <= len(dims) <= 4:
        raise ValueError(
            f"scale_cache_shape: payload rank {len(dims)} ({list(dims)}) is neither the "
            "flat [slots, kv_heads, head_dim] nor the paged "
            "[blocks, page_size, kv_heads, head_dim] layout"
        )
    bad = [d for d in dims if not _is_count(d) or d < 1]
    if bad:
        raise ValueError(f"scale_cache_shape: every payload dimension must be an int >= 1, got {list(dims)}")
    return dims[:-1]


def kv_token_layer_bytes(*, num_kv_heads: int, head_dim: int, token_head_scales: bool = True,
                         payload_itemsize: int = 1) -> int:
    """Bytes that one token occupies in one layer: K and V rows plus their scales."""

    row = num_kv_heads * head_dim * payload_itemsize
    if token_head_scales:
        row += num_kv_heads * _SCALE_ITEMSIZE
    return KV_COMPONENT_COUNT * row


def kv_block_storage_bytes(
    *,
    num_layers: int,
    page_size: int,
    num_kv_heads: int,
    head_dim: int,
    payload_dtype: torch.dtype,
    token_head_scales: bool,
) -> KVStorageBytes:
    """Bytes that one physical page (block) owns summed over every layer.

    A 36-layer page of 256 tokens, 8 kv heads and 128 dims is 18,874,368 B of
    E4M3FN payload and 589,824 B of scales; the same page in bf16 without
    scales is 37,748,736 B (ratio 0.515625).
    """

    _require_counts({"num_layers": num_layers, "page_size": page_size,
                     "num_kv_heads": num_kv_heads, "head_dim": head_dim})
    if not isinstance(payload_dtype, torch.dtype):
        raise TypeError(f"payload_dtype: expected a torch.dtype, received {payload_dtype!r}")
    if not isinstance(token_head_scales, bool):
        raise TypeError(f"token_head_scales: expected a bool, received {token_head_scales!r}")
    rows = KV_COMPONENT_COUNT * num_layers * page_size * num_kv_heads
    return KVStorageBytes(
        payload=rows * head_dim * payload_dtype.itemsize,
        scales=rows * _SCALE_ITEMSIZE if token_head_scales else 0,
    )


def tensor_storage_bytes(tensor: Optional[torch.Tensor]) -> int:
    """Bytes of the elements a tensor views (0 for an absent tensor).

    Counts ``numel * itemsize`` of the view, not the size of the storage
    behind it.
    """

    if tensor is None:
        return 0
    if not isinstance(tensor, torch.Tensor):
        raise TypeError(f"tensor_storage_bytes: expected a torch.Tensor or None, "
                        f"received {type(tensor).__name__}")
    return math.prod(tensor.shape) * tensor.dtype.itemsize


def kv_cache_storage_bytes(payload_cache: torch.Tensor,
                           scale_cache: Optional[torch.Tensor]) -> KVStorageBytes:
    """Payload and scale bytes of an allocated cache (no scale tensor counts 0)."""

    if not isinstance(payload_cache, torch.Tensor):
        raise TypeError(f"kv_cache_storage_bytes: payload_cache must be a torch.Tensor, "
                        f"received {type(payload_cache).__name__}")
    return KVStorageBytes(tensor_storage_bytes(payload_cache), tensor_storage_bytes(scale_cache))


__all__ = [
    "FP8_E4M3FN_MAX",
    "FP8_E4M3FN_MIN",
    "KV_COMPONENT_COUNT",
    "KV_SCALE_DTYPE",
    "KVStorageBytes",
    "PER_TOKEN_HEAD_SCALE_FLOOR",
    "kv_block_storage_bytes",
    "kv_cache_storage_bytes",
    "kv_token_layer_bytes",
    "scale_cache_shape",
    "tensor_storage_bytes",
]
