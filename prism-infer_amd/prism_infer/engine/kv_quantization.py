"""Format constants and byte accounting for scaled-FP8 KV storage.

Restates prism_infer/engine/kv_quantization.py:9-80 (same names and values):
E4M3FN payload with a per-token, per-KV-head fp32 scale
``max(amax|x| / 448, 1e-6)``; the scale cache shape is the payload shape
without ``head_dim``.
"""

from __future__ import annotations

from typing import NamedTuple

import torch

FP8_E4M3FN_MAX = 448.0
FP8_E4M3FN_MIN = -FP8_E4M3FN_MAX
PER_TOKEN_HEAD_SCALE_FLOOR = 1.0e-6
KV_SCALE_DTYPE = torch.float32
KV_COMPONENT_COUNT = 2  # independent K and V storage


class KVStorageBytes(NamedTuple):
    """Physical bytes owned by one paged KV block across all layers."""

    payload: int
    scales: int

    @property
    def total(self) -> int:
        return self.payload + self.scales


def _positive_dimension(value: int, *, name: str) -> int:
    if isinstance(value, bool) or not isinstance(value, int) or value <= 0:
        raise ValueError(f"{name} must be a positive integer, got {value!r}")
    return value


def scale_cache_shape(payload_shape) -> tuple[int, ...]:
    """Return the token-head scale shape for one paged KV payload tensor."""

    shape = tuple(payload_shape)
    if len(shape) not in (3, 4):
        raise ValueError(
            "KV payload must be [slots, heads, dim] or "
            f"[blocks, page, heads, dim], got {list(shape)}"
        )
    if any(isinstance(d, bool) or not isinstance(d, int) or d <= 0 for d in shape):
        raise ValueError(f"KV payload dimensions must be positive, got {list(shape)}")
    return shape[:-1]


def kv_block_storage_bytes(
    *,
    num_layers: int,
    page_size: int,
    num_kv_heads: int,
    head_dim: int,
    payload_dtype: torch.dtype,
    token_head_scales: bool,
) -> KVStorageBytes:
    """Return payload/scale bytes for one physical block across all layers."""

    for name, value in (
        ("num_layers", num_layers),
        ("page_size", page_size),
        ("num_kv_heads", num_kv_heads),
        ("head_dim", head_dim),
    ):
        _positive_dimension(value, name=name)
    if not isinstance(payload_dtype, torch.dtype):
        raise TypeError(f"payload_dtype must be torch.dtype, got {payload_dtype!r}")
    if not isinstance(token_head_scales, bool):
        raise TypeError("token_head_scales must be bool")
    elements = KV_COMPONENT_COUNT * num_layers * page_size * num_kv_heads
    payload = elements * head_dim * torch.empty((), dtype=payload_dtype).element_size()
    scales = elements * torch.empty((), dtype=KV_SCALE_DTYPE).element_size() if token_head_scales else 0
    return KVStorageBytes(payload=payload, scales=scales)


def kv_token_layer_bytes(*, num_kv_heads: int, head_dim: int, token_head_scales: bool = True) -> int:
    """Bytes one token occupies in one layer (K and V payload plus scales)."""

    per = num_kv_heads * head_dim + (num_kv_heads * 4 if token_head_scales else 0)
    return KV_COMPONENT_COUNT * per


__all__ = [
    "FP8_E4M3FN_MAX",
    "FP8_E4M3FN_MIN",
    "KV_COMPONENT_COUNT",
    "KV_SCALE_DTYPE",
    "KVStorageBytes",
    "PER_TOKEN_HEAD_SCALE_FLOOR",
    "kv_block_storage_bytes",
    "kv_token_layer_bytes",
    "scale_cache_shape",
]
